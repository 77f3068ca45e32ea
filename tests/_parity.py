"""Step-by-step parity check of a greedy token stream against the oracle
(shared by the GPU model tests; not a test module)."""

from __future__ import annotations

import torch


def check_steps(oracle, tokens, ref, gpu_hidden, ref_hidden, bounds):
    """The GPU's hidden state within ``bounds`` = (mean, per-step) relative
    error of the oracle's; at every step the tokens equal, or the flip
    explained: the oracle's logit gap between the two tokens is no larger than
    the measured GPU-vs-oracle difference of those two logits plus one bf16
    ulp."""
    mean_bound, step_bound = bounds
    emb = oracle.w["embed"].double()
    bad, errs = [], []
    for step, (tok, (rt, margin)) in enumerate(zip(tokens, ref)):
        hg, ho = gpu_hidden[step].double(), ref_hidden[step].double()
        err = float((hg - ho).norm() / ho.norm())
        errs.append(err)
        if err > step_bound:
            bad.append((step, "hidden", err))
        if tok != rt:
            rows = emb[[tok, rt]]
            lg = (hg @ rows.t()).float().to(torch.bfloat16).double()[0]
            lo = (ho @ rows.t()).float().to(torch.bfloat16).double()[0]
            gap = float(lo[1] - lo[0])
            noise = float((lg - lo).abs().sum())
            ulp = 2.0 ** (torch.floor(torch.log2(lo.abs().max())).item() - 7)
            print(f"step {step}: gpu {tok} oracle {rt} oracle margin {margin:.4f} gap {gap:.4f} "
                  f"logit noise {noise:.4f} hidden err {err:.2e}", flush=True)
            if gap > noise + ulp:
                bad.append((step, tok, rt, gap, noise))
    same = sum(t == r for t, (r, _) in zip(tokens, ref))
    mean = sum(errs) / len(errs)
    print(f"{len(tokens)} steps, {same} identical tokens, hidden rel err max {max(errs):.2e} "
          f"mean {mean:.2e}", flush=True)
    assert not bad, f"steps outside the parity bound: {bad}"
    assert mean <= mean_bound, f"mean hidden error {mean:.3e} above {mean_bound}"




def eager_greedy(state, cfg, prompt, steps: int):
    """Greedy tokens of Transformers' own eager Qwen3.5 forward on the CPU
    (bf16, DynamicCache; the path the reference runs for CPU tensors,
    integration.py:51-52) on the same weights: ``steps`` tokens (the prefill's
    token first) and, per token, the top-2 logit margin."""
    from transformers.cache_utils import DynamicCache
    from transformers.models.qwen3_5.modeling_qwen3_5 import Qwen3_5ForCausalLM

    old = torch.get_default_dtype()
    torch.set_default_dtype(torch.bfloat16)
    try:
        with torch.device("meta"):
            model = Qwen3_5ForCausalLM(cfg)
    finally:
        torch.set_default_dtype(old)
    model.load_state_dict(state, assign=True, strict=False)
    model.tie_weights()
    rot = model.model.rotary_emb
    inv_freq, _ = rot.compute_default_rope_parameters(cfg, "cpu")
    rot.inv_freq = inv_freq
    rot.original_inv_freq = inv_freq
    model.eval()
    tokens, margins = [], []
    with torch.inference_mode():
        cache = DynamicCache(config=cfg)
        ids = prompt
        for _ in range(steps):
            logits = model(input_ids=ids, past_key_values=cache, use_cache=True,
                           logits_to_keep=1).logits[0, -1].float()
            top = torch.topk(logits, 2)
            tokens.append(int(top.indices[0]))
            margins.append(float(top.values[0] - top.values[1]))
            ids = torch.tensor([[tokens[-1]]])
    return tokens, margins


def report_eager_agreement(gpu_tokens, eager_tokens, eager_margins) -> int | None:
    """Print how many greedy tokens the GPU and Transformers eager share and
    the first divergence with eager's top-2 margin there; returns its step."""
    same = sum(a == b for a, b in zip(gpu_tokens, eager_tokens))
    first = next((i for i, (a, b) in enumerate(zip(gpu_tokens, eager_tokens)) if a != b), None)
    prefix = first if first is not None else len(gpu_tokens)
    msg = (f"GPU vs Transformers eager (CPU): {same}/{len(gpu_tokens)} identical tokens, "
           f"identical prefix {prefix}")
    if first is not None:
        msg += (f"; first divergence at step {first}: gpu {gpu_tokens[first]} eager "
                f"{eager_tokens[first]}, eager top-2 margin {eager_margins[first]:.4f}")
    print(msg, flush=True)
    return first
