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


