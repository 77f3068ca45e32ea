"""End-to-end parity of the integrated MI355X path against the CPU oracle decoder.

A Transformers Qwen3.5 model (synthetic seeded weights) is patched with
``apply_fusions`` and run on the GPU: prefill, then greedy decode through the
captured graph. The oracle decoder gets the identical weights on the CPU and
is teacher-forced with the GPU's tokens, so every step compares the two paths
on the same history: the final hidden states must agree to HIDDEN_BOUNDS (set from the measured
summation-order noise floor of the oracle itself), and a
token may differ only where the oracle's logit gap between the two tokens is
within the measured GPU-vs-oracle difference of those two logits (random-init
logits often tie to the bf16 ulp). Every flip is printed with its numbers.
"""

from __future__ import annotations

import pytest
import torch

from oracle.model import OracleDecoder
from ppu_amd import synth
from tests._parity import check_steps, eager_greedy, report_eager_agreement

pytestmark = pytest.mark.gpu

# Relative L2 error between the GPU's and the oracle's final hidden state at a
# teacher-forced step: (bound on the mean over the steps, bound on every
# step), set from the oracle's own noise floor. Two CPU oracle variants that
# differ only in the fp32 summation order of their linear layers diverge by
# 1.1 % (4 layers) and 2.4 % (12 layers) on these random-init weights
# (tests/test_oracle_model.py). On the 24-layer 2B shape a one-ulp change of the
# RMSNorm variances moves the hidden state, over 64 steps, by 2.3 % mean /
# 2.9 % max in bf16 and 8.2 % mean / 10 % max in A8W8, where the per-token int8
# quantisation turns ulp changes into whole int8 steps (the perturbation of
# tests/test_oracle_model.py::_variance_order_noise run once at the 2B shape).
# The GPU perturbs every reduction, not one: mean bounds are about twice the
# floor mean, per-step bounds about 2.4x (bf16) and 3x (A8W8) the floor max.
# The 2B bounds are about 1.5x what the GPU path measures (bf16 mean 0.032 /
# max 0.044, A8W8 0.083 / 0.094 over the 64 steps), so a data-flow change in
# a late decode step that moves the state by a few percent fails them.
HIDDEN_BOUNDS = {"tiny": (0.03, 0.03), "2b": (0.045, 0.06), "2b-a8w8": (0.12, 0.14)}

# Relative L2 error of one layer's outputs and written states, the layer run
# from the oracle's own input and state (test_2b_layerwise_teacher_forced).
LAYER_BOUND = {"bf16": 0.01, "a8w8": 0.01}
# The late decode step the layer-wise test also checks (the states then hold
# 63 decode tokens on top of the 1024-token prefill).
LATE = 64


def _build(cfg, gpu, fusion):
    from ppu_amd.integration import apply_fusions

    model = synth.build_model(cfg, device=gpu)
    state = {k: v.detach().cpu() for k, v in model.state_dict().items()}
    stats = apply_fusions(model, fusion)
    return model, state, stats


@torch.inference_mode()
def _gpu_hidden_states(model, prompt, tokens, bucket):
    """Final-normed hidden state of every step of the GPU path, teacher-forced
    on ``tokens`` (prefill, then one fused decode step per token)."""
    from transformers.cache_utils import StaticCache

    dev = prompt.device
    cache = StaticCache(config=model.config, max_cache_len=bucket)
    pos = torch.arange(prompt.shape[1], device=dev).view(1, -1)
    out = model.model(input_ids=prompt, position_ids=pos, past_key_values=cache, use_cache=True)
    hidden = [out.last_hidden_state[:, -1].float().cpu()]
    p = torch.full((1, 1), prompt.shape[1], device=dev, dtype=torch.long)
    for tok in tokens[:-1]:
        out = model.model(input_ids=torch.tensor([[tok]], device=dev), position_ids=p,
                          past_key_values=cache, use_cache=True)
        hidden.append(out.last_hidden_state[:, -1].float().cpu())
        p.add_(1)
    return hidden


def _check_teacher_forced(oracle, prompt, tokens, max_len, gpu_hidden, bounds):
    ref, ref_hidden = oracle.teacher_forced(prompt.cpu(), tokens[:-1], max_len, return_hidden=True)
    check_steps(oracle, tokens, ref, gpu_hidden, ref_hidden, bounds)


@pytest.mark.parametrize("fused,a8w8", [(True, False), (False, False), (True, True)])
def test_tiny_model_greedy_vs_oracle(gpu, fused, a8w8):
    from ppu_amd.generate import FusedGreedyGenerator
    from ppu_amd.integration import FusionConfig

    cfg = synth.config_tiny()
    model, state, stats = _build(cfg, gpu, FusionConfig(fused_decode=fused, a8w8=a8w8))
    assert stats["delta"] == 3 and stats["attention"] == 1
    g = torch.Generator().manual_seed(20260625)
    prompt = torch.randint(0, cfg.vocab_size, (1, 70), generator=g).to(gpu)
    res = FusedGreedyGenerator(model).generate(prompt, max_new_tokens=24)
    assert len(res.tokens) == 24
    hidden = _gpu_hidden_states(model, prompt, res.tokens, res.meta["cache_bucket"])
    oracle = OracleDecoder(state, cfg, a8w8=a8w8)
    _check_teacher_forced(oracle, prompt, res.tokens, res.meta["cache_bucket"], hidden,
                          HIDDEN_BOUNDS["tiny"])


def test_fused_cache_reset_matches_transformers(gpu):
    """reset_cache (one zeroing launch) leaves a used cache exactly as
    Transformers' Cache.reset() does, and a generator reusing its cache
    reproduces the first run's tokens."""
    from transformers.cache_utils import StaticCache

    from ppu_amd.generate import FusedGreedyGenerator, reset_cache

    cfg = synth.config_tiny()
    model, _, _ = _build(cfg, gpu, None)
    g = torch.Generator().manual_seed(11)
    prompt = torch.randint(0, cfg.vocab_size, (1, 70), generator=g).to(gpu)

    def used_cache():
        cache = StaticCache(config=cfg, max_cache_len=512)
        with torch.inference_mode():
            pos = torch.arange(70, device=gpu).view(1, -1)
            model.model(input_ids=prompt, position_ids=pos, past_key_values=cache, use_cache=True)
        return cache

    def snapshot(cache):
        out = []
        for layer in cache.layers:
            for name in ("keys", "values", "cumulative_length"):
                v = getattr(layer, name, None)
                out.append(v.clone() if isinstance(v, torch.Tensor) else v)
            for d in ("conv_states", "recurrent_states", "has_previous_state"):
                v = getattr(layer, d, None)
                if isinstance(v, dict):
                    out += [x.clone() if isinstance(x, torch.Tensor) else x for x in v.values()]
        return out

    ca, cb = used_cache(), used_cache()
    assert any(isinstance(t, torch.Tensor) and t.any() for t in snapshot(cb))
    with torch.inference_mode():  # the states are inference tensors, as in generate()
        ca.reset()
        reset_cache(cb)
    torch.cuda.synchronize()
    sa, sb = snapshot(ca), snapshot(cb)
    assert len(sa) == len(sb)
    for a, b in zip(sa, sb):
        if isinstance(a, torch.Tensor):
            assert torch.equal(a, b) and not b.any()
        else:
            assert a == b
    gen_ = FusedGreedyGenerator(model)
    first = gen_.generate(prompt, max_new_tokens=12)
    again = gen_.generate(prompt, max_new_tokens=12)
    assert again.meta["cache_reused"] and again.tokens == first.tokens


def test_a8w8_int8_handoff_prefill_equals_layer_chain(gpu):
    """The A8W8 prefill that hands int8 activations and int32 accumulators
    between the GEMMs (fused dequant / norm / quant kernels) leaves the same
    bits as the layer-by-layer chain of separate kernels: final hidden state,
    every conv and recurrent state and every K/V cache row."""
    from transformers.cache_utils import StaticCache

    from ppu_amd import kernels as K
    from ppu_amd.integration import FusionConfig, prefill_layer, text_stack

    cfg = synth.config_tiny()
    model, _, _ = _build(cfg, gpu, FusionConfig(a8w8=True))
    stack = text_stack(model)
    g = torch.Generator().manual_seed(13)
    prompt = torch.randint(0, cfg.vocab_size, (1, 90), generator=g).to(gpu)
    pos = torch.arange(90, device=gpu).view(1, -1)
    with torch.inference_mode():
        c1 = StaticCache(config=model.config, max_cache_len=512)
        fused = model.model(input_ids=prompt, position_ids=pos, past_key_values=c1,
                            use_cache=True).last_hidden_state
        c2 = StaticCache(config=model.config, max_cache_len=512)
        embeds = stack.embed_tokens(prompt)
        rope = stack.rotary_emb(embeds, pos)
        residual = embeds.contiguous()
        hidden = K.rms_norm(residual, stack.layers[0].input_layernorm.weight,
                            stack.layers[0].input_layernorm.eps)
        for i in range(cfg.num_hidden_layers):
            residual, hidden = prefill_layer(stack, i, residual, hidden, c2, rope,
                                             model._qwen35_fusion_config)
    torch.cuda.synchronize()
    assert torch.equal(fused, hidden)
    for a, b in zip(c1.layers, c2.layers):
        for name in ("keys", "values", "conv_states", "recurrent_states"):
            x, y = getattr(a, name, None), getattr(b, name, None)
            if isinstance(x, torch.Tensor):
                assert torch.equal(x, y), name
            elif isinstance(x, (dict, list, tuple)):
                keys = x.keys() if isinstance(x, dict) else range(len(x))
                for key in keys:
                    if isinstance(x[key], torch.Tensor):
                        assert torch.equal(x[key], y[key]), name


@pytest.mark.parametrize("a8w8", [False, True])
def test_prefill_graph_matches_eager(gpu, a8w8):
    """A prompt length seen before runs its prefill as one captured graph:
    the same tokens as the eager first call, for the same prompt and for a
    different prompt of that length (the graph reads the ids from its input
    buffer), with the cache's device state and host flags as after an eager
    prefill; a new length runs eagerly again."""
    from ppu_amd.generate import FusedGreedyGenerator
    from ppu_amd.integration import FusionConfig

    cfg = synth.config_tiny()
    model, _, _ = _build(cfg, gpu, FusionConfig(a8w8=a8w8))
    g = torch.Generator().manual_seed(12)
    p1 = torch.randint(0, cfg.vocab_size, (1, 90), generator=g).to(gpu)
    p2 = torch.randint(0, cfg.vocab_size, (1, 90), generator=g).to(gpu)
    p3 = torch.randint(0, cfg.vocab_size, (1, 33), generator=g).to(gpu)
    eager = {}
    for name, p in (("p1", p1), ("p2", p2), ("p3", p3)):
        eager[name] = FusedGreedyGenerator(model).generate(p, max_new_tokens=10).tokens
    gen_ = FusedGreedyGenerator(model)
    first = gen_.generate(p1, max_new_tokens=10)
    assert not first.meta["prefill_graph"] and first.tokens == eager["p1"]
    for name, p in (("p1", p1), ("p2", p2), ("p1", p1)):
        res = gen_.generate(p, max_new_tokens=10)
        assert res.meta["prefill_graph"], name
        assert res.tokens == eager[name], name
    res = gen_.generate(p3, max_new_tokens=10)
    assert not res.meta["prefill_graph"] and res.tokens == eager["p3"]
    res = gen_.generate(p2, max_new_tokens=10)  # the 90-token graph survives another length
    assert res.meta["prefill_graph"] and res.tokens == eager["p2"]


def test_graph_replay_matches_eager_decode(gpu):
    """Graph replays advance the cache exactly as eager decode steps do."""
    from transformers.cache_utils import StaticCache

    from ppu_amd.graph import GreedyDecodeGraph
    from ppu_amd.kernels import lm_head_argmax

    cfg = synth.config_tiny()
    model, _, _ = _build(cfg, gpu, None)
    g = torch.Generator().manual_seed(7)
    prompt = torch.randint(0, cfg.vocab_size, (1, 33), generator=g).to(gpu)

    def prefill(cache):
        pos = torch.arange(33, device=gpu).view(1, -1)
        out = model.model(input_ids=prompt, position_ids=pos, past_key_values=cache, use_cache=True)
        return lm_head_argmax(out.last_hidden_state[:, -1].contiguous(), model.lm_head.weight)

    with torch.inference_mode():
        cache_a = StaticCache(config=cfg, max_cache_len=512)
        tok = prefill(cache_a)
        eager = []
        pos = torch.full((1, 1), 33, device=gpu, dtype=torch.long)
        for _ in range(6):
            out = model.model(input_ids=tok, position_ids=pos, past_key_values=cache_a, use_cache=True)
            tok = lm_head_argmax(out.last_hidden_state[:, -1].contiguous(), model.lm_head.weight)
            eager.append(int(tok))
            pos.add_(1)
        cache_b = StaticCache(config=cfg, max_cache_len=512)
        tok = prefill(cache_b)
        runner = GreedyDecodeGraph(model, cache_b, tok, torch.full((1, 1), 33, device=gpu,
                                                                   dtype=torch.long))
        # capture itself ran one step on cache_b: restart from the prefill state
        cache_b.reset()
        tok = prefill(cache_b)
        runner.set_inputs(tok, torch.full((1, 1), 33, device=gpu, dtype=torch.long))
        graphed = []
        for _ in range(6):
            graphed.append(int(runner.replay()))
            torch.cuda.synchronize()
        assert graphed == eager


@pytest.mark.timeout(900)
@pytest.mark.parametrize("variant", ["bf16", "a8w8"])
def test_2b_prefill_1024_decode_64_vs_oracle(gpu, variant):
    """Benchmark config 5: the full 2B-shaped decoder, 1024-token uniform-random
    prompt, 64 greedy tokens on the GPU (fused decode graph); the CPU oracle
    decoder is teacher-forced on the same tokens and must agree at every step
    whose top-2 margin exceeds the bf16 rounding noise."""
    from ppu_amd.generate import FusedGreedyGenerator
    from ppu_amd.integration import FusionConfig

    torch.set_num_threads(16)
    cfg = synth.config_2b()
    model, state, _ = _build(cfg, gpu, FusionConfig(a8w8=variant == "a8w8"))
    g = torch.Generator().manual_seed(synth.MODEL_SEED)
    prompt = torch.randint(0, cfg.vocab_size, (1, 1024), generator=g)
    res = FusedGreedyGenerator(model).generate(prompt.to(gpu), max_new_tokens=64)
    print(f"GPU TTFT {res.ttft_seconds * 1e3:.2f} ms, decode {res.decode_tokens_per_second:.1f} tok/s",
          flush=True)
    hidden = _gpu_hidden_states(model, prompt.to(gpu), res.tokens, res.meta["cache_bucket"])
    del model
    torch.cuda.empty_cache()
    # Transformers' own eager forward on the CPU (the reference's fallback
    # path, bf16) on the same weights, free-running for all 64 tokens: the
    # streams may part only where eager's own top-2 margin is within bf16
    # noise (A8W8 is compared with the bf16 eager model: printed only).
    eager, margins = eager_greedy(state, cfg, prompt, len(res.tokens))
    first = report_eager_agreement(res.tokens, eager, margins)
    if variant == "bf16" and first is not None:
        assert margins[first] <= 0.25, (first, margins[first])
    oracle = OracleDecoder(state, cfg, a8w8=variant == "a8w8")
    _check_teacher_forced(oracle, prompt, res.tokens, res.meta["cache_bucket"], hidden,
                          HIDDEN_BOUNDS["2b" if variant == "bf16" else "2b-a8w8"])


def _rel(gpu_t, ref_t) -> float:
    a, b = gpu_t.detach().double().cpu(), ref_t.detach().double()
    return float((a - b).norm() / b.norm())


def _set_layer_state(cache, index, states, length):
    """Load the oracle's cache state of one layer into the GPU cache."""
    slot = cache.layers[index]
    if "rec" in states:
        slot.conv_states[0].copy_(states["conv"])
        slot.recurrent_states[0].copy_(states["rec"])
    else:
        slot.keys.copy_(states["k"])
        slot.values.copy_(states["v"])
        slot.cumulative_length.fill_(length)


def _layer_state_errors(cache, index, states, rows):
    slot = cache.layers[index]
    if "rec" in states:
        return {"conv": _rel(slot.conv_states[0], states["conv"]),
                "state": _rel(slot.recurrent_states[0], states["rec"])}
    return {"k": _rel(slot.keys[:, :, :rows], states["k"][:, :, :rows]),
            "v": _rel(slot.values[:, :, :rows], states["v"][:, :, :rows])}


@pytest.mark.timeout(900)
@pytest.mark.parametrize("variant", ["bf16", "a8w8"])
def test_2b_layerwise_teacher_forced(gpu, variant):
    """Benchmark config 5, one layer at a time: every GPU layer is run from the
    oracle's own input and cache state, so an error cannot hide in the
    amplification of 24 chaotic random-init layers. Prefill (1024 tokens, the
    product prefill path per layer) and the second decode step (the fused
    decode launches per layer, state from prefill + one decode step) and a
    late decode step (step LATE = 64, states from the oracle's own greedy
    continuation): the
    layer's mixer output and stream after the mixer add,
    the MLP output, the next normed input and every cache state it writes,
    each within LAYER_BOUND relative L2 of the oracle's. (The mixer output
    and the MLP output are compared directly, not as differences of the bf16
    residual stream, whose rounding is larger than a small update.)"""
    from transformers.cache_utils import StaticCache

    from ppu_amd.integration import DecodeContext, FusionConfig, decode_layer, prefill_layer, text_stack

    bound = LAYER_BOUND[variant]
    torch.set_num_threads(16)
    cfg = synth.config_2b()
    fusion = FusionConfig(a8w8=variant == "a8w8")
    model, state, _ = _build(cfg, gpu, fusion)
    stack = text_stack(model)
    n = cfg.num_hidden_layers
    prompt = synth.prompt_ids(1024, cfg.vocab_size)
    bucket = 1152
    oracle = OracleDecoder(state, cfg, a8w8=variant == "a8w8")
    ocache = oracle.new_cache(bucket)
    pre, d1, d2 = [], [], []
    h = oracle.forward(prompt, ocache, pre)
    t1 = oracle.top1(h[:, -1])[0]
    h = oracle.forward(torch.tensor([[t1]]), ocache, d1)
    t2 = oracle.top1(h[:, -1])[0]
    h = oracle.forward(torch.tensor([[t2]]), ocache, d2)
    # A late decode step (LATE): the oracle continues greedily; the states
    # after step LATE - 1 and the trace of step LATE are kept.
    tok = oracle.top1(h[:, -1])[0]
    for _ in range(3, LATE - 1):
        h = oracle.forward(torch.tensor([[tok]]), ocache)
        tok = oracle.top1(h[:, -1])[0]
    dprev, dlate = [], []
    h = oracle.forward(torch.tensor([[tok]]), ocache, dprev)
    t_late = oracle.top1(h[:, -1])[0]
    oracle.forward(torch.tensor([[t_late]]), ocache, dlate)

    worst: dict[str, float] = {}
    fails = []

    def record(where, errs):
        for k, v in errs.items():
            worst[k] = max(worst.get(k, 0.0), v)
            if v > bound:
                fails.append((where, k, v))

    cache = StaticCache(config=cfg, max_cache_len=bucket)
    with torch.inference_mode():
        pos = torch.arange(1024, device=gpu).view(1, -1)
        model.model(input_ids=prompt.to(gpu), position_ids=pos, past_key_values=cache,
                    use_cache=True)  # allocates every cache layer
        rope = stack.rotary_emb(torch.zeros(1, 1024, 8, device=gpu, dtype=torch.bfloat16), pos)
        for i in range(n):
            t = pre[i]
            zero = {k: torch.zeros_like(v) for k, v in t["states"].items()}
            _set_layer_state(cache, i, zero, 0)
            got = {}
            _, n_out = prefill_layer(stack, i, t["residual_in"].to(gpu), t["normalized_in"].to(gpu),
                                     cache, rope, fusion, trace=got)
            errs = {"update": _rel(got["update"], t["update"]),
                    "residual_mid": _rel(got["residual_mid"], t["residual_mid"]),
                    "mlp_out": _rel(got["mlp_out"], t["mlp_out"]),
                    "normalized": _rel(n_out, t["normalized_out"])}
            errs.update(_layer_state_errors(cache, i, t["states"], 1024))
            record(f"prefill layer {i}", errs)
            print(f"prefill layer {i:2d} " + " ".join(f"{k} {v:.2e}" for k, v in errs.items()), flush=True)
        # decode step s consumes its token at position 1024 + s - 1, from the
        # states after step s - 1
        for step, prev, cur, tok_in in ((2, d1, d2, t2), (LATE, dprev, dlate, t_late)):
            at = 1024 + step - 1
            ctx = DecodeContext(cache, torch.tensor([[at]], device=gpu), True)
            token = torch.tensor([tok_in], device=gpu, dtype=torch.long)
            for i in range(n):
                t = cur[i]
                _set_layer_state(cache, i, prev[i]["states"], at)
                residual = update = None
                if i:
                    residual, update = cur[i - 1]["residual_mid"].to(gpu), cur[i - 1]["mlp_out"].to(gpu)
                got = {}
                r, u = decode_layer(stack, i, residual, update, ctx, token, trace=got)
                errs = {"update": _rel(got["update"], t["update"]),
                        "residual_mid": _rel(r, t["residual_mid"]),
                        "mlp_out": _rel(u, t["mlp_out"])}
                errs.update(_layer_state_errors(cache, i, t["states"], at + 1))
                record(f"decode step {step} layer {i}", errs)
                print(f"decode step {step} layer {i:2d} " + " ".join(f"{k} {v:.2e}" for k, v in errs.items()),
                      flush=True)
    print(f"{variant}: worst per quantity " + " ".join(f"{k} {v:.2e}" for k, v in worst.items()), flush=True)
    assert not fails, fails
