"""End-to-end parity of the integrated MI355X path against the CPU oracle decoder.

A Transformers Qwen3.5 model (synthetic seeded weights) is patched with
``apply_fusions`` and run on the GPU: prefill, then greedy decode through the
captured graph. The oracle decoder gets the identical weights on the CPU and
is teacher-forced with the GPU's tokens, so every step compares the GPU token
with the oracle's argmax on the same history. A step may differ only where
the oracle's top-2 bf16 logit margin is within the accumulated bf16 rounding
noise of the two paths (MARGIN); every mismatch is printed with its margin.
"""

from __future__ import annotations

import pytest
import torch

from oracle.model import OracleDecoder
from ppu_amd import synth

pytestmark = pytest.mark.gpu

# Two bf16 ulps at logit magnitude ~4: the largest gap a different fp32
# summation order can close between otherwise identical paths.
MARGIN = 0.0625


def _build(cfg, gpu, fusion):
    from ppu_amd.integration import apply_fusions

    model = synth.build_model(cfg, device=gpu)
    state = {k: v.detach().cpu() for k, v in model.state_dict().items()}
    stats = apply_fusions(model, fusion)
    return model, state, stats


def _check_teacher_forced(oracle, prompt, tokens, max_len):
    ref = oracle.teacher_forced(prompt.cpu(), tokens[:-1], max_len)
    bad = []
    for step, (tok, (rt, margin)) in enumerate(zip(tokens, ref)):
        if tok != rt:
            print(f"step {step}: gpu {tok} oracle {rt} margin {margin:.4f}", flush=True)
            if margin > MARGIN:
                bad.append((step, tok, rt, margin))
    margins = [m for _, m in ref]
    print(f"{len(tokens)} steps, {sum(t == r for t, (r, _) in zip(tokens, ref))} identical, "
          f"min margin {min(margins):.4f}", flush=True)
    assert not bad, f"mismatches beyond the rounding margin: {bad}"


@pytest.mark.parametrize("fused", [True, False])
def test_tiny_model_greedy_vs_oracle(gpu, fused):
    from ppu_amd.generate import FusedGreedyGenerator
    from ppu_amd.integration import FusionConfig

    cfg = synth.config_tiny()
    model, state, stats = _build(cfg, gpu, FusionConfig(fused_decode=fused))
    assert stats["delta"] == 3 and stats["attention"] == 1
    g = torch.Generator().manual_seed(20260625)
    prompt = torch.randint(0, cfg.vocab_size, (1, 70), generator=g).to(gpu)
    res = FusedGreedyGenerator(model).generate(prompt, max_new_tokens=24)
    assert len(res.tokens) == 24
    oracle = OracleDecoder(state, cfg)
    _check_teacher_forced(oracle, prompt, res.tokens, res.meta["cache_bucket"])


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
