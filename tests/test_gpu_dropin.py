"""The drop-in boundary on the GPU, driven the way the reference's callers drive it.

* ``test_vlm_generation_call_sequence`` restates the call sequence of the
  reference's fused greedy generation (evaluation_wrapper.py:307-419) on the
  image-text model class, through the ``qwen35_fused`` import names:
  ``apply_fusions``, ``precompute_vision_kwargs``, a bucketed StaticCache,
  ``model.model(**inputs)`` prefill with an image (the vision tower on the
  fused vision path; the text stack receives ``inputs_embeds`` and 3-row
  multimodal positions), ``lm_head_argmax``, the ``rope_deltas`` position arithmetic, one
  eager decode step and ``GreedyDecodeGraph`` replays. The text path is checked
  against the oracle decoder on the embeddings and positions the text stack
  received.
* ``test_graph_multistep_equals_single_steps``: ``steps=4`` replays continue
  the sequence exactly as single-step replays do.
* Wrappers reject tensors on the wrong device before any launch.
* A library capture under inference mode leaves later captures outside
  inference mode working (the first GPU test of the suite, so in a full run
  the process has captured nothing before it).
"""

from __future__ import annotations

import pytest
import torch

from oracle.model import OracleDecoder
from ppu_amd import synth
from tests._parity import check_steps

pytestmark = pytest.mark.gpu

TINY_BOUNDS = (0.03, 0.03)  # as the tiny text-model test (tests/test_gpu_model.py)


def _text_state(model) -> dict[str, torch.Tensor]:
    """The text stack's parameters under the causal-LM names the oracle packs."""
    out = {}
    for k, v in model.state_dict().items():
        if k.startswith("model.language_model."):
            out["model." + k[len("model.language_model."):]] = v.detach().cpu()
    return out


def _image_prompt(cfg, gpu):
    g = torch.Generator().manual_seed(synth.MODEL_SEED + 3)
    vocab = cfg.text_config.vocab_size - 4
    grid = torch.tensor([[1, 8, 8]])  # 64 patches, 16 merged image tokens
    n_img = int(grid.prod()) // cfg.vision_config.spatial_merge_size ** 2
    ids = torch.cat([
        torch.randint(0, vocab, (1, 37), generator=g),
        torch.tensor([[cfg.vision_start_token_id]]),
        torch.full((1, n_img), cfg.image_token_id),
        torch.tensor([[cfg.vision_end_token_id]]),
        torch.randint(0, vocab, (1, 29), generator=g),
    ], dim=1)
    types = torch.zeros_like(ids, dtype=torch.int32)
    types[ids == cfg.image_token_id] = 1
    c, t, p = cfg.vision_config.in_channels, cfg.vision_config.temporal_patch_size, cfg.vision_config.patch_size
    pixels = torch.randn(int(grid.prod()), c * t * p * p, generator=g).to(torch.bfloat16)
    from transformers import BatchFeature

    return BatchFeature(dict(input_ids=ids, attention_mask=torch.ones_like(ids), pixel_values=pixels,
                             image_grid_thw=grid, mm_token_type_ids=types))


def test_capture_outside_inference_mode_after_library_capture_inside(gpu):
    """A decode graph captured under ``torch.inference_mode``, then a plain
    capture outside it, which must not fail in ``capture_begin`` (the
    generator's capture state is created at the process's first capture; the
    library makes that first registration outside inference mode)."""
    from transformers import StaticCache

    from ppu_amd.graph import GreedyDecodeGraph
    from ppu_amd.integration import apply_fusions

    cfg = synth.config_tiny()
    model = synth.build_model(cfg, device=gpu)
    apply_fusions(model)
    prompt = synth.prompt_ids(12, cfg.vocab_size, seed=synth.MODEL_SEED + 9).to(gpu)
    cache = StaticCache(config=model.config, max_cache_len=512)
    with torch.inference_mode():
        out = model.model(input_ids=prompt, position_ids=torch.arange(12, device=gpu).view(1, -1),
                          past_key_values=cache, use_cache=True)
        tok = out.last_hidden_state[:, -1:, 0].long().abs() % cfg.vocab_size
        runner = GreedyDecodeGraph(model, cache, tok, torch.full((1, 1), 12, device=gpu))
        runner.replay()
    x = torch.zeros(4, device=gpu)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        x.add_(1)
    graph.replay()
    torch.cuda.synchronize()
    assert x.sum().item() == 4.0


def test_vlm_generation_call_sequence(gpu):
    from transformers.cache_utils import StaticCache

    from qwen35_fused.graph import GreedyDecodeGraph
    from qwen35_fused.integration import apply_fusions, precompute_vision_kwargs
    from qwen35_fused.kernels import lm_head_argmax

    cfg = synth.config_vlm()
    model = synth.build_model(cfg, device=gpu)
    state = _text_state(model)
    stats = apply_fusions(model)
    assert stats["delta"] == 3 and stats["attention"] == 1 and stats["mlp"] == 4

    seen = {}

    def capture(module, args, kwargs):
        if kwargs.get("inputs_embeds") is not None and kwargs["inputs_embeds"].shape[1] > 1:
            seen["embeds"] = kwargs["inputs_embeds"].detach().float().cpu()
            seen["positions"] = kwargs["position_ids"].detach().cpu()

    model.model.language_model.register_forward_pre_hook(capture, with_kwargs=True)

    # evaluation_wrapper.py:333-419, text generation part
    inputs = _image_prompt(cfg, gpu)
    precompute_vision_kwargs(model, inputs)
    inputs = inputs.to(gpu)
    input_len = int(inputs.input_ids.shape[-1])
    max_new_tokens = 20
    bucket = max(512, ((input_len + max_new_tokens + 1 + 127) // 128) * 128)
    cache = StaticCache(config=model.config, max_cache_len=bucket)
    with torch.inference_mode():
        prefill = model.model(**inputs, past_key_values=cache, use_cache=True, return_dict=True)
        token = lm_head_argmax(prefill.last_hidden_state[:, -1, :].contiguous(), model.lm_head.weight)
        generated = [int(token.item())]
        assert model.model.rope_deltas is not None and int(model.model.rope_deltas) != 0
        first_position = (inputs.attention_mask.long().sum(dim=-1, keepdim=True).unsqueeze(0)
                          + model.model.rope_deltas.unsqueeze(0))
        start_position = int(first_position)
        decode = model.model(input_ids=token, attention_mask=None, position_ids=first_position,
                             past_key_values=cache, use_cache=True, return_dict=True)
        token = lm_head_argmax(decode.last_hidden_state[:, -1, :].contiguous(), model.lm_head.weight)
        generated.append(int(token.item()))
        first_position.add_(1)
        runner = GreedyDecodeGraph(model, cache, token, first_position, fused_lm_head=True, steps=1)
        while len(generated) < max_new_tokens:
            generated.extend(int(t) for t in runner.replay().reshape(-1).tolist())
    generated = generated[:max_new_tokens]
    assert seen["positions"].shape == (3, 1, input_len)
    # The capture recorded one step without running it; the graph's position
    # tensor has advanced once per replay.
    assert int(runner.position_ids) == start_position + max_new_tokens - 1

    # Eager teacher-forced pass on a fresh cache: the final hidden state of
    # every step, and the same greedy tokens as the graph produced.
    hidden_gpu = []
    cache2 = StaticCache(config=model.config, max_cache_len=bucket)
    with torch.inference_mode():
        out = model.model(**inputs, past_key_values=cache2, use_cache=True, return_dict=True)
        hidden_gpu.append(out.last_hidden_state[:, -1].float().cpu())
        pos = torch.full((1, 1, 1), start_position, device=gpu, dtype=torch.long)
        for tok in generated[:-1]:
            out = model.model(input_ids=torch.tensor([[tok]], device=gpu), attention_mask=None,
                              position_ids=pos, past_key_values=cache2, use_cache=True,
                              return_dict=True)
            hidden_gpu.append(out.last_hidden_state[:, -1].float().cpu())
            pos.add_(1)
    assert all(torch.isfinite(h).all() for h in hidden_gpu)

    # Oracle: the text stack on the embeddings and 3-row positions it received.
    oracle = OracleDecoder(state, cfg.text_config)
    ocache = oracle.new_cache(bucket)
    h = oracle.forward(None, ocache, embeds=seen["embeds"].to(torch.bfloat16),
                       rope_positions=seen["positions"])
    ref, ref_hidden = [oracle.top1(h[:, -1])], [h[:, -1].clone()]
    for i, tok in enumerate(generated[:-1]):
        rp = torch.full((1, 1), start_position + i, dtype=torch.long)
        h = oracle.forward(torch.tensor([[tok]]), ocache, rope_positions=rp)
        ref.append(oracle.top1(h[:, -1]))
        ref_hidden.append(h[:, -1].clone())
    check_steps(oracle, generated, ref, hidden_gpu, ref_hidden, TINY_BOUNDS)


def _prefilled(model, cfg, gpu, prompt):
    from transformers.cache_utils import StaticCache

    from ppu_amd.kernels import lm_head_argmax

    cache = StaticCache(config=cfg, max_cache_len=512)
    pos = torch.arange(prompt.shape[1], device=gpu).view(1, -1)
    out = model.model(input_ids=prompt, position_ids=pos, past_key_values=cache, use_cache=True)
    tok = lm_head_argmax(out.last_hidden_state[:, -1].contiguous(), model.lm_head.weight)
    return cache, tok


def _state_tensors(cache):
    out = []
    for layer in cache.layers:
        for name in ("keys", "values", "cumulative_length"):
            v = getattr(layer, name, None)
            if isinstance(v, torch.Tensor):
                out.append(v.clone())
        for d in ("conv_states", "recurrent_states"):
            v = getattr(layer, d, None)
            if isinstance(v, dict):
                out += [x.clone() for x in v.values() if isinstance(x, torch.Tensor)]
    return out


def test_graph_multistep_equals_single_steps(gpu):
    """Two replays of a 4-step graph give the 8 tokens, the position and the
    cache state that eight replays of a 1-step graph give (the multi-token
    graph option of the reference's scheduling notes)."""
    from ppu_amd.graph import GreedyDecodeGraph
    from ppu_amd.integration import apply_fusions
    from ppu_amd.kernels import lm_head_argmax

    cfg = synth.config_tiny()
    model = synth.build_model(cfg, device=gpu)
    apply_fusions(model)
    prompt = synth.prompt_ids(45, cfg.vocab_size, seed=synth.MODEL_SEED + 4).to(gpu)
    results = {}
    with torch.inference_mode():
        for steps, replays in ((1, 8), (4, 2)):
            cache, tok = _prefilled(model, cfg, gpu, prompt)
            start = torch.full((1, 1), 45, device=gpu, dtype=torch.long)
            runner = GreedyDecodeGraph(model, cache, tok, start, steps=steps)
            # restart from the prefill state on the captured cache object
            cache.reset()
            pos = torch.arange(45, device=gpu).view(1, -1)
            out = model.model(input_ids=prompt, position_ids=pos, past_key_values=cache, use_cache=True)
            tok = lm_head_argmax(out.last_hidden_state[:, -1].contiguous(), model.lm_head.weight)
            runner.set_inputs(tok, start)
            tokens = []
            for _ in range(replays):
                tokens += runner.replay().reshape(-1).tolist()
            torch.cuda.synchronize()
            results[steps] = (tokens, int(runner.position_ids), _state_tensors(cache))
    (t1, p1, s1), (t4, p4, s4) = results[1], results[4]
    assert t1 == t4 and len(t1) == 8
    assert p1 == p4 == 45 + 8
    assert len(s1) == len(s4) and all(torch.equal(a, b) for a, b in zip(s1, s4))


def test_pipelined_graph_equals_single_steps(gpu):
    """The pipelined decode loop (two captures alternating, the token read from
    pinned host memory the top-1 launch writes, the next step queued before the
    previous token is read) gives the tokens, the position and the cache state
    of plain one-step replays; an EOS stops it after that token with nothing
    left outstanding; misuse is refused before any launch."""
    from ppu_amd.graph import GreedyDecodeGraph, decode_tokens
    from ppu_amd.integration import apply_fusions
    from ppu_amd.kernels import lm_head_argmax

    cfg = synth.config_tiny()
    model = synth.build_model(cfg, device=gpu)
    apply_fusions(model)
    prompt = synth.prompt_ids(45, cfg.vocab_size, seed=synth.MODEL_SEED + 5).to(gpu)
    start = torch.full((1, 1), 45, device=gpu, dtype=torch.long)
    results = {}
    with torch.inference_mode():
        def restart(runner, cache):
            cache.reset()
            pos = torch.arange(45, device=gpu).view(1, -1)
            out = model.model(input_ids=prompt, position_ids=pos, past_key_values=cache, use_cache=True)
            tok = lm_head_argmax(out.last_hidden_state[:, -1].contiguous(), model.lm_head.weight)
            runner.set_inputs(tok, start)

        for pipelined in (False, True):
            cache, tok = _prefilled(model, cfg, gpu, prompt)
            runner = GreedyDecodeGraph(model, cache, tok, start, pipelined=pipelined)
            restart(runner, cache)
            if pipelined:
                tokens = decode_tokens(runner, 9)
            else:
                tokens = [int(runner.replay()) for _ in range(9)]
            torch.cuda.synchronize()
            results[pipelined] = (tokens, int(runner.position_ids), _state_tensors(cache))
        (t0, p0, s0), (t1, p1, s1) = results[False], results[True]
        assert t0 == t1 and len(t1) == 9
        assert p0 == p1 == 45 + 9
        assert len(s0) == len(s1) and all(torch.equal(a, b) for a, b in zip(s0, s1))

        # no step asked: nothing launched; one step: one token, nothing queued past it
        restart(runner, cache)
        assert decode_tokens(runner, 0) == [] and int(runner.position_ids) == 45
        assert decode_tokens(runner, 1) == t0[:1] and int(runner.position_ids) == 46
        # a plain replay (capture 0, whose top-1 also writes host slot 0), not
        # waited for, then the pipelined loop: it continues with the next tokens
        restart(runner, cache)
        runner.replay()
        assert decode_tokens(runner, 3) == t0[1:4]
        # an EOS at the fourth token: four tokens back, the queued fifth step drained
        restart(runner, cache)
        assert decode_tokens(runner, 9, eos_ids={t0[3]}) == t0[: t0.index(t0[3]) + 1]
        assert int(runner.position_ids) == 45 + t0.index(t0[3]) + 2
        # misuse: a third launch, an out-of-order read, new inputs or a plain
        # replay while launches are outstanding
        restart(runner, cache)
        a = runner.launch()
        b = runner.launch()
        with pytest.raises(RuntimeError):
            runner.launch()
        with pytest.raises(RuntimeError):
            runner.result(b)
        with pytest.raises(RuntimeError):
            runner.set_inputs(t0[0] * torch.ones((1, 1), device=gpu, dtype=torch.long), start)
        with pytest.raises(RuntimeError):
            runner.replay()
        assert [runner.result(a), runner.result(b)] == t0[:2]
        with pytest.raises(ValueError):
            GreedyDecodeGraph(model, cache, tok, start, pipelined=True, steps=2)


def test_wrappers_reject_wrong_device_before_launch(gpu):
    """A CPU ``out``/``advance``/``positions`` tensor, or mis-shaped state,
    raises ValueError on the host (no kernel sees a host address)."""
    from ppu_amd import kernels as K

    bf = torch.bfloat16
    h = torch.randn(1, 2048, device=gpu).to(bf)
    w = torch.randn(300, 2048, device=gpu).to(bf)
    with pytest.raises(ValueError):
        K.lm_head_argmax(h, w, out=torch.zeros(1, 1, dtype=torch.long))
    with pytest.raises(ValueError):
        K.lm_head_argmax(h, w, advance=torch.zeros(1, 1, dtype=torch.long))
    packed = torch.randn(1, 1, 5120, device=gpu).to(bf)
    kc = torch.zeros(1, 2, 64, 256, device=gpu, dtype=bf)
    with pytest.raises(ValueError):
        K.gqa_decode_fused(packed, torch.zeros(256, device=gpu, dtype=bf),
                           torch.zeros(256, device=gpu, dtype=bf),
                           torch.ones(32, device=gpu), torch.zeros(1, 1, dtype=torch.long),
                           kc, kc.clone(), torch.zeros((), device=gpu, dtype=torch.long), 0.0625,
                           q_heads=8)
    # delta_decode_fused: recurrent state of the wrong head count
    with pytest.raises(ValueError):
        K.delta_decode_fused(torch.zeros(1, 1, 8320, device=gpu, dtype=bf),
                             torch.zeros(6144, 4, device=gpu, dtype=bf),
                             torch.zeros(1, 6144, 4, device=gpu, dtype=bf),
                             torch.zeros(16, device=gpu), torch.zeros(16, device=gpu),
                             torch.zeros(1, 8, 128, 128, device=gpu),
                             torch.ones(128, device=gpu, dtype=bf), 1e-6)
    torch.cuda.synchronize()


@pytest.mark.parametrize("a8w8", [False, True])
def test_checkpoint_loader_generates_like_the_built_model(gpu, tmp_path, a8w8):
    """A checkpoint written from the seeded model and read back by the
    loader (packed at load, int8-quantised at load with ``a8w8``) generates
    the same greedy tokens as the same model built in memory and packed by
    ``apply_fusions``."""
    from ppu_amd.checkpoint import load_checkpoint
    from ppu_amd.generate import FusedGreedyGenerator
    from ppu_amd.integration import FusionConfig, apply_fusions
    from tests.test_checkpoint import write_checkpoint

    cfg = synth.config_tiny()
    built = synth.build_model(cfg, device=gpu)
    write_checkpoint(built, cfg, tmp_path)
    apply_fusions(built, FusionConfig(a8w8=a8w8))
    loaded, _ = load_checkpoint(tmp_path, device=gpu, fusion=FusionConfig(a8w8=a8w8))
    prompt = synth.prompt_ids(50, cfg.vocab_size, seed=synth.MODEL_SEED + 9).to(gpu)
    a = FusedGreedyGenerator(built).generate(prompt, max_new_tokens=16).tokens
    b = FusedGreedyGenerator(loaded).generate(prompt, max_new_tokens=16).tokens
    assert a == b

