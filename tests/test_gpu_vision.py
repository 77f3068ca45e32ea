"""GPU parity of the vision-encoder operators (layer_norm,
residual_add_layer_norm, position_embed_add, vision_qkv_rope) against the CPU
oracle on identical seeded bf16 inputs.

Tolerances (per assertion): bf16 outputs rtol 1e-2 / atol 1e-3, and where the
only difference from the oracle is the order of an fp32 sum, at least 97 % of
the elements bit-identical; the residual sum, the position-embedding add (the
same fused multiply-add chain on both sides) and the RoPE split (no fused
multiply-add on either side) bit-exact.
"""

from __future__ import annotations

import copy

import pytest
import torch

from oracle import ops as ref
from tests.conftest import KERNEL_SEED, gen

pytestmark = pytest.mark.gpu

BF = torch.bfloat16


def randn(g, *shape, scale=1.0, mean=0.0):
    return (torch.randn(*shape, generator=g) * scale + mean).to(BF)


def close_mostly_exact(actual, expected, frac=0.97):
    a, e = actual.detach().cpu(), expected.detach().cpu()
    torch.testing.assert_close(a.float(), e.float(), rtol=1e-2, atol=1e-3)
    assert (a == e).float().mean().item() >= frac


@pytest.mark.parametrize("rows,width", [(7, 1152), (1000, 1024), (3, 2048), (5, 72), (4, 100),
                                        (2, 4096), (1, 8)])
@pytest.mark.parametrize("f32_params", [False, True])
def test_layer_norm(gpu, rows, width, f32_params):
    from ppu_amd import kernels as K

    g = gen(KERNEL_SEED + width)
    x = randn(g, rows, width, scale=2.0, mean=0.3)
    w = randn(g, width, scale=0.1, mean=1.0)
    b = randn(g, width, scale=0.1)
    if f32_params:
        w, b = w.float(), b.float()
    got = K.layer_norm(x.to(gpu), w.to(gpu), b.to(gpu), 1e-6)
    close_mostly_exact(got, ref.layer_norm(x, w, b, 1e-6))


@pytest.mark.parametrize("rows,width", [(9, 1152), (6, 100), (1, 2048)])
def test_residual_add_layer_norm(gpu, rows, width):
    from ppu_amd import kernels as K

    g = gen(KERNEL_SEED + 1)
    r = randn(g, 1, rows, width)
    u = randn(g, 1, rows, width)
    w = randn(g, width, scale=0.1, mean=1.0)
    b = randn(g, width, scale=0.1)
    r_out, y = K.residual_add_layer_norm(r.to(gpu), u.to(gpu), w.to(gpu), b.to(gpu), 1e-6)
    er, ey = ref.residual_add_layer_norm(r, u, w, b, 1e-6)
    assert torch.equal(r_out.cpu(), er)
    close_mostly_exact(y, ey)


@pytest.mark.parametrize("mode,width", [("bilinear", 1152), ("bicubic", 1152), ("bilinear", 100)])
@pytest.mark.parametrize("bf16_weights", [False, True])
def test_position_embed_add(gpu, mode, width, bf16_weights):
    from transformers.vision_utils import get_vision_interpolation_indices_and_weights

    from ppu_amd import kernels as K

    g = gen(KERNEL_SEED + 2)
    side = 12
    table = randn(g, side * side, width, scale=0.5)
    grid = torch.tensor([[1, 8, 6], [2, 4, 4]])
    idx, wts = get_vision_interpolation_indices_and_weights(
        grid, num_grid_per_side=side, mode=mode, align_corners=True, spatial_merge_size=2)
    if bf16_weights:
        wts = wts.to(BF)
    hidden = randn(g, idx.shape[0], width)
    got = K.position_embed_add(hidden.to(gpu), table.to(gpu), idx.to(gpu), wts.to(gpu))
    # same fused multiply-add chain on both sides: bit-exact
    assert torch.equal(got.cpu(), ref.position_embed_add(hidden, table, idx, wts))


def test_position_embed_add_clamps_indices(gpu):
    from ppu_amd import kernels as K

    g = gen(KERNEL_SEED + 3)
    table = randn(g, 16, 64)
    hidden = torch.zeros(3, 64, dtype=BF)
    idx = torch.tensor([[0, 40], [-3, 15], [15, 15]])
    wts = torch.tensor([[0.0, 1.0], [1.0, 0.0], [0.5, 0.5]])
    got = K.position_embed_add(hidden.to(gpu), table.to(gpu), idx.to(gpu), wts.to(gpu)).cpu()
    assert torch.equal(got[0], table[15])  # 40 -> 15
    assert torch.equal(got[1], table[0])   # -3 -> 0
    assert torch.equal(got[2], table[15])


@pytest.mark.parametrize("tokens,heads,dim", [(10, 16, 72), (257, 16, 64), (33, 12, 80), (5, 2, 128),
                                               (7, 3, 18), (4, 2, 6)])
@pytest.mark.parametrize("cs_dtype", [torch.float32, BF])
def test_vision_qkv_rope(gpu, tokens, heads, dim, cs_dtype):
    from ppu_amd import kernels as K

    g = gen(KERNEL_SEED + 4)
    packed = randn(g, tokens, 3 * heads * dim)
    ang = torch.randn(tokens, dim // 2, generator=g) * 3
    emb = torch.cat((ang, ang), dim=-1)
    cos, sin = emb.cos().to(cs_dtype), emb.sin().to(cs_dtype)
    q, k, v = K.vision_qkv_rope(packed.to(gpu), cos.to(gpu), sin.to(gpu), heads=heads, dim=dim)
    eq, ek, ev = ref.vision_qkv_rope(packed, cos, sin, heads=heads, dim=dim)
    assert q.shape == (1, heads, tokens, dim)
    assert torch.equal(q.cpu(), eq)
    assert torch.equal(k.cpu(), ek)
    assert torch.equal(v.cpu(), ev)


def test_vision_ops_reject_bad_shapes(gpu):
    from ppu_amd import kernels as K

    x = torch.zeros(4, 64, dtype=BF, device=gpu)
    with pytest.raises(ValueError):
        K.layer_norm(x, torch.ones(63, device=gpu), torch.zeros(64, device=gpu))
    with pytest.raises(ValueError):
        K.residual_add_layer_norm(x, torch.zeros(4, 32, dtype=BF, device=gpu), torch.ones(64, device=gpu),
                                  torch.zeros(64, device=gpu))
    with pytest.raises(ValueError):
        K.position_embed_add(x, torch.zeros(16, 64, dtype=BF, device=gpu),
                             torch.zeros(3, 4, dtype=torch.int64, device=gpu), torch.zeros(3, 4, device=gpu))
    with pytest.raises(ValueError):
        K.vision_qkv_rope(torch.zeros(4, 3 * 2 * 8, dtype=BF, device=gpu), torch.zeros(4, 8, device=gpu),
                          torch.zeros(4, 8, device=gpu), heads=2, dim=16)
    with pytest.raises(ValueError):
        K.layer_norm(x.cpu(), torch.ones(64), torch.zeros(64))
    q = torch.zeros(1, 2, 16, 64, dtype=BF, device=gpu)
    with pytest.raises(ValueError):  # head dim not a multiple of 8
        K.vision_attention(*(torch.zeros(1, 2, 16, 12, dtype=BF, device=gpu),) * 3, 0.3)
    with pytest.raises(ValueError):  # batch of two
        K.vision_attention(*(torch.zeros(2, 2, 16, 64, dtype=BF, device=gpu),) * 3, 0.125)
    with pytest.raises(ValueError):  # image offsets on the host
        K.vision_attention(q, q, q, 0.125, torch.tensor([0, 8, 16], dtype=torch.int32))
    with pytest.raises(ValueError):  # fewer than two offsets
        K.vision_attention(q, q, q, 0.125, torch.tensor([0], dtype=torch.int32, device=gpu))


# ------------------------------------------------------------- vision tower
def _vision_setup(gpu):
    from transformers.models.qwen3_5 import modeling_qwen3_5 as impl

    from ppu_amd import synth

    vision = dict(depth=2, hidden_size=128, intermediate_size=256, num_heads=4, in_channels=3,
                  patch_size=16, spatial_merge_size=2, temporal_patch_size=2,
                  out_hidden_size=64, num_position_embeddings=64)
    cfg = synth.config_vlm(vision_config=vision)
    model = synth.build_model(cfg, device=gpu)
    # fp32 CPU copy of the tower with Transformers' own forward (eager attention)
    vcfg = copy.deepcopy(model.model.visual.config)
    vcfg._attn_implementation = "eager"
    ref_tower = impl.Qwen3_5VisionModel(vcfg).float().eval()
    ref_tower.load_state_dict({k: v.float().cpu() for k, v in model.model.visual.state_dict().items()})
    ref_tower.rotary_pos_emb.inv_freq.copy_(model.model.visual.rotary_pos_emb.inv_freq.cpu())
    return cfg, model, ref_tower


def _pixels(cfg, grid, seed):
    vc = cfg.vision_config
    g = torch.Generator().manual_seed(seed)
    n = int(grid.prod(-1).sum())
    return torch.randn(n, vc.in_channels * vc.temporal_patch_size * vc.patch_size ** 2, generator=g)


def _rel(a, b):
    a, b = a.detach().float().cpu(), b.detach().float().cpu()
    return ((a - b).norm() / b.norm()).item()


def test_vision_tower_matches_transformers_and_graph_replays(gpu):
    """The fused vision forward (our LayerNorm / position-embedding / RoPE
    kernels, library GEMMs, the vision_attn_fa flash kernel) against Transformers' fp32 CPU forward
    of the same weights; the second call of a patch count replays the captured
    graph and every replay (with eager work in between) equals the eager call."""
    from qwen35_fused.integration import apply_fusions

    cfg, model, ref_tower = _vision_setup(gpu)
    stats = apply_fusions(model)
    assert stats["vision"] == 2
    grid = torch.tensor([[1, 8, 12]])
    pix = _pixels(cfg, grid, 11)
    with torch.inference_mode():
        exp = ref_tower(pix, grid_thw=grid)
        first = model.model.visual(pix.to(gpu, torch.bfloat16), grid_thw=grid.to(gpu))
        # bf16 path against the fp32 reference: relative L2 error of the outputs
        assert _rel(first.last_hidden_state, exp.last_hidden_state) < 2e-2
        assert _rel(first.pooler_output, exp.pooler_output) < 2e-2
        base_h = first.last_hidden_state.clone()
        base_p = first.pooler_output.clone()
        for r in range(3):
            other = model.model.visual(_pixels(cfg, grid, 100 + r).to(gpu, torch.bfloat16),
                                       grid_thw=grid.to(gpu))
            torch.cuda.synchronize()
            again = model.model.visual(pix.to(gpu, torch.bfloat16), grid_thw=grid.to(gpu))
            assert torch.equal(again.last_hidden_state, base_h)
            assert torch.equal(again.pooler_output, base_p)
            assert not torch.equal(other.last_hidden_state, base_h)


def test_vision_tower_two_images_and_precomputed_kwargs(gpu):
    """Two images in one call (attention per image, no graph) and the
    precomputed tensors of precompute_vision_kwargs give the same output as
    computing them inside the forward."""
    from transformers import BatchFeature

    from qwen35_fused.integration import apply_fusions, precompute_vision_kwargs

    cfg, model, ref_tower = _vision_setup(gpu)
    apply_fusions(model)
    grid = torch.tensor([[1, 8, 8], [1, 4, 6]])
    pix = _pixels(cfg, grid, 12)
    with torch.inference_mode():
        exp = ref_tower(pix, grid_thw=grid)
        got = model.model.visual(pix.to(gpu, torch.bfloat16), grid_thw=grid.to(gpu))
        assert _rel(got.last_hidden_state, exp.last_hidden_state) < 2e-2
        assert _rel(got.pooler_output, exp.pooler_output) < 2e-2
        inputs = precompute_vision_kwargs(model, BatchFeature({"image_grid_thw": grid}))
        for name in ("image_interp_indices", "image_interp_weights", "image_position_ids",
                     "image_cu_seqlens"):
            assert name in inputs
        pre = {k[len("image_"):]: (v.to(gpu) if isinstance(v, torch.Tensor) else v)
               for k, v in inputs.items() if k.startswith("image_") and k != "image_grid_thw"}
        got2 = model.model.visual(pix.to(gpu, torch.bfloat16), grid_thw=grid.to(gpu), **pre)
        assert torch.equal(got2.last_hidden_state, got.last_hidden_state)


@pytest.mark.parametrize("tokens,heads,dim", [(784, 16, 72), (100, 4, 64), (257, 2, 80), (64, 3, 128),
                                              (5, 2, 8), (130, 1, 96), (2048, 16, 72)])
def test_vision_attention_one_image(gpu, tokens, heads, dim):
    from ppu_amd import kernels as K

    g = gen(KERNEL_SEED + 5)
    q, k, v = (randn(g, 1, heads, tokens, dim) for _ in range(3))
    got = K.vision_attention(q.to(gpu), k.to(gpu), v.to(gpu), dim ** -0.5)
    exp = ref.vision_attention(q, k, v, dim ** -0.5)
    assert got.shape == (tokens, heads * dim)
    # P is rounded to bf16 before the P.V product (as fused attention kernels do)
    torch.testing.assert_close(got.float().cpu(), exp.float(), rtol=1e-2, atol=1e-2)


# (grids of 512 workgroups and more take the one-block-per-stage form)
@pytest.mark.parametrize("bounds,heads", [([0, 64, 100, 257], 4), ([0, 1, 130, 131], 4), ([0, 200, 257], 4),
                                          ([0, 1000, 2100], 16)])
def test_vision_attention_per_image(gpu, bounds, heads):
    from ppu_amd import kernels as K

    g = gen(KERNEL_SEED + 6)
    dim, tokens = 72, bounds[-1]
    q, k, v = (randn(g, 1, heads, tokens, dim, scale=2.0) for _ in range(3))
    cu = torch.tensor(bounds, dtype=torch.int32)
    got = K.vision_attention(q.to(gpu), k.to(gpu), v.to(gpu), dim ** -0.5, cu.to(gpu))
    exp = ref.vision_attention(q, k, v, dim ** -0.5, cu)
    torch.testing.assert_close(got.float().cpu(), exp.float(), rtol=1e-2, atol=1e-2)
    # a one-token image returns its value row exactly
    for a, b in zip(bounds[:-1], bounds[1:]):
        if b - a == 1:
            assert torch.equal(got[a].cpu().reshape(heads, dim), v[0, :, a])


def test_vision_mlp_fused_gelu_matches_module(gpu):
    """The block MLP with the tanh GELU as the fc1 GEMM's epilogue (one bf16
    rounding fewer) against the module's own bf16 forward and an fp32 one,
    then on zero-padded weights."""
    from transformers.models.qwen3_5 import modeling_qwen3_5 as impl
    from transformers.models.qwen3_5.configuration_qwen3_5 import Qwen3_5VisionConfig
    from ppu_amd import integration

    cfg = Qwen3_5VisionConfig(hidden_size=256, intermediate_size=688)
    torch.manual_seed(KERNEL_SEED + 7)
    mlp = impl.Qwen3_5VisionMLP(cfg)
    x = torch.randn(300, 256)
    exp32 = mlp(x)
    mlp = mlp.to(gpu, torch.bfloat16)
    xb = x.to(gpu, torch.bfloat16)
    with torch.no_grad():
        mod = mlp(xb).float().cpu()
        got = integration._vision_mlp(mlp, xb).float().cpu()
        # zero-padded to 768 intermediate columns: the module's own forward
        # (on views of the padded weights) is unchanged, the fused one close
        integration._pad_vision_mlp(mlp)
        padded = mlp.q35_fc1_w
        integration._pad_vision_mlp(mlp)  # a second call keeps the padded weights
        assert mlp.q35_fc1_w is padded
        assert mlp.q35_fc1_w.shape == (768, 256) and mlp.linear_fc1.weight.shape == (688, 256)
        assert torch.equal(mlp(xb).float().cpu(), mod)
        got_pad = integration._vision_mlp(mlp, xb).float().cpu()
    rel = lambda a, b: ((a - b).norm() / b.norm()).item()
    assert rel(got, exp32.detach()) <= rel(mod, exp32.detach()) * 1.5 + 1e-3
    assert rel(got, mod) < 1e-2
    assert rel(got_pad, got) < 1e-3
