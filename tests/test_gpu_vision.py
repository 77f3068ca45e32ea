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


@pytest.mark.parametrize("tokens,heads,dim", [(10, 16, 72), (257, 16, 64), (33, 12, 80), (5, 2, 128)])
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
