"""GPU parity of every operator against the CPU oracle on identical seeded inputs.

Inputs are drawn on the CPU in fp32 from seeded generators, cast to bf16 and
copied to the GPU, so both sides see the same bits. Tolerances (written per
assertion): bf16/fp32 outputs rtol 1e-2 / atol 1e-3; int8 quantisation, int32
accumulators and argmax indices bit-exact; delta-rule state 1e-3 relative.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import a8w8 as oa
from oracle import ops as ref
from tests.conftest import KERNEL_SEED, gen

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-2, 1e-3
BF = torch.bfloat16


def randn(g, *shape, scale=1.0, mean=0.0):
    return (torch.randn(*shape, generator=g) * scale + mean).to(BF)


def close(actual, expected, rtol=RTOL, atol=ATOL):
    torch.testing.assert_close(actual.detach().float().cpu(), expected.detach().float().cpu(),
                               rtol=rtol, atol=atol)


# ------------------------------------------------------------------ norms
@pytest.mark.parametrize("width", [128, 256, 2048, 100])
def test_rms_norm(gpu, width):
    from ppu_amd import kernels as K

    g = gen(KERNEL_SEED)
    x = randn(g, 7, width)
    w = randn(g, width)
    out = K.rms_norm(x.to(gpu), w.to(gpu))
    close(out, ref.rms_norm(x, w))


def test_rms_norm_fp32_weight(gpu):
    from ppu_amd import kernels as K

    g = gen(KERNEL_SEED + 1)
    x = randn(g, 3, 2048)
    w = torch.randn(2048, generator=g) * 0.02
    close(K.rms_norm(x.to(gpu), w.to(gpu)), ref.rms_norm(x, w))


@pytest.mark.parametrize("rows", [1, 7])
def test_residual_add_rms_norm(gpu, rows):
    from ppu_amd import kernels as K

    g = gen(KERNEL_SEED + 2)
    r = randn(g, rows, 2048)
    u = randn(g, rows, 2048)
    w = randn(g, 2048, scale=0.02, mean=1.0)
    r_out, y = K.residual_add_rms_norm(r.to(gpu), u.to(gpu), w.to(gpu))
    er, ey = ref.residual_add_rms_norm(r, u, w)
    assert torch.equal(r_out.cpu(), er), "bf16 residual add must be exact"
    close(y, ey)


def test_gated_rms_norm(gpu):
    from ppu_amd import kernels as K

    g = gen(KERNEL_SEED + 3)
    x = randn(g, 32, 128)
    gate = randn(g, 32, 128)
    w = randn(g, 128)
    close(K.gated_rms_norm(x.to(gpu), gate.to(gpu), w.to(gpu)), ref.gated_rms_norm(x, gate, w))


def test_gated_rms_norm_packed(gpu):
    """The prefill form reads z in place from the packed projection [L, 8320]
    (z = columns 6144..8191, 16 heads of 128): same bits as the copied z."""
    from ppu_amd import kernels as K

    g = gen(KERNEL_SEED + 6)
    tokens, heads = 37, 16
    core = randn(g, tokens * heads, 128)
    packed = randn(g, 1, tokens, 8320)
    w = randn(g, 128, scale=0.02, mean=1.0)
    z = packed[..., 6144:8192].reshape(tokens * heads, 128)
    exp = ref.gated_rms_norm(core, z, w)
    got = K.gated_rms_norm_packed(core.to(gpu), packed.to(gpu), 6144, heads, w.to(gpu))
    close(got, exp)
    copied = K.gated_rms_norm(core.to(gpu), z.contiguous().to(gpu), w.to(gpu))
    assert torch.equal(got, copied)


def test_silu_and_mul(gpu):
    from ppu_amd import kernels as K

    g = gen(KERNEL_SEED + 4)
    p = randn(g, 7, 12288)
    close(K.silu_and_mul(p.to(gpu)), ref.silu_and_mul(p))


@pytest.mark.parametrize("rows,width", [(8, 64), (72, 128), (1024, 6144), (200, 192)])
def test_silu_and_mul_t_equals_silu_and_mul_of_transpose(gpu, rows, width):
    """The transposing form on W @ X^T's channel-major product: bit-equal to
    silu_and_mul of the token-major product (same arithmetic), for token
    counts that do not fill the last 64-token tile too."""
    from ppu_amd import kernels as K

    g = gen(KERNEL_SEED + 16)
    packed = randn(g, rows, 2 * width, scale=2.0).to(gpu)
    got = K.silu_and_mul_t(packed.t().contiguous())
    assert torch.equal(got, K.silu_and_mul(packed))
    with pytest.raises(ValueError):
        K.silu_and_mul_t(packed.t().contiguous()[:, : rows - 1].contiguous() if rows > 8 else
                         torch.zeros(2 * width, 7, dtype=BF, device=gpu))


def test_attention_gate_mul(gpu):
    from ppu_amd import kernels as K

    g = gen(KERNEL_SEED + 5)
    packed = randn(g, 1, 5, 5120)
    x = randn(g, 1, 5, 2048)
    close(K.attention_gate_mul(x.to(gpu), packed.to(gpu), 256), ref.attention_gate_mul(x, packed, 256))


@pytest.mark.parametrize("tokens,hidden,head_dim", [(70, 2048, 256), (9, 36, 12), (0, 2048, 256)])
def test_attention_gate_mul_advance(gpu, tokens, hidden, head_dim):
    """The gate kernel's counter advance (the prefill's cache-length add_ moved
    into it): the counter grows by `amount` exactly once whatever the grid
    (16-byte form over 70 tokens, element form at head_dim 12, no tokens), and
    the output bits are those of the call without it."""
    from ppu_amd import kernels as K

    g = gen(KERNEL_SEED + 6)
    packed = randn(g, 1, tokens, 2 * hidden + 8).to(gpu)
    x = randn(g, 1, tokens, hidden).to(gpu)
    counter = torch.tensor(37, dtype=torch.int64, device=gpu)
    plain = K.attention_gate_mul(x, packed, head_dim)
    got = K.attention_gate_mul(x, packed, head_dim, advance=counter, amount=tokens + 5)
    torch.cuda.synchronize()
    assert int(counter) == 37 + tokens + 5
    assert torch.equal(got, plain)
    if tokens:
        close(got.cpu(), ref.attention_gate_mul(x.cpu(), packed.cpu(), head_dim))
    with pytest.raises(ValueError):
        K.attention_gate_mul(x, packed, head_dim, advance=counter.to(torch.int32), amount=1)


@pytest.mark.parametrize("screened", [False, True])
def test_lm_head_top1_mirror(gpu, screened):
    """The top-1 launch also stores the token into a mirror: pinned host
    memory (through its device address) or a second GPU tensor; pageable host
    memory is refused before any launch."""
    from ppu_amd import kernels as K

    g = torch.Generator(device=gpu).manual_seed(KERNEL_SEED + 63)
    v = 50000
    w = (torch.randn(v, 2048, device=gpu, generator=g) * 0.02).to(BF)
    h = torch.randn(1, 2048, device=gpu, generator=g).to(BF)
    screen = K.lm_head_screen_prep(w) if screened else None
    plain = int(K.lm_head_argmax(h, w, screen=screen))
    host = torch.full((1,), -1, dtype=torch.int64, pin_memory=True)
    dev2 = torch.full((1, 1), -1, device=gpu, dtype=torch.int64)
    out = torch.full((1, 1), -1, device=gpu, dtype=torch.int64)
    K.lm_head_argmax(h, w, out=out, mirror=host, screen=screen)
    K.lm_head_argmax(h, w, mirror=dev2, screen=screen)
    torch.cuda.synchronize()
    assert int(out) == int(host[0]) == int(dev2) == plain
    with pytest.raises(ValueError):
        K.lm_head_argmax(h, w, mirror=torch.zeros(1, dtype=torch.int64), screen=screen)
    with pytest.raises(ValueError):
        K.host_device_address(torch.zeros(1, dtype=torch.int64))


@pytest.mark.parametrize("width", [512, 2048, 4096])
def test_embed_rms_norm_equals_gather_then_norm(gpu, width):
    """The embedding lookup + first input norm launch gives the bits of the
    table gather followed by rms_norm (ids of any shape, repeats included);
    ids outside the table read its nearest end row, as the decode gather."""
    from ppu_amd import kernels as K

    g = gen(KERNEL_SEED + 9)
    table = randn(g, 300, width).to(gpu)
    w = randn(g, width, scale=0.02, mean=1.0).to(gpu)
    ids = torch.randint(0, 300, (2, 37), generator=g).to(gpu)
    ids[0, 5] = ids[1, 7]
    res, y = K.embed_rms_norm(table, ids, w, 1e-6)
    ref_res = table[ids]
    torch.cuda.synchronize()
    assert torch.equal(res, ref_res)
    assert torch.equal(y, K.rms_norm(ref_res, w, 1e-6))
    oob = torch.tensor([[-4, 300, 10**9]], device=gpu)
    r2, _ = K.embed_rms_norm(table, oob, w)
    assert torch.equal(r2[0], table[[0, 299, 299]])
    with pytest.raises(ValueError):
        K.embed_rms_norm(table[:, :100].contiguous(), ids, w[:100])


@pytest.mark.parametrize("tokens,hidden,head_dim", [(70, 2048, 256), (9, 4096, 128), (0, 2048, 256)])
def test_attention_gate_quant_equals_gate_then_quant(gpu, tokens, hidden, head_dim):
    """The gate + per-token quantisation launch gives the bits of the gate
    kernel followed by the quantiser (int8 rows and scales), and advances the
    counter once; all-zero gated rows keep the quantiser's zero rule."""
    from ppu_amd import kernels as K

    g = gen(KERNEL_SEED + 8)
    packed = randn(g, 1, tokens, 2 * hidden + 16).to(gpu)
    x = randn(g, 1, tokens, hidden).to(gpu)
    if tokens:
        x[0, 3] = 0.0  # a row whose gated values are all zero
    counter = torch.tensor(5, dtype=torch.int64, device=gpu)
    xq, sx = K.attention_gate_quant(x, packed, head_dim, advance=counter, amount=tokens + 1)
    eq, es = K.quantize_act_i8(K.attention_gate_mul(x, packed, head_dim))
    torch.cuda.synchronize()
    assert int(counter) == 5 + tokens + 1
    assert xq.shape == eq.shape and sx.shape == es.shape
    assert torch.equal(xq, eq) and torch.equal(sx, es)
    with pytest.raises(ValueError):
        K.attention_gate_quant(x, packed, 12)


def test_zero_tensors_many(gpu):
    """zero_tensors over 300 buffers (three launches of at most 128): every
    buffer is cleared, odd byte counts and empty ones included, and the bytes
    between the buffers are left as they were."""
    from ppu_amd import kernels as K

    g = gen(KERNEL_SEED + 7)
    sizes = torch.randint(0, 5000, (300,), generator=g).tolist()
    sizes[3], sizes[4], sizes[200] = 0, 1, 15
    starts, at = [], 0
    for n in sizes:
        starts.append(at)
        at += -(-n // 16) * 16 + 32  # a 16-byte aligned start and a gap after each buffer
    pool = torch.full((at,), 0xAB, dtype=torch.uint8, device=gpu)
    views = [pool[st : st + n] for st, n in zip(starts, sizes)]
    K.zero_tensors(views)
    torch.cuda.synchronize()
    mask = torch.zeros(at, dtype=torch.bool)
    for st, n in zip(starts, sizes):
        mask[st : st + n] = True
    host = pool.cpu()
    assert not host[mask].any()
    assert bool((host[~mask] == 0xAB).all())


# ------------------------------------------------------------------ GEMV
@pytest.mark.parametrize("n,k", [(6144, 2048), (8320, 2048), (5120, 2048), (2048, 2048),
                                 (2048, 6144), (257, 128), (100, 40)])
def test_linear(gpu, n, k):
    from ppu_amd import kernels as K

    g = gen(KERNEL_SEED + 6)
    x = randn(g, 1, 1, k)
    w = randn(g, n, k, scale=0.02)
    close(K.linear(x.to(gpu), w.to(gpu)), ref.linear(x, w))


def test_config1_residual_norm_gemv(gpu):
    """Benchmark config 1: x, residual ~N(0,1) [1,2048], w ~N(1,0.02), eps 1e-6,
    then W[6144,2048] ~N(0,0.02), fused in one launch."""
    from ppu_amd import kernels as K

    g = gen(KERNEL_SEED)
    x = randn(g, 1, 2048)
    r = randn(g, 1, 2048)
    nw = randn(g, 2048, scale=0.02, mean=1.0)
    W = randn(g, 6144, 2048, scale=0.02)
    r_out, y = K.residual_norm_linear(r.to(gpu), x.to(gpu), nw.to(gpu), 1e-6, W.to(gpu))
    er, en = ref.residual_add_rms_norm(r, x, nw, 1e-6)
    assert torch.equal(r_out.cpu(), er)
    close(y, ref.linear(en, W))


@pytest.mark.parametrize("k", [2048, 6144])
def test_swiglu_gemv(gpu, k):
    from ppu_amd import kernels as K

    g = gen(KERNEL_SEED + 7)
    x = randn(g, 1, 1, k)
    w = randn(g, 12288, k, scale=0.02)
    close(K.ppu_swiglu_gemv(x.to(gpu), w.to(gpu)), ref.swiglu_gemv(x, w))


def test_swiglu_fused_residual(gpu):
    from ppu_amd import kernels as K

    g = gen(KERNEL_SEED + 8)
    r = randn(g, 1, 1, 2048)
    u = randn(g, 1, 1, 2048)
    nw = randn(g, 2048, scale=0.02)
    w = randn(g, 12288, 2048, scale=0.02)
    r_out, y = K.residual_norm_linear(r.to(gpu), u.to(gpu), nw.to(gpu), 1e-6, w.to(gpu), swiglu=True)
    er, en = ref.residual_add_rms_norm(r, u, nw)
    assert torch.equal(r_out.cpu(), er)
    close(y, ref.swiglu_gemv(en, w))


# ------------------------------------------------------------------ lm_head
@pytest.mark.parametrize("v,k", [(257, 128), (248320, 2048), (5000, 2048)])
def test_lm_head_argmax(gpu, v, k):
    from ppu_amd import kernels as K

    g = gen(KERNEL_SEED + 9)
    h = randn(g, 1, k)
    w = randn(g, v, k, scale=0.02 if k == 2048 else 1.0)
    got = K.lm_head_argmax(h.to(gpu), w.to(gpu))
    assert got.dtype == torch.int64 and got.shape == (1, 1)
    exp = ref.lm_head_argmax(h, w)
    if int(got) != int(exp):
        # Only acceptable when the two bf16 logits tie within one fp32 rounding.
        logits = h.float() @ w.float().t()
        a, b = float(logits[0, int(got)]), float(logits[0, int(exp)])
        pytest.fail(f"argmax {int(got)} vs {int(exp)}: logits {a} vs {b}")


def test_lm_head_ties(gpu):
    from ppu_amd import kernels as K

    h = torch.zeros(1, 128, dtype=BF)
    w = torch.zeros(257, 128, dtype=BF)
    assert int(K.lm_head_argmax(h.to(gpu), w.to(gpu))) == 0
    g = gen(KERNEL_SEED + 10)
    h = randn(g, 1, 2048)
    w = randn(g, 9000, 2048, scale=0.02)
    w[7777] = w[123]
    w[8000] = w[123] * 4  # larger
    w[8500] = w[8000]
    got = int(K.lm_head_argmax(h.to(gpu), w.to(gpu)))
    assert got == int(ref.lm_head_argmax(h, w))


def _screened(gpu, h, w, **kw):
    from ppu_amd import kernels as K

    return K.lm_head_argmax(h, w, screen=K.lm_head_screen_prep(w), **kw)


@pytest.mark.parametrize("v", [248320, 50000, 1, 63, 4099])
def test_lm_head_screened_equals_full(gpu, v):
    """The int8-screened top-1 returns the full kernel's index, for the 2B
    vocabulary and ragged small ones, over hidden vectors of several scales
    (the screen's bound grows with |x|), and the oracle's index where the
    full kernel's is checked against it."""
    from ppu_amd import kernels as K

    g = torch.Generator(device=gpu).manual_seed(KERNEL_SEED + 60)
    w = (torch.randn(v, 2048, device=gpu, generator=g) * 0.02).to(BF)
    screen = K.lm_head_screen_prep(w)
    for scale in (0.25, 1.0, 4.0, 30.0):
        for _ in range(3):
            h = (torch.randn(1, 2048, device=gpu, generator=g) * scale).to(BF)
            full = int(K.lm_head_argmax(h, w))
            assert int(K.lm_head_argmax(h, w, screen=screen)) == full
    if v <= 50000:
        h = (torch.randn(1, 2048, device=gpu, generator=g)).to(BF)
        assert int(K.lm_head_argmax(h, w, screen=screen)) == int(ref.lm_head_argmax(h.cpu(), w.cpu()))


def test_lm_head_screened_ties_and_adversarial(gpu):
    """Planted exact ties (lowest index wins), a larger copy of a row, rows
    one bf16 ulp apart, all rows equal (every row a candidate), an all-zero
    hidden vector, a row far outside the others' range (an outlier scale) and
    an inf row (NaN bound: always recomputed): the same index as the full
    kernel every time."""
    from ppu_amd import kernels as K

    g = gen(KERNEL_SEED + 61)
    h = randn(g, 1, 2048)
    w = randn(g, 9000, 2048, scale=0.02)
    w[7777] = w[123]
    w[8000] = w[123] * 4
    w[8500] = w[8000]
    hg, wg = h.to(gpu), w.to(gpu)
    assert int(_screened(gpu, hg, wg)) == int(K.lm_head_argmax(hg, wg)) == int(ref.lm_head_argmax(h, w))
    # rows one ulp apart around the current winner
    best = int(K.lm_head_argmax(hg, wg))
    w2 = w.clone()
    w2[4000] = w[best]
    w2[4000, 0] = torch.nextafter(w[best, 0].float(), torch.tensor(1e9)).to(BF)
    w2g = w2.to(gpu)
    assert int(_screened(gpu, hg, w2g)) == int(K.lm_head_argmax(hg, w2g))
    same = w[5].expand(3000, 2048).contiguous().to(gpu)
    assert int(_screened(gpu, hg, same)) == 0 == int(K.lm_head_argmax(hg, same))
    _, n_same = _screened(gpu, hg, same, return_candidates=True)
    assert int(n_same) == 3000  # no row can be excluded
    zero_h = torch.zeros(1, 2048, dtype=BF, device=gpu)
    assert int(_screened(gpu, zero_h, wg)) == 0 == int(K.lm_head_argmax(zero_h, wg))
    w3 = w.clone()
    w3[17] = w[17] * 300
    w3g = w3.to(gpu)
    assert int(_screened(gpu, hg, w3g)) == int(K.lm_head_argmax(hg, w3g))
    w4 = w.clone()
    w4[29, 7] = float("inf")
    w4g = w4.to(gpu)
    assert int(_screened(gpu, hg, w4g)) == int(K.lm_head_argmax(hg, w4g))


def test_lm_head_screen_bound_holds(gpu):
    """The screen's upper bounds (left in the workspace) are at least every
    row's exact logit plus the bf16 rounding, and the largest lower bound is
    at most the largest logit: checked against fp64 dot products."""
    from ppu_amd import _lib
    from ppu_amd import kernels as K

    g = torch.Generator(device=gpu).manual_seed(KERNEL_SEED + 62)
    v = 60000
    w = (torch.randn(v, 2048, device=gpu, generator=g) * 0.02).to(BF)
    h = torch.randn(1, 2048, device=gpu, generator=g).to(BF)
    wq, sw, cr = K.lm_head_screen_prep(w)
    nbytes = _lib.load().q35_lm_head_top1_screened_workspace(v, 2048)
    ws = torch.empty(nbytes, device=gpu, dtype=torch.uint8)
    out = torch.empty(1, 1, device=gpu, dtype=torch.int64)
    _lib.call("q35_lm_head_top1_screened", w.data_ptr(), wq.data_ptr(), sw.data_ptr(), cr.data_ptr(),
              h.data_ptr(), v, 2048, ws.data_ptr(), nbytes, out.data_ptr(), None, None, 0,
              torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    upper = ws[: v * 4].view(torch.float32).double().cpu()
    exact = (w.double() @ h.double().t()).reshape(-1).cpu()
    assert bool((upper >= exact + exact.abs() * 2.0**-8).all())
    # per-workgroup largest lower bounds follow U (256-byte aligned), one per
    # workgroup of the screen's persistent grid (1 per CU)
    nb = torch.cuda.get_device_properties(gpu).multi_processor_count
    at = (v * 4 + 255) // 256 * 256
    lower_max = float(ws[at : at + 4 * nb].view(torch.float32).max())
    assert lower_max <= float(exact.max()) * (1 - 2.0**-8 * (1 if exact.max() > 0 else -1))
    # candidates: a few percent of the rows for these random weights
    frac = float((upper >= lower_max).double().mean())
    print(f"candidate fraction {frac:.4f}")
    assert frac < 0.2
    assert int(out) == int(K.lm_head_argmax(h, w))
    # the per-workgroup recomputed-row counts add up to exactly those rows
    import ctypes

    n = ctypes.c_int(0)
    off = _lib.load().q35_lm_head_screened_counts(v, ctypes.byref(n))
    nr = 2 * nb  # rescore workgroups (2 per CU) each count their rows
    assert n.value == nr and off + 4 * nr <= nbytes
    counts = ws[off : off + 4 * nr].view(torch.int32).long().cpu()
    assert int(counts.sum()) == int((upper >= lower_max).sum())
    _, total = K.lm_head_argmax(h, w, screen=(wq, sw, cr), return_candidates=True)
    assert int(total) == int(counts.sum())


def test_lm_head_screened_in_graph_with_feedback(gpu):
    """Captured in a graph with the token written to ``out`` and positions
    advanced: every replay equals the eager full kernel on the same input."""
    from ppu_amd import kernels as K

    g = torch.Generator(device=gpu).manual_seed(KERNEL_SEED + 63)
    w = (torch.randn(20000, 2048, device=gpu, generator=g) * 0.02).to(BF)
    screen = K.lm_head_screen_prep(w)
    h = torch.randn(1, 2048, device=gpu, generator=g).to(BF)
    tok = torch.zeros(1, 1, dtype=torch.int64, device=gpu)
    pos = torch.tensor([[7]], dtype=torch.int64, device=gpu)
    K.lm_head_argmax(h, w, out=tok, advance=pos, screen=screen)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        K.lm_head_argmax(h, w, out=tok, advance=pos, screen=screen)
    for r in range(3):
        h.copy_(torch.randn(1, 2048, device=gpu, generator=g).to(BF))
        tok.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert int(tok) == int(K.lm_head_argmax(h, w)) and int(pos) == 9 + r


# ------------------------------------------------------------------ DeltaNet
@pytest.mark.parametrize("seq_len", [1, 17])
@pytest.mark.parametrize("extra", [0, 32])
def test_causal_conv1d(gpu, seq_len, extra):
    from ppu_amd import kernels as K

    g = gen(KERNEL_SEED + 11)
    c = 64
    x = randn(g, 1, seq_len, c + extra)
    w = randn(g, c, 4)
    st0 = randn(g, 1, c, 4)
    st_ref = st0.clone()
    exp = ref.causal_conv1d(x, w, st_ref)
    st = st0.to(gpu)
    got = K.causal_conv1d_fused(x.to(gpu), w.to(gpu), st)
    close(got, exp)
    assert torch.equal(st.cpu(), st_ref)


def _delta_inputs(g, seq_len, heads=16, dim=128):
    qkv_w = 3 * heads * dim
    packed_w = qkv_w + heads * dim + 2 * heads
    qkv = randn(g, 1, seq_len, qkv_w)
    packed = randn(g, 1, seq_len, packed_w)
    packed[..., :qkv_w] = qkv
    a_log = randn(g, heads)
    dt_bias = randn(g, heads)
    state = torch.randn(1, heads, dim, dim, generator=g) * 0.01
    return qkv, packed, a_log, dt_bias, state


@pytest.mark.parametrize("seq_len", [1, 3, 63, 64, 200, 1024])
def test_delta_recurrent(gpu, seq_len):
    """Token scan below 64 tokens, the chunked closed form (64-token chunks on
    the matrix cores, partial last chunk) from 64 on; the incoming state is
    nonzero, so the carried state enters every chunk."""
    from ppu_amd import kernels as K

    g = gen(KERNEL_SEED + 12)
    qkv, packed, a_log, dt_bias, state = _delta_inputs(g, seq_len)
    st_ref = state.clone()
    exp = ref.delta_recurrent(qkv, packed, a_log, dt_bias, st_ref)
    st = state.to(gpu)
    got = K.delta_recurrent_fused(qkv.to(gpu), packed.to(gpu), a_log.to(gpu), dt_bias.to(gpu), st,
                                  precompute_factors=True)
    close(got, exp)
    # state: 1e-3 relative (the state tolerance of the parity contract), plus a tiny absolute floor.
    torch.testing.assert_close(st.cpu(), st_ref, rtol=1e-3, atol=1e-6)


@pytest.mark.parametrize("batch,heads,seq_len", [(2, 8, 130), (2, 6, 64), (1, 6, 257)])
def test_delta_chunked_batch_and_head_counts(gpu, batch, heads, seq_len):
    """The chunked form with several sequences and head counts that do and do
    not fill the 8-XCD placement of the chunk scan (H % 8 == 0 or not), ragged
    last chunks included: output and state against the oracle token loop, the
    gated form against the oracle norm of the same core."""
    from ppu_amd import kernels as K

    g = gen(KERNEL_SEED + 16)
    dim = 128
    qkv_w = 3 * heads * dim
    qkv = randn(g, batch, seq_len, qkv_w)
    width = qkv_w + heads * dim + 2 * heads
    packed = randn(g, batch, seq_len, (width + 7) // 8 * 8)  # rows padded to 16 bytes, as the model packs them
    packed[..., :qkv_w] = qkv
    a_log, dt_bias = randn(g, heads), randn(g, heads)
    state = torch.randn(batch, heads, dim, dim, generator=g) * 0.01
    norm_w = randn(g, dim, scale=0.02, mean=1.0)
    st_ref = state.clone()
    core_ref = ref.delta_recurrent(qkv, packed, a_log, dt_bias, st_ref)
    args = (qkv.to(gpu), packed.to(gpu), a_log.to(gpu), dt_bias.to(gpu))
    st = state.to(gpu)
    core = K.delta_recurrent_fused(*args, st)
    close(core, core_ref)
    torch.testing.assert_close(st.cpu(), st_ref, rtol=1e-3, atol=1e-6)
    st2 = state.to(gpu)
    got = K.delta_prefill_gated(*args, st2, norm_w.to(gpu), 1e-6)
    z = packed[..., 3 * heads * dim : 4 * heads * dim].reshape(-1, dim)
    exp = ref.gated_rms_norm(core.cpu().reshape(-1, dim), z, norm_w).reshape(batch, seq_len, heads, dim)
    close(got, exp)
    assert torch.equal(st2, st)


@pytest.mark.parametrize("seq_len", [3, 63, 200, 1024])
def test_delta_prefill_gated(gpu, seq_len):
    """Prefill recurrence + gated RMSNorm in one call (the norm is fused into
    the chunked output kernel from 64 tokens on). The core output of the
    unfused call is checked against the oracle recurrence, and the fused
    result against the oracle norm of that same core: the chain has four bf16
    roundings, so comparing it end to end against an oracle core that differs
    by one ulp in a few places would test the rounding chain, not the kernel.
    The final state equals the unfused call's bit for bit."""
    from ppu_amd import kernels as K

    g = gen(KERNEL_SEED + 14)
    heads, dim = 16, 128
    qkv, packed, a_log, dt_bias, state = _delta_inputs(g, seq_len)
    norm_w = randn(g, dim, scale=0.02, mean=1.0)
    st_ref = state.clone()
    core_ref = ref.delta_recurrent(qkv, packed, a_log, dt_bias, st_ref)
    args = (qkv.to(gpu), packed.to(gpu), a_log.to(gpu), dt_bias.to(gpu))
    st2 = state.to(gpu)
    core = K.delta_recurrent_fused(*args, st2)
    close(core, core_ref)
    st = state.to(gpu)
    got = K.delta_prefill_gated(*args, st, norm_w.to(gpu), 1e-6)
    z = packed[..., 3 * heads * dim : 4 * heads * dim].reshape(-1, dim)
    exp = ref.gated_rms_norm(core.cpu().reshape(-1, dim), z, norm_w).reshape(1, seq_len, heads, dim)
    close(got, exp)
    assert torch.equal(st, st2)
    torch.testing.assert_close(st.cpu(), st_ref, rtol=1e-3, atol=1e-6)


@pytest.mark.parametrize("seq_len", [64, 67, 200, 1024])
def test_delta_prefill_gated_conv_equals_conv_then_prefill(gpu, seq_len):
    """The causal conv folded into the chunk prep gives the output, recurrent
    state and conv state of the separate conv launch followed by the gated
    prefill, bit for bit (same conv arithmetic, same bf16 conv output), and
    rejects fewer than 64 tokens."""
    from ppu_amd import kernels as K

    g = gen(KERNEL_SEED + 15)
    heads, dim = 16, 128
    conv_dim = 3 * heads * dim
    _, packed, a_log, dt_bias, state = _delta_inputs(g, seq_len)
    conv_w = randn(g, conv_dim, 4, scale=0.3).to(gpu)
    norm_w = randn(g, dim, scale=0.02, mean=1.0).to(gpu)
    packed, a_log, dt_bias = packed.to(gpu), a_log.to(gpu), dt_bias.to(gpu)
    cs_a = torch.full((1, conv_dim, 4), 7.0, dtype=BF, device=gpu)  # prefill ignores the old state
    cs_b = cs_a.clone()
    st_a, st_b = state.to(gpu), state.to(gpu)
    qkv = K.causal_conv1d_fused(packed, conv_w, cs_a)
    y_a = K.delta_prefill_gated(qkv, packed, a_log, dt_bias, st_a, norm_w, 1e-6)
    y_b = K.delta_prefill_gated_conv(packed, conv_w, cs_b, a_log, dt_bias, st_b, norm_w, 1e-6)
    assert torch.equal(y_a, y_b)
    assert torch.equal(st_a, st_b)
    assert torch.equal(cs_a, cs_b)
    with pytest.raises(ValueError):
        K.delta_prefill_gated_conv(packed[:, :63].contiguous(), conv_w, cs_b, a_log, dt_bias, st_b,
                                   norm_w, 1e-6)


def test_config4_delta_64_steps(gpu):
    """Benchmark config 4: 16 heads x 128, S ~N(0,0.1), conv width 4 on q/k/v,
    beta = sigmoid(N(0,1)), g = -softplus(N(0,1)) (A_log = 0, dt_bias = 0),
    64 sequential decode tokens through the fused conv+delta+gated-norm kernel,
    against the oracle chain conv -> delta -> gated norm."""
    from ppu_amd import kernels as K

    g = gen(KERNEL_SEED + 13)
    heads, dim = 16, 128
    conv_dim = 3 * heads * dim
    packed_w = 8320
    conv_w = randn(g, conv_dim, 4, scale=0.02)
    a_log = torch.zeros(heads, dtype=BF)
    dt_bias = torch.zeros(heads, dtype=BF)
    norm_w = randn(g, dim, scale=0.02, mean=1.0)
    state = torch.randn(1, heads, dim, dim, generator=g) * 0.1
    conv_state = torch.zeros(1, conv_dim, 4, dtype=BF)
    st_ref, cs_ref = state.clone(), conv_state.clone()
    st_gpu, cs_gpu = state.to(gpu), conv_state.to(gpu)
    args_gpu = (conv_w.to(gpu), cs_gpu, a_log.to(gpu), dt_bias.to(gpu), st_gpu, norm_w.to(gpu), 1e-6)
    worst = 0.0
    for step in range(64):
        packed = randn(g, 1, 1, packed_w)
        qkv = ref.causal_conv1d(packed, conv_w, cs_ref)
        core = ref.delta_recurrent(qkv, packed, a_log, dt_bias, st_ref)
        z = packed[..., conv_dim : conv_dim + heads * dim].reshape(-1, dim)
        exp = ref.gated_rms_norm(core.reshape(-1, dim), z, norm_w)
        got = K.delta_decode_fused(packed.to(gpu), *args_gpu)
        close(got, exp)
        worst = max(worst, float(((st_gpu.cpu() - st_ref).abs().max() / st_ref.abs().max())))
    assert torch.equal(cs_gpu.cpu(), cs_ref)
    torch.testing.assert_close(st_gpu.cpu(), st_ref, rtol=1e-3, atol=1e-5)
    assert worst < 1e-3


def test_config4_delta_64_steps_production_chain(gpu):
    """Benchmark config 4 through the kernels the model's decode step runs: the
    single-token conv update (``causal_conv1d_fused``, L = 1) then the
    256-wave delta step (``delta_recurrent_fused``, L = 1) and the packed gated
    norm, 64 sequential tokens. Each step's core output within the bf16
    tolerance of the oracle's, and the recurrent state within 1e-3 relative
    (max-abs over max-abs, and L2) after every step, not only the last."""
    from ppu_amd import kernels as K

    g = gen(KERNEL_SEED + 23)
    heads, dim = 16, 128
    conv_dim = 3 * heads * dim
    packed_w = 8320
    conv_w = randn(g, conv_dim, 4, scale=0.02)
    a_log = torch.zeros(heads, dtype=BF)
    dt_bias = torch.zeros(heads, dtype=BF)
    norm_w = randn(g, dim, scale=0.02, mean=1.0)
    state = torch.randn(1, heads, dim, dim, generator=g) * 0.1
    conv_state = torch.zeros(1, conv_dim, 4, dtype=BF)
    st_ref, cs_ref = state.clone(), conv_state.clone()
    st_gpu, cs_gpu = state.to(gpu), conv_state.to(gpu)
    conv_w_gpu, a_gpu, dt_gpu, nw_gpu = conv_w.to(gpu), a_log.to(gpu), dt_bias.to(gpu), norm_w.to(gpu)
    worst_max = worst_l2 = 0.0
    for step in range(64):
        packed = randn(g, 1, 1, packed_w)
        qkv = ref.causal_conv1d(packed, conv_w, cs_ref)
        core = ref.delta_recurrent(qkv, packed, a_log, dt_bias, st_ref)
        z = packed[..., conv_dim : conv_dim + heads * dim].reshape(-1, dim)
        exp = ref.gated_rms_norm(core.reshape(-1, dim), z, norm_w)
        pg = packed.to(gpu)
        qkv_g = K.causal_conv1d_fused(pg, conv_w_gpu, cs_gpu)
        core_g = K.delta_recurrent_fused(qkv_g, pg, a_gpu, dt_gpu, st_gpu)
        close(qkv_g, qkv)
        close(core_g, core)
        got = K.gated_rms_norm_packed(core_g.reshape(-1, dim), pg, conv_dim, heads, nw_gpu, 1e-6)
        close(got, exp)
        d = st_gpu.cpu() - st_ref
        worst_max = max(worst_max, float(d.abs().max() / st_ref.abs().max()))
        worst_l2 = max(worst_l2, float(d.norm() / st_ref.norm()))
    print(f"state after 64 steps: worst max-abs rel {worst_max:.2e}, worst L2 rel {worst_l2:.2e}")
    assert torch.equal(cs_gpu.cpu(), cs_ref)
    torch.testing.assert_close(st_gpu.cpu(), st_ref, rtol=1e-3, atol=1e-5)
    assert worst_max < 1e-3 and worst_l2 < 1e-3


def test_delta_invariant_beta0_alpha1(gpu):
    """With beta = 0 (b -> -inf) and alpha = 1 (A_log -> -inf) the state is unchanged."""
    from ppu_amd import kernels as K

    g = gen(KERNEL_SEED + 14)
    qkv, packed, _, _, state = _delta_inputs(g, 1)
    packed[..., -32:] = -1e4  # a and b: beta = sigmoid(-1e4) = 0
    a_log = torch.full((16,), -1e4)
    dt_bias = torch.zeros(16)
    st = state.to(gpu)
    K.delta_recurrent_fused(qkv.to(gpu), packed.to(gpu), a_log.to(gpu), dt_bias.to(gpu), st)
    assert torch.equal(st.cpu(), state)


# ------------------------------------------------------------------ attention
def _qgkv_inputs(g, seq_len):
    q_heads, kv_heads, dim, rot = 8, 2, 256, 64
    packed = randn(g, 1, seq_len, 2 * q_heads * dim + 2 * kv_heads * dim)
    qw = randn(g, dim)
    kw = randn(g, dim)
    cos = randn(g, 1, seq_len, rot)
    sin = randn(g, 1, seq_len, rot)
    return packed, qw, kw, cos, sin


@pytest.mark.parametrize("seq_len,w_dtype", [(5, torch.float32), (70, torch.bfloat16)])
def test_qgkv_norm_rope(gpu, seq_len, w_dtype):
    """Prefill Q/K norm + RoPE (the 256-wide vector path) against the oracle,
    with fp32 and bf16 norm weights."""
    from ppu_amd import kernels as K

    g = gen(KERNEL_SEED + 15)
    packed, qw, kw, cos, sin = _qgkv_inputs(g, seq_len)
    qw, kw = qw.to(w_dtype), kw.to(w_dtype)
    kwargs = dict(q_heads=8, kv_heads=2, dim=256, rotary_dim=64)
    eq, ek, ev = ref.qgkv_norm_rope(packed, qw, kw, cos, sin, **kwargs)
    q, k, v = K.qgkv_norm_rope(packed.to(gpu), qw.to(gpu), kw.to(gpu), cos.to(gpu), sin.to(gpu), **kwargs)
    close(q, eq)
    close(k, ek)
    assert torch.equal(v.cpu(), ev)


def test_qgkv_cache_write(gpu):
    from ppu_amd import kernels as K

    g = gen(KERNEL_SEED + 16)
    packed, qw, kw, cos, sin = _qgkv_inputs(g, 5)
    kwargs = dict(q_heads=8, kv_heads=2, dim=256, rotary_dim=64)
    eq, ek, ev = ref.qgkv_norm_rope(packed, qw, kw, cos, sin, **kwargs)
    kc = torch.zeros(1, 2, 13, 256, dtype=BF, device=gpu)
    vc = torch.zeros_like(kc)
    start = torch.tensor(3, dtype=torch.int64, device=gpu)
    q, k, v = K.qgkv_norm_rope(packed.to(gpu), qw.to(gpu), kw.to(gpu), cos.to(gpu), sin.to(gpu),
                               cache_key=kc, cache_value=vc, cache_start=start, **kwargs)
    close(q, eq)
    close(kc[:, :, 3:8], ek)
    assert torch.equal(vc[:, :, 3:8].cpu(), ev)
    assert not kc[:, :, :3].any() and not vc[:, :, 8:].any()
    # A start past the end writes nothing (no out-of-bounds store).
    start.fill_(12)
    kc.zero_()
    K.qgkv_norm_rope(packed.to(gpu), qw.to(gpu), kw.to(gpu), cos.to(gpu), sin.to(gpu),
                     cache_key=kc, cache_value=vc, cache_start=start, **kwargs)
    assert kc[:, :, 12].abs().sum() > 0


@pytest.mark.parametrize("cache_len,n_valid", [(512, 1), (512, 7), (512, 370), (512, 512),
                                                (2048, 2048), (8192, 8192), (8192, 5000)])
def test_gqa_decode_attention(gpu, cache_len, n_valid):
    from ppu_amd import kernels as K

    g = gen(KERNEL_SEED + 17)
    q = randn(g, 1, 8, 1, 256)
    kc = randn(g, 1, 2, cache_len, 256)
    vc = randn(g, 1, 2, cache_len, 256)
    length = torch.tensor(n_valid, dtype=torch.int64)
    exp = ref.gqa_decode_attention(q, kc, vc, length, 0.0625)
    got = K.gqa_decode_attention(q.to(gpu), kc.to(gpu), vc.to(gpu), length.to(gpu), 0.0625)
    close(got, exp)


@pytest.mark.parametrize("fused", [False, True])
@pytest.mark.parametrize("cache_len,n_valid", [(1152, 1040), (512, 5), (8192, 6000)])
def test_gqa_decode_rows_past_valid_end_ignored(gpu, fused, cache_len, n_valid):
    """Cache rows at and past the valid length hold NaN / inf (a static
    cache's unwritten tail may hold any bits): the kernels request those rows
    before they know the length, so they must mask their scores and zero
    their V values. The output equals the oracle over the valid rows."""
    from ppu_amd import kernels as K

    g = gen(KERNEL_SEED + 21)
    kc = randn(g, 1, 2, cache_len, 256)
    vc = randn(g, 1, 2, cache_len, 256)
    kc[:, :, n_valid:] = float("nan")
    vc[:, :, n_valid:] = float("inf")
    vc[:, 1, n_valid + 1 :: 3] = float("nan")
    if not fused:
        q = randn(g, 1, 8, 1, 256)
        length = torch.tensor(n_valid, dtype=torch.int64)
        exp = ref.gqa_decode_attention(q, kc, vc, length, 0.0625)
        got = K.gqa_decode_attention(q.to(gpu), kc.to(gpu), vc.to(gpu), length.to(gpu), 0.0625)
        close(got, exp)
        return
    from transformers.models.qwen3_5.modeling_qwen3_5 import Qwen3_5TextRotaryEmbedding

    from ppu_amd import synth

    packed = randn(g, 1, 1, 5120)
    qw, kw = randn(g, 256, scale=0.1), randn(g, 256, scale=0.1)
    rot = Qwen3_5TextRotaryEmbedding(synth.config_tiny())
    pos = torch.tensor((n_valid,) * 3, dtype=torch.int64).view(3, 1, 1)
    cos, sin = rot(torch.zeros(1, 1, 8, dtype=BF), pos)
    kr, vr = kc.clone(), vc.clone()
    q, _, _ = ref.qgkv_norm_rope(packed, qw, kw, cos, sin, q_heads=8, kv_heads=2, dim=256,
                                 rotary_dim=64, cache_key=kr, cache_value=vr, cache_start=n_valid)
    att = ref.gqa_decode_attention(q, kr, vr, n_valid + 1, 0.0625)
    exp = ref.attention_gate_mul(att, packed, 256)
    length = torch.tensor(n_valid, dtype=torch.int64, device=gpu)
    got = K.gqa_decode_fused(packed.to(gpu), qw.to(gpu), kw.to(gpu), rot.inv_freq.to(gpu),
                             pos.to(gpu), kc.to(gpu), vc.to(gpu), length, 0.0625, q_heads=8)
    assert bool(torch.isfinite(got).all())
    close(got, exp)


@pytest.mark.parametrize("q_heads,kv_heads", [(2, 2), (4, 2), (16, 2), (4, 4), (8, 1)])
def test_gqa_decode_back_to_back(gpu, q_heads, kv_heads):
    """Head groupings G = 1, 2, 4, 8 and several launches queued without a host
    sync in between: the in-kernel split merge keeps per-KV-head arrival
    counters that each launch must leave at zero for the next one."""
    from ppu_amd import kernels as K

    g = gen(KERNEL_SEED + 20)
    cache_len = 1152
    kc = randn(g, 1, kv_heads, cache_len, 256)
    vc = randn(g, 1, kv_heads, cache_len, 256)
    kg, vg = kc.to(gpu), vc.to(gpu)
    cases = []
    for n_valid in (1152, 65, 3, 700):
        q = randn(g, 1, q_heads, 1, 256)
        length = torch.tensor(n_valid, dtype=torch.int64)
        got = K.gqa_decode_attention(q.to(gpu), kg, vg, length.to(gpu), 0.0625)
        cases.append((got, ref.gqa_decode_attention(q, kc, vc, length, 0.0625)))
    for got, exp in cases:
        close(got, exp)


def test_gqa_decode_gate_fused(gpu):
    from ppu_amd import kernels as K

    g = gen(KERNEL_SEED + 18)
    q = randn(g, 1, 8, 1, 256)
    kc = randn(g, 1, 2, 512, 256)
    vc = randn(g, 1, 2, 512, 256)
    packed = randn(g, 1, 1, 5120)
    length = torch.tensor(300, dtype=torch.int64)
    att = ref.gqa_decode_attention(q, kc, vc, length, 0.0625)
    exp = ref.attention_gate_mul(att, packed, 256)
    got = K.gqa_decode_attention(q.to(gpu), kc.to(gpu), vc.to(gpu), length.to(gpu), 0.0625,
                                 packed_gate=packed.to(gpu))
    close(got, exp)


@pytest.mark.parametrize("seq_len,kv_start", [(33, 0), (64, 16), (1, 0), (100, 37), (1024, 0),
                                             (300, 500)])
def test_prefill_attention(gpu, seq_len, kv_start):
    """Causal GQA prefill (MFMA flash attention, P as bf16 hi + lo parts)
    against the fp64 oracle, rtol 1e-2 / atol 1e-3 on the bf16 output. Cache
    rows past the prompt hold NaN, which must not reach the output."""
    from ppu_amd import kernels as K

    g = gen(KERNEL_SEED + 19)
    q = randn(g, 1, 8, seq_len, 256)
    kc = randn(g, 1, 2, kv_start + seq_len + 5, 256)
    vc = randn(g, 1, 2, kv_start + seq_len + 5, 256)
    exp = ref.prefill_attention(q, kc, vc, 0.0625, kv_start)
    kg, vg = kc.to(gpu), vc.to(gpu)
    kg[:, :, kv_start + seq_len:] = float("nan")
    vg[:, :, kv_start + seq_len:] = float("nan")
    got = K.gqa_prefill_attention(q.to(gpu), kg, vg, 0.0625, kv_start=kv_start)
    close(got, exp)


@pytest.mark.parametrize("q_heads,kv_heads", [(2, 2), (8, 1), (4, 2)])
def test_prefill_attention_groupings(gpu, q_heads, kv_heads):
    """Head groupings G = 1, 8, 2 and the device-length form (start = valid
    length - L, as the static-cache prefill passes it)."""
    from ppu_amd import kernels as K

    g = gen(KERNEL_SEED + 23)
    seq_len, start = 77, 20
    q = randn(g, 1, q_heads, seq_len, 256)
    kc = randn(g, 1, kv_heads, 128, 256)
    vc = randn(g, 1, kv_heads, 128, 256)
    exp = ref.prefill_attention(q, kc, vc, 0.0625, start)
    valid = torch.tensor(start + seq_len, dtype=torch.int64, device=gpu)
    got = K.gqa_prefill_attention(q.to(gpu), kc.to(gpu), vc.to(gpu), 0.0625, valid_length=valid)
    close(got, exp)
    # the length before the prompt (its advance deferred to the gate kernel): same bits
    before = torch.tensor(start, dtype=torch.int64, device=gpu)
    got_s = K.gqa_prefill_attention(q.to(gpu), kc.to(gpu), vc.to(gpu), 0.0625, valid_length=before,
                                    length_is_start=True)
    assert torch.equal(got_s, got)


@pytest.mark.parametrize("q_heads,kv_heads", [(8, 2), (4, 2)])
def test_prefill_attention_split_keys(gpu, q_heads, kv_heads):
    """Query tiles with more than 4 key blocks of 64 split their key range over
    workgroups and are merged by a second launch; with no workspace the same
    call runs unsplit. Device length with a prompt that starts at 600 of a
    1024-row cache (tiles cover 10-13 key blocks)."""
    from ppu_amd import _lib
    from ppu_amd import kernels as K

    g = gen(KERNEL_SEED + 24)
    seq_len, start, cache = 200, 600, 1024
    q = randn(g, 1, q_heads, seq_len, 256)
    kc = randn(g, 1, kv_heads, cache, 256)
    vc = randn(g, 1, kv_heads, cache, 256)
    exp = ref.prefill_attention(q, kc, vc, 0.0625, start)
    valid = torch.tensor(start + seq_len, dtype=torch.int64, device=gpu)
    qg, kg, vg = q.to(gpu), kc.to(gpu), vc.to(gpu)
    kg[:, :, start + seq_len:] = float("nan")
    vg[:, :, start + seq_len:] = float("nan")
    assert _lib.load().q35_gqa_prefill_workspace(1, q_heads, kv_heads, seq_len, cache) > 0
    got = K.gqa_prefill_attention(qg, kg, vg, 0.0625, valid_length=valid)
    close(got, exp)
    before = torch.tensor(start, dtype=torch.int64, device=gpu)
    assert torch.equal(K.gqa_prefill_attention(qg, kg, vg, 0.0625, valid_length=before,
                                               length_is_start=True), got)
    unsplit = torch.empty_like(got)
    _lib.call("q35_gqa_prefill", qg.data_ptr(), kg.data_ptr(), vg.data_ptr(), unsplit.data_ptr(),
              1, q_heads, kv_heads, 256, seq_len, cache, 0, valid.data_ptr(), 0.0625, None, 0,
              torch.cuda.current_stream().cuda_stream)
    close(unsplit, exp)


# ------------------------------------------------------------------ A8W8
@pytest.mark.parametrize("n,k", [(12288, 2048), (2048, 6144), (96, 64)])
def test_quantize_weight_bit_exact(gpu, n, k):
    from ppu_amd import kernels as K

    g = gen(KERNEL_SEED + 20)
    w = randn(g, n, k, scale=0.02)
    w[0] = 0  # zero row -> scale 1
    wq, s = K.quantize_weight_i8(w.to(gpu))
    ewq, es = oa.quantize_weight(w)
    assert np.array_equal(wq.cpu().numpy(), ewq)
    assert np.array_equal(s.cpu().numpy(), es)


@pytest.mark.parametrize("m", [1, 2, 4, 7, 13, 16, 17])
@pytest.mark.parametrize("n,k", [(12288, 2048), (2048, 6144), (1000, 2048), (1000, 6144)])
def test_a8w8_linear_config2(gpu, m, n, k):
    """Benchmark config 2: int8 quantisation and int32 accumulators bit-exact,
    bf16 dequant output within rtol 1e-2 / atol 1e-3."""
    from ppu_amd import kernels as K

    g = gen(KERNEL_SEED + 21)
    w = randn(g, n, k, scale=0.02)
    x = randn(g, m, k)
    x[0, :5] = 0
    wq, sw = K.quantize_weight_i8(w.to(gpu))
    y, xq, sx, acc = K.a8w8_linear(x.to(gpu), wq, sw, return_quant=True, return_acc=True)
    ewq, esw = oa.quantize_weight(w)
    ey, exq, esx, eacc = oa.a8w8_linear(x, ewq, esw)
    assert np.array_equal(xq.cpu().numpy(), exq)
    assert np.array_equal(sx.cpu().numpy(), esx)
    assert np.array_equal(acc.cpu().numpy(), eacc)
    close(y, ey)
    # the dequant is the oracle's expression on exact accumulators: bit-exact
    assert torch.equal(y.cpu(), ey)
    if m > 16 and k % 256 == 0:  # the hand-written int8 GEMM: the same bits
        assert torch.equal(K.gemm_a8w8(xq, sx, wq, sw).cpu(), ey)


@pytest.mark.parametrize("m", [4, 300])
def test_a8w8_swiglu_prefill(gpu, m):
    """Fused int32 dequant + SwiGLU equals a8w8_linear followed by silu_and_mul
    bit for bit, and the oracle's A8W8 linear + SiLU-mul within tolerance."""
    from ppu_amd import kernels as K

    g = gen(KERNEL_SEED + 24)
    n, k = 6144, 2048
    w = randn(g, 2 * n, k, scale=0.02)
    x = randn(g, m, k)
    wq, sw = K.quantize_weight_i8(w.to(gpu))
    xg = x.to(gpu)
    y = K.a8w8_swiglu(xg, wq, sw)
    two_step = K.silu_and_mul(K.a8w8_linear(xg, wq, sw))
    assert torch.equal(y, two_step)
    ewq, esw = oa.quantize_weight(w)
    close(y, ref.silu_and_mul(oa.a8w8_linear(x, ewq, esw)[0]))


@pytest.mark.parametrize("m", [1, 4, 16])
def test_a8w8_zero_row(gpu, m):
    """An all-zero token row quantises to 0 with scale 0 (0 * inf -> NaN -> 0)."""
    from ppu_amd import kernels as K

    g = gen(KERNEL_SEED + 22)
    w = randn(g, 64, 2048, scale=0.02)
    x = randn(g, m, 2048)
    x[m - 1] = 0
    wq, sw = K.quantize_weight_i8(w.to(gpu))
    y, xq, sx = K.a8w8_linear(x.to(gpu), wq, sw, return_quant=True)
    assert not xq[m - 1].any() and float(sx[m - 1]) == 0.0 and not y[m - 1].float().any()
    if m > 1:
        assert xq[0].any() and float(sx[0]) > 0.0


@pytest.mark.parametrize("m,n,k", [(1024, 12288, 2048), (300, 1000, 2048), (64, 2048, 6144),
                                   (1, 200, 128)])
def test_gemm_bf16(gpu, m, n, k):
    """Matrix-core GEMM vs the fp32 product, rounded once to bf16: rtol 1e-2 /
    atol 1e-3 against the bf16-rounded reference (ragged M and N tiles)."""
    from ppu_amd import kernels as K

    g = gen(KERNEL_SEED + 90)
    x, w = randn(g, m, k), randn(g, n, k, scale=0.02)
    y = K.gemm_bf16(x.to(gpu), w.to(gpu))
    close(y, (x.float() @ w.float().t()).to(BF))


_STAGE_BYTES = {t: 128 for t in range(9)}


@pytest.mark.parametrize("tile,splits", [(0, 1), (4, 1), (5, 1), (1, 1), (1, 2), (1, 3), (1, 8),
                                         (2, 1), (2, 2), (2, 4), (3, 1), (3, 3), (6, 1), (6, 2), (7, 4),
                                         (8, 1), (8, 2)])
@pytest.mark.parametrize("m,n,k", [(1024, 2048, 6144), (300, 700, 1536)])
def test_gemm_bf16_split_plans(gpu, tile, splits, m, n, k):
    """Every tile shape with K split over workgroups (the last one to finish a
    tile sums the partials): the fp32 product within the bf16 bar, ragged
    tiles included; the same launch twice in a row and three graph replays
    give identical bits (the arrival counters in the workspace reset
    themselves and the split order of the sum is fixed)."""
    from ppu_amd import kernels as K

    if (2 * k // _STAGE_BYTES[tile]) % splits:
        pytest.skip("the stage count must divide into the splits")
    g = gen(KERNEL_SEED + 92)
    x, w = randn(g, m, k), randn(g, n, k, scale=0.02)
    xg, wg = x.to(gpu), w.to(gpu)
    y1 = K.gemm_bf16(xg, wg, plan=(tile, splits))
    y2 = K.gemm_bf16(xg, wg, plan=(tile, splits))
    close(y1, (x.float() @ w.float().t()).to(BF))
    assert torch.equal(y1, y2)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        y3 = K.gemm_bf16(xg, wg, plan=(tile, splits))
    for _ in range(3):
        y3.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(y3, y1)


def test_gemm_rejects_invalid_plans(gpu):
    """Split K is refused for the 256x192 tiles and for SwiGLU kinds, and for a
    split that does not divide the stage count; the direct-store tiles refuse
    the dequant and SwiGLU kinds; a K that is not a multiple of the stage
    width is refused before any launch."""
    from ppu_amd import kernels as K

    x = torch.zeros(64, 2048, dtype=BF, device=gpu)
    w = torch.zeros(256, 2048, dtype=BF, device=gpu)
    for plan in ((0, 2), (4, 2), (5, 2), (1, 5), (9, 1)):
        with pytest.raises((ValueError, RuntimeError)):
            K.gemm_bf16(x, w, plan=plan)
    with pytest.raises((ValueError, RuntimeError)):
        K.gemm_bf16(x, w, swiglu=True, plan=(1, 2))
    with pytest.raises((ValueError, RuntimeError)):
        K.gemm_bf16(x, w, swiglu=True, plan=(5, 1))
    with pytest.raises(ValueError):
        K.gemm_bf16(x[:, :96].contiguous(), w[:, :96].contiguous())


_EXACT_CACHE: dict = {}


def _exact_i8_product(xq, wq):
    """int8 x int8 dot products summed exactly (|sum| < 2^53 in float64)."""
    return (xq.cpu().double() @ wq.cpu().double().t()).to(torch.int64)


@pytest.mark.parametrize("plan", [None, (0, 1), (4, 1), (1, 1), (1, 2), (1, 4), (2, 1), (2, 2),
                                  (3, 1), (3, 4)])
@pytest.mark.parametrize("m,n,k", [(1024, 2048, 6144), (300, 1000, 2048), (17, 200, 256)])
def test_gemm_a8w8(gpu, plan, m, n, k):
    """int8 matrix-core GEMM with the dequant epilogue: bit-exact against the
    oracle's dequant of the exact integer product, for every tile shape and
    K split (ragged tiles included); repeated launches and three graph
    replays give the same bits."""
    from ppu_amd import kernels as K

    if plan is not None and (k // _STAGE_BYTES[plan[0]]) % plan[1]:
        pytest.skip("the stage count must divide into the splits")
    g = gen(KERNEL_SEED + 93)
    w, x = randn(g, n, k, scale=0.02), randn(g, m, k)
    x[m // 2] = 0  # a zero row: scale 0, output 0
    wq, sw = K.quantize_weight_i8(w.to(gpu))
    xq, sx = K.quantize_act_i8(x.to(gpu))
    y1 = K.gemm_a8w8(xq, sx, wq, sw, plan=plan)
    y2 = K.gemm_a8w8(xq, sx, wq, sw, plan=plan)
    acc = _exact_i8_product(xq, wq)
    assert int(acc.abs().max()) < 2**31
    exp = oa.dequant(acc.numpy().astype(np.int32), sx.cpu().numpy(), sw.cpu().numpy())
    assert torch.equal(y1.cpu(), exp)
    assert torch.equal(y1, y2)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        y3 = K.gemm_a8w8(xq, sx, wq, sw, plan=plan)
    for _ in range(3):
        y3.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(y3, y1)


@pytest.mark.parametrize("plan", [None, (0, 1), (4, 1), (5, 1), (1, 2), (2, 3), (3, 8), (6, 2), (8, 1),
                                  (8, 4)])
@pytest.mark.parametrize("m,n,k", [(1024, 2048, 6144), (1024, 8320, 2048), (33, 520, 1024)])
def test_int8_gemm_int32_exact(gpu, plan, m, n, k):
    """The int8 GEMM's int32 accumulators (what the A8W8 prefill hands to the
    fused dequant kernels) equal the exact integer product, split plans
    included; graph replays give the same values."""
    from ppu_amd import kernels as K

    if plan is not None and (k // _STAGE_BYTES[plan[0]]) % plan[1]:
        pytest.skip("the stage count must divide into the splits")
    g = torch.Generator(device=gpu).manual_seed(KERNEL_SEED + 97)
    xq = torch.randint(-128, 128, (m, k), device=gpu, dtype=torch.int8, generator=g)
    wq = torch.randint(-127, 128, (n, k), device=gpu, dtype=torch.int8, generator=g)
    if (m, n, k) not in _EXACT_CACHE:  # the same seeded operands for every plan
        _EXACT_CACHE[(m, n, k)] = _exact_i8_product(xq, wq)
    exp = _EXACT_CACHE[(m, n, k)]
    acc = torch.empty((m, n), device=gpu, dtype=torch.int32)
    K.gemm_into(xq, wq, acc, K.GEMM_I32, plan=plan)
    torch.cuda.synchronize()
    assert torch.equal(acc.cpu().to(torch.int64), exp)
    if plan is None:
        assert torch.equal(K.a8w8_int_gemm(xq, wq), acc)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        K.gemm_into(xq, wq, acc, K.GEMM_I32, plan=plan)
    for _ in range(2):
        acc.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(acc.cpu().to(torch.int64), exp)


@pytest.mark.parametrize("plan", [None, (0, 1), (4, 1), (2, 1), (3, 1)])
@pytest.mark.parametrize("m,n,k", [(1024, 6144, 2048), (200, 504, 2048)])
def test_gemm_a8w8_swiglu(gpu, plan, m, n, k):
    """Packed gate/up int8 GEMM with dequant + SwiGLU in the epilogue: the same
    bits as the exact integer product put through q35_dequant_swiglu_i32 (the
    separate dequant + SwiGLU kernel), which a8w8_swiglu runs for prefill."""
    from ppu_amd import _lib
    from ppu_amd import kernels as K

    g = gen(KERNEL_SEED + 94)
    w, x = randn(g, 2 * n, k, scale=0.02), randn(g, m, k)
    wq, sw = K.quantize_weight_i8(w.to(gpu))
    xq, sx = K.quantize_act_i8(x.to(gpu))
    y = K.gemm_a8w8(xq, sx, wq, sw, swiglu=True, plan=plan)
    acc = _exact_i8_product(xq, wq).to(torch.int32).to(gpu)
    exp = torch.empty((m, n), device=gpu, dtype=BF)
    _lib.call("q35_dequant_swiglu_i32", acc.data_ptr(), sx.data_ptr(), sw.data_ptr(),
              exp.data_ptr(), m, n, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert torch.equal(y, exp)
    if plan is None:
        assert torch.equal(K.a8w8_swiglu(x.to(gpu), wq, sw), exp)


@pytest.mark.parametrize("rows", [1024, 37])
@pytest.mark.parametrize("w_f32", [False, True])
def test_residual_rmsnorm_dequant_quant(gpu, rows, w_f32):
    """The fused A8W8 prefill row kernel gives the same bits as the separate
    chain: dequant of the int32 accumulators -> residual add + RMSNorm ->
    per-token int8 quantisation (and the bf16 rows when asked), a zero row
    included."""
    from ppu_amd import kernels as K

    g = torch.Generator(device=gpu).manual_seed(KERNEL_SEED + 95)
    acc = torch.randint(-2**20, 2**20, (rows, 2048), device=gpu, dtype=torch.int32, generator=g)
    sx = torch.rand(rows, 1, device=gpu, generator=g) * 1e-3
    sw = torch.rand(2048, device=gpu, generator=g) * 1e-3
    res = torch.randn(rows, 2048, device=gpu, generator=g).to(BF)
    nw = (torch.randn(2048, device=gpu, generator=g) * 0.05).to(torch.float32 if w_f32 else BF)
    acc[rows // 2] = 0
    res[rows // 2] = 0
    upd = K.dequant_linear_i32(acc, sx, sw)
    r_exp, y_exp = K.residual_add_rms_norm(res, upd, nw, 1e-6)
    q_exp, s_exp = K.quantize_act_i8(y_exp)
    r, y, q, sy = K.residual_rmsnorm_dequant_quant(res, acc, sx, sw, nw, 1e-6, normalized=True)
    assert torch.equal(r, r_exp) and torch.equal(y, y_exp)
    assert torch.equal(q, q_exp) and torch.equal(sy, s_exp)
    r2, y2, q2, s2 = K.residual_rmsnorm_dequant_quant(res, acc, sx, sw, nw, 1e-6)
    assert y2 is None and torch.equal(r2, r_exp) and torch.equal(q2, q_exp) and torch.equal(s2, s_exp)


@pytest.mark.parametrize("m,n", [(1024, 6144), (300, 1024), (17, 200)])
def test_dequant_swiglu_quant(gpu, m, n):
    """SwiGLU of the packed gate/up accumulators quantised per token: the same
    bits as q35_dequant_swiglu_i32 followed by the activation quantiser."""
    from ppu_amd import _lib
    from ppu_amd import kernels as K

    g = torch.Generator(device=gpu).manual_seed(KERNEL_SEED + 96)
    acc = torch.randint(-2**20, 2**20, (m, 2 * n), device=gpu, dtype=torch.int32, generator=g)
    sx = torch.rand(m, 1, device=gpu, generator=g) * 1e-3
    sw = torch.rand(2 * n, device=gpu, generator=g) * 1e-3
    act = torch.empty((m, n), device=gpu, dtype=BF)
    _lib.call("q35_dequant_swiglu_i32", acc.data_ptr(), sx.data_ptr(), sw.data_ptr(), act.data_ptr(),
              m, n, torch.cuda.current_stream().cuda_stream)
    q_exp, s_exp = K.quantize_act_i8(act)
    q, s = K.dequant_swiglu_quant(acc, sx, sw)
    assert torch.equal(q, q_exp) and torch.equal(s, s_exp)


@pytest.mark.parametrize("m", [1024, 90])
def test_gemm_i8_swiglu_then_quant_equals_dequant_swiglu_quant(gpu, m):
    """The A8W8 prefill MLP runs the SwiGLU in the int8 GEMM's epilogue and
    quantises its bf16 output per token: the same int8 rows and scales as
    quantising the SwiGLU of the int32 [gate; up] accumulators."""
    from ppu_amd import kernels as K

    g = torch.Generator(device=gpu).manual_seed(KERNEL_SEED + 97)
    w = torch.randint(-127, 128, (2 * 6144, 2048), device=gpu, dtype=torch.int8, generator=g)
    sw = torch.rand(2 * 6144, device=gpu, generator=g) * 1e-3
    x = torch.randn(m, 2048, device=gpu, generator=g).to(BF)
    xq, sx = K.quantize_act_i8(x)
    q_exp, s_exp = K.dequant_swiglu_quant(K.a8w8_int_gemm(xq, w), sx, sw)
    q, s = K.quantize_act_i8(K.gemm_a8w8(xq, sx, w, sw, swiglu=True))
    assert torch.equal(q, q_exp) and torch.equal(s.reshape(-1), s_exp.reshape(-1))


@pytest.mark.parametrize("m,n,k", [(1024, 6144, 2048), (200, 500, 2048)])
def test_gemm_swiglu_bf16(gpu, m, n, k):
    """Packed gate/up GEMM with the SwiGLU epilogue vs F.linear + silu_and_mul
    rounding points on the fp32 product. g and u are each rounded to bf16 from
    fp32 sums taken in another order, so a one-ulp flip in g and in u can
    compound with the final rounding: every element within rtol 2e-2 /
    atol 2e-3, and all but 1e-5 of them within the rtol 1e-2 / atol 1e-3 bar."""
    from ppu_amd import kernels as K

    g = gen(KERNEL_SEED + 91)
    x, w = randn(g, m, k), randn(g, 2 * n, k, scale=0.02)
    y = K.gemm_bf16(x.to(gpu), w.to(gpu), swiglu=True).float().cpu()
    exp = ref.silu_and_mul((x.float() @ w.float().t()).to(BF)).float()
    close(y, exp, rtol=2e-2, atol=2e-3)
    outside = ((y - exp).abs() > 1e-3 + 1e-2 * exp.abs()).sum().item()
    assert outside <= 1e-5 * exp.numel()


@pytest.mark.parametrize("one_round", [False, True])
@pytest.mark.parametrize("nbytes", [16, 1 << 20, (9 << 20) + 48])
def test_stream_read(gpu, nbytes, one_round):
    """The read-rate probe reads every 16-byte group exactly once: the XOR of
    its per-thread words is the XOR of all words of the buffer (sizes below,
    above and past one full 8-load sweep of the grid, with a tail), for the
    persistent grid and the one-round grid."""
    import numpy as np

    from ppu_amd import kernels as K

    g = gen(KERNEL_SEED + 15)
    words = torch.randint(-(2**31), 2**31 - 1, (nbytes // 4,), generator=g, dtype=torch.int32)
    out = K.stream_read(words.to(gpu), one_round=one_round)
    torch.cuda.synchronize()
    got = np.bitwise_xor.reduce(out.cpu().numpy())
    assert got == np.bitwise_xor.reduce(words.numpy())


def test_gemm_bf16_rejects_k():
    from ppu_amd import kernels as K

    with pytest.raises(ValueError):
        K.gemm_bf16(torch.zeros(4, 96, dtype=BF), torch.zeros(8, 96, dtype=BF))


@pytest.mark.parametrize("m", [3, 8, 16])
@pytest.mark.parametrize("n,k", [(12288, 2048), (2048, 6144)])
def test_a8w8_prequantised_abi(gpu, m, n, k):
    """q35_gemv_a8w8 with x = NULL: the int8 rows and their scales are inputs
    (the skinny matrix-core path without the fused quantisation); int32
    accumulators bit-exact, one all-zero token row included."""
    from ppu_amd import _lib
    from ppu_amd import kernels as K

    g = gen(KERNEL_SEED + 23)
    w = randn(g, n, k, scale=0.02)
    x = randn(g, m, k)
    x[1] = 0
    wq, sw = K.quantize_weight_i8(w.to(gpu))
    ewq, esw = oa.quantize_weight(w)
    ey, exq, esx, eacc = oa.a8w8_linear(x, ewq, esw)
    xq = torch.from_numpy(exq).to(gpu)
    sx = torch.from_numpy(esx).reshape(m, 1).to(gpu)
    swf = sw.reshape(-1).float().contiguous()
    y = torch.empty(m, n, dtype=BF, device=gpu)
    acc = torch.empty(m, n, dtype=torch.int32, device=gpu)
    _lib.call("q35_gemv_a8w8", None, xq.data_ptr(), sx.data_ptr(), wq.data_ptr(), swf.data_ptr(),
              y.data_ptr(), acc.data_ptr(), m, n, k, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert np.array_equal(acc.cpu().numpy(), eacc)
    close(y, ey)
    # the dequant is the oracle's expression on exact accumulators: bit-exact
    assert torch.equal(y.cpu(), ey)
    if m > 16 and k % 256 == 0:  # the hand-written int8 GEMM: the same bits
        assert torch.equal(K.gemm_a8w8(xq, sx, wq, sw).cpu(), ey)


def _i8_row(prologue, x, u, nw):
    """The oracle's normalised activation row for a GEMV prologue."""
    if prologue == 0:
        return x
    if prologue == 1:
        return ref.rms_norm(x, nw)
    if prologue == 2:
        return ref.residual_add_rms_norm(x, u, nw)[1]
    k = x.shape[-1]
    return ref.gated_rms_norm(x.reshape(-1, 128), u.reshape(-1, 128), nw).reshape(1, k)


def _rel(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return float((a - b).norm() / b.norm())


@pytest.mark.parametrize("prologue", [0, 1, 2, 3])
@pytest.mark.parametrize("n,k", [(2048, 2048), (1000, 6144), (4352, 1024)])
def test_gemv_i8_prologues(gpu, prologue, n, k):
    """int8-weight GEMV (A8W8, one token) with each prologue. Bit-exact on the
    kernel's own normalised row (x_norm_out): its quantisation (xq, s_x), the
    int32 accumulators and the dequantised bf16 output; the normalised row
    matches the oracle's within rtol 1e-2, and the output the oracle's
    end-to-end A8W8 linear within 1 % (a one-ulp difference in the row can move
    an int8 step)."""
    from ppu_amd import _lib
    from ppu_amd import kernels as K

    g = gen(KERNEL_SEED + 60 + prologue)
    w = randn(g, n, k, scale=0.02)
    x, u = randn(g, 1, k), randn(g, 1, k)
    nw = randn(g, 128, scale=0.02, mean=1.0) if prologue == 3 else randn(g, k, scale=0.02)
    wq, sw = K.quantize_weight_i8(w.to(gpu))
    xg, ug, nwg = x.to(gpu), u.to(gpu), nw.to(gpu)
    y = torch.empty(1, n, dtype=BF, device=gpu)
    acc = torch.empty(n, dtype=torch.int32, device=gpu)
    xq = torch.empty(k, dtype=torch.int8, device=gpu)
    sx = torch.empty(1, dtype=torch.float32, device=gpu)
    xn = torch.empty(1, k, dtype=BF, device=gpu)
    r = torch.empty(1, k, dtype=BF, device=gpu)
    _lib.call("q35_gemv_i8", wq.data_ptr(), sw.data_ptr(), xg.data_ptr(),
              ug.data_ptr() if prologue >= 2 else None, nwg.data_ptr() if prologue else None, 0,
              1e-6, r.data_ptr() if prologue == 2 else None, xn.data_ptr() if prologue else None,
              y.data_ptr(), acc.data_ptr(), xq.data_ptr(), sx.data_ptr(), n, k, prologue,
              torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    row = _i8_row(prologue, x, u, nw)
    got_row = x if prologue == 0 else xn.cpu()
    if prologue:
        close(xn, row)
    if prologue == 2:
        close(r, ref.residual_add_rms_norm(x, u, nw)[0])
    exq, esx = oa.quantize_act(got_row)
    assert np.array_equal(xq.cpu().numpy().reshape(1, -1), exq)
    assert np.array_equal(sx.cpu().numpy().reshape(1, 1), esx)
    ewq, esw = wq.cpu().numpy(), sw.cpu().numpy()
    eacc = oa.int_gemm(exq, ewq)
    assert np.array_equal(acc.cpu().numpy().reshape(1, -1), eacc)
    assert torch.equal(y.cpu(), oa.dequant(eacc, esx, esw))
    assert _rel(y, oa.a8w8_linear(row, ewq, esw)[0]) < 1e-2


def test_swiglu_gemv_i8(gpu):
    """A8W8 [gate; up] GEMV with the residual-norm prologue and SwiGLU
    epilogue: accumulators exact for both halves, output = silu_and_mul of the
    dequantised gate and up (bit-exact), and the wrapper's result matches."""
    from ppu_amd import _lib
    from ppu_amd import kernels as K

    g = gen(KERNEL_SEED + 65)
    n, k = 6144, 2048
    w = randn(g, 2 * n, k, scale=0.02)
    r, u, nw = randn(g, 1, k), randn(g, 1, k), randn(g, k, scale=0.02)
    wq, sw = K.quantize_weight_i8(w.to(gpu))
    rg, ug, nwg = r.to(gpu), u.to(gpu), nw.to(gpu)
    y = torch.empty(1, n, dtype=BF, device=gpu)
    acc = torch.empty(2 * n, dtype=torch.int32, device=gpu)
    xn = torch.empty(1, k, dtype=BF, device=gpu)
    r_out = torch.empty(1, k, dtype=BF, device=gpu)
    _lib.call("q35_swiglu_gemv_i8", wq.data_ptr(), sw.data_ptr(), rg.data_ptr(), ug.data_ptr(),
              nwg.data_ptr(), 0, 1e-6, r_out.data_ptr(), xn.data_ptr(), y.data_ptr(), acc.data_ptr(),
              n, k, 2, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    close(xn, ref.residual_add_rms_norm(r, u, nw)[1])
    exq, esx = oa.quantize_act(xn.cpu())
    eacc = oa.int_gemm(exq, wq.cpu().numpy())
    assert np.array_equal(acc.cpu().numpy().reshape(1, -1), eacc)
    packed = oa.dequant(eacc, esx, sw.cpu().numpy())
    assert torch.equal(y.cpu(), ref.silu_and_mul(packed))
    r2, y2 = K.residual_norm_linear(rg, ug, nwg, 1e-6, wq, swiglu=True, weight_scale=sw)
    assert torch.equal(y2, y) and torch.equal(r2, r_out)


def test_norm_linear_conv_i8(gpu):
    """A8W8 DeltaNet input projection with the conv1d epilogue, including the
    embedding gather of the first layer: packed output within 1 % of the
    oracle A8W8 linear, conv output and state exactly the oracle conv of the
    kernel's own packed output."""
    from ppu_amd import kernels as K

    g = gen(KERNEL_SEED + 66)
    table = randn(g, 500, 2048)
    nw = randn(g, 2048, scale=0.02)
    w = randn(g, 8320, 2048, scale=0.02)
    cw = randn(g, 6144, 4, scale=0.3)
    state0 = randn(g, 1, 6144, 4)
    wq, sw = K.quantize_weight_i8(w.to(gpu))
    ewq, esw = wq.cpu().numpy(), sw.cpu().numpy()
    cs = state0.to(gpu)
    tok = torch.tensor([321], dtype=torch.int64, device=gpu)
    r, packed, qkv = K.norm_linear_conv(table.to(gpu), None, nw.to(gpu), 1e-6, wq, cw.to(gpu), cs,
                                        token=tok, weight_scale=sw)
    assert torch.equal(r.cpu().reshape(-1), table[321])
    row = ref.rms_norm(table[321:322], nw)
    assert _rel(packed.reshape(1, -1), oa.a8w8_linear(row, ewq, esw)[0]) < 1e-2
    st = state0.clone()
    exp = ref.causal_conv1d(packed.cpu()[..., :6144], cw, st)
    close(qkv, exp)
    close(cs, st)
    # second layer form: residual + update prologue
    res, upd = randn(g, 1, 1, 2048), randn(g, 1, 1, 2048)
    r2, packed2, _ = K.norm_linear_conv(res.to(gpu), upd.to(gpu), nw.to(gpu), 1e-6, wq, cw.to(gpu),
                                        cs, weight_scale=sw)
    er, erow = ref.residual_add_rms_norm(res, upd, nw)
    close(r2, er)
    assert _rel(packed2.reshape(1, -1), oa.a8w8_linear(erow.reshape(1, -1), ewq, esw)[0]) < 1e-2


# ------------------------------------------------------------------ boundary
def test_single_hip_runtime(gpu):
    """libq35 binds to the HIP runtime torch loaded (one libamdhip64 mapped)."""
    maps = open("/proc/self/maps").read().splitlines()
    hip = {line.split()[-1] for line in maps if "libamdhip64" in line}
    assert len(hip) == 1, hip
    assert any("libq35.so" in line for line in maps)


def test_graph_capture_replay(gpu):
    """ctypes launches on torch's current stream are captured by
    torch.cuda.graph; replays (with eager work and syncs between) match eager."""
    from ppu_amd import kernels as K

    g = gen(KERNEL_SEED + 30)
    r = randn(g, 1, 2048).to(gpu)
    u = randn(g, 1, 2048).to(gpu)
    nw = randn(g, 2048, scale=0.02, mean=1.0).to(gpu)
    W = randn(g, 6144, 2048, scale=0.02).to(gpu)
    lw = randn(g, 3000, 6144, scale=0.02).to(gpu)
    _, y0 = K.residual_norm_linear(r, u, nw, 1e-6, W)
    t0 = K.lm_head_argmax(y0.reshape(1, -1), lw)
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            K.residual_norm_linear(r, u, nw, 1e-6, W)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        _, y = K.residual_norm_linear(r, u, nw, 1e-6, W)
        t = K.lm_head_argmax(y.reshape(1, -1), lw)
    for i in range(3):
        y.zero_()
        t.fill_(-1)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, y0), f"replay {i}"
        assert int(t) == int(t0), f"replay {i}"
        _ = (r * 2).sum().item()  # eager work between replays


# ------------------------------------------------------------------ fused DeltaNet decode entries
@pytest.mark.parametrize("first", [True, False])
def test_norm_linear_conv(gpu, first):
    """Input RMSNorm (+ residual add) -> packed projection GEMV -> conv1d update
    epilogue, against the oracle chain rms_norm/residual_add_rms_norm ->
    linear -> causal_conv1d."""
    from ppu_amd import kernels as K

    g = gen(KERNEL_SEED + 40)
    r = randn(g, 1, 1, 2048)
    u = randn(g, 1, 1, 2048)
    nw = randn(g, 2048, scale=0.02)
    W = randn(g, 8320, 2048, scale=0.02)
    cw = randn(g, 6144, 4, scale=0.3)
    cs0 = randn(g, 1, 6144, 4)
    if first:
        er, xn = None, ref.rms_norm(r, nw)
    else:
        er, xn = ref.residual_add_rms_norm(r, u, nw)
    ep = ref.linear(xn, W)
    cs_ref = cs0.clone()
    eqkv = ref.causal_conv1d(ep, cw, cs_ref)
    cs = cs0.to(gpu)
    r_out, packed, qkv = K.norm_linear_conv(r.to(gpu), None if first else u.to(gpu), nw.to(gpu),
                                            1e-6, W.to(gpu), cw.to(gpu), cs)
    if not first:
        assert torch.equal(r_out.cpu(), er)
    close(packed, ep)
    close(qkv, eqkv)
    # state shift is exact; the appended value is this kernel's own bf16 projection
    assert torch.equal(cs.cpu()[..., :3], cs0[..., 1:])
    assert torch.equal(cs.cpu()[0, :, 3], packed.cpu()[0, 0, :6144])


def test_gated_norm_linear(gpu):
    from ppu_amd import kernels as K

    g = gen(KERNEL_SEED + 41)
    core = randn(g, 16, 128)
    packed = randn(g, 1, 1, 8320)
    z = packed[..., 6144:8192]
    nw = randn(g, 128, scale=0.02, mean=1.0)
    W = randn(g, 2048, 2048, scale=0.02)
    exp = ref.linear(ref.gated_rms_norm(core, z.reshape(16, 128), nw).reshape(1, 1, 2048), W)
    pg = packed.to(gpu)
    got = K.gated_norm_linear(core.to(gpu), pg[..., 6144:8192], nw.to(gpu), 1e-6, W.to(gpu))
    close(got, exp)


@pytest.mark.parametrize("cache_len", [1152, 4096])
@pytest.mark.parametrize("positions", [(777, 777, 777), (100, 57, 33)])
@pytest.mark.parametrize("n_old", [0, 300, 1151])
def test_gqa_decode_fused_step(gpu, positions, n_old, cache_len):
    """Fused attention decode step (Q/K norm + RoPE from device positions, cache
    write, split-K attention incl. the new token, combine, gate, length += 1)
    against the oracle chain qgkv_norm_rope -> cache write -> decode attention
    -> attention gate, with Transformers' rotary table for cos/sin."""
    from transformers.models.qwen3_5.modeling_qwen3_5 import Qwen3_5TextRotaryEmbedding

    from ppu_amd import kernels as K
    from ppu_amd import synth

    g = gen(KERNEL_SEED + 50)
    packed = randn(g, 1, 1, 5120)
    qw, kw = randn(g, 256, scale=0.1), randn(g, 256, scale=0.1)
    kc = randn(g, 1, 2, cache_len, 256)
    vc = randn(g, 1, 2, cache_len, 256)
    kc[:, :, n_old:] = 0
    vc[:, :, n_old:] = 0
    rot = Qwen3_5TextRotaryEmbedding(synth.config_tiny())
    pos = torch.tensor(positions, dtype=torch.int64).view(3, 1, 1)
    cos, sin = rot(torch.zeros(1, 1, 8, dtype=BF), pos)
    kr, vr = kc.clone(), vc.clone()
    q, _, _ = ref.qgkv_norm_rope(packed, qw, kw, cos, sin, q_heads=8, kv_heads=2, dim=256,
                                 rotary_dim=64, cache_key=kr, cache_value=vr, cache_start=n_old)
    att = ref.gqa_decode_attention(q, kr, vr, n_old + 1, 0.0625)
    exp = ref.attention_gate_mul(att, packed, 256)
    kg, vg = kc.to(gpu), vc.to(gpu)
    length = torch.tensor(n_old, dtype=torch.int64, device=gpu)
    got = K.gqa_decode_fused(packed.to(gpu), qw.to(gpu), kw.to(gpu), rot.inv_freq.to(gpu),
                             pos.to(gpu), kg, vg, length, 0.0625, q_heads=8)
    close(got, exp)
    assert int(length) == n_old + 1
    close(kg[:, :, n_old], kr[:, :, n_old])
    assert torch.equal(vg[:, :, n_old].cpu(), vr[:, :, n_old])
    assert torch.equal(kg[:, :, :n_old].cpu(), kc[:, :, :n_old])


@pytest.mark.parametrize("cache_len", [1152, 4096])
def test_gqa_decode_fused_graph_replays(gpu, cache_len):
    """The fused decode step (split kernel + combine) captured in a graph:
    every replay appends one cache row, advances the length by exactly one
    and gives the same bits as the same sequence of eager calls on a copy of
    the cache, with eager work and host syncs between the replays."""
    from transformers.models.qwen3_5.modeling_qwen3_5 import Qwen3_5TextRotaryEmbedding

    from ppu_amd import kernels as K
    from ppu_amd import synth

    g = gen(KERNEL_SEED + 53)
    n_old = 700
    packed = randn(g, 1, 1, 5120).to(gpu)
    qw, kw = randn(g, 256, scale=0.1).to(gpu), randn(g, 256, scale=0.1).to(gpu)
    kc = randn(g, 1, 2, cache_len, 256).to(gpu)
    vc = randn(g, 1, 2, cache_len, 256).to(gpu)
    rot = Qwen3_5TextRotaryEmbedding(synth.config_tiny())
    inv = rot.inv_freq.to(gpu)
    pos = torch.tensor((900, 900, 900), dtype=torch.int64, device=gpu).view(3, 1, 1)
    ke, ve = kc.clone(), vc.clone()
    le = torch.tensor(n_old, dtype=torch.int64, device=gpu)
    eager = [K.gqa_decode_fused(packed, qw, kw, inv, pos, ke, ve, le, 0.0625, q_heads=8)
             for _ in range(4)]
    assert int(le) == n_old + 4
    length = torch.tensor(n_old, dtype=torch.int64, device=gpu)
    K.gqa_decode_fused(packed, qw, kw, inv, pos, kc.clone(), vc.clone(), length.clone(), 0.0625,
                       q_heads=8)  # warm the allocator outside the capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = K.gqa_decode_fused(packed, qw, kw, inv, pos, kc, vc, length, 0.0625, q_heads=8)
    assert int(length) == n_old  # capture ran nothing
    for r in range(4):
        graph.replay()
        torch.cuda.synchronize()
        assert int(length) == n_old + r + 1
        assert torch.equal(out, eager[r])
        K.gqa_decode_attention(packed[..., :2048].reshape(1, 8, 1, 256).contiguous(), ke, ve,
                               le, 0.0625)  # eager work between the replays
    assert torch.equal(kc[:, :, : n_old + 4], ke[:, :, : n_old + 4])


def test_norm_linear_conv_embedding_gather(gpu):
    from ppu_amd import kernels as K

    g = gen(KERNEL_SEED + 51)
    table = randn(g, 1000, 2048)
    nw = randn(g, 2048, scale=0.02)
    W = randn(g, 8320, 2048, scale=0.02)
    cw = randn(g, 6144, 4, scale=0.3)
    cs = torch.zeros(1, 6144, 4, dtype=BF, device=gpu)
    tok = torch.tensor([737], dtype=torch.int64, device=gpu)
    r, packed, _ = K.norm_linear_conv(table.to(gpu), None, nw.to(gpu), 1e-6, W.to(gpu), cw.to(gpu), cs,
                                      token=tok)
    assert torch.equal(r.cpu().reshape(-1), table[737])
    close(packed.reshape(1, -1), ref.linear(ref.rms_norm(table[737:738], nw), W))


def test_lm_head_feedback(gpu):
    from ppu_amd import kernels as K

    g = gen(KERNEL_SEED + 52)
    h = randn(g, 1, 2048)
    w = randn(g, 5000, 2048, scale=0.02)
    tok = torch.zeros(1, 1, dtype=torch.int64, device=gpu)
    pos = torch.tensor([[41]], dtype=torch.int64, device=gpu)
    out = K.lm_head_argmax(h.to(gpu), w.to(gpu), out=tok, advance=pos)
    assert out is tok and int(tok) == int(ref.lm_head_argmax(h, w)) and int(pos) == 42
