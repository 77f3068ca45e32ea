"""Pins the CPU oracle to things other than itself: Transformers 5.15.0 eager
modules (the semantics the reference kernels restate), closed forms, brute
force on tiny inputs and the committed golden vectors. Each check is chosen so
that a plausible slip in the oracle (a dropped term, a wrong rounding point, a
transposed operand, a wrong tie rule) fails it."""

from __future__ import annotations

import math
from pathlib import Path

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import a8w8 as oa
from oracle import ops as ref
from tests.conftest import KERNEL_SEED, gen

BF = torch.bfloat16
GOLDEN = Path(__file__).resolve().parent / "golden" / "golden.npz"


def randn(g, *shape, scale=1.0, mean=0.0):
    return (torch.randn(*shape, generator=g) * scale + mean).to(BF)


def ulp_close(a, b, frac_exact=0.99):
    """bf16 tensors equal up to one bf16 ulp, and identical in at least
    ``frac_exact`` of the elements (reduction-order differences only)."""
    a32, b32 = a.float(), b.float()
    torch.testing.assert_close(a32, b32, rtol=2 ** -7, atol=1e-6)
    assert (a == b).float().mean().item() >= frac_exact


def tf_impl():
    from transformers.models.qwen3_5 import modeling_qwen3_5 as m

    return m


# ---------------------------------------------------------------- norms
@pytest.mark.parametrize("width", [128, 256, 2048])
def test_rms_norm_matches_transformers(width):
    m = tf_impl()
    g = gen(KERNEL_SEED)
    x = randn(g, 7, width)
    w = randn(g, width, scale=0.1)
    mod = m.Qwen3_5RMSNorm(width, eps=1e-6)
    mod.weight.data = w.float()
    ulp_close(ref.rms_norm(x, w), mod(x))


def test_residual_add_rms_norm_matches_eager():
    m = tf_impl()
    g = gen(KERNEL_SEED + 1)
    r, u = randn(g, 7, 2048), randn(g, 7, 2048)
    w = randn(g, 2048, scale=0.02)
    mod = m.Qwen3_5RMSNorm(2048, eps=1e-6)
    mod.weight.data = w.float()
    out_r, out_n = ref.residual_add_rms_norm(r, u, w)
    assert torch.equal(out_r, r + u)  # eager bf16 add rounds once
    ulp_close(out_n, mod(r + u))


def test_gated_rms_norm_matches_transformers():
    m = tf_impl()
    g = gen(KERNEL_SEED + 2)
    x, z = randn(g, 32, 128), randn(g, 32, 128)
    w = randn(g, 128, mean=1.0, scale=0.1)
    mod = m.Qwen3_5RMSNormGated(128, eps=1e-6).to(BF)
    mod.weight.data = w
    ulp_close(ref.gated_rms_norm(x, z, w), mod(x, z))


def test_rms_norm_closed_form():
    # constant row c: rms = |c|, so y = sign(c) * (1 + w) / sqrt(1 + eps/c^2)
    x = torch.full((1, 64), -3.0, dtype=BF)
    w = torch.zeros(64, dtype=BF)
    y = ref.rms_norm(x, w, eps=0.0)
    assert torch.all(y.float() == -1.0)


# ---------------------------------------------------------------- elementwise
def test_silu_and_mul_closed_form():
    p = torch.tensor([[0.0, 10.0, -10.0, 2.0, 3.0, 4.0]], dtype=BF)  # gate | up
    out = ref.silu_and_mul(p).float()
    assert out[0, 0] == 0.0  # silu(0) * 2 = 0
    silu10 = float(torch.tensor(10.0 / (1 + math.exp(-10.0))).to(BF))
    assert out[0, 1].item() == float(torch.tensor(silu10 * 3.0).to(BF))  # bf16(bf16(silu) * up)
    assert abs(out[0, 2].item()) < 0.01  # silu(-10) ~ -4.5e-4


def test_silu_and_mul_matches_eager():
    g = gen(KERNEL_SEED + 3)
    p = randn(g, 7, 512)
    exp = (F.silu(p[:, :256]) * p[:, 256:])  # bf16 eager: silu -> bf16, product -> bf16
    ulp_close(ref.silu_and_mul(p), exp)


def test_attention_gate_matches_eager():
    g = gen(KERNEL_SEED + 4)
    packed = randn(g, 1, 3, 2 * 4 * 64 + 2 * 2 * 64)
    x = randn(g, 1, 3, 4 * 64)
    gate = packed[..., : 2 * 4 * 64].reshape(1, 3, 4, 128)[..., 64:].reshape(1, 3, 256)
    ulp_close(ref.attention_gate_mul(x, packed, 64), x * torch.sigmoid(gate))


# ---------------------------------------------------------------- linear / lm_head
def test_linear_fp32_accumulate():
    g = gen(KERNEL_SEED + 5)
    x, w = randn(g, 1, 512), randn(g, 96, 512, scale=0.02)
    exact = (x.double() @ w.double().t())
    torch.testing.assert_close(ref.linear(x, w).double(), exact, rtol=2 ** -8, atol=1e-6)
    # torch's CPU bf16 F.linear (used by the oracle decoder) agrees to one ulp
    torch.testing.assert_close(F.linear(x, w).float(), ref.linear(x, w).float(), rtol=2 ** -7, atol=1e-6)


def test_swiglu_equals_linear_then_silu_and_mul():
    g = gen(KERNEL_SEED + 6)
    x, w = randn(g, 1, 1, 256), randn(g, 64, 256, scale=0.05)
    assert torch.equal(ref.swiglu_gemv(x, w), ref.silu_and_mul(ref.linear(x, w)))


def test_lm_head_argmax_ties_and_brute_force():
    assert int(ref.lm_head_argmax(torch.zeros(1, 128, dtype=BF), torch.zeros(257, 128, dtype=BF))) == 0
    g = gen(KERNEL_SEED + 7)
    h, w = randn(g, 1, 64), randn(g, 300, 64)
    w[250] = w[17]  # planted duplicate of row 17
    w[17] *= 3
    w[250] = w[17]
    got = int(ref.lm_head_argmax(h, w))
    logits = [float(torch.tensor(sum(float(a) * float(b) for a, b in zip(h[0], w[v]))).to(BF))
              for v in range(300)]
    best = max(logits)
    assert got == logits.index(best)  # lowest index among equal bf16 maxima
    if logits[17] == best:
        assert got == 17


# ---------------------------------------------------------------- conv1d
def test_conv1d_update_matches_transformers():
    m = tf_impl()
    g = gen(KERNEL_SEED + 8)
    c = 64
    x = randn(g, 1, 1, c + 32)
    w = randn(g, c, 4)
    st = randn(g, 1, c, 4)
    st_tf = st.clone()
    exp = m.causal_conv1d_update(x[..., :c].transpose(1, 2).contiguous(), st_tf, w, None, "silu")
    st_o = st.clone()
    got = ref.causal_conv1d(x, w, st_o)
    ulp_close(got, exp.transpose(1, 2))
    assert torch.equal(st_o, st_tf)


def test_conv1d_prefill_matches_transformers():
    m = tf_impl()
    g = gen(KERNEL_SEED + 9)
    c, seq = 64, 17
    x = randn(g, 1, seq, c)
    w = randn(g, c, 4)
    st = torch.zeros(1, c, 4, dtype=BF)
    exp = m.causal_conv1d_fn(x.transpose(1, 2), w, None, activation="silu")
    got = ref.causal_conv1d(x, w, st)
    ulp_close(got, exp.transpose(1, 2), frac_exact=0.97)
    assert torch.equal(st, x[:, -4:].transpose(1, 2))


# ---------------------------------------------------------------- delta rule
def _delta_inputs(g, seq, heads=4, dim=128):
    qkv = randn(g, 1, seq, 3 * heads * dim)
    packed = randn(g, 1, seq, 4 * heads * dim + 2 * heads)
    packed[..., : 3 * heads * dim] = qkv
    return qkv, packed, randn(g, heads), randn(g, heads), torch.randn(1, heads, dim, dim, generator=g) * 0.01


def test_delta_matches_transformers_recurrent():
    m = tf_impl()
    g = gen(KERNEL_SEED + 10)
    heads, dim, seq = 4, 128, 5
    qkv, packed, a_log, dt_bias, st = _delta_inputs(g, seq, heads, dim)
    st_o = st.clone()
    got = ref.delta_recurrent(qkv, packed, a_log, dt_bias, st_o)
    q, k, v = qkv.float().reshape(1, seq, 3, heads, dim).unbind(2)
    a_off = 4 * heads * dim
    a = packed[..., a_off : a_off + heads].float()
    b = packed[..., a_off + heads :].float()
    gg = -a_log.float().exp() * F.softplus(a + dt_bias.float())
    out, final = m.torch_recurrent_gated_delta_rule(q, k, v, g=gg, beta=b.sigmoid(),
                                                    initial_state=st.clone(), output_final_state=True,
                                                    use_qk_l2norm_in_kernel=True)
    torch.testing.assert_close(st_o, final, rtol=1e-4, atol=1e-6)
    torch.testing.assert_close(got.float(), out.float().to(BF).float(), rtol=2 ** -7, atol=1e-3)


def test_delta_invariant_and_single_step_closed_form():
    g = gen(KERNEL_SEED + 11)
    heads, dim = 2, 128
    qkv, packed, _, _, st = _delta_inputs(g, 1, heads, dim)
    # beta = 0 and alpha = 1: state unchanged
    p0 = packed.clone()
    p0[..., -2 * heads :] = -1e4
    st0 = st.clone()
    ref.delta_recurrent(qkv, p0, torch.full((heads,), -1e4), torch.zeros(heads), st0)
    assert torch.equal(st0, st)
    # zero state, beta = 1 (b -> +inf), alpha = 1: S = k^ v^T, o = (q^ . k^) v
    p1 = packed.clone()
    p1[..., -2 * heads : -heads] = -1e4  # a: softplus(-1e4) = 0 -> alpha = 1
    p1[..., -heads:] = 1e4               # b: beta = 1
    z = torch.zeros(1, heads, dim, dim)
    out = ref.delta_recurrent(qkv, p1, torch.zeros(heads), torch.zeros(heads), z)
    q, k, v = qkv.double().reshape(1, 1, 3, heads, dim).unbind(2)
    qh = q / q.norm(dim=-1, keepdim=True) / math.sqrt(dim)
    kh = k / k.norm(dim=-1, keepdim=True)
    exp_o = (qh * kh).sum(-1, keepdim=True) * v
    torch.testing.assert_close(out.double(), exp_o.to(BF).double(), rtol=2 ** -7, atol=1e-4)
    torch.testing.assert_close(z.double(), (kh[0, 0][..., :, None] * v[0, 0][..., None, :])[None],
                               rtol=1e-5, atol=1e-6)


# ---------------------------------------------------------------- QGKV norm + RoPE
def test_qgkv_norm_rope_matches_transformers():
    m = tf_impl()
    g = gen(KERNEL_SEED + 12)
    qh, kvh, d, rot, seq = 8, 2, 256, 64, 5
    packed = randn(g, 1, seq, 2 * qh * d + 2 * kvh * d)
    qw, kw = randn(g, d, scale=0.1), randn(g, d, scale=0.1)
    cos, sin = randn(g, 1, seq, rot), randn(g, 1, seq, rot)
    q, k, v = ref.qgkv_norm_rope(packed, qw, kw, cos, sin, q_heads=qh, kv_heads=kvh, dim=d, rotary_dim=rot)
    qn = m.Qwen3_5RMSNorm(d)
    qn.weight.data = qw.float()
    kn = m.Qwen3_5RMSNorm(d)
    kn.weight.data = kw.float()
    q_raw = packed[..., : 2 * qh * d].reshape(1, seq, qh, 2 * d)[..., :d]
    k_raw = packed[..., 2 * qh * d : 2 * qh * d + kvh * d].reshape(1, seq, kvh, d)
    v_raw = packed[..., 2 * qh * d + kvh * d :].reshape(1, seq, kvh, d)
    eq, ek = m.apply_rotary_pos_emb(qn(q_raw).transpose(1, 2), kn(k_raw).transpose(1, 2), cos, sin)
    ulp_close(q, eq)
    ulp_close(k, ek)
    assert torch.equal(v, v_raw.transpose(1, 2))
    # cache write at offset 3 of 13 leaves the prefix and suffix untouched
    kc = torch.zeros(1, kvh, 13, d, dtype=BF)
    vc = torch.zeros_like(kc)
    ref.qgkv_norm_rope(packed, qw, kw, cos, sin, q_heads=qh, kv_heads=kvh, dim=d, rotary_dim=rot,
                       cache_key=kc, cache_value=vc, cache_start=3)
    assert torch.equal(kc[:, :, 3:8], k) and not kc[:, :, :3].any() and not vc[:, :, 8:].any()


def test_rotary_table_matches_transformers():
    from ppu_amd import synth

    m = tf_impl()
    cfg = synth.config_tiny()
    rot = m.Qwen3_5TextRotaryEmbedding(cfg)
    pos = torch.arange(0, 300).view(1, -1)
    x = torch.zeros(1, 300, 8, dtype=BF)
    cos_tf, sin_tf = rot(x, pos[None].expand(3, 1, -1))
    cos, sin = ref.rotary_cos_sin(pos, 64, 1e7)
    assert torch.equal(cos, cos_tf) and torch.equal(sin, sin_tf)


def test_multimodal_rotary_table_matches_transformers():
    """Distinct temporal / height / width rows (an image's 2-D positions):
    the interleaved mrope row choice must match Transformers bit for bit, and
    a plan that ignores the rows (text table of row 0) must not."""
    from ppu_amd import synth

    m = tf_impl()
    cfg = synth.config_tiny()
    rot = m.Qwen3_5TextRotaryEmbedding(cfg)
    g = gen(KERNEL_SEED + 21)
    pos = torch.randint(0, 5000, (3, 1, 40), generator=g)
    x = torch.zeros(1, 40, 8, dtype=BF)
    cos_tf, sin_tf = rot(x, pos)
    cos, sin = ref.rotary_cos_sin(pos, 64, 1e7, (11, 11, 10))
    assert torch.equal(cos, cos_tf) and torch.equal(sin, sin_tf)
    cos0, _ = ref.rotary_cos_sin(pos[0], 64, 1e7)
    assert not torch.equal(cos0, cos_tf)


# ---------------------------------------------------------------- attention
def test_decode_attention_matches_sdpa_and_split_invariance():
    g = gen(KERNEL_SEED + 13)
    q = randn(g, 1, 8, 1, 256)
    kc, vc = randn(g, 1, 2, 64, 256), randn(g, 1, 2, 64, 256)
    for n in (1, 7, 40, 64):
        got = ref.gqa_decode_attention(q, kc, vc, n, 0.0625)
        exp = F.scaled_dot_product_attention(q.float(), kc[:, :, :n].float(), vc[:, :, :n].float(),
                                             scale=0.0625, enable_gqa=True).reshape(1, 1, -1)
        torch.testing.assert_close(got.float(), exp.to(BF).float(), rtol=2 ** -7, atol=1e-3)
    # keys past the valid length do not matter
    kc2 = kc.clone()
    kc2[:, :, 40:] = 100.0
    assert torch.equal(ref.gqa_decode_attention(q, kc2, vc, 40, 0.0625),
                       ref.gqa_decode_attention(q, kc, vc, 40, 0.0625))


def test_prefill_attention_is_causal():
    g = gen(KERNEL_SEED + 14)
    q = randn(g, 1, 8, 6, 256)
    kc, vc = randn(g, 1, 2, 6, 256), randn(g, 1, 2, 6, 256)
    out = ref.prefill_attention(q, kc, vc, 0.0625)
    exp = F.scaled_dot_product_attention(q.float(), kc.float(), vc.float(), scale=0.0625,
                                         is_causal=True, enable_gqa=True)
    torch.testing.assert_close(out.float(), exp.transpose(1, 2).reshape(1, 6, -1).to(BF).float(),
                               rtol=2 ** -7, atol=1e-3)
    # row 0 attends only to key 0: output = V[0] of its kv head
    assert torch.equal(out[0, 0, :256], vc[0, 0, 0])


# ---------------------------------------------------------------- A8W8
def test_weight_quant_matches_torch_rule():
    g = gen(KERNEL_SEED + 15)
    w = randn(g, 64, 96, scale=0.02)
    w[3] = 0
    q, s = oa.quantize_weight(w)
    w32 = w.float()
    absmax = w32.abs().amax(dim=1, keepdim=True)
    ts = torch.where(absmax > 0, absmax / 127.0, torch.ones_like(absmax))
    tq = torch.round(w32 / ts).clamp_(-127, 127).to(torch.int8)
    assert np.array_equal(q, tq.numpy()) and np.array_equal(s, ts.numpy())
    assert s[3, 0] == 1.0 and not q[3].any()


def test_act_quant_known_answers():
    # absmax 2.0 -> scale 2/127; x * 63.5: 1.0 -> 63.5 -> 64 (ties to even), -2 -> -127
    x = torch.tensor([[1.0, -2.0, 0.5, 0.0078125]], dtype=BF)
    q, s = oa.quantize_act(x)
    assert q.tolist() == [[64, -127, 32, 0]]  # 31.75 -> 32; 0.496 -> 0
    assert s[0, 0] == np.float32(2.0) / np.float32(127.0)
    # a zero row quantises to zeros with scale 0
    q0, s0 = oa.quantize_act(torch.zeros(1, 8, dtype=BF))
    assert not q0.any() and s0[0, 0] == 0.0


def test_int_gemm_brute_force():
    rng = np.random.default_rng(0)
    xq = rng.integers(-128, 128, size=(3, 40), dtype=np.int8)
    wq = rng.integers(-127, 128, size=(5, 40), dtype=np.int8)
    acc = oa.int_gemm(xq, wq)
    for m in range(3):
        for n in range(5):
            assert acc[m, n] == sum(int(a) * int(b) for a, b in zip(xq[m], wq[n]))


# ---------------------------------------------------------------- golden vectors
@pytest.mark.skipif(not GOLDEN.exists(), reason="golden vectors not generated")
def test_oracle_reproduces_golden_vectors():
    data = np.load(GOLDEN, allow_pickle=False)

    def bf(name):
        return torch.from_numpy(data[name].astype(np.uint16).view(np.int16)).view(BF)

    ulp_close(ref.rms_norm(bf("rms_x"), bf("rms_w")), bf("rms_out"))
    ulp_close(ref.gated_rms_norm(bf("g_x"), bf("g_z"), bf("g_w")), bf("g_out"))
    st = torch.from_numpy(data["delta_state0"])
    out = ref.delta_recurrent(bf("delta_qkv"), bf("delta_packed"), bf("delta_alog"), bf("delta_dt"), st)
    torch.testing.assert_close(st, torch.from_numpy(data["delta_state1"]), rtol=1e-4, atol=1e-6)
    torch.testing.assert_close(out.float(), bf("delta_out").float(), rtol=2 ** -7, atol=1e-3)
    q, k, _ = ref.qgkv_norm_rope(bf("qg_packed"), bf("qg_qw"), bf("qg_kw"), bf("qg_cos"), bf("qg_sin"),
                                 q_heads=8, kv_heads=2, dim=256, rotary_dim=64)
    ulp_close(q, bf("qg_q"))
    ulp_close(k, bf("qg_k"))
    assert int(ref.lm_head_argmax(bf("lm_h"), bf("lm_w"))) == int(data["lm_idx"])


# ---------------------------------------------------------------- vision
@pytest.mark.parametrize("width", [64, 1152])
def test_layer_norm_matches_fp64_and_invariants(width):
    g = gen(KERNEL_SEED)
    x = randn(g, 9, width, scale=2.0, mean=0.5)
    w = randn(g, width, scale=0.1, mean=1.0)
    b = randn(g, width, scale=0.1)
    got = ref.layer_norm(x, w, b)
    exp = F.layer_norm(x.double(), (width,), w.double(), b.double(), eps=1e-6)
    # one bf16 rounding of the output apart
    torch.testing.assert_close(got.double(), exp, rtol=2 ** -8, atol=1e-5)
    # a constant row normalises to exactly the bias
    const = torch.full((2, width), 3.0).to(BF)
    assert torch.equal(ref.layer_norm(const, w, b), b.expand(2, width))
    # shift invariance: x and x + 1 (exact in bf16 here) give the same output
    xs = torch.randint(-8, 8, (3, width), generator=g).to(BF)
    torch.testing.assert_close(ref.layer_norm(xs + 1, w, b).float(), ref.layer_norm(xs, w, b).float(),
                               rtol=2 ** -7, atol=1e-3)


def test_residual_add_layer_norm_is_add_then_norm():
    g = gen(KERNEL_SEED)
    r = randn(g, 5, 256)
    u = randn(g, 5, 256)
    w = randn(g, 256, scale=0.1, mean=1.0)
    b = randn(g, 256, scale=0.1)
    added, normed = ref.residual_add_layer_norm(r, u, w, b)
    assert torch.equal(added, (r.float() + u.float()).to(BF))
    exp = F.layer_norm(added.double(), (256,), w.double(), b.double(), eps=1e-6)
    torch.testing.assert_close(normed.double(), exp, rtol=2 ** -8, atol=1e-5)


def test_position_embed_add_matches_transformers_sum():
    from transformers.vision_utils import get_vision_interpolation_indices_and_weights

    g = gen(KERNEL_SEED)
    side, width = 8, 64
    table = randn(g, side * side, width, scale=0.5)
    grid = torch.tensor([[1, 6, 4]])
    idx, wts = get_vision_interpolation_indices_and_weights(
        grid, num_grid_per_side=side, mode="bilinear", align_corners=True, spatial_merge_size=2)
    hidden = randn(g, idx.shape[0], width)
    got = ref.position_embed_add(hidden, table, idx, wts)
    # Qwen3_5VisionModel.forward: (pos_embed(indices) * weights[:, :, None]).sum(1), cast, added
    emb = torch.nn.functional.embedding(idx, table.float())
    pos = (emb * wts.float()[:, :, None]).sum(1).to(BF)
    exp = (hidden.float() + pos.float()).to(BF)
    ulp_close(got, exp, frac_exact=0.98)
    # one-hot weights select the table row exactly
    one = torch.zeros_like(wts)
    one[:, 2] = 1.0
    got1 = ref.position_embed_add(torch.zeros_like(hidden), table, idx, one)
    assert torch.equal(got1, table[idx[:, 2]])


def test_vision_qkv_rope_matches_transformers():
    m = tf_impl()
    g = gen(KERNEL_SEED)
    tokens, heads, dim = 10, 4, 72
    packed = randn(g, tokens, 3 * heads * dim)
    ang = torch.randn(tokens, dim // 2, generator=g)
    emb = torch.cat((ang, ang), dim=-1)
    cos, sin = emb.cos(), emb.sin()
    q, k, v = ref.vision_qkv_rope(packed, cos, sin, heads=heads, dim=dim)
    qs, ks, vs = packed.reshape(tokens, 3, heads, dim).permute(1, 0, 2, 3).unbind(0)
    qe, ke = m.apply_rotary_pos_emb_vision(qs, ks, cos, sin)
    assert torch.equal(q, qe.transpose(0, 1).unsqueeze(0))
    assert torch.equal(k, ke.transpose(0, 1).unsqueeze(0))
    assert torch.equal(v, vs.transpose(0, 1).unsqueeze(0))
    # cos = 1, sin = 0 is the identity on q and k
    q1, k1, _ = ref.vision_qkv_rope(packed, torch.ones(tokens, dim), torch.zeros(tokens, dim),
                                    heads=heads, dim=dim)
    assert torch.equal(q1, qs.transpose(0, 1).unsqueeze(0))
    assert torch.equal(k1, ks.transpose(0, 1).unsqueeze(0))


def test_vision_attention_matches_sdpa_per_image():
    g = gen(KERNEL_SEED)
    heads, tokens, dim = 3, 11, 16
    q, k, v = (randn(g, 1, heads, tokens, dim) for _ in range(3))
    cu = torch.tensor([0, 4, 10, 11])
    got = ref.vision_attention(q, k, v, dim ** -0.5, cu)
    for a, b in ((0, 4), (4, 10), (10, 11)):
        exp = F.scaled_dot_product_attention(q[:, :, a:b].double(), k[:, :, a:b].double(),
                                             v[:, :, a:b].double(), scale=dim ** -0.5)
        torch.testing.assert_close(got[a:b].double(), exp[0].permute(1, 0, 2).reshape(b - a, -1),
                                   rtol=2 ** -8, atol=1e-5)
    # a one-token image attends to itself only
    assert torch.equal(got[10].reshape(heads, dim), v[0, :, 10])
