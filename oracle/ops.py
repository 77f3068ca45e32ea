"""CPU restatement of the reference operators (test infrastructure only).

Each function follows one reference kernel of PingGuoLiZiJvZi/ppu
``qwen35_fused/kernels.py`` (cited per function): inputs are upcast from bf16
to fp32, reductions run in fp32, and every place where the reference kernel
stores or casts to bf16 is an explicit ``.to(torch.bfloat16)`` here (round to
nearest even). ``rsqrt`` is ``1/sqrt`` in fp32, the same two correctly
rounded steps as torch's CPU ``rsqrt``.

Pinning (tests/test_oracle.py):
  rms_norm, residual_add_rms_norm, gated_rms_norm — bit-exact against
      Transformers 5.15.0 Qwen3_5RMSNorm / Qwen3_5RMSNormGated (CPU eager) and
      the committed golden vectors;
  silu_and_mul, swiglu_gemv, linear — against F.silu / F.linear in fp64, and
      the closed form silu(0)=0, silu(x)->x;
  qgkv_norm_rope — bit-exact against Transformers eager q_norm/k_norm +
      apply_rotary_pos_emb, and the cache-offset prefix/suffix checks;
  causal_conv1d — against Transformers causal_conv1d_update / causal_conv1d_fn;
  delta_recurrent — against Transformers torch_recurrent_gated_delta_rule on
      the same fp32 inputs, the beta=0/alpha=1 invariant and a hand-derived
      single-step closed form;
  gqa_decode_attention, prefill_attention — fp64 textbook softmax attention,
      split invariance;
  lm_head_argmax — brute force F.linear + argmax, the all-zero tie (index 0)
      and planted duplicate maxima;
  layer_norm, residual_add_layer_norm — against torch's F.layer_norm in fp64
      on the same inputs (one bf16 rounding of the output apart), constant
      rows (output = bias) and mean/scale invariance;
  position_embed_add — against Transformers 5.15.0's weighted
      pos_embed(indices) sum (Qwen3_5VisionModel.forward; unfused products,
      so one bf16 ulp of the position term apart) and one-hot weights (an
      exact table row);
  vision_qkv_rope — bit-exact against Transformers 5.15.0
      apply_rotary_pos_emb_vision, and cos = 1, sin = 0 (identity);
  vision_attention — against torch's scaled_dot_product_attention in fp64
      per image, and a one-key image (output = its value row).
"""

from __future__ import annotations

import math

import torch
import torch.nn.functional as F

BF16 = torch.bfloat16


def _bf(x: torch.Tensor) -> torch.Tensor:
    return x.to(BF16)


def _f(x: torch.Tensor) -> torch.Tensor:
    return x.to(torch.float32)


def _rsqrt(x: torch.Tensor) -> torch.Tensor:
    return 1.0 / torch.sqrt(x)


def _silu(x: torch.Tensor) -> torch.Tensor:
    return x / (1.0 + torch.exp(-x))


def _sigmoid(x: torch.Tensor) -> torch.Tensor:
    return 1.0 / (1.0 + torch.exp(-x))


# ---------------------------------------------------------------- norms
def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """reference kernels.py:24-53: bf16(x * rsqrt(sum(x^2)/n + eps) * (1 + w))."""
    x32 = _f(x)
    var = (x32 * x32).sum(-1, keepdim=True) / x.shape[-1]
    return _bf(x32 * _rsqrt(var + eps) * (1.0 + _f(weight)))


def residual_add_rms_norm(residual, update, weight, eps: float = 1e-6):
    """reference kernels.py:56-112: r' = bf16(r + u), then rms_norm(r')."""
    r = _bf(_f(residual) + _f(update))
    return r, rms_norm(r, weight, eps)


def gated_rms_norm(x, gate, weight, eps: float = 1e-6):
    """reference kernels.py:115-155: bf16(bf16(bf16(rms(x)) * bf16(w)) * silu(gate))."""
    x32 = _f(x)
    var = (x32 * x32).sum(-1, keepdim=True) / x.shape[-1]
    norm_bf = _bf(x32 * _rsqrt(var + eps))
    weighted = _bf(_f(norm_bf) * _f(_bf(weight)))
    return _bf(_f(weighted) * _silu(_f(gate)))


def silu_and_mul(packed: torch.Tensor) -> torch.Tensor:
    """reference kernels.py:158-180: bf16(bf16(silu(g)) * u)."""
    w = packed.shape[-1] // 2
    g = _f(packed[..., :w])
    u = _f(packed[..., w:])
    return _bf(_f(_bf(_silu(g))) * u)


def attention_gate_mul(x, packed_qgkv, head_dim: int):
    """reference kernels.py:285-333: bf16(x * bf16(sigmoid(gate_h))); the gate
    of head h is packed[..., h*2*hd + hd : (h+1)*2*hd]."""
    hidden = x.shape[-1]
    heads = hidden // head_dim
    lead = x.shape[:-1]
    q_part = packed_qgkv[..., : 2 * hidden].reshape(*lead, heads, 2 * head_dim)
    gate = q_part[..., head_dim:].reshape(*lead, hidden)
    return _bf(_f(x) * _f(_bf(_sigmoid(_f(gate)))))


# ---------------------------------------------------------------- GEMV
def linear(x: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """bf16 F.linear: fp32 sum over K, one bf16 round (integration.py:185 etc.)."""
    return _bf(_f(x) @ _f(weight).t())


def swiglu_gemv(x: torch.Tensor, packed_weight: torch.Tensor) -> torch.Tensor:
    """reference kernels.py:183-263: gate, up rounded to bf16; silu -> bf16; product -> bf16."""
    n = packed_weight.shape[0] // 2
    acc = _f(x) @ _f(packed_weight).t()
    g = _f(_bf(acc[..., :n]))
    u = _f(_bf(acc[..., n:]))
    return _bf(_f(_bf(_silu(g))) * u)


def lm_head_argmax(hidden: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """reference kernels.py:1093-1143: argmax of bf16-rounded logits, lowest index on ties."""
    logits = _f(_bf(_f(hidden) @ _f(weight).t()))
    return logits.argmax(dim=-1, keepdim=True).to(torch.int64)


# ---------------------------------------------------------------- DeltaNet
def causal_conv1d(x: torch.Tensor, weight: torch.Tensor, state: torch.Tensor) -> torch.Tensor:
    """reference kernels.py:576-656. x [B,L,S] (first C channels used),
    weight [C,K], state [B,C,K] updated in place; returns [B,L,C] bf16.

    L == 1: window = (state[1:], x); state shifted. L > 1: zero history,
    the last K inputs (where they exist) are written to the state.
    conv -> bf16 -> silu (fp32) -> bf16.
    """
    batch, seq_len, _ = x.shape
    channels, ksize = weight.shape
    xs = _f(x[..., :channels])
    w32 = _f(weight)
    if seq_len == 1:
        window = torch.cat((_f(state[..., 1:]), xs.transpose(1, 2)), dim=-1)  # [B,C,K]
        acc = torch.zeros(batch, channels)
        for t in range(ksize):
            acc = acc + window[..., t] * w32[:, t]
        state.copy_(_bf(window))
        out = _bf(_silu(_f(_bf(acc))))
        return out.unsqueeze(1)
    acc = torch.zeros(batch, seq_len, channels)
    for tap in range(ksize):
        shift = ksize - 1 - tap
        src = torch.zeros_like(xs)
        if shift < seq_len:
            src[:, shift:] = xs[:, : seq_len - shift]
        acc = acc + src * w32[:, tap]
    out = _bf(_silu(_f(_bf(acc))))
    for pos in range(ksize):
        t = seq_len - ksize + pos
        if 0 <= t < seq_len:
            state[:, :, pos] = x[:, t, :channels]
    return out


def delta_factors(qkv, packed, a_log, dt_bias, heads: int, dim: int):
    """reference kernels.py:713-765: per (token, head) q_inv, k_inv, alpha, beta."""
    b, l, width = qkv.shape
    q, k, _ = _f(qkv).reshape(b, l, 3, heads, dim).unbind(2)
    q_inv = _rsqrt((q * q).sum(-1) + 1e-6)
    k_inv = _rsqrt((k * k).sum(-1) + 1e-6)
    a_off = width + heads * dim
    a = _f(packed[..., a_off : a_off + heads]) + _f(dt_bias)
    bb = _f(packed[..., a_off + heads : a_off + 2 * heads])
    softplus = torch.where(a > 20.0, a, torch.log(1.0 + torch.exp(a)))
    alpha = torch.exp(-torch.exp(_f(a_log)) * softplus)
    beta = 1.0 / (1.0 + torch.exp(-bb))
    return q_inv, k_inv, alpha, beta


def delta_recurrent(qkv, packed, a_log, dt_bias, state: torch.Tensor) -> torch.Tensor:
    """reference kernels.py:768-851 (fp32 rule, kernel operation order):
    q^ = q*q_inv*fp32(1/sqrt(D)); k^ = k*k_inv; S *= alpha; m = S^T k^;
    d = beta*(v - m); S += k^ d^T; o = S^T q^. state [B,H,D,D] fp32 in place;
    returns [B,L,H,D] bf16."""
    b, l, width = qkv.shape
    heads, dim = state.shape[1], state.shape[2]
    q, k, v = _f(qkv).reshape(b, l, 3, heads, dim).unbind(2)
    q_inv, k_inv, alpha, beta = delta_factors(qkv, packed, a_log, dt_bias, heads, dim)
    scale = torch.tensor(1.0 / math.sqrt(dim), dtype=torch.float32)
    outs = []
    s = state
    for t in range(l):
        qh = q[:, t] * q_inv[:, t, :, None] * scale  # [B,H,D]
        kh = k[:, t] * k_inv[:, t, :, None]
        s.mul_(alpha[:, t, :, None, None])
        mem = (s * kh[..., :, None]).sum(-2)  # [B,H,Dv]
        delta = beta[:, t, :, None] * (v[:, t] - mem)
        s.add_(kh[..., :, None] * delta[..., None, :])
        outs.append((s * qh[..., :, None]).sum(-2))
    return _bf(torch.stack(outs, dim=1))


# ---------------------------------------------------------------- attention
def qgkv_norm_rope(packed, q_weight, k_weight, cos, sin, *, q_heads, kv_heads, dim, rotary_dim,
                   cache_key=None, cache_value=None, cache_start=None):
    """reference kernels.py:419-573. Returns (q [B,QH,L,D], k, v); with a cache,
    K/V are written at cache_start + t and the cache tensors are returned."""
    b, l, _ = packed.shape
    qg = packed[..., : 2 * q_heads * dim].reshape(b, l, q_heads, 2 * dim)
    q_raw = qg[..., :dim]
    ks = 2 * q_heads * dim
    k_raw = packed[..., ks : ks + kv_heads * dim].reshape(b, l, kv_heads, dim)
    v_raw = packed[..., ks + kv_heads * dim :].reshape(b, l, kv_heads, dim)

    def norm(x, w):
        x32 = _f(x)
        var = (x32 * x32).sum(-1, keepdim=True) / dim
        return _bf(x32 * _rsqrt(var + 1.0e-6) * (1.0 + _f(w)))

    half = rotary_dim // 2
    cs = _f(_bf(cos))[:, :, None, :]  # [B,L,1,R]
    sn = _f(_bf(sin))[:, :, None, :]

    def rope(n):
        n32 = _f(n)
        front = n32[..., :rotary_dim]
        rot_half = torch.cat((-front[..., half:], front[..., :half]), dim=-1)
        qc = _f(_bf(front * cs))
        qs = _f(_bf(rot_half * sn))
        rotated = _bf(qc + qs)
        return torch.cat((rotated, n[..., rotary_dim:]), dim=-1)

    q = rope(norm(q_raw, q_weight)).transpose(1, 2).contiguous()
    k = rope(norm(k_raw, k_weight)).transpose(1, 2).contiguous()
    v = v_raw.transpose(1, 2).contiguous()
    if cache_key is None:
        return q, k, v
    start = int(cache_start)
    cache_key[:, :, start : start + l] = k
    cache_value[:, :, start : start + l] = v
    return q, cache_key, cache_value


def gqa_decode_attention(q, cache_keys, cache_values, valid_length, scale):
    """reference kernels.py:940-1090 (textbook fp64 softmax over the valid
    prefix, output rounded to bf16): q [1,H,1,D], K/V [1,KVH,L,D] -> [1,1,H*D]."""
    n = int(valid_length)
    heads, dim = q.shape[1], q.shape[3]
    group = heads // cache_keys.shape[1]
    k = cache_keys[0, :, :n].double().repeat_interleave(group, dim=0)  # [H,n,D]
    v = cache_values[0, :, :n].double().repeat_interleave(group, dim=0)
    qd = q[0, :, 0].double() * float(torch.tensor(scale, dtype=torch.float32))
    s = torch.einsum("hd,hnd->hn", qd, k)
    p = torch.softmax(s, dim=-1)
    o = torch.einsum("hn,hnd->hd", p, v)
    return _bf(o).reshape(1, 1, heads * dim)


def prefill_attention(q, keys, values, scale, kv_start: int = 0):
    """Causal GQA attention in fp64 (the prefill attention of integration.py:360-380):
    q [B,QH,L,D] row i sees keys [0, kv_start+i]; returns [B,L,QH*D] bf16."""
    b, heads, l, dim = q.shape
    group = heads // keys.shape[1]
    n = kv_start + l
    k = keys[:, :, :n].double().repeat_interleave(group, dim=1)
    v = values[:, :, :n].double().repeat_interleave(group, dim=1)
    s = torch.matmul(q.double() * scale, k.transpose(-1, -2))  # [B,H,L,n]
    mask = torch.arange(n)[None, :] > (kv_start + torch.arange(l))[:, None]
    s = s.masked_fill(mask, float("-inf"))
    o = torch.matmul(torch.softmax(s, dim=-1), v)  # [B,H,L,D]
    return _bf(o.transpose(1, 2).reshape(b, l, heads * dim))


# ---------------------------------------------------------------- rotary
def rotary_cos_sin(positions: torch.Tensor, rotary_dim: int = 64, theta: float = 1e7,
                   mrope_section=(11, 11, 10)):
    """Qwen3.5 rotary table (Transformers Qwen3_5TextRotaryEmbedding, default
    rope): inv_freq = 1/theta^(2i/R) in fp32; freqs = pos * inv_freq (fp32);
    emb = [freqs, freqs]; cos/sin -> bf16.

    ``positions`` [B, L] int64 (text: the same position on the temporal,
    height and width rows) or [3, B, L] multimodal rows, combined by the
    interleaved mrope rule: frequency j takes row 1 when j % 3 == 1 and
    j < 3 * section[1], row 2 when j % 3 == 2 and j < 3 * section[2], else
    row 0 (modeling_qwen3_5.py apply_interleaved_mrope)."""
    inv_freq = 1.0 / (theta ** (torch.arange(0, rotary_dim, 2, dtype=torch.int64).float() / rotary_dim))
    if positions.ndim == 2:
        positions = positions[None].expand(3, *positions.shape)
    freqs = positions.float()[..., None] * inv_freq  # [3, B, L, R/2]
    j = torch.arange(rotary_dim // 2)
    row = torch.zeros_like(j)
    row[(j % 3 == 1) & (j < 3 * mrope_section[1])] = 1
    row[(j % 3 == 2) & (j < 3 * mrope_section[2])] = 2
    freqs = torch.gather(freqs, 0, row.view(1, 1, 1, -1).expand(1, *freqs.shape[1:]))[0]
    emb = torch.cat((freqs, freqs), dim=-1)
    return _bf(emb.cos()), _bf(emb.sin())


# ---------------------------------------------------------------- vision
def layer_norm(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor,
               eps: float = 1e-6) -> torch.Tensor:
    """reference kernels.py:1186-1218: mean and variance of the fp32 row,
    bf16((x - mean) * rsqrt(var + eps) * w + b)."""
    xf = _f(x)
    mean = xf.sum(-1, keepdim=True) / xf.shape[-1]
    c = xf - mean
    var = (c * c).sum(-1, keepdim=True) / xf.shape[-1]
    return _bf(c * _rsqrt(var + eps) * _f(weight) + _f(bias))


def residual_add_layer_norm(residual, update, weight, bias, eps: float = 1e-6):
    """reference kernels.py:1221-1280: r' = bf16(r + u), then layer_norm(r')."""
    added = _bf(_f(residual) + _f(update))
    return added, layer_norm(added, weight, bias, eps)


def position_embed_add(hidden, table, indices, weights):
    """reference kernels.py:1283-1336: p = sum_n table[idx_n] * w_n as an fp32
    multiply-add chain in neighbour order (the kernel's `position +=
    embedding * weight`, contracted to one fused multiply-add by Triton's
    default fp fusion), out = bf16(hidden + bf16(p)). Each fused step is
    computed in fp64 (the fp32 product is exact there) and rounded to fp32."""
    pos = torch.zeros(hidden.shape, dtype=torch.float32)
    for n in range(indices.shape[-1]):
        e = table[indices[:, n]].to(torch.float64)
        w = _f(weights[:, n : n + 1]).to(torch.float64)
        pos = (e * w + pos.to(torch.float64)).to(torch.float32)
    return _bf(_f(hidden) + _f(_bf(pos)))


def vision_qkv_rope(packed, cos, sin, *, heads: int, dim: int):
    """reference kernels.py:336-416: packed [T, 3*H*D] -> q, k, v [1, H, T, D];
    q and k get x*cos + rotate_half(x)*sin in fp32 (no fused multiply-add),
    rounded to bf16; v is copied."""
    tokens = packed.shape[0]
    parts = packed.reshape(tokens, 3, heads, dim)
    c = _f(cos)[:, None, :]
    s = _f(sin)[:, None, :]
    half = dim // 2

    def rope(x):
        xf = _f(x)
        rot = torch.cat((-xf[..., half:], xf[..., :half]), dim=-1)
        return _bf(xf * c + rot * s).permute(1, 0, 2).unsqueeze(0).contiguous()

    v = parts[:, 2].permute(1, 0, 2).unsqueeze(0).contiguous()
    return rope(parts[:, 0]), rope(parts[:, 1]), v


def vision_attention(q, k, v, scale: float, cu_seqlens=None):
    """Non-causal attention per image (the Transformers attention interface
    the reference's vision attention calls, integration.py:671-731): fp32
    softmax(q k^T * scale) v over each image's tokens, bf16 out, [T, H*D]."""
    _, heads, tokens, dim = q.shape
    bounds = [0, tokens] if cu_seqlens is None else [int(x) for x in cu_seqlens]
    out = torch.empty(tokens, heads, dim, dtype=torch.float32)
    for a, b in zip(bounds[:-1], bounds[1:]):
        qs, ks, vs = (_f(t[0, :, a:b]) for t in (q, k, v))
        w = torch.softmax(qs @ ks.transpose(-1, -2) * scale, dim=-1)
        out[a:b] = (w @ vs).permute(1, 0, 2)
    return _bf(out.reshape(tokens, heads * dim))
