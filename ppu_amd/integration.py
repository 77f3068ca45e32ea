"""Install the MI355X Qwen3.5 fast path on a Transformers model.

Public interface of reference qwen35_fused/integration.py (``FusionConfig``
:32-48, ``apply_fusions(model, config) -> stats`` :778-814,
``precompute_vision_kwargs`` :738-775): the same config fields and stats keys,
the same packed weight layouts and the same module forwards taking over, with
every decode and prefill operator on the gfx950 kernels of ``ppu_amd.kernels``.

How it is put together here:

* Each packed projection is a ``_Weight`` submodule (bf16 ``[N, K]``, or with
  A8W8 an int8 ``[N, K]`` + fp32 per-row scales) attached to the module that
  owns it, so the packed tensors follow ``model.to()`` and stay out of the
  state dict.
* ``_take_over`` routes a module's ``forward`` through a fast function that
  answers ``NotImplemented`` for inputs it does not handle (CPU or non-bf16
  tensors, as reference integration.py:51-52); the original forward then runs.
* The decoder stack is driven layer by layer by ``prefill_layer`` and
  ``decode_layer``; ``decode_layer`` is the fused batch-1 decode of one layer
  (residual add + RMSNorm in the prologue of the layer's first GEMV, the conv
  update in its epilogue, the gated norm in the output projection's prologue,
  Q/K norm + RoPE + cache write + split-K attention in one launch and the
  combine + gate in another, the post-attention norm in the SwiGLU GEMV).

Fields added for MI355X: ``fused_decode`` (use ``decode_layer`` for batch-1
single-token steps over a static cache) and ``a8w8`` (the packed projections
and the other linears as A8W8, as reference explore_runtime_quantization.py
applies PPUA8W8Linear; the lm_head stays bf16).
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Any, Callable

import torch
from transformers.activations import GELUTanh
from transformers.cache_utils import DynamicCache
from transformers.models.qwen3_5 import modeling_qwen3_5 as qwen_impl

from . import kernels as K
from .capture import prime_capture_state


@dataclass(frozen=True)
class FusionConfig:
    """Switches of reference integration.py:32-48, plus ``fused_decode`` and ``a8w8``."""

    delta: bool = True
    rms_norm: bool = True
    residual_norm: bool = True
    swiglu: bool = True
    attention: bool = True
    vision: bool = True
    release_original_weights: bool = True
    delta_projection_padding: int = 128
    delta_block_v: int = 8
    delta_precompute_factors: bool = True
    ppu_swiglu_gemv: bool = True
    ppu_swiglu_block_n: int = 8
    gqa_decode_attention: bool = True
    vision_graph: bool = True
    vision_graph_max_entries: int = 48
    fused_decode: bool = True
    a8w8: bool = False
    # greedy top-1 through an int8 screen of the lm_head plus an exact
    # recomputation of the rows it cannot exclude (same token, about half the
    # bytes; 0.5 GB more device memory for the 2B vocabulary). Its cost grows
    # with the rows the bound cannot exclude: lm_head_screen_candidates()
    # counts them for a hidden state; past about V/4 (a quarter of the
    # vocabulary) the screen reads more than 3/4 of the plain top-1's bytes
    # and gains little, so switch it off for such weights
    lm_head_screen: bool = True
    # prefill of 64+ tokens: the DeltaNet causal conv computed inside the
    # chunk prep from the raw projection (one launch and one 12 MB
    # intermediate fewer per layer; same values)
    delta_conv_in_prep: bool = True


def _gpu_bf16(t: Any) -> bool:
    return isinstance(t, torch.Tensor) and t.is_cuda and t.dtype == torch.bfloat16


def text_stack(model: torch.nn.Module) -> torch.nn.Module:
    """The decoder stack: ``model.model.language_model`` (VLM) or ``model.model``."""
    inner = model.model
    return getattr(inner, "language_model", inner)


# ----------------------------------------------------------------- weights
class _Weight(torch.nn.Module):
    """A projection weight in the form the kernels read."""

    def __init__(self, weight: torch.Tensor, int8: bool) -> None:
        super().__init__()
        weight = weight.detach().contiguous()
        if int8:
            q, scale = K.quantize_weight_i8(weight)
            self.register_buffer("w", q, persistent=False)
            self.register_buffer("s", scale.reshape(-1).contiguous(), persistent=False)
        else:
            self.register_buffer("w", weight, persistent=False)
            self.s = None

    @property
    def int8(self) -> bool:
        return self.w.dtype == torch.int8

    @property
    def out_features(self) -> int:
        return self.w.shape[0]

    def operands(self) -> tuple[torch.Tensor, torch.Tensor | None]:
        """(weight, per-row scales or None) for the fused decode GEMVs."""
        return self.w, self.s

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if self.int8:
            return K.a8w8_linear(x.contiguous(), self.w, self.s)
        if x.numel() == x.shape[-1]:
            return K.linear(x.contiguous(), self.w)
        return K.prefill_linear(x, self.w)

    def from_int8(self, xq: torch.Tensor, sx: torch.Tensor) -> torch.Tensor:
        """The A8W8 prefill product of already quantised rows ``xq [..., K]``
        (scales ``sx``): the int8 GEMM with the dequant in its epilogue, bf16
        ``[..., N]``."""
        y = K.gemm_a8w8(xq.reshape(-1, xq.shape[-1]), sx, self.w, self.s)
        return y.reshape(*xq.shape[:-1], self.out_features)

    def to_int32(self, x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        """The A8W8 prefill product left as ``(int32 accumulators [rows, N],
        activation scales)`` for a consumer that dequantises on load."""
        xq, sx = K.quantize_act_i8(x.contiguous())
        return K.a8w8_int_gemm(xq, self.w), sx


def _stack_rows(parts: list[torch.Tensor], multiple: int) -> torch.Tensor:
    """Concatenate weights along the output dimension, zero rows appended up
    to a multiple of ``multiple`` (reference integration.py:78-97)."""
    rows = sum(p.shape[0] for p in parts)
    total = -(-rows // multiple) * multiple if multiple else rows
    out = parts[0].new_zeros((total, parts[0].shape[1]))
    at = 0
    for p in parts:
        out[at : at + p.shape[0]].copy_(p.detach())
        at += p.shape[0]
    return out


def _free_linears(*linears: torch.nn.Module) -> int:
    """Drop the original projection weights; returns the bytes given back
    (weights never materialised, on the meta device, count as zero)."""
    freed = 0
    for lin in linears:
        if lin.weight is not None and not lin.weight.is_meta:
            freed += lin.weight.numel() * lin.weight.element_size()
        lin.weight = None
    return freed


def layer_projections(layer: torch.nn.Module, config: FusionConfig) -> dict[str, torch.Tensor]:
    """The packed projection weights of one decoder layer, from its modules
    (reference integration.py:69-140): ``in`` = DeltaNet ``[qkv | z | a | b]``
    zero-padded to a multiple of ``delta_projection_padding`` rows, ``out``;
    ``qgkv`` = attention ``[q (+gate); k; v]``, ``o``; ``gate_up`` = MLP
    ``[gate; up]``, ``down``."""
    out: dict[str, torch.Tensor] = {}
    if hasattr(layer, "linear_attn") and config.delta:
        m = layer.linear_attn
        parts = [m.in_proj_qkv.weight, m.in_proj_z.weight, m.in_proj_a.weight, m.in_proj_b.weight]
        out["in"] = _stack_rows(parts, config.delta_projection_padding)
        out["out"] = m.out_proj.weight.detach()
    if config.swiglu:
        out["gate_up"] = _stack_rows([layer.mlp.gate_proj.weight, layer.mlp.up_proj.weight], 0)
        out["down"] = layer.mlp.down_proj.weight.detach()
    if hasattr(layer, "self_attn") and config.attention:
        a = layer.self_attn
        if any(p.bias is not None for p in (a.q_proj, a.k_proj, a.v_proj)):
            raise ValueError("the MI355X path supports bias-free Qwen3.5 attention projections only")
        out["qgkv"] = _stack_rows([a.q_proj.weight, a.k_proj.weight, a.v_proj.weight], 0)
        out["o"] = a.o_proj.weight.detach()
    return out


def attach_layer(layer: torch.nn.Module, config: FusionConfig, stats: dict[str, int],
                 packed: dict[str, torch.Tensor]) -> None:
    """Give one layer its packed weights (``layer_projections`` layout; A8W8
    quantises them here) and, with ``release_original_weights``, drop the
    original projection weights."""
    int8 = config.a8w8
    free = config.release_original_weights
    if "in" in packed:
        m = layer.linear_attn
        m.q35_in = _Weight(packed["in"], int8)
        m.q35_out = _Weight(packed["out"], int8)
        m.q35_conv_w = m.conv1d.weight.detach().reshape(m.conv_dim, -1).contiguous()
        if free:
            stats["released_weight_bytes"] += _free_linears(m.in_proj_qkv, m.in_proj_z,
                                                            m.in_proj_a, m.in_proj_b)
        stats["delta"] += 1
    if "gate_up" in packed:
        mlp = layer.mlp
        mlp.q35_gate_up = _Weight(packed["gate_up"], int8)
        mlp.q35_down = _Weight(packed["down"], int8)
        if free:
            stats["released_weight_bytes"] += _free_linears(mlp.gate_proj, mlp.up_proj)
        stats["mlp"] += 1
    if "qgkv" in packed:
        a = layer.self_attn
        a.q35_qgkv = _Weight(packed["qgkv"], int8)
        a.q35_o = _Weight(packed["o"], int8)
        if free:
            stats["released_weight_bytes"] += _free_linears(a.q_proj, a.k_proj, a.v_proj)
        stats["attention"] += 1


# ----------------------------------------------------------------- forwards
def _take_over(module: torch.nn.Module, fast: Callable[..., Any]) -> None:
    """Route ``module.forward`` through ``fast``; when ``fast`` returns
    ``NotImplemented`` the module's original forward handles the call."""
    if getattr(module, "_q35_original_forward", None) is not None:
        return
    original = module.forward

    def forward(*args, **kwargs):
        out = fast(*args, **kwargs)
        return original(*args, **kwargs) if out is NotImplemented else out

    module._q35_original_forward = original
    module.forward = forward


def _norm_fast(module):
    def fast(x, *args, **kwargs):
        if args or kwargs or not _gpu_bf16(x) or not x.is_contiguous():
            return NotImplemented
        return K.rms_norm(x, module.weight, module.eps)
    return fast


def _gated_norm_fast(module):
    def fast(hidden_states, gate=None, *args, **kwargs):
        if gate is None or args or kwargs or not _gpu_bf16(hidden_states):
            return NotImplemented
        return K.gated_rms_norm(hidden_states.contiguous(), gate.contiguous(), module.weight,
                                module.variance_epsilon)
    return fast


def _mlp_fast(module, config: FusionConfig):
    def fast(x, *args, **kwargs):
        if args or kwargs or not _gpu_bf16(x):
            return NotImplemented
        return _mlp_apply(module, x.contiguous(), config)
    return fast


def _mlp_apply(mlp, x: torch.Tensor, config: FusionConfig) -> torch.Tensor:
    """SwiGLU MLP (reference integration.py:169-187): decode one token through
    the SwiGLU GEMV, prefill through the matrix-core GEMM with the SwiGLU in
    its epilogue (the packed gate/up product is never stored)."""
    gate_up = mlp.q35_gate_up
    if gate_up.int8:
        act = K.a8w8_swiglu(x, gate_up.w, gate_up.s)
    elif config.ppu_swiglu_gemv and x.shape[:-1] == (1, 1):
        act = K.ppu_swiglu_gemv(x, gate_up.w, block_n=config.ppu_swiglu_block_n)
    elif x.numel() > x.shape[-1] and x.shape[-1] % 64 == 0:
        act = K.gemm_bf16(x, gate_up.w, swiglu=True)  # SwiGLU in the GEMM epilogue
    else:
        act = K.silu_and_mul(gate_up(x))
    return mlp.q35_down(act)


# ----------------------------------------------------------------- cache state
def _delta_state(mixer, cache, batch: int, device: torch.device) -> tuple[torch.Tensor, torch.Tensor]:
    """Conv state ``[B, C, kw]`` bf16 and recurrent state ``[B, H, Dk, Dv]``
    fp32 of a DeltaNet layer: the cache layer's own tensors (created on first
    use, as Transformers' LinearAttentionLayer does), or fresh zeros without a
    cache (reference integration.py:191-217)."""
    conv_shape = (batch, mixer.conv_dim, mixer.conv_kernel_size)
    rec_shape = (batch, mixer.num_v_heads, mixer.head_k_dim, mixer.head_v_dim)
    if cache is None:
        return (torch.zeros(conv_shape, device=device, dtype=torch.bfloat16),
                torch.zeros(rec_shape, device=device, dtype=torch.float32))
    slot = cache.layers[mixer.layer_idx]
    if slot.record_past:
        raise RuntimeError("the fused DeltaNet path keeps no rollback history (record_past)")
    if not slot.is_conv_states_initialized[0]:
        slot.lazy_initialization(conv_states=torch.empty(conv_shape, device=device,
                                                         dtype=torch.bfloat16))
    if not slot.is_recurrent_states_initialized[0]:
        slot.lazy_initialization(recurrent_states=torch.empty(rec_shape, device=device,
                                                              dtype=torch.float32))
    slot.has_previous_state[0] = True
    return slot.conv_states[0], slot.recurrent_states[0]


def _kv_slot(attn, cache, like: torch.Tensor):
    """The static cache layer of an attention module (allocated on first use),
    or None for a dynamic cache / no cache."""
    if cache is None:
        return None
    slot = cache.layers[attn.layer_idx]
    if not hasattr(slot, "max_cache_len"):
        return None
    if not slot.is_initialized:
        shape = (like.shape[0], attn.config.num_key_value_heads, like.shape[1], attn.head_dim)
        probe = torch.empty(shape, device=like.device, dtype=like.dtype)
        slot.lazy_initialization(probe, probe)
    return slot


# ----------------------------------------------------------------- mixers
def _delta_prefill(mixer, hidden: torch.Tensor, cache, config: FusionConfig, quant=None,
                   int32_out: bool = False):
    """DeltaNet mixer on the GPU (reference integration.py:220-274). A8W8
    prefill: ``quant`` = the input already quantised ``(xq [B, L, K], sx)``
    (``hidden`` then only gives the shape), and ``int32_out`` leaves the
    output projection as ``(accumulators, activation scales)``."""
    batch, length, _ = hidden.shape
    packed = mixer.q35_in(hidden.contiguous()) if quant is None else mixer.q35_in.from_int8(*quant)
    conv_state, rec_state = _delta_state(mixer, cache, batch, hidden.device)
    dv = mixer.head_v_dim
    if (config.delta_conv_in_prep and dv == 128 and length >= 64 and mixer.conv_dim == 3 * mixer.value_dim
            and mixer.q35_conv_w.shape[1] == 4 and conv_state.dtype == torch.bfloat16):
        core = K.delta_prefill_gated_conv(packed, mixer.q35_conv_w, conv_state, mixer.A_log,
                                          mixer.dt_bias, rec_state, mixer.norm.weight,
                                          mixer.layer_norm_epsilon)
        core = core.reshape(batch, length, mixer.value_dim)
        return mixer.q35_out.to_int32(core) if int32_out else mixer.q35_out(core)
    qkv = K.causal_conv1d_fused(packed, mixer.q35_conv_w, conv_state)
    if dv == 128 and length > 1 and mixer.conv_dim == 3 * mixer.value_dim:
        core = K.delta_prefill_gated(qkv, packed, mixer.A_log, mixer.dt_bias, rec_state,
                                     mixer.norm.weight, mixer.layer_norm_epsilon)
    else:
        core = K.delta_recurrent_fused(qkv, packed, mixer.A_log, mixer.dt_bias, rec_state,
                                       block_v=config.delta_block_v,
                                       precompute_factors=config.delta_precompute_factors)
        core = core.reshape(-1, dv)
        if dv == 128:
            core = K.gated_rms_norm_packed(core, packed, mixer.conv_dim, mixer.value_dim // dv,
                                           mixer.norm.weight, mixer.layer_norm_epsilon)
        else:
            z = packed[..., mixer.conv_dim : mixer.conv_dim + mixer.value_dim]
            core = K.gated_rms_norm(core, z.reshape(-1, dv).contiguous(), mixer.norm.weight,
                                    mixer.layer_norm_epsilon)
    core = core.reshape(batch, length, mixer.value_dim)
    return mixer.q35_out.to_int32(core) if int32_out else mixer.q35_out(core)


def _delta_fast(mixer, config: FusionConfig):
    def fast(hidden_states, cache_params=None, attention_mask=None, **kwargs):
        if not _gpu_bf16(hidden_states):
            return NotImplemented
        if attention_mask is not None:
            hidden_states = qwen_impl.apply_mask_to_padding_states(hidden_states, attention_mask)
        return _delta_prefill(mixer, hidden_states, cache_params, config)
    return fast


def _attention_prefill(attn, hidden: torch.Tensor, position_embeddings, cache,
                       config: FusionConfig, quant=None, int32_out: bool = False):
    """Attention mixer on the GPU (reference integration.py:277-382): packed
    projection, Q/K norm + RoPE with the static-cache write, decode attention
    for one token or causal GQA prefill attention, sigmoid gate, o_proj.
    ``quant`` / ``int32_out`` as for ``_delta_prefill``."""
    length = hidden.shape[1]
    packed = (attn.q35_qgkv(hidden.contiguous()) if quant is None
              else attn.q35_qgkv.from_int8(*quant))
    cos, sin = position_embeddings
    slot = _kv_slot(attn, cache, hidden)
    q, k, v = K.qgkv_norm_rope(
        packed, attn.q_norm.weight, attn.k_norm.weight, cos, sin,
        q_heads=attn.config.num_attention_heads, kv_heads=attn.config.num_key_value_heads,
        dim=attn.head_dim, rotary_dim=cos.shape[-1],
        cache_key=None if slot is None else slot.keys,
        cache_value=None if slot is None else slot.values,
        cache_start=None if slot is None else slot.cumulative_length,
    )
    kv_start, valid = 0, None
    decode = slot is not None and length == 1 and config.gqa_decode_attention
    if decode:
        slot.cumulative_length.add_(length)
        valid = slot.cumulative_length
    elif slot is not None:
        # the cache length still holds the start here: the attention reads it
        # as such and the gate kernel advances it by `length` (one launch
        # fewer than the reference's add_ before the attention)
        valid = slot.cumulative_length
    elif cache is not None:
        k, v = cache.update(k, v, attn.layer_idx)
        kv_start = k.shape[2] - length
    if decode:
        out = K.gqa_decode_attention(q, slot.keys, slot.values, valid, attn.scaling,
                                     packed_gate=packed)
    else:
        out = K.gqa_prefill_attention(q, k.contiguous(), v.contiguous(), attn.scaling,
                                      kv_start=kv_start, valid_length=valid,
                                      length_is_start=valid is not None)
        hidden = out.shape[-1]
        if (int32_out and attn.q35_o.int8 and hidden % 8 == 0 and attn.head_dim % 8 == 0
                and hidden <= 8192 and packed.shape[-1] % 8 == 0):
            # the gate and the o_proj input's quantisation in one launch
            aq, sa = K.attention_gate_quant(out, packed, attn.head_dim, advance=valid, amount=length)
            return K.a8w8_int_gemm(aq, attn.q35_o.w), sa
        out = K.attention_gate_mul(out, packed, attn.head_dim, advance=valid, amount=length)
    return attn.q35_o.to_int32(out) if int32_out else attn.q35_o(out)


def _attention_fast(attn, config: FusionConfig):
    def fast(hidden_states, position_embeddings, attention_mask, past_key_values=None, **kwargs):
        if not _gpu_bf16(hidden_states):
            return NotImplemented
        return _attention_prefill(attn, hidden_states, position_embeddings, past_key_values,
                                  config), None
    return fast


# ----------------------------------------------------------------- layers
@dataclass
class DecodeContext:
    """What every layer of one fused decode step shares: the cache, the rope
    positions of the token and, when the rotary table is not computed inside
    the attention kernel, the token's cos/sin."""

    cache: Any
    rope_positions: torch.Tensor
    in_kernel_rope: bool
    cos: torch.Tensor | None = None
    sin: torch.Tensor | None = None


def _rope_in_kernel(stack) -> bool:
    """The fused attention kernel builds cos/sin itself for the default
    (unscaled, fp32 inverse-frequency) rotary table."""
    rot = stack.rotary_emb
    return (getattr(rot, "rope_type", "default") == "default"
            and float(getattr(rot, "attention_scaling", 1.0)) == 1.0
            and rot.inv_freq.dtype == torch.float32)


def decode_layer(stack, index: int, residual: torch.Tensor | None, update: torch.Tensor | None,
                 ctx: DecodeContext, token: torch.Tensor | None = None, trace: dict | None = None):
    """One decoder layer of a batch-1 decode step in fused launches.

    The layer's input is the pending pair ``(residual, update)``: its input
    RMSNorm runs on ``residual + update`` inside the first GEMV (``update`` is
    None for the first layer; with ``token`` given, ``residual`` is None and
    the first layer gathers the embedding row itself). Returns the pending pair
    after the layer: ``(residual after the mixer, MLP output)``. ``trace`` (a
    dict) receives the mixer output as ``update``.
    """
    layer = stack.layers[index]
    ln = layer.input_layernorm
    if hasattr(layer, "linear_attn"):
        m = layer.linear_attn
        w_in, s_in = m.q35_in.operands()
        conv_state, rec_state = _delta_state(m, ctx.cache, 1, w_in.device)
        if residual is None:
            r_new, packed, qkv = K.norm_linear_conv(
                stack.embed_tokens.weight, None, ln.weight, ln.eps, w_in, m.q35_conv_w, conv_state,
                token=token, weight_scale=s_in)
        else:
            r_new, packed, qkv = K.norm_linear_conv(residual, update, ln.weight, ln.eps, w_in,
                                                    m.q35_conv_w, conv_state, weight_scale=s_in)
        residual = residual if r_new is None else r_new
        core = K.delta_recurrent_fused(qkv, packed, m.A_log, m.dt_bias, rec_state)
        z = packed[..., m.conv_dim : m.conv_dim + m.value_dim]
        w_out, s_out = m.q35_out.operands()
        update = K.gated_norm_linear(core, z, m.norm.weight, m.layer_norm_epsilon, w_out,
                                     weight_scale=s_out)
    else:
        a = layer.self_attn
        w_in, s_in = a.q35_qgkv.operands()
        if residual is None:
            residual = stack.embed_tokens(token.view(1, 1))
        if update is None:
            packed = K.norm_linear(residual, ln.weight, ln.eps, w_in, weight_scale=s_in)
        else:
            residual, packed = K.residual_norm_linear(residual, update, ln.weight, ln.eps, w_in,
                                                      weight_scale=s_in)
        slot = _kv_slot(a, ctx.cache, residual)
        if ctx.in_kernel_rope:
            rot = stack.rotary_emb
            out = K.gqa_decode_fused(
                packed, a.q_norm.weight, a.k_norm.weight, rot.inv_freq, ctx.rope_positions,
                slot.keys, slot.values, slot.cumulative_length, a.scaling,
                q_heads=a.config.num_attention_heads, mrope_section=tuple(rot.mrope_section))
        else:
            q, _, _ = K.qgkv_norm_rope(
                packed, a.q_norm.weight, a.k_norm.weight, ctx.cos, ctx.sin,
                q_heads=a.config.num_attention_heads, kv_heads=a.config.num_key_value_heads,
                dim=a.head_dim, rotary_dim=ctx.cos.shape[-1], cache_key=slot.keys,
                cache_value=slot.values, cache_start=slot.cumulative_length)
            slot.cumulative_length.add_(1)
            out = K.gqa_decode_attention(q, slot.keys, slot.values, slot.cumulative_length,
                                         a.scaling, packed_gate=packed)
        update = a.q35_o(out)
    if trace is not None:
        trace["update"] = update
    pln = layer.post_attention_layernorm
    w_gu, s_gu = layer.mlp.q35_gate_up.operands()
    residual, act = K.residual_norm_linear(residual, update, pln.weight, pln.eps, w_gu, swiglu=True,
                                           weight_scale=s_gu)
    return residual, layer.mlp.q35_down(act)


def prefill_layer(stack, index: int, residual: torch.Tensor, normalized: torch.Tensor, cache,
                  position_embeddings, config: FusionConfig, trace: dict | None = None):
    """One decoder layer of the unfused-decode / prefill text forward
    (reference integration.py:456-499): mixer on the normalised input, residual
    add + post-attention RMSNorm, MLP, residual add + the next layer's input
    RMSNorm (the final norm after the last layer). Returns ``(residual,
    normalised)`` for the next layer; after the last layer ``residual`` is the
    stream before the final add. ``trace`` (a dict) receives ``update`` (mixer
    output), ``residual_mid`` and ``mlp_out``."""
    layer = stack.layers[index]
    if hasattr(layer, "linear_attn"):
        update = layer.linear_attn(hidden_states=normalized, cache_params=cache,
                                   attention_mask=None)
    else:
        update, _ = layer.self_attn(hidden_states=normalized, position_embeddings=position_embeddings,
                                    attention_mask=None, past_key_values=cache)
    residual, mlp_in = K.residual_add_rms_norm(residual, update.contiguous(),
                                               layer.post_attention_layernorm.weight,
                                               layer.post_attention_layernorm.eps)
    mlp_out = layer.mlp(mlp_in)
    if trace is not None:
        trace.update(update=update, residual_mid=residual, mlp_out=mlp_out)
    last = index + 1 == stack.config.num_hidden_layers
    norm = stack.norm if last else stack.layers[index + 1].input_layernorm
    summed, normalized = K.residual_add_rms_norm(residual, mlp_out.contiguous(), norm.weight, norm.eps)
    return (residual if last else summed), normalized


def prefill_layer_a8w8(stack, index: int, residual: torch.Tensor, shape_of: torch.Tensor, quant,
                       cache, position_embeddings, config: FusionConfig):
    """``prefill_layer`` for A8W8 linears with the activations handed between
    the int8 GEMMs in int8 form: the layer's input arrives quantised
    (``quant`` = ``(xq, sx)``; ``shape_of`` gives its shape), each output
    projection's int32 accumulators are dequantised inside the following
    residual add + RMSNorm, which also quantises its output for the next
    GEMM, and the gate/up GEMM's SwiGLU epilogue output is quantised per
    token for the down projection. The same
    bits as ``prefill_layer`` (each fused kernel keeps the separate kernels'
    arithmetic). Returns ``(residual, normalised or None, quant or None)``:
    after the last layer the final norm's bf16 output and no quant."""
    layer = stack.layers[index]
    if hasattr(layer, "linear_attn"):
        acc, sx = _delta_prefill(layer.linear_attn, shape_of, cache, config, quant=quant,
                                 int32_out=True)
        out_w = layer.linear_attn.q35_out
    else:
        acc, sx = _attention_prefill(layer.self_attn, shape_of, position_embeddings, cache, config,
                                     quant=quant, int32_out=True)
        out_w = layer.self_attn.q35_o
    ln = layer.post_attention_layernorm
    residual, _, mq, ms = K.residual_rmsnorm_dequant_quant(residual, acc, sx, out_w.s, ln.weight, ln.eps)
    gate_up, down = layer.mlp.q35_gate_up, layer.mlp.q35_down
    # SwiGLU in the int8 GEMM's epilogue (bf16 [M, I]), then the per-token
    # quantiser: the same bits as dequant_swiglu_quant on the int32 [M, 2I]
    # accumulators, without writing and re-reading them (~2 us per layer)
    aq, sa = K.quantize_act_i8(K.gemm_a8w8(mq.reshape(-1, mq.shape[-1]), ms, gate_up.w, gate_up.s,
                                           swiglu=True))
    acc = K.a8w8_int_gemm(aq, down.w)
    last = index + 1 == stack.config.num_hidden_layers
    norm = stack.norm if last else stack.layers[index + 1].input_layernorm
    summed, normalized, nq, ns = K.residual_rmsnorm_dequant_quant(
        residual, acc, sa, down.s, norm.weight, norm.eps, normalized=last, quant=not last)
    if last:
        return residual, normalized, None
    return summed, None, (nq.view(shape_of.shape), ns)


def _a8w8_prefill_ok(stack, config: FusionConfig, length: int) -> bool:
    """The int8-handoff prefill applies: A8W8 packed projections on every
    mixer and MLP, hidden width 2048, SwiGLU width <= 6144, and more than 16
    tokens (fewer run on the int8 GEMV)."""
    return (config.a8w8 and config.delta and config.attention and config.swiglu and length > 16
            and stack.config.hidden_size == 2048 and stack.config.intermediate_size <= 6144)


def _rope_positions(position_ids, past_seen: int, batch: int, length: int, device) -> torch.Tensor:
    """Positions the rotary embedding takes: Transformers' Qwen3.5 text model
    accepts ``[B, L]`` text positions, ``[3, B, L]`` rope rows or ``[4, B, L]``
    with the text row first (reference integration.py:409-418)."""
    if position_ids is None:
        return torch.arange(past_seen, past_seen + length, device=device).expand(batch, length)
    if position_ids.ndim == 3 and position_ids.shape[0] == 4:
        return position_ids[1:]
    return position_ids


def _static_cache(stack, cache) -> bool:
    return cache is not None and all(
        hasattr(cache.layers[i], "max_cache_len")
        for i, kind in enumerate(stack.config.layer_types) if kind == "full_attention")


def _text_fast(stack, config: FusionConfig):
    def fast(input_ids=None, attention_mask=None, position_ids=None, past_key_values=None,
             inputs_embeds=None, use_cache=None, **kwargs):
        if (input_ids is None) == (inputs_embeds is None):
            raise ValueError("specify exactly one of input_ids and inputs_embeds")
        if inputs_embeds is not None:
            if not _gpu_bf16(inputs_embeds):
                return NotImplemented
            device, (batch, length) = inputs_embeds.device, inputs_embeds.shape[:2]
        else:
            if not (input_ids.is_cuda and _gpu_bf16(stack.embed_tokens.weight)):
                return NotImplemented
            device, (batch, length) = input_ids.device, input_ids.shape[:2]
        if position_ids is not None and position_ids.device != device:
            raise ValueError(f"position_ids are on {position_ids.device}, the inputs on {device}")
        if (isinstance(attention_mask, torch.Tensor) and not torch.cuda.is_current_stream_capturing()
                and not bool(attention_mask.all())):
            raise ValueError("the fused MI355X path does not support padded inputs")
        cache = past_key_values
        if use_cache and cache is None:
            cache = DynamicCache(config=stack.config)
        past = cache.get_seq_length() if cache is not None else 0
        rope_pos = _rope_positions(position_ids, past, batch, length, device)
        n = stack.config.num_hidden_layers
        if (config.fused_decode and length == 1 and batch == 1 and _static_cache(stack, cache)
                and config.delta and config.attention and config.swiglu):
            ctx = DecodeContext(cache, rope_pos, _rope_in_kernel(stack))
            if not ctx.in_kernel_rope:
                ref = inputs_embeds if inputs_embeds is not None else stack.embed_tokens.weight[:1]
                ctx.cos, ctx.sin = stack.rotary_emb(ref, rope_pos)
            token = None
            residual = inputs_embeds.contiguous() if inputs_embeds is not None else None
            if residual is None:
                token = input_ids.reshape(-1)[:1].to(torch.int64)
            update = None
            for i in range(n):
                residual, update = decode_layer(stack, i, residual, update, ctx, token)
            _, hidden = K.residual_add_rms_norm(residual, update, stack.norm.weight, stack.norm.eps)
        else:
            ln0 = stack.layers[0].input_layernorm
            table = stack.embed_tokens.weight
            if (inputs_embeds is None and table.shape[1] in (512, 1024, 2048, 4096)
                    and table.is_contiguous() and input_ids.dtype == torch.int64):
                # the embedding lookup and the first input norm in one launch
                residual, hidden = K.embed_rms_norm(table, input_ids, ln0.weight, ln0.eps)
            else:
                embeds = inputs_embeds if inputs_embeds is not None else stack.embed_tokens(input_ids)
                residual = embeds.contiguous()
                hidden = K.rms_norm(residual, ln0.weight, ln0.eps)
            rope = kwargs.get("position_embeddings")  # (cos, sin) computed by the caller
            if rope is None:
                rope = stack.rotary_emb(residual, rope_pos)
            if _a8w8_prefill_ok(stack, config, length):
                xq, sx = K.quantize_act_i8(hidden)
                quant = (xq, sx)
                for i in range(n):
                    residual, out, quant = prefill_layer_a8w8(stack, i, residual, hidden, quant, cache,
                                                              rope, config)
                hidden = out
            else:
                for i in range(n):
                    residual, hidden = prefill_layer(stack, i, residual, hidden, cache, rope, config)
        return qwen_impl.Qwen3_5ModelOutputWithPast(last_hidden_state=hidden, past_key_values=cache)
    return fast


# ----------------------------------------------------------------- vision
def _vision_attention(attn, x: torch.Tensor, cos, sin, cu) -> torch.Tensor:
    """One vision block's attention (reference integration.py:644-735): the
    packed QKV projection, the split + RoPE kernel straight into
    ``[1, heads, tokens, dim]``, non-causal attention per image on the
    matrix-core kernel (``vision_attention``: head dims that are multiples of
    8 up to 128, Qwen3.5's 72 included; other head dims raise), output
    projection. ``cu``: the images' int32 row bounds on the device (None for
    one image), built once per call."""
    if attn.head_dim % 8 or attn.head_dim > 128:
        raise ValueError(f"the fused vision attention supports head dims that are multiples of 8 "
                         f"up to 128, not {attn.head_dim}")
    packed = attn.qkv(x).contiguous()
    q, k, v = K.vision_qkv_rope(packed, cos, sin, heads=attn.num_heads, dim=attn.head_dim)
    return attn.proj(K.vision_attention(q, k, v, attn.scaling, cu))


def _patch_embed(visual, pixels: torch.Tensor) -> torch.Tensor:
    """The patch embedding as one GEMM: its Conv3d has kernel = stride = one
    (temporal x patch x patch) block, so each output row is the flattened
    block times the flattened filter bank (same products, one launch instead
    of an im2col per patch)."""
    proj = visual.patch_embed.proj
    w = proj.weight
    x = pixels.reshape(-1, w[0].numel()).to(w.dtype)
    return torch.nn.functional.linear(x, w.reshape(w.shape[0], -1), proj.bias)


def _pad_vision_mlp(mlp, multiple: int = 128) -> None:
    """Give a vision MLP whose intermediate width is not a multiple of
    ``multiple`` zero-padded weights: fc1 gets zero rows and zero bias (its
    extra outputs are act(0)), fc2 zero columns, so the padded product equals
    the original one and both GEMMs run on the library's whole-tile kernels
    (Qwen3.5's 4304 -> 4352: fc2 29.4 -> 22.7 µs, fc1 20.4 -> 18.9 µs at 784
    rows). The module's own weights become views of the padded ones, so no
    memory is duplicated and its forward is unchanged. Only for GPU bf16
    weights with a bias on fc1."""
    fc1, fc2 = mlp.linear_fc1, mlp.linear_fc2
    w1, b1, w2 = fc1.weight, fc1.bias, fc2.weight
    if getattr(mlp, "q35_fc1_w", None) is not None:
        return  # already padded
    if b1 is None or not (_gpu_bf16(w1) and _gpu_bf16(w2) and _gpu_bf16(b1)):
        return
    inter = w1.shape[0]
    padded = -(-inter // multiple) * multiple
    if padded == inter or w2.shape[1] != inter:
        return
    with torch.no_grad():
        w1p = torch.zeros((padded, w1.shape[1]), dtype=w1.dtype, device=w1.device)
        w1p[:inter].copy_(w1)
        b1p = torch.zeros(padded, dtype=b1.dtype, device=b1.device)
        b1p[:inter].copy_(b1)
        w2p = torch.zeros((w2.shape[0], padded), dtype=w2.dtype, device=w2.device)
        w2p[:, :inter].copy_(w2)
    mlp.register_buffer("q35_fc1_w", w1p, persistent=False)
    mlp.register_buffer("q35_fc1_b", b1p, persistent=False)
    mlp.register_buffer("q35_fc2_w", w2p, persistent=False)
    fc1.weight = torch.nn.Parameter(w1p[:inter], requires_grad=False)
    fc1.bias = torch.nn.Parameter(b1p[:inter], requires_grad=False)
    fc2.weight = torch.nn.Parameter(w2p[:, :inter], requires_grad=False)


def _vision_mlp(mlp, x: torch.Tensor) -> torch.Tensor:
    """Qwen3_5VisionMLP (fc1 -> tanh-approximated GELU -> fc2), on the
    zero-padded weights when ``_pad_vision_mlp`` made them. With the tanh GELU
    the activation is the library GEMM's epilogue applied to the fp32
    accumulator plus bias (one launch and one bf16 rounding fewer than
    rounding fc1's output and running GELU on it); other activations run as
    the module wrote them."""
    fc1, fc2 = mlp.linear_fc1, mlp.linear_fc2
    w1 = getattr(mlp, "q35_fc1_w", None)
    if w1 is None:
        w1, b1, w2 = fc1.weight, fc1.bias, fc2.weight
    else:
        b1, w2 = mlp.q35_fc1_b, mlp.q35_fc2_w
    if isinstance(mlp.act_fn, GELUTanh) and b1 is not None and x.dim() == 2:
        h = torch._addmm_activation(b1, x, w1.t(), use_gelu=True)
    else:
        h = mlp.act_fn(torch.nn.functional.linear(x, w1, b1))
    return torch.nn.functional.linear(h, w2, fc2.bias)


def _vision_merger(merger, hidden: torch.Tensor) -> torch.Tensor:
    """Qwen3_5VisionPatchMerger: LayerNorm (before or after the spatial
    shuffle), then fc1 -> GELU -> fc2 on groups of merged rows."""
    width = merger.hidden_size
    if merger.use_postshuffle_norm:
        x = K.layer_norm(hidden.reshape(-1, width).contiguous(), merger.norm.weight, merger.norm.bias,
                         merger.norm.eps)
    else:
        x = K.layer_norm(hidden, merger.norm.weight, merger.norm.bias, merger.norm.eps).reshape(-1, width)
    return merger.linear_fc2(merger.act_fn(merger.linear_fc1(x)))


def _vision_rotary(visual, position_ids: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """cos / sin ``[tokens, head_dim]`` of the tower's 2-D rotary embedding
    for these position ids (Transformers' rotary module, halves repeated)."""
    freqs = visual.rotary_pos_emb(position_ids).reshape(position_ids.shape[0], -1)
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos().contiguous(), emb.sin().contiguous()


def _vision_forward(visual, pixels, interp_indices, interp_weights, cos, sin, cu):
    """The whole tower for the patches of one call (reference
    integration.py:514-562 plus the patch embedding and the merger): position
    embedding, every block with the given rotary table (the residual stream
    stays bf16; each block's second norm and the next block's first norm run
    as residual-add + LayerNorm launches), merger. Returns (last hidden
    state, merged rows)."""
    patches = _patch_embed(visual, pixels).contiguous()
    hidden = K.position_embed_add(patches, visual.pos_embed.weight, interp_indices, interp_weights)
    blocks = visual.blocks
    n1 = blocks[0].norm1
    normed = K.layer_norm(hidden, n1.weight, n1.bias, n1.eps)
    residual = hidden
    for i, blk in enumerate(blocks):
        update = _vision_attention(blk.attn, normed, cos, sin, cu)
        residual, mlp_in = K.residual_add_layer_norm(residual, update.contiguous(), blk.norm2.weight,
                                                     blk.norm2.bias, blk.norm2.eps)
        mlp_out = _vision_mlp(blk.mlp, mlp_in).contiguous()
        if i + 1 < len(blocks):
            nxt = blocks[i + 1].norm1
            residual, normed = K.residual_add_layer_norm(residual, mlp_out, nxt.weight, nxt.bias, nxt.eps)
        else:
            residual = residual + mlp_out
    return residual, _vision_merger(visual.merger, residual)


class _VisionGraph:
    """The tower for one patch count captured as a graph over static inputs
    (reference integration.py:587-632): the first call of a size runs eagerly
    and captures; later calls copy their inputs in and replay. Outputs are
    returned as copies (the next replay overwrites the graph's buffers)."""

    def __init__(self, visual, pixels, interp_indices, interp_weights, cos, sin) -> None:
        self.inputs = [t.contiguous().clone() for t in (pixels, interp_indices, interp_weights, cos, sin)]
        prime_capture_state(pixels.device)
        torch.cuda.synchronize(pixels.device)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self.out = _vision_forward(visual, *self.inputs, None)

    def run(self, *inputs) -> tuple[torch.Tensor, torch.Tensor]:
        """Copy in the pixels and any further inputs given (in capture
        order), replay, return copies of the outputs."""
        for dst, src in zip(self.inputs, inputs):
            dst.copy_(src)
        self.graph.replay()
        return self.out[0].clone(), self.out[1].clone()


_VISION_PRECOMPUTED = ("interp_indices", "interp_weights", "position_ids", "cu_seqlens")


def _vision_prep(visual, grid_thw: torch.Tensor, kw: dict, device) -> tuple:
    """The tower's per-call inputs derived from ``grid_thw`` (Transformers'
    helpers, which take precomputed values out of ``kw`` when the caller
    passed them): interpolation indices / weights, the images' int32 row
    bounds (None for one image) and the rotary cos / sin of the position ids,
    on ``device``."""
    idx, wts = qwen_impl.get_vision_interpolation_indices_and_weights(
        grid_thw, num_grid_per_side=visual.num_grid_per_side, mode=visual.interpolation_mode,
        align_corners=visual.interpolation_align_corners,
        spatial_merge_size=visual.config.spatial_merge_size, kwargs=kw)
    position_ids = qwen_impl.get_vision_position_ids(grid_thw, visual.spatial_merge_size, kwargs=kw)
    cu_seqlens, _ = qwen_impl.get_vision_attention_seqlens(grid_thw, visual.config, kwargs=kw)
    cu = None
    if cu_seqlens.numel() != 2:
        cu = cu_seqlens.to(device=device, dtype=torch.int32).contiguous()
    cos, sin = _vision_rotary(visual, position_ids.to(device))
    return idx.to(device).contiguous(), wts.to(device).contiguous(), cu, cos, sin


def _vision_model_fast(visual, config: FusionConfig):
    graphs: dict[tuple, _VisionGraph] = {}
    preps: dict[tuple, tuple] = {}

    def fast(hidden_states, grid_thw=None, **kwargs):
        if (grid_thw is None or not hidden_states.is_cuda or not _gpu_bf16(visual.pos_embed.weight)
                or kwargs.get("output_attentions") or kwargs.get("output_hidden_states")):
            return NotImplemented
        kw = dict(kwargs)
        device = hidden_states.device
        inv_freq = getattr(visual.rotary_pos_emb, "inv_freq", None)
        rot_key = (inv_freq.data_ptr(), inv_freq._version) if inv_freq is not None else ()
        grid_key = (str(device), *rot_key) + tuple(int(g) for g in grid_thw.reshape(-1).tolist())
        given = any(kw.get(name) is not None for name in _VISION_PRECOMPUTED)
        if given:
            prep = _vision_prep(visual, grid_thw, kw, device)
        else:
            # Pure functions of the grid: computed once per grid (a few dozen
            # small launches and host syncs fewer per call).
            prep = preps.get(grid_key)
            if prep is None:
                prep = _vision_prep(visual, grid_thw, kw, device)
                if len(preps) < 64:
                    preps[grid_key] = prep
        idx, wts, cu, cos, sin = prep
        pixels = hidden_states.to(visual.patch_embed.proj.weight.dtype).contiguous()
        single = cu is None
        key = (tuple(pixels.shape), wts.dtype, grid_key)
        entry = graphs.get(key) if config.vision_graph and single else None
        if entry is not None:
            # The captured grid's inputs are already in place unless the
            # caller handed in its own.
            hidden, merged = entry.run(pixels, *((idx, wts, cos, sin) if given else ()))
        else:
            hidden, merged = _vision_forward(visual, pixels, idx, wts, cos, sin, cu)
            if (config.vision_graph and single and len(graphs) < config.vision_graph_max_entries
                    and not torch.cuda.is_current_stream_capturing()):
                graphs[key] = _VisionGraph(visual, pixels, idx, wts, cos, sin)
        return qwen_impl.BaseModelOutputWithPooling(last_hidden_state=hidden, pooler_output=merged)
    return fast


def install_vision(visual, config: FusionConfig) -> int:
    """Take over a Qwen3.5 vision tower's forward (the fused tower, its graph
    per image size and grid) after padding its MLP weights; returns the
    number of blocks."""
    for blk in visual.blocks:
        _pad_vision_mlp(blk.mlp)
    _take_over(visual, _vision_model_fast(visual, config))
    return len(visual.blocks)


def _vision_tower(model: torch.nn.Module):
    inner = getattr(model, "model", None)
    return getattr(inner, "visual", None)


# ----------------------------------------------------------------- entry points
def precompute_vision_kwargs(model: torch.nn.Module, inputs: Any) -> Any:
    """reference integration.py:738-775: for an image input (``image_grid_thw``
    present), add the vision tower's interpolation indices / weights, rotary
    position ids and sequence bounds under the ``image_``-prefixed names that
    Transformers' ``get_image_features`` hands to the vision forward, so they
    are computed once on the processor output (CPU) and travel with
    ``inputs.to(device)``. Text-only inputs are returned unchanged."""
    grid = inputs.get("image_grid_thw")
    if grid is None:
        return inputs
    visual = _vision_tower(model)
    sink: dict[str, Any] = {}
    idx, wts = qwen_impl.get_vision_interpolation_indices_and_weights(
        grid, num_grid_per_side=visual.num_grid_per_side, mode=visual.interpolation_mode,
        align_corners=visual.interpolation_align_corners,
        spatial_merge_size=visual.config.spatial_merge_size, kwargs=sink)
    position_ids = qwen_impl.get_vision_position_ids(grid, visual.spatial_merge_size, kwargs=sink)
    cu_seqlens, max_seqlen = qwen_impl.get_vision_attention_seqlens(grid, visual.config, kwargs=sink)
    inputs["image_interp_indices"] = idx
    inputs["image_interp_weights"] = wts
    inputs["image_position_ids"] = position_ids
    inputs["image_cu_seqlens"] = cu_seqlens
    if max_seqlen is not None:
        inputs["image_max_seqlen"] = max_seqlen
    return inputs


def attach_lm_head_screen(model: torch.nn.Module) -> bool:
    """Give ``model.lm_head`` the operands of the screened greedy top-1 (an
    int8 copy of its weight and per-row scale / error-bound factors), keyed
    to the weight's storage and version; False where the weight does not fit
    the kernel (not a contiguous bf16 GPU [V, 2048] tensor)."""
    lm = getattr(model, "lm_head", None)
    w = getattr(lm, "weight", None)
    if w is None or w.dim() != 2 or w.shape[1] != 2048 or not _gpu_bf16(w) or not w.is_contiguous():
        return False
    wq, sw, cr = K.lm_head_screen_prep(w)
    lm.register_buffer("q35_screen_wq", wq, persistent=False)
    lm.register_buffer("q35_screen_s", sw, persistent=False)
    lm.register_buffer("q35_screen_c", cr, persistent=False)
    lm._q35_screen_of = (w.data_ptr(), w._version)
    return True


def lm_head_screen(model: torch.nn.Module):
    """The screen operands for ``lm_head_argmax(..., screen=)``, or None when
    there are none or the weight changed (storage or in-place version) since
    they were made; the full top-1 kernel then runs."""
    lm = getattr(model, "lm_head", None)
    wq = getattr(lm, "q35_screen_wq", None)
    if wq is None:
        return None
    w = lm.weight
    if (w.data_ptr(), w._version) != getattr(lm, "_q35_screen_of", None) or wq.device != w.device:
        return None
    return wq, lm.q35_screen_s, lm.q35_screen_c


def lm_head_screen_candidates(model: torch.nn.Module, hidden: torch.Tensor) -> int | None:
    """How many lm_head rows the screened top-1 recomputes in bf16 for the
    final hidden state ``hidden`` ([1, 2048] or [2048]) of ``model``: the
    bytes it reads are the int8 copy plus 4 KB per such row. None without
    installed screen operands."""
    screen = lm_head_screen(model)
    if screen is None:
        return None
    _, n = K.lm_head_argmax(hidden.reshape(1, -1), model.lm_head.weight, screen=screen,
                            return_candidates=True)
    return int(n)


def apply_fusions(model: torch.nn.Module, config: FusionConfig | None = None) -> dict[str, int]:
    """Pack the projection weights and take over the enabled module forwards
    (reference integration.py:778-814). Returns the packing statistics."""
    config = config or FusionConfig()
    if model.training:
        raise ValueError("apply_fusions requires model.eval()")
    stack = text_stack(model)
    return install(model, config, [layer_projections(layer, config) for layer in stack.layers])


def install(model: torch.nn.Module, config: FusionConfig,
            packed: list[dict[str, torch.Tensor]]) -> dict[str, int]:
    """``apply_fusions`` with the packed weights given (one
    ``layer_projections``-layout dict per layer), as the checkpoint loader
    builds them straight from the files."""
    if model.training:
        raise ValueError("apply_fusions requires model.eval()")
    stack = text_stack(model)
    stats = {"delta": 0, "mlp": 0, "attention": 0, "vision": 0, "released_weight_bytes": 0}
    for layer, weights in zip(stack.layers, packed):
        attach_layer(layer, config, stats, weights)
    for layer in stack.layers:
        if config.rms_norm:
            _take_over(layer.input_layernorm, _norm_fast(layer.input_layernorm))
            _take_over(layer.post_attention_layernorm, _norm_fast(layer.post_attention_layernorm))
        if config.swiglu:
            _take_over(layer.mlp, _mlp_fast(layer.mlp, config))
        if hasattr(layer, "linear_attn") and config.delta:
            _take_over(layer.linear_attn.norm, _gated_norm_fast(layer.linear_attn.norm))
            _take_over(layer.linear_attn, _delta_fast(layer.linear_attn, config))
        if hasattr(layer, "self_attn") and config.attention:
            _take_over(layer.self_attn.q_norm, _norm_fast(layer.self_attn.q_norm))
            _take_over(layer.self_attn.k_norm, _norm_fast(layer.self_attn.k_norm))
            _take_over(layer.self_attn, _attention_fast(layer.self_attn, config))
    if config.rms_norm:
        _take_over(stack.norm, _norm_fast(stack.norm))
    if config.residual_norm:
        _take_over(stack, _text_fast(stack, config))
    visual = _vision_tower(model)
    if config.vision and visual is not None:
        stats["vision"] = install_vision(visual, config)
    model._qwen35_fusion_config = config
    stats["lm_head_screen"] = int(config.lm_head_screen and attach_lm_head_screen(model))
    stats["delta_precompute_factors"] = int(config.delta and config.delta_precompute_factors)
    stats["ppu_swiglu_gemv"] = int(config.swiglu and config.ppu_swiglu_gemv)
    stats["fused_decode"] = int(config.fused_decode)
    stats["a8w8"] = int(config.a8w8)
    return stats
