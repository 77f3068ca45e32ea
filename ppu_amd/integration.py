"""Install the MI355X fused Qwen3.5 inference path on a Transformers model.

Drop-in for the reference's qwen35_fused/integration.py: the same
``FusionConfig`` fields, ``apply_fusions(model, config) -> stats`` and
``precompute_vision_kwargs``, the same weight packing and the same patched
module forwards, with every decode and prefill operator running on the
gfx950 kernels of ``ppu_amd.kernels``. Fields added for MI355X:

  fused_decode : at L == 1 the patched text forward runs each layer as a few
                 fused launches (residual add + RMSNorm in the prologue of the
                 next GEMV, conv1d + delta rule + gated RMSNorm in one kernel,
                 attention combine + sigmoid gate in one kernel) instead of the
                 reference's per-op sequence;
  a8w8         : the packed projections and the other linears run as A8W8
                 (per-channel int8 weights quantised once here, per-token int8
                 activations), as reference explore_runtime_quantization.py
                 applies PPUA8W8Linear to the M, F and L module groups. The
                 lm_head stays bf16.

Patched forwards fall back to the original Transformers forward for inputs
that are not GPU bf16 tensors, as the reference does (integration.py:51-52);
with ``release_original_weights`` that fallback cannot run (the reference has
the same limitation).
"""

from __future__ import annotations

import types
from dataclasses import dataclass
from typing import Any

import torch
import torch.nn.functional as F
from transformers.cache_utils import DynamicCache
from transformers.models.qwen3_5 import modeling_qwen3_5 as qwen_impl

from . import kernels as K


@dataclass(frozen=True)
class FusionConfig:
    """reference integration.py:32-48, plus ``fused_decode`` and ``a8w8``."""

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


def _is_fast_tensor(x: torch.Tensor) -> bool:
    return x.is_cuda and x.dtype == torch.bfloat16


def _register_buffer(module: torch.nn.Module, name: str, value: torch.Tensor | None) -> None:
    if hasattr(module, name):
        setattr(module, name, value)
    else:
        module.register_buffer(name, value, persistent=False)


def _release_linear_weight(module: torch.nn.Module) -> int:
    weight = module.weight
    released = weight.numel() * weight.element_size()
    module.register_parameter("weight", None)
    return released


def _text_model(model: torch.nn.Module) -> torch.nn.Module:
    inner = model.model
    return getattr(inner, "language_model", inner)


# ----------------------------------------------------------------- linears
class _Linear:
    """A projection weight as the decode/prefill kernels consume it: bf16
    [N, K], or int8 [N, K] + fp32 [N, 1] scales when A8W8 is on."""

    def __init__(self, weight: torch.Tensor, a8w8: bool):
        self.a8w8 = a8w8
        if a8w8:
            self.wq, self.scale = K.quantize_weight_i8(weight.contiguous())
            self.weight = None
        else:
            self.weight = weight.contiguous()
            self.wq = self.scale = None
        self.out_features = weight.shape[0]

    def gemv_args(self) -> tuple[torch.Tensor, torch.Tensor | None]:
        """(weight, scale) for the fused decode GEMVs: bf16 weight and None, or
        int8 weight and its fp32 per-channel scales."""
        return (self.wq, self.scale) if self.a8w8 else (self.weight, None)

    def __call__(self, x: torch.Tensor) -> torch.Tensor:
        if self.a8w8:
            return K.a8w8_linear(x.contiguous(), self.wq, self.scale)
        if x.numel() == x.shape[-1]:
            return K.linear(x, self.weight)
        return K.prefill_linear(x, self.weight)


def _pack_linear_weights(model: torch.nn.Module, config: FusionConfig) -> dict[str, int]:
    """reference integration.py:69-140: packed [qkv|z|a|b] (padded), [gate; up]
    and [q; k; v] projections; originals released when configured."""
    text_model = _text_model(model)
    stats = {"delta": 0, "mlp": 0, "attention": 0, "vision": 0, "released_weight_bytes": 0}
    q8 = config.a8w8
    for layer in text_model.layers:
        if hasattr(layer, "linear_attn") and config.delta:
            delta = layer.linear_attn
            packed = torch.cat(
                (delta.in_proj_qkv.weight, delta.in_proj_z.weight, delta.in_proj_a.weight,
                 delta.in_proj_b.weight),
                dim=0,
            ).contiguous().detach()
            if config.delta_projection_padding:
                pad_rows = (-packed.shape[0]) % config.delta_projection_padding
                if pad_rows:
                    packed = F.pad(packed, (0, 0, 0, pad_rows))
            _register_buffer(delta, "_fused_in_proj_weight", packed)
            delta._q35_in = _Linear(packed, q8)
            delta._q35_out = _Linear(delta.out_proj.weight.detach(), q8)
            delta._q35_conv_w = delta.conv1d.weight.detach().squeeze(1).contiguous()
            if q8:
                _register_buffer(delta, "_fused_in_proj_weight", None)
            if config.release_original_weights:
                stats["released_weight_bytes"] += sum(
                    _release_linear_weight(p)
                    for p in (delta.in_proj_qkv, delta.in_proj_z, delta.in_proj_a, delta.in_proj_b)
                )
            stats["delta"] += 1

        if config.swiglu:
            mlp = layer.mlp
            gate_up = torch.cat((mlp.gate_proj.weight, mlp.up_proj.weight), dim=0).contiguous().detach()
            _register_buffer(mlp, "_fused_gate_up_weight", gate_up)
            mlp._q35_gate_up = _Linear(gate_up, q8)
            mlp._q35_down = _Linear(mlp.down_proj.weight.detach(), q8)
            if q8:
                _register_buffer(mlp, "_fused_gate_up_weight", None)
            if config.release_original_weights:
                stats["released_weight_bytes"] += _release_linear_weight(mlp.gate_proj)
                stats["released_weight_bytes"] += _release_linear_weight(mlp.up_proj)
            stats["mlp"] += 1

        if hasattr(layer, "self_attn") and config.attention:
            attn = layer.self_attn
            qgkv = torch.cat(
                (attn.q_proj.weight, attn.k_proj.weight, attn.v_proj.weight), dim=0
            ).contiguous().detach()
            biases = (attn.q_proj.bias, attn.k_proj.bias, attn.v_proj.bias)
            if any(b is not None for b in biases):
                raise ValueError("the MI355X path supports bias-free Qwen3.5 attention projections only")
            _register_buffer(attn, "_fused_qgkv_weight", qgkv)
            attn._q35_qgkv = _Linear(qgkv, q8)
            attn._q35_o = _Linear(attn.o_proj.weight.detach(), q8)
            if q8:
                _register_buffer(attn, "_fused_qgkv_weight", None)
            if config.release_original_weights:
                for p in (attn.q_proj, attn.k_proj, attn.v_proj):
                    stats["released_weight_bytes"] += _release_linear_weight(p)
            stats["attention"] += 1
    return stats


# ----------------------------------------------------------------- module patches
def _patch_norm_module(module: torch.nn.Module) -> None:
    if hasattr(module, "_fused_original_forward"):
        return
    module._fused_original_forward = module.forward

    def forward(self, x: torch.Tensor):
        if _is_fast_tensor(x) and x.is_contiguous():
            return K.rms_norm(x, self.weight, self.eps)
        return self._fused_original_forward(x)

    module.forward = types.MethodType(forward, module)


def _patch_gated_norm_module(module: torch.nn.Module) -> None:
    if hasattr(module, "_fused_original_forward"):
        return
    module._fused_original_forward = module.forward

    def forward(self, hidden_states: torch.Tensor, gate: torch.Tensor | None = None):
        if gate is not None and _is_fast_tensor(hidden_states):
            return K.gated_rms_norm(hidden_states.contiguous(), gate.contiguous(), self.weight,
                                    self.variance_epsilon)
        return self._fused_original_forward(hidden_states, gate)

    module.forward = types.MethodType(forward, module)


def _patch_mlp(module: torch.nn.Module, config: FusionConfig) -> None:
    """reference integration.py:169-187."""
    if hasattr(module, "_fused_original_forward"):
        return
    module._fused_original_forward = module.forward

    def forward(self, x: torch.Tensor):
        if not _is_fast_tensor(x):
            return self._fused_original_forward(x)
        gate_up = self._q35_gate_up
        if (config.ppu_swiglu_gemv and x.shape[:2] == (1, 1) and not gate_up.a8w8):
            activated = K.ppu_swiglu_gemv(x.contiguous(), gate_up.weight,
                                          block_n=config.ppu_swiglu_block_n)
        elif gate_up.a8w8:
            activated = K.a8w8_swiglu(x.contiguous(), gate_up.wq, gate_up.scale)
        else:
            activated = K.silu_and_mul(gate_up(x.contiguous()))
        return self._q35_down(activated)

    module.forward = types.MethodType(forward, module)


def _delta_cache_tensors(module, cache_params, batch, seq_len, device, dtype):
    """reference integration.py:191-217: conv and recurrent state tensors of a
    DeltaNet layer (lazily initialised in the Transformers cache layer)."""
    conv_shape = (batch, module.conv_dim, module.conv_kernel_size)
    recurrent_shape = (batch, module.num_v_heads, module.head_k_dim, module.head_v_dim)
    if cache_params is None:
        return (
            torch.zeros(conv_shape, device=device, dtype=dtype),
            torch.zeros(recurrent_shape, device=device, dtype=torch.float32),
        )
    cache_layer = cache_params.layers[module.layer_idx]
    if cache_layer.record_past:
        raise RuntimeError("fused DeltaNet does not support rollback cache recording")
    if not cache_layer.is_conv_states_initialized[0]:
        example = torch.empty((batch, module.conv_dim, seq_len), device=device, dtype=dtype)
        cache_layer.lazy_initialization(conv_states=example, conv_kernel_size=module.conv_kernel_size)
    if not cache_layer.is_recurrent_states_initialized[0]:
        example = torch.empty(recurrent_shape, device=device, dtype=torch.float32)
        cache_layer.lazy_initialization(recurrent_states=example)
    cache_layer.has_previous_state[0] = True
    return cache_layer.conv_states[0], cache_layer.recurrent_states[0]


def _patch_delta(module: torch.nn.Module, config: FusionConfig) -> None:
    """reference integration.py:220-274."""
    if hasattr(module, "_fused_original_forward"):
        return
    module._fused_original_forward = module.forward

    def forward(self, hidden_states, cache_params=None, attention_mask=None, **kwargs):
        if not _is_fast_tensor(hidden_states):
            return self._fused_original_forward(hidden_states, cache_params=cache_params,
                                                attention_mask=attention_mask, **kwargs)
        if attention_mask is not None:
            hidden_states = qwen_impl.apply_mask_to_padding_states(hidden_states, attention_mask)
        batch, seq_len, _ = hidden_states.shape
        packed = self._q35_in(hidden_states.contiguous())
        conv_state, recurrent_state = _delta_cache_tensors(
            self, cache_params, batch, seq_len, hidden_states.device, hidden_states.dtype)
        qkv = K.causal_conv1d_fused(packed, self._q35_conv_w, conv_state)
        if self.head_v_dim == 128 and seq_len > 1 and self.conv_dim == 3 * self.value_dim:
            # prefill: recurrence and gated norm (z read in place) in one call
            core = K.delta_prefill_gated(qkv, packed, self.A_log, self.dt_bias, recurrent_state,
                                         self.norm.weight, self.layer_norm_epsilon)
            return self._q35_out(core.reshape(batch, seq_len, self.value_dim))
        core = K.delta_recurrent_fused(qkv, packed, self.A_log, self.dt_bias, recurrent_state,
                                       block_v=config.delta_block_v,
                                       precompute_factors=config.delta_precompute_factors)
        core = core.reshape(-1, self.head_v_dim)
        if self.head_v_dim == 128:
            # z read in place from the packed projection (no copy)
            core = K.gated_rms_norm_packed(core, packed, self.conv_dim,
                                           self.value_dim // self.head_v_dim, self.norm.weight,
                                           self.layer_norm_epsilon)
        else:
            z_start = self.conv_dim
            z = packed[..., z_start : z_start + self.value_dim].reshape(-1, self.head_v_dim)
            core = K.gated_rms_norm(core, z.contiguous(), self.norm.weight,
                                    self.layer_norm_epsilon)
        return self._q35_out(core.reshape(batch, seq_len, self.value_dim))

    module.forward = types.MethodType(forward, module)


def _static_cache_layer(module, past_key_values, hidden_states):
    if past_key_values is None:
        return None
    candidate = past_key_values.layers[module.layer_idx]
    if not hasattr(candidate, "max_cache_len"):
        return None
    if not candidate.is_initialized:
        batch, seq_len = hidden_states.shape[:2]
        shape = (batch, module.config.num_key_value_heads, seq_len, module.head_dim)
        initial_key = torch.empty(shape, device=hidden_states.device, dtype=hidden_states.dtype)
        candidate.lazy_initialization(initial_key, torch.empty_like(initial_key))
    return candidate


def _patch_attention(module: torch.nn.Module, config: FusionConfig) -> None:
    """reference integration.py:277-382; prefill attention runs on the gfx950
    causal GQA kernel instead of the attention interface."""
    if hasattr(module, "_fused_original_forward"):
        return
    module._fused_original_forward = module.forward

    def forward(self, hidden_states, position_embeddings, attention_mask, past_key_values=None,
                **kwargs):
        if not _is_fast_tensor(hidden_states):
            return self._fused_original_forward(hidden_states, position_embeddings, attention_mask,
                                                past_key_values=past_key_values, **kwargs)
        packed = self._q35_qgkv(hidden_states.contiguous())
        cos, sin = position_embeddings
        cache_layer = _static_cache_layer(self, past_key_values, hidden_states)
        seq_len = hidden_states.shape[1]
        q, k, v = K.qgkv_norm_rope(
            packed, self.q_norm.weight, self.k_norm.weight, cos, sin,
            q_heads=self.config.num_attention_heads, kv_heads=self.config.num_key_value_heads,
            dim=self.head_dim, rotary_dim=cos.shape[-1],
            cache_key=None if cache_layer is None else cache_layer.keys,
            cache_value=None if cache_layer is None else cache_layer.values,
            cache_start=None if cache_layer is None else cache_layer.cumulative_length,
        )
        valid = None
        kv_start = 0
        if cache_layer is not None:
            cache_layer.cumulative_length.add_(seq_len)
            valid = cache_layer.cumulative_length
        elif past_key_values is not None:
            k, v = past_key_values.update(k, v, self.layer_idx)
            kv_start = k.shape[2] - seq_len
        if config.gqa_decode_attention and cache_layer is not None and seq_len == 1:
            out = K.gqa_decode_attention(q, cache_layer.keys, cache_layer.values, valid,
                                         self.scaling, packed_gate=packed)
            return self._q35_o(out), None
        out = K.gqa_prefill_attention(q, k.contiguous(), v.contiguous(), self.scaling,
                                      kv_start=kv_start, valid_length=valid)
        out = K.attention_gate_mul(out, packed, self.head_dim)
        return self._q35_o(out), None

    module.forward = types.MethodType(forward, module)


# ----------------------------------------------------------------- text forward
def _rope_in_kernel(text_model) -> bool:
    """The fused attention kernel computes cos/sin itself for the default
    (unscaled) rotary table; other rope types keep Transformers' table."""
    rot = text_model.rotary_emb
    return (getattr(rot, "rope_type", "default") == "default"
            and float(getattr(rot, "attention_scaling", 1.0)) == 1.0
            and rot.inv_freq.dtype == torch.float32)


def _fused_decode_layers(text_model, input_ids, inputs_embeds, config, past_key_values,
                         rotary_position_ids):
    """One token through all layers with fused launches; returns the final-normed hidden.

    Per DeltaNet layer: [residual add + RMSNorm -> packed projection -> conv1d
    update] [delta rule] [gated RMSNorm -> out_proj] [residual add + RMSNorm ->
    gate/up GEMV -> SwiGLU] [down]. Per attention layer: [residual add +
    RMSNorm -> packed projection] [Q/K norm + RoPE + cache write + split-K
    attention] [combine + gate + length += 1] [o_proj] and the same MLP. The
    embedding row is gathered by the first projection when layer 0 is a
    DeltaNet layer. With A8W8 the same launches take int8 weights: each GEMV
    quantises its (normalised) input row per token inside the launch.
    """
    layers = text_model.layers[: text_model.config.num_hidden_layers]
    in_kernel_rope = _rope_in_kernel(text_model)
    cos = sin = None
    if not in_kernel_rope:
        ref = inputs_embeds if inputs_embeds is not None else text_model.embed_tokens.weight[:1]
        cos, sin = text_model.rotary_emb(ref, rotary_position_ids)
    residual = inputs_embeds
    update = None
    for index, layer in enumerate(layers):
        ln = layer.input_layernorm
        delta = layer.block_type == "linear_attention"
        mod = layer.linear_attn if delta else layer.self_attn
        lin = mod._q35_in if delta else mod._q35_qgkv
        w_in, s_in = lin.gemv_args()
        if residual is None and not (index == 0 and delta):
            residual = text_model.embed_tokens(input_ids.view(1, 1))
        if delta:
            conv_state, rec_state = _delta_cache_tensors(
                mod, past_key_values, 1, 1, lin_device(lin), torch.bfloat16)
            # residual add + input RMSNorm in the packed projection's prologue,
            # the conv1d update in its epilogue (embedding gather for layer 0)
            if residual is None:
                r_new, packed, qkv = K.norm_linear_conv(
                    text_model.embed_tokens.weight, None, ln.weight, ln.eps, w_in,
                    mod._q35_conv_w, conv_state, token=input_ids, weight_scale=s_in)
            else:
                r_new, packed, qkv = K.norm_linear_conv(residual, update, ln.weight, ln.eps, w_in,
                                                        mod._q35_conv_w, conv_state,
                                                        weight_scale=s_in)
            if r_new is not None:
                residual = r_new
            # delta rule on the convolved qkv, then gated RMSNorm as the
            # prologue of the output projection
            core = K.delta_recurrent_fused(qkv, packed, mod.A_log, mod.dt_bias, rec_state)
            z = packed[..., mod.conv_dim : mod.conv_dim + mod.value_dim]
            w_out, s_out = mod._q35_out.gemv_args()
            update = K.gated_norm_linear(core, z, mod.norm.weight, mod.layer_norm_epsilon, w_out,
                                         weight_scale=s_out)
        else:
            if update is None:
                packed = K.norm_linear(residual, ln.weight, ln.eps, w_in, weight_scale=s_in)
            else:
                residual, packed = K.residual_norm_linear(residual, update, ln.weight, ln.eps, w_in,
                                                          weight_scale=s_in)
            cache_layer = _static_cache_layer(mod, past_key_values, residual)
            if in_kernel_rope:
                out = K.gqa_decode_fused(
                    packed, mod.q_norm.weight, mod.k_norm.weight, text_model.rotary_emb.inv_freq,
                    rotary_position_ids, cache_layer.keys, cache_layer.values,
                    cache_layer.cumulative_length, mod.scaling,
                    q_heads=mod.config.num_attention_heads,
                    mrope_section=tuple(text_model.rotary_emb.mrope_section))
            else:
                q, _, _ = K.qgkv_norm_rope(
                    packed, mod.q_norm.weight, mod.k_norm.weight, cos, sin,
                    q_heads=mod.config.num_attention_heads, kv_heads=mod.config.num_key_value_heads,
                    dim=mod.head_dim, rotary_dim=cos.shape[-1], cache_key=cache_layer.keys,
                    cache_value=cache_layer.values, cache_start=cache_layer.cumulative_length)
                cache_layer.cumulative_length.add_(1)
                out = K.gqa_decode_attention(q, cache_layer.keys, cache_layer.values,
                                             cache_layer.cumulative_length, mod.scaling,
                                             packed_gate=packed)
            update = mod._q35_o(out)
        # post-attention residual + RMSNorm fused into the SwiGLU GEMV
        pln = layer.post_attention_layernorm
        w_gu, s_gu = layer.mlp._q35_gate_up.gemv_args()
        residual, act = K.residual_norm_linear(residual, update, pln.weight, pln.eps, w_gu,
                                               swiglu=True, weight_scale=s_gu)
        update = layer.mlp._q35_down(act)
    _, normalized = K.residual_add_rms_norm(residual, update, text_model.norm.weight,
                                            text_model.norm.eps)
    return normalized


def lin_device(lin: "_Linear") -> torch.device:
    return (lin.weight if lin.weight is not None else lin.wq).device


def _patch_text_model(text_model: torch.nn.Module, config: FusionConfig) -> None:
    """reference integration.py:385-506."""
    if hasattr(text_model, "_fused_original_forward"):
        return
    text_model._fused_original_forward = text_model.forward

    def forward(self, input_ids=None, attention_mask=None, position_ids=None, past_key_values=None,
                inputs_embeds=None, use_cache=None, **kwargs):
        if (input_ids is None) == (inputs_embeds is None):
            raise ValueError("specify exactly one of input_ids and inputs_embeds")
        probe = inputs_embeds if inputs_embeds is not None else self.embed_tokens.weight
        if not _is_fast_tensor(probe) or (input_ids is not None and not input_ids.is_cuda):
            if inputs_embeds is None:
                inputs_embeds = self.embed_tokens(input_ids)
            return self._fused_original_forward(
                input_ids=None, attention_mask=attention_mask, position_ids=position_ids,
                past_key_values=past_key_values, inputs_embeds=inputs_embeds, use_cache=use_cache,
                **kwargs)
        if use_cache and past_key_values is None:
            past_key_values = DynamicCache(config=self.config)
        src = inputs_embeds if inputs_embeds is not None else input_ids
        batch, seq_len = src.shape[0], src.shape[1]
        if position_ids is None:
            past_seen = past_key_values.get_seq_length() if past_key_values is not None else 0
            position_ids = torch.arange(seq_len, device=src.device) + past_seen
            position_ids = position_ids.view(1, 1, -1).expand(4, batch, -1)
        elif position_ids.ndim == 2:
            position_ids = position_ids[None, ...].expand(4, position_ids.shape[0], -1)
        if position_ids.ndim == 3 and position_ids.shape[0] == 4:
            text_position_ids = position_ids[0]
            rotary_position_ids = position_ids[1:]
        else:
            text_position_ids = None
            rotary_position_ids = position_ids
        if isinstance(attention_mask, torch.Tensor) and not torch.cuda.is_current_stream_capturing():
            if not bool(attention_mask.all()):
                raise ValueError("the fused MI355X path does not support padded inputs")
        static = past_key_values is not None and all(
            hasattr(past_key_values.layers[i], "max_cache_len")
            for i, t in enumerate(self.config.layer_types) if t == "full_attention")
        if (config.fused_decode and seq_len == 1 and batch == 1 and static
                and config.delta and config.attention and config.swiglu):
            token = None
            if inputs_embeds is None:
                token = input_ids.reshape(-1)[:1]
                if input_ids.dtype != torch.int64:
                    token = token.to(torch.int64)
            normalized = _fused_decode_layers(
                self, token, None if inputs_embeds is None else inputs_embeds.contiguous(), config,
                past_key_values, rotary_position_ids)
            return qwen_impl.Qwen3_5ModelOutputWithPast(last_hidden_state=normalized,
                                                        past_key_values=past_key_values)
        if inputs_embeds is None:
            inputs_embeds = self.embed_tokens(input_ids)
        position_embeddings = self.rotary_emb(inputs_embeds, rotary_position_ids)
        residual = inputs_embeds.contiguous()
        normalized = K.rms_norm(residual, self.layers[0].input_layernorm.weight,
                                self.layers[0].input_layernorm.eps)
        n_layers = self.config.num_hidden_layers
        for index, layer in enumerate(self.layers[:n_layers]):
            if layer.block_type == "linear_attention":
                update = layer.linear_attn(hidden_states=normalized, cache_params=past_key_values,
                                           attention_mask=None, **kwargs)
            else:
                update, _ = layer.self_attn(hidden_states=normalized, attention_mask=None,
                                            position_ids=text_position_ids,
                                            past_key_values=past_key_values,
                                            position_embeddings=position_embeddings, **kwargs)
            residual, mlp_in = K.residual_add_rms_norm(residual, update.contiguous(),
                                                       layer.post_attention_layernorm.weight,
                                                       layer.post_attention_layernorm.eps)
            mlp_out = layer.mlp(mlp_in)
            nxt = self.layers[index + 1].input_layernorm if index + 1 < n_layers else self.norm
            res_next, normalized = K.residual_add_rms_norm(residual, mlp_out.contiguous(),
                                                           nxt.weight, nxt.eps)
            if index + 1 < n_layers:
                residual = res_next
        return qwen_impl.Qwen3_5ModelOutputWithPast(last_hidden_state=normalized,
                                                    past_key_values=past_key_values)

    text_model.forward = types.MethodType(forward, text_model)


def precompute_vision_kwargs(model: torch.nn.Module, inputs: Any) -> Any:
    """reference integration.py:738-775. The vision encoder is outside this
    build; for text-only inputs (no ``image_grid_thw``) the mapping is returned
    unchanged, and image inputs are passed through for Transformers' own
    vision path."""
    return inputs


def apply_fusions(model: torch.nn.Module, config: FusionConfig | None = None) -> dict[str, int]:
    """Pack weights and install the enabled fast paths (reference integration.py:778-814)."""
    config = config or FusionConfig()
    if model.training:
        raise ValueError("apply_fusions requires model.eval()")
    stats = _pack_linear_weights(model, config)
    text_model = _text_model(model)
    for layer in text_model.layers:
        if config.rms_norm:
            _patch_norm_module(layer.input_layernorm)
            _patch_norm_module(layer.post_attention_layernorm)
        if config.swiglu:
            _patch_mlp(layer.mlp, config)
        if hasattr(layer, "linear_attn") and config.delta:
            _patch_gated_norm_module(layer.linear_attn.norm)
            _patch_delta(layer.linear_attn, config)
        if hasattr(layer, "self_attn") and config.attention:
            _patch_norm_module(layer.self_attn.q_norm)
            _patch_norm_module(layer.self_attn.k_norm)
            _patch_attention(layer.self_attn, config)
    if config.rms_norm:
        _patch_norm_module(text_model.norm)
    if config.residual_norm:
        _patch_text_model(text_model, config)
    model._qwen35_fusion_config = config
    stats["delta_precompute_factors"] = int(config.delta and config.delta_precompute_factors)
    stats["ppu_swiglu_gemv"] = int(config.swiglu and config.ppu_swiglu_gemv)
    stats["fused_decode"] = int(config.fused_decode)
    stats["a8w8"] = int(config.a8w8)
    return stats
