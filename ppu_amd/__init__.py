"""MI355X-native Qwen3.5 decode hot path.

``ppu_amd.kernels`` mirrors the reference operator API (qwen35_fused.kernels)
on hand-written gfx950 kernels from libq35.so; ``ppu_amd.integration`` and
``ppu_amd.graph`` mirror the reference model integration and decode-graph
runner. The top-level ``qwen35_fused`` package re-exports these modules under
the reference's import names.
"""

from .kernels import (  # noqa: F401
    attention_gate_mul,
    causal_conv1d_fused,
    delta_recurrent_fused,
    gated_rms_norm,
    gqa_decode_attention,
    layer_norm,
    lm_head_argmax,
    position_embed_add,
    ppu_swiglu_gemv,
    qgkv_norm_rope,
    residual_add_layer_norm,
    residual_add_rms_norm,
    rms_norm,
    sigmoid_mul,
    silu_and_mul,
    vision_qkv_rope,
)
