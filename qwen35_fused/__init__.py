"""Reference import names (qwen35_fused) for the MI355X implementation.

``qwen35_fused.kernels``, ``.integration`` and ``.graph`` are the modules of
``ppu_amd`` under the names the reference's callers import
(reference qwen35_fused/__init__.py:1-40, evaluation_wrapper.py:115-117,317-318).
"""

from ppu_amd.integration import precompute_vision_kwargs  # noqa: F401
from ppu_amd.kernels import (  # noqa: F401
    attention_gate_mul,
    causal_conv1d_fused,
    delta_recurrent_fused,
    gated_rms_norm,
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

__all__ = [
    "attention_gate_mul",
    "causal_conv1d_fused",
    "delta_recurrent_fused",
    "gated_rms_norm",
    "layer_norm",
    "lm_head_argmax",
    "position_embed_add",
    "ppu_swiglu_gemv",
    "qgkv_norm_rope",
    "residual_add_layer_norm",
    "residual_add_rms_norm",
    "rms_norm",
    "sigmoid_mul",
    "silu_and_mul",
    "vision_qkv_rope",
    "precompute_vision_kwargs",
]
