"""Synthetic Qwen3.5-2B-shaped text decoder (random-init bf16 weights).

The model object is Transformers' ``Qwen3_5ForCausalLM`` built from an
explicit ``Qwen3_5TextConfig`` (the config defaults are not the 2B shape), so
the reference's model integration applies to it unchanged. Construction runs
on the meta device (no host-side init of 1.9B parameters); every parameter is
then drawn from one seeded generator in ``named_parameters()`` order:

  * all weights ~N(0, 0.02) in fp32, cast to bf16 — including the RMSNorm
    weights, which Qwen3.5 applies as ``(1 + w)``, A_log, dt_bias and conv1d;
  * except the gated RMSNorm weight of each DeltaNet layer, which multiplies
    the normalised core output directly (no ``1 + w``): ~N(1, 0.02), so the
    DeltaNet branch keeps unit scale as Transformers' ones-init does.

The embedding is tied to the LM head (248320 x 2048, 1.017 GB).
"""

from __future__ import annotations

import torch

MODEL_SEED = 20260625  # reference benchmark_public.py:72


def config_2b(**overrides):
    from transformers.models.qwen3_5.configuration_qwen3_5 import Qwen3_5TextConfig

    fields = dict(
        vocab_size=248320,
        hidden_size=2048,
        intermediate_size=6144,
        num_hidden_layers=24,
        num_attention_heads=8,
        num_key_value_heads=2,
        head_dim=256,
        linear_num_key_heads=16,
        linear_num_value_heads=16,
        linear_key_head_dim=128,
        linear_value_head_dim=128,
        linear_conv_kernel_dim=4,
        rms_norm_eps=1e-6,
        tie_word_embeddings=True,
        max_position_embeddings=262144,
        rope_parameters={
            "rope_type": "default",
            "rope_theta": 1e7,
            "partial_rotary_factor": 0.25,
            "mrope_section": [11, 11, 10],
            "mrope_interleaved": True,
        },
    )
    fields.update(overrides)
    return Qwen3_5TextConfig(**fields)


def config_tiny(**overrides):
    """Same layer pattern and head shapes (the kernels' D = 128 / 256), fewer
    layers and a small vocabulary, for fast CPU/GPU tests."""
    fields = dict(vocab_size=4096, num_hidden_layers=4, intermediate_size=1024, hidden_size=2048)
    fields.update(overrides)
    return config_2b(**fields)


def _init_param(name: str, shape, gen: torch.Generator, device) -> torch.Tensor:
    t = torch.randn(shape, generator=gen, device=device, dtype=torch.float32) * 0.02
    if name.endswith("linear_attn.norm.weight"):
        t += 1.0
    return t.to(torch.bfloat16)


def build_model(config=None, *, device="cuda", seed: int = MODEL_SEED):
    """-> ``Qwen3_5ForCausalLM`` in eval mode, bf16, on ``device``, seeded."""
    from transformers.models.qwen3_5.modeling_qwen3_5 import Qwen3_5ForCausalLM

    config = config or config_2b()
    device = torch.device(device)
    # bf16 parameters as from_pretrained(torch_dtype=bf16) gives; the rotary
    # inverse frequencies are built explicitly in fp32 and stay fp32.
    old = torch.get_default_dtype()
    torch.set_default_dtype(torch.bfloat16)
    try:
        with torch.device("meta"):
            model = Qwen3_5ForCausalLM(config)
    finally:
        torch.set_default_dtype(old)
    model = model.to_empty(device=device)
    gen = torch.Generator(device=device).manual_seed(seed)
    with torch.no_grad():
        for name, p in model.named_parameters():
            p.copy_(_init_param(name, p.shape, gen, device))
        rot = model.model.rotary_emb
        inv_freq, _ = rot.compute_default_rope_parameters(config, device)
        rot.inv_freq.copy_(inv_freq)
        rot.original_inv_freq.copy_(inv_freq)
    model.tie_weights()
    model.eval()
    return model


def text_model(model):
    """The decoder stack: ``model.model.language_model`` for the VLM wrapper,
    ``model.model`` for a text-only causal LM."""
    inner = model.model
    return getattr(inner, "language_model", inner)
