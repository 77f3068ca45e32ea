"""Synthetic Qwen3.5-2B-shaped text decoder (random-init bf16 weights).

The model object is Transformers' ``Qwen3_5ForCausalLM`` built from an
explicit ``Qwen3_5TextConfig`` (the config defaults are not the 2B shape), so
the reference's model integration applies to it unchanged. Construction runs
on the meta device; every parameter is then drawn on the host from one seeded
CPU generator (mt19937: the same bits on every host and torch/ROCm build, so
the CPU oracle and the GPU start from identical weights) in
``named_parameters()`` order and copied to the device:

  * all weights ~N(0, 0.02) in fp32, cast to bf16 — including the RMSNorm
    weights, which Qwen3.5 applies as ``(1 + w)``, A_log, dt_bias and conv1d;
  * except the gated RMSNorm weight of each DeltaNet layer, which multiplies
    the normalised core output directly (no ``1 + w``): ~N(1, 0.02), so the
    DeltaNet branch keeps unit scale as Transformers' ones-init does.

The embedding is tied to the LM head (248320 x 2048, 1.017 GB).
"""

from __future__ import annotations

import hashlib

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


def _init_param(name: str, shape, gen: torch.Generator) -> torch.Tensor:
    t = torch.randn(shape, generator=gen, dtype=torch.float32) * 0.02
    if name.endswith("linear_attn.norm.weight"):
        t += 1.0
    return t.to(torch.bfloat16)


def tensor_sha256(t: torch.Tensor) -> str:
    """SHA-256 of a tensor's bytes (host copy, native byte order)."""
    raw = t.detach().contiguous().cpu().reshape(-1).view(torch.uint8)
    return hashlib.sha256(raw.numpy().tobytes()).hexdigest()


def config_vlm(text=None, **overrides):
    """``Qwen3_5Config`` of the image-text model class with a small vision
    tower (one block, 64 wide) in front of ``text`` (default: the tiny text
    config); the image / video / vision-bracket token ids are moved inside the
    text vocabulary."""
    from transformers.models.qwen3_5.configuration_qwen3_5 import Qwen3_5Config

    text = text or config_tiny()
    tc = text.to_dict()
    tc.pop("model_type", None)
    vocab = text.vocab_size
    vision = dict(depth=1, hidden_size=64, intermediate_size=128, num_heads=2, in_channels=3,
                  patch_size=16, spatial_merge_size=2, temporal_patch_size=2,
                  out_hidden_size=text.hidden_size, num_position_embeddings=64)
    fields = dict(text_config=tc, vision_config=vision, image_token_id=vocab - 4,
                  video_token_id=vocab - 3, vision_start_token_id=vocab - 2,
                  vision_end_token_id=vocab - 1, tie_word_embeddings=True)
    fields.update(overrides)
    return Qwen3_5Config(**fields)


def build_model(config=None, *, device="cuda", seed: int = MODEL_SEED, digest: list | None = None):
    """-> ``Qwen3_5ForCausalLM`` (a text config) or
    ``Qwen3_5ForConditionalGeneration`` (a ``Qwen3_5Config``, see
    ``config_vlm``) in eval mode, bf16, on ``device``, seeded.

    ``digest`` (a list) receives the SHA-256 over every parameter's name and
    bf16 bytes in generation order, to pin the inputs across builds."""
    from transformers.models.qwen3_5 import modeling_qwen3_5 as impl

    config = config or config_2b()
    vlm = hasattr(config, "text_config") and hasattr(config, "vision_config")
    cls = impl.Qwen3_5ForConditionalGeneration if vlm else impl.Qwen3_5ForCausalLM
    device = torch.device(device)
    # bf16 parameters as from_pretrained(torch_dtype=bf16) gives; the rotary
    # inverse frequencies are built explicitly in fp32 and stay fp32.
    old = torch.get_default_dtype()
    torch.set_default_dtype(torch.bfloat16)
    try:
        with torch.device("meta"):
            model = cls(config)
    finally:
        torch.set_default_dtype(old)
    model = model.to_empty(device=device)
    gen = torch.Generator().manual_seed(seed)
    h = hashlib.sha256() if digest is not None else None
    with torch.no_grad():
        for name, p in model.named_parameters():
            t = _init_param(name, p.shape, gen)
            if h is not None:
                h.update(name.encode())
                h.update(t.reshape(-1).view(torch.uint8).numpy().tobytes())
            p.copy_(t)
        stack = text_model(model)
        rot = stack.rotary_emb
        inv_freq, _ = rot.compute_default_rope_parameters(stack.config, device)
        rot.inv_freq.copy_(inv_freq)
        rot.original_inv_freq.copy_(inv_freq)
        if vlm:  # the vision rotary table (a non-persistent buffer left empty by to_empty)
            vr = model.model.visual.rotary_pos_emb
            vr.inv_freq.copy_(1.0 / (vr.theta ** (torch.arange(0, vr.dim, 2, dtype=torch.float32,
                                                               device=device) / vr.dim)))
    model.tie_weights()
    model.eval()
    if digest is not None:
        digest.append(h.hexdigest())
    return model


def prompt_ids(length: int, vocab: int, seed: int = MODEL_SEED) -> torch.Tensor:
    """Uniform-random token ids ``[1, length]`` int64 from a seeded CPU generator."""
    g = torch.Generator().manual_seed(seed)
    return torch.randint(0, vocab, (1, length), generator=g)


def text_model(model):
    """The decoder stack: ``model.model.language_model`` for the VLM wrapper,
    ``model.model`` for a text-only causal LM."""
    inner = model.model
    return getattr(inner, "language_model", inner)
