"""Load a local Qwen3.5 safetensors checkpoint straight into the packed layouts.

The reference loads a local model directory with Transformers
(``from_pretrained(path, local_files_only=True)``, evaluation_wrapper.py:100-111)
and then packs the projections (integration.py:69-140), holding every
projection twice on the device while it packs. Here the directory is read
tensor by tensor (``safetensors.safe_open``, any number of shards) and each
projection is copied straight into its rows of the packed
``[qkv | z | a | b | zero pad]``, ``[gate; up]`` and ``[q (+gate); k; v]``
buffers on the device; the unpacked projection weights are never
materialised. With ``a8w8`` the packed buffers are quantised on the device as
they are attached (per-row int8 + fp32 scales). Everything else (embedding,
norms, conv taps, ``A_log``, ``dt_bias``, a vision tower) is loaded into the
model as is. Nothing is fetched: ``path`` must be a local directory holding
``config.json`` and ``*.safetensors``.
"""

from __future__ import annotations

import json
from pathlib import Path

import torch

from .integration import FusionConfig, install, text_stack

# (packed buffer, projections in row order) per module kind; the names are
# the Transformers Qwen3.5 submodule names.
_GROUPS = {
    "linear_attn": (("in", ("in_proj_qkv", "in_proj_z", "in_proj_a", "in_proj_b")),
                    ("out", ("out_proj",))),
    "self_attn": (("qgkv", ("q_proj", "k_proj", "v_proj")), ("o", ("o_proj",))),
    "mlp": (("gate_up", ("gate_proj", "up_proj")), ("down", ("down_proj",))),
}


def _config(path: Path):
    from transformers import AutoConfig

    return AutoConfig.from_pretrained(str(path), local_files_only=True)


def _empty_model(config, dtype: torch.dtype):
    from transformers.models.qwen3_5 import modeling_qwen3_5 as impl

    cls = (impl.Qwen3_5ForConditionalGeneration if hasattr(config, "vision_config")
           else impl.Qwen3_5ForCausalLM)
    old = torch.get_default_dtype()
    torch.set_default_dtype(dtype)
    try:
        with torch.device("meta"):
            model = cls(config)
    finally:
        torch.set_default_dtype(old)
    return model.eval()


def _plan(model, stack_prefix: str, fusion: FusionConfig, device, dtype):
    """Packed buffers per layer (zeros, so padding rows stay zero) and the
    checkpoint name -> (layer, buffer key, first row) routing table."""
    enabled = {"linear_attn": fusion.delta, "self_attn": fusion.attention, "mlp": fusion.swiglu}
    packed, route = [], {}
    for i, layer in enumerate(text_stack(model).layers):
        bufs = {}
        for kind, groups in _GROUPS.items():
            if not hasattr(layer, kind) or not enabled[kind]:
                continue
            owner = getattr(layer, kind)
            for key, names in groups:
                row = 0
                for name in names:
                    w = getattr(owner, name).weight
                    route[f"{stack_prefix}layers.{i}.{kind}.{name}.weight"] = (i, key, row)
                    row += w.shape[0]
                pad = fusion.delta_projection_padding if key == "in" else 0
                rows = -(-row // pad) * pad if pad else row
                bufs[key] = torch.zeros((rows, w.shape[1]), device=device, dtype=dtype)
        packed.append(bufs)
    return packed, route


def _shards(path: Path) -> list[Path]:
    index = path / "model.safetensors.index.json"
    if index.exists():
        files = sorted(set(json.loads(index.read_text())["weight_map"].values()))
        return [path / f for f in files]
    files = sorted(path.glob("*.safetensors"))
    if not files:
        raise FileNotFoundError(f"no *.safetensors in {path}")
    return files


def load_checkpoint(path, *, device="cuda", fusion: FusionConfig | None = None,
                    dtype: torch.dtype = torch.bfloat16):
    """-> ``(model, stats)``: the Transformers Qwen3.5 model of the local
    checkpoint at ``path`` (``Qwen3_5ForCausalLM`` for a text config,
    ``Qwen3_5ForConditionalGeneration`` for an image-text one) in eval mode on
    ``device``, with the fused MI355X path installed (``fusion``, default
    ``FusionConfig()``; ``a8w8=True`` quantises the packed projections at
    load) and the packing statistics of ``apply_fusions``."""
    from safetensors import safe_open

    path = Path(path)
    fusion = fusion or FusionConfig()
    if not fusion.release_original_weights:
        raise ValueError("the checkpoint loader never materialises the unpacked projections: "
                         "release_original_weights must stay True")
    device = torch.device(device)
    config = _config(path)
    model = _empty_model(config, dtype)
    stack = text_stack(model)
    prefix = "model.language_model." if hasattr(model.model, "language_model") else "model."
    packed, route = _plan(model, prefix, fusion, device, dtype)
    wanted = {k for k, _ in model.named_parameters() if k not in route}
    for name in route:  # the unpacked projections are never given storage
        mod, _, leaf = name.rpartition(".")
        setattr(model.get_submodule(mod), leaf, None)
    model.to_empty(device=device)
    state: dict[str, torch.Tensor] = {}
    seen = set()
    for shard in _shards(path):
        with safe_open(str(shard), framework="pt", device="cpu") as f:
            for name in f.keys():
                if name in route:
                    i, key, row = route[name]
                    t = f.get_tensor(name)
                    packed[i][key][row : row + t.shape[0]].copy_(t.to(dtype))
                    seen.add(name)
                elif name in wanted:
                    state[name] = f.get_tensor(name).to(device=device, dtype=dtype)
    missing = (set(route) - seen) | (wanted - set(state))
    tied = bool(getattr(config, "tie_word_embeddings", False) or getattr(
        getattr(config, "text_config", None), "tie_word_embeddings", False))
    if tied:
        missing.discard("lm_head.weight")
    if missing:
        raise KeyError(f"checkpoint {path} lacks {len(missing)} tensors, e.g. {sorted(missing)[:4]}")
    with torch.no_grad():
        model.load_state_dict(state, strict=False)
    del state
    if tied:
        model.tie_weights()
    _init_buffers(model, stack, device)
    stats = install(model, fusion, packed)
    return model, stats


def _init_buffers(model, stack, device) -> None:
    """Non-persistent buffers are not in a checkpoint: the text rotary table
    (fp32) and, for the image-text class, the vision rotary table."""
    with torch.no_grad():
        rot = stack.rotary_emb
        inv_freq, _ = rot.compute_default_rope_parameters(stack.config, device)
        rot.inv_freq = inv_freq.to(device)
        rot.original_inv_freq = rot.inv_freq.clone()
        visual = getattr(model.model, "visual", None)
        if visual is not None:
            vr = visual.rotary_pos_emb
            vr.inv_freq = 1.0 / (vr.theta ** (torch.arange(0, vr.dim, 2, dtype=torch.float32,
                                                           device=device) / vr.dim))
