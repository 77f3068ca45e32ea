"""The local safetensors loader (ppu_amd.checkpoint) on the CPU: a checkpoint
written from the seeded synthetic model, split into two shards with an index
file, loads into the packed layouts bit for bit, and every other tensor
equals the source model's; a missing tensor is reported."""

from __future__ import annotations

import json

import pytest
import torch

from ppu_amd import synth

PACKED = {"in": "linear_attn.q35_in", "out": "linear_attn.q35_out", "gate_up": "mlp.q35_gate_up",
          "down": "mlp.q35_down", "qgkv": "self_attn.q35_qgkv", "o": "self_attn.q35_o"}


def write_checkpoint(model, cfg, directory, drop=()):
    """Two safetensors shards + index, as Transformers' save_pretrained lays them out."""
    from safetensors.torch import save_file

    cfg.save_pretrained(directory)
    sd = {k: v.detach().cpu().contiguous() for k, v in model.state_dict().items()
          if k != "lm_head.weight" and k not in drop}
    keys = sorted(sd)
    shards = {"model-00001-of-00002.safetensors": keys[: len(keys) // 2],
              "model-00002-of-00002.safetensors": keys[len(keys) // 2 :]}
    weight_map = {}
    for fname, ks in shards.items():
        save_file({k: sd[k] for k in ks}, str(directory / fname))
        weight_map.update({k: fname for k in ks})
    (directory / "model.safetensors.index.json").write_text(json.dumps({"weight_map": weight_map}))
    return sd


def test_checkpoint_loads_into_packed_layouts(tmp_path):
    from ppu_amd.checkpoint import load_checkpoint
    from ppu_amd.integration import FusionConfig, layer_projections, text_stack

    cfg = synth.config_tiny()
    src = synth.build_model(cfg, device="cpu")
    expect = [layer_projections(layer, FusionConfig()) for layer in text_stack(src).layers]
    sd = write_checkpoint(src, cfg, tmp_path)
    model, stats = load_checkpoint(tmp_path, device="cpu")
    assert (stats["delta"], stats["attention"], stats["mlp"]) == (3, 1, 4)
    stack = text_stack(model)
    for layer, packed in zip(stack.layers, expect):
        for key, w in packed.items():
            got = layer.get_submodule(PACKED[key]).w
            assert got.shape == w.shape and torch.equal(got, w), key
        assert layer.mlp.gate_proj.weight is None  # never materialised
    loaded = model.state_dict()
    for k, v in sd.items():
        if loaded.get(k) is not None:
            assert torch.equal(loaded[k], v), k
    assert torch.equal(stack.rotary_emb.inv_freq, text_stack(src).rotary_emb.inv_freq)
    assert model.lm_head.weight.data_ptr() == stack.embed_tokens.weight.data_ptr()


def test_checkpoint_missing_tensor_is_reported(tmp_path):
    from ppu_amd.checkpoint import load_checkpoint

    cfg = synth.config_tiny()
    src = synth.build_model(cfg, device="cpu")
    write_checkpoint(src, cfg, tmp_path, drop=("model.layers.2.mlp.up_proj.weight",))
    with pytest.raises(KeyError, match="lacks 1 tensors"):
        load_checkpoint(tmp_path, device="cpu")
