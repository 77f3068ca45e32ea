"""The C-ABI library: it loads without a GPU, exports every function that
include/q35.h declares, and the ctypes table matches the header's arity."""

from __future__ import annotations

import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


def _header_functions() -> dict[str, int]:
    text = (ROOT / "include" / "q35.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    funcs = {}
    for m in re.finditer(r"\b(?:int|long long)\s+(q35_\w+)\s*\(([^)]*)\)\s*;", text, flags=re.S):
        args = m.group(2).strip()
        funcs[m.group(1)] = 0 if args in ("", "void") else len(args.split(","))
    return funcs


def test_header_parses():
    funcs = _header_functions()
    assert "q35_gemv_bf16" in funcs and "q35_lm_head_top1" in funcs
    assert len(funcs) >= 20


def test_library_exports_every_declared_symbol():
    from ppu_amd import _lib

    lib = _lib.load()
    for name in _header_functions():
        assert hasattr(lib, name), f"{name} declared in q35.h but not exported"


def test_ctypes_table_matches_header():
    from ppu_amd import _lib

    funcs = _header_functions()
    assert set(funcs) == set(_lib.SIGNATURES), set(funcs) ^ set(_lib.SIGNATURES)
    for name, arity in funcs.items():
        assert len(_lib.SIGNATURES[name][1]) == arity, name


def test_abi_version_and_host_queries():
    from ppu_amd import _lib

    lib = _lib.load()
    assert lib.q35_abi_version() == _lib.ABI_VERSION
    assert lib.q35_lm_head_top1_workspace(248320, 2048) >= 248320 // 16
    # factors (4 floats per token and head), plus for L >= 64 the chunked form's
    # 28800 operand + 1 decay + 24576 snapshot floats per (head, 64-token chunk)
    # and 3 floats of alignment slack
    assert lib.q35_delta_prefill_workspace(1, 63, 16) == 4 * 63 * 16
    assert lib.q35_delta_prefill_workspace(1, 1024, 16) == 4 * 1024 * 16 + 16 * 16 * 53377 + 3
    splits = lib.q35_gqa_decode_splits(8192, 2, None)
    assert 1 <= splits <= 1024
    assert lib.q35_gqa_decode_workspace(8192, 8, 2, 256) == 8 * splits * 258


def test_invalid_sizes_rejected_before_launch():
    """Argument checks run on the host and return hipErrorInvalidValue (1)."""
    from ppu_amd import _lib

    lib = _lib.load()
    assert lib.q35_gemv_bf16(None, None, None, None, 0, 0.0, None, None, None, 0, 0, 0, None) == 1
    assert lib.q35_gqa_decode(None, None, None, None, 1.0, None, None, None, 0, 8, 2, 128, 512, None) == 1
    assert lib.q35_delta_decode(None, 0, None, 0, None, None, 0, None, None, 0, None, None, 0, 0.0,
                                None, 1, 16, 64, 0, 0, None) == 1
    assert lib.q35_stream_read(None, 16, None, 1 << 20, None, None) == 1
    assert lib.q35_stream_read_round(None, 16, None, 1 << 20, None, None) == 1


def test_wrappers_reject_cpu_tensors():
    """The operators have no CPU path: CPU inputs raise ValueError, as the
    reference wrappers do (kernels.py:16-21)."""
    import torch

    from ppu_amd import kernels as K

    x = torch.zeros(1, 2048, dtype=torch.bfloat16)
    w = torch.zeros(2048, dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        K.rms_norm(x, w)
    with pytest.raises(ValueError):
        K.residual_add_rms_norm(x, x, w)
    with pytest.raises(ValueError):
        K.lm_head_argmax(x, torch.zeros(16, 2048, dtype=torch.bfloat16))
    with pytest.raises(ValueError):
        K.ppu_swiglu_gemv(x.view(1, 1, -1), torch.zeros(16, 2048, dtype=torch.bfloat16))
    with pytest.raises(ValueError):
        K.ppu_swiglu_gemv(x.view(1, 1, -1), torch.zeros(16, 2048, dtype=torch.bfloat16), block_n=3)
    with pytest.raises(ValueError):
        K.stream_read(x)


def test_reference_import_names():
    import qwen35_fused
    import qwen35_fused.graph
    import qwen35_fused.integration
    import qwen35_fused.kernels

    from ppu_amd import graph, integration, kernels

    assert qwen35_fused.kernels is kernels
    assert qwen35_fused.integration is integration
    assert qwen35_fused.graph is graph
    for name in ("rms_norm", "residual_add_rms_norm", "gated_rms_norm", "silu_and_mul",
                 "ppu_swiglu_gemv", "attention_gate_mul", "qgkv_norm_rope", "causal_conv1d_fused",
                 "delta_recurrent_fused", "gqa_decode_attention", "lm_head_argmax"):
        assert callable(getattr(qwen35_fused.kernels, name))
    assert hasattr(integration, "apply_fusions") and hasattr(integration, "FusionConfig")
    assert hasattr(graph, "GreedyDecodeGraph")
