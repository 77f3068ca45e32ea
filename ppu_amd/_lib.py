"""ctypes binding of libq35.so, the gfx950 C-ABI kernel library.

The library is loaded after torch so that it binds to the HIP runtime torch
already loaded (same SONAME), and kernels are enqueued on torch's current
stream; a graph captured with ``torch.cuda.graph`` therefore records them.
There is no fallback: if the library is missing, every operator raises.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().with_name("libq35.so")
ABI_VERSION = 5

_P = ctypes.c_void_p
_I = ctypes.c_int
_L = ctypes.c_longlong
_F = ctypes.c_float

# name -> (restype, argtypes); mirrors include/q35.h (checked by the CPU tests).
SIGNATURES: dict[str, tuple[object, list[object]]] = {
    "q35_abi_version": (_I, []),
    "q35_zero_buffers": (_I, [_P, _P, _I, _P]),
    "q35_stream_read": (_I, [_P, _L, _P, _L, _P, _P]),
    "q35_stream_read_round": (_I, [_P, _L, _P, _L, _P, _P]),
    "q35_layernorm": (_I, [_P, _P, _P, _I, _P, _I, _I, _F, _P]),
    "q35_residual_layernorm": (_I, [_P, _P, _P, _P, _I, _P, _P, _I, _I, _F, _P]),
    "q35_position_embed_add": (_I, [_P, _P, _I, _P, _P, _I, _P, _I, _I, _I, _P]),
    "q35_vision_qkv_rope": (_I, [_P, _P, _P, _I, _P, _P, _P, _I, _I, _I, _P]),
    "q35_vision_attention": (_I, [_P, _P, _P, _P, _P, _I, _I, _I, _I, _F, _P]),
    "q35_rmsnorm": (_I, [_P, _P, _I, _P, _I, _I, _F, _P]),
    "q35_residual_rmsnorm": (_I, [_P, _P, _P, _I, _P, _P, _I, _I, _F, _P]),
    "q35_gated_rmsnorm": (_I, [_P, _P, _P, _I, _P, _I, _I, _F, _P]),
    "q35_gated_rmsnorm_grouped": (_I, [_P, _P, _I, _L, _P, _I, _P, _I, _F, _P]),
    "q35_silu_mul": (_I, [_P, _P, _L, _I, _P]),
    "q35_silu_mul_t": (_I, [_P, _P, _I, _I, _P]),
    "q35_attn_gate_mul": (_I, [_P, _P, _P, _L, _I, _I, _I, _P, _L, _P]),
    "q35_gemv_bf16": (_I, [_P, _P, _P, _P, _I, _F, _P, _P, _P, _I, _I, _I, _P]),
    "q35_swiglu_gemv": (_I, [_P, _P, _P, _P, _I, _F, _P, _P, _P, _I, _I, _I, _P]),
    "q35_gemv_conv": (
        _I, [_P, _P, _P, _P, _I, _F, _P, _P, _I, _I, _I, _P, _P, _P, _I, _I, _P, _I, _P]),
    "q35_gemv_i8": (
        _I, [_P, _P, _P, _P, _P, _I, _F, _P, _P, _P, _P, _P, _P, _I, _I, _I, _P]),
    "q35_gemv_i8_conv": (
        _I, [_P, _P, _P, _P, _P, _I, _F, _P, _P, _I, _I, _I, _P, _P, _P, _I, _I, _P, _I, _P]),
    "q35_swiglu_gemv_i8": (
        _I, [_P, _P, _P, _P, _P, _I, _F, _P, _P, _P, _P, _I, _I, _I, _P]),
    "q35_lm_head_top1_workspace": (_L, [_I, _I]),
    "q35_lm_head_top1": (_I, [_P, _P, _I, _I, _P, _L, _P, _P, _P, _I, _P]),
    "q35_lm_head_top1_noalloc": (_I, [_P, _P, _I, _I, _P, _P, _I, _P]),
    "q35_init": (_I, []),
    "q35_conv1d_update": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _P]),
    "q35_conv1d_prefill": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _I, _P]),
    "q35_delta_decode": (
        _I,
        [_P, _I, _P, _I, _P, _P, _I, _P, _P, _I, _P, _P, _I, _F, _P, _I, _I, _I, _I, _I, _P],
    ),
    "q35_delta_prefill_workspace": (_L, [_I, _I, _I]),
    "q35_delta_prefill": (_I, [_P, _I, _P, _I, _P, _P, _I, _P, _P, _P, _L, _I, _I, _I, _I, _P]),
    "q35_delta_prefill_gated": (
        _I, [_P, _I, _P, _I, _P, _P, _I, _P, _P, _P, _L, _I, _I, _I, _I, _P, _I, _F, _P, _P]),
    "q35_delta_prefill_gated_conv": (
        _I, [_P, _I, _P, _P, _P, _P, _I, _P, _P, _P, _L, _I, _I, _I, _I, _P, _I, _F, _P, _P]),
    "q35_qgkv_norm_rope": (
        _I,
        [_P, _P, _P, _I, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _P],
    ),
    "q35_gqa_decode_splits": (_I, [_I, _I, ctypes.POINTER(_I)]),
    "q35_gqa_decode_workspace": (_L, [_I, _I, _I, _I]),
    "q35_gqa_decode": (_I, [_P, _P, _P, _P, _F, _P, _P, _P, _L, _I, _I, _I, _I, _P]),
    "q35_gqa_prefill": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _P, _F, _P, _L, _P]),
    "q35_gqa_prefill_workspace": (_L, [_I, _I, _I, _I, _I]),
    "q35_gqa_decode_fused": (
        _I,
        [_P, _P, _P, _I, _P, _P, _P, _P, _I, _I, _I, _P, _P, _P, _F, _P, _P, _L, _I, _I, _I, _I,
         _P],
    ),
    "q35_quant_weight_i8": (_I, [_P, _P, _P, _I, _I, _P]),
    "q35_quant_act_i8": (_I, [_P, _P, _P, _I, _I, _P]),
    "q35_gemv_a8w8": (_I, [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _P]),
    "q35_dequant_i32": (_I, [_P, _P, _P, _P, _I, _I, _P]),
    "q35_dequant_swiglu_i32": (_I, [_P, _P, _P, _P, _I, _I, _P]),
    "q35_gemm_workspace": (_L, [_I, _I, _I, _I, _I, _I]),
    "q35_gemm": (_I, [_P, _P, _P, _I, _I, _I, _I, _P, _P, _I, _I, _P, _L, _P]),
    "q35_residual_rmsnorm_dequant_quant": (
        _I, [_P, _P, _P, _P, _P, _I, _P, _P, _P, _P, _I, _I, _F, _P]),
    "q35_dequant_swiglu_quant": (_I, [_P, _P, _P, _P, _P, _I, _I, _P]),
    "q35_lm_head_screen_prep": (_I, [_P, _I, _I, _P, _P, _P, _P]),
    "q35_lm_head_top1_screened_workspace": (_L, [_I, _I]),
    "q35_lm_head_screened_counts": (_L, [_I, ctypes.POINTER(_I)]),
    "q35_lm_head_top1_screened": (_I, [_P, _P, _P, _P, _P, _I, _I, _P, _L, _P, _P, _P, _I, _P]),
    "q35_host_device_ptr": (_I, [_P, _P]),
    "q35_attn_gate_quant": (_I, [_P, _P, _P, _P, _L, _I, _I, _I, _P, _L, _P]),
    "q35_embed_rmsnorm": (_I, [_P, _I, _P, _P, _I, _P, _P, _I, _I, _F, _P]),
}

_lib: ctypes.CDLL | None = None


def load(path: Path | None = None) -> ctypes.CDLL:
    """Load (once) and return the library with argtypes set."""

    global _lib
    if _lib is not None and path is None:
        return _lib
    p = Path(path) if path is not None else LIB_PATH
    if not p.exists():
        raise RuntimeError(
            f"{p} is missing: build it with `python -m ppu_amd.build` (hipcc, gfx950); "
            "there is no fallback implementation"
        )
    lib = ctypes.CDLL(str(p))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    version = lib.q35_abi_version()
    if version != ABI_VERSION:
        raise RuntimeError(f"libq35 ABI version {version}, expected {ABI_VERSION}")
    if torch.cuda.is_available():
        # per-device set-up (the no-alloc top-1's scratch address) before any
        # call can be made under graph capture
        check(lib.q35_init(), "q35_init")
    if path is None:
        _lib = lib
    return lib


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stream(device: torch.device | None = None) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def check(rc: int, name: str) -> None:
    if rc != 0:
        raise RuntimeError(f"{name} failed with HIP status {rc}")


def call(name: str, *args) -> int:
    lib = load()
    rc = getattr(lib, name)(*args)
    check(rc, name)
    return rc
