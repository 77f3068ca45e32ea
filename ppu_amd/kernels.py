"""Operator API of the Qwen3.5 decode hot path on MI355X.

Same names, signatures, return shapes/dtypes and ``ValueError`` conditions as
the reference operator module (qwen35_fused/kernels.py), so the model
integration and graph runner can call them unchanged. Every operator launches
hand-written gfx950 kernels from libq35.so on the current torch stream; none
has a torch or CPU fallback. Outputs and workspaces are allocated with
``torch.empty`` on the input's device (from the graph pool under capture);
state tensors (conv state, recurrent state, KV cache) are updated in place.

Tuning keywords of the reference (``block_n``, ``block_v``, ``splits`` ...)
are accepted and validated as the reference does, but the MI355X kernels pick
their own decomposition.
"""

from __future__ import annotations

import functools
import itertools

import torch

from . import _lib

_BF16 = torch.bfloat16



def _device_checked(fn):
    """Validate the device of every tensor argument before the wrapper runs.

    Each tensor an operator receives reaches a kernel as a raw address, so all
    of them (inputs, weights, states, ``out``/``advance`` targets, positions)
    must be GPU tensors on one device; a CPU tensor would otherwise become a
    host address inside a kernel. Raises ``ValueError`` before any launch.
    The one exception is a ``mirror`` argument in host memory, which the
    wrapper itself accepts only when it is pinned and device-mapped.
    """

    code = fn.__code__
    names = code.co_varnames[: code.co_argcount + code.co_kwonlyargcount]

    @functools.wraps(fn)
    def checked(*args, **kwargs):
        device = None
        flat = []
        for name, value in itertools.chain(zip(names, args), kwargs.items()):
            if isinstance(value, (tuple, list)):
                flat.extend((name, v) for v in value)
            else:
                flat.append((name, value))
        for name, value in flat:
            if not isinstance(value, torch.Tensor):
                continue
            if name == "mirror" and not value.is_cuda:
                continue  # checked by the wrapper (host_device_address)
            if not value.is_cuda:
                raise ValueError(f"fused kernels require GPU tensors: {name} is on {value.device}")
            if device is None:
                device = value.device
            elif value.device != device:
                raise ValueError(f"{name} is on {value.device}, the other operands on {device}")
        return fn(*args, **kwargs)

    return checked


def _rows_and_width(x: torch.Tensor) -> tuple[int, int]:
    """reference kernels.py:16-21."""
    if not x.is_cuda:
        raise ValueError("fused kernels require a GPU tensor")
    if not x.is_contiguous():
        raise ValueError("fused kernels require contiguous input")
    return x.numel() // x.shape[-1], x.shape[-1]


def _need_bf16(*tensors: torch.Tensor) -> None:
    for t in tensors:
        if t.dtype != _BF16:
            raise ValueError(f"MI355X kernels take bfloat16 tensors, got {t.dtype}")


def _param(t: torch.Tensor) -> tuple[torch.Tensor, int]:
    """A small parameter vector as (contiguous tensor, is_fp32 flag)."""
    if t.dtype == torch.float32:
        return t.contiguous(), 1
    if t.dtype == _BF16:
        return t.contiguous(), 0
    return t.float().contiguous(), 1


def _stream(x: torch.Tensor) -> int:
    return _lib.stream(x.device)


# ------------------------------------------------------------------ norms
@_device_checked
def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """Qwen3.5 RMSNorm ``(1 + w)``: fp32 reduction, bf16 output. reference kernels.py:44."""

    rows, width = _rows_and_width(x)
    if weight.numel() != width:
        raise ValueError(f"weight has {weight.numel()} values, expected {width}")
    _need_bf16(x)
    w, wf = _param(weight)
    out = torch.empty_like(x)
    _lib.call("q35_rmsnorm", x.data_ptr(), w.data_ptr(), wf, out.data_ptr(), rows, width,
              float(eps), _stream(x))
    return out


@_device_checked
def embed_rms_norm(table: torch.Tensor, ids: torch.Tensor, weight: torch.Tensor,
                   eps: float = 1e-6) -> tuple[torch.Tensor, torch.Tensor]:
    """``(table[ids], rms_norm(table[ids]))`` in one launch: the embedding
    lookup (reference integration.py:403, ids clamped to the table as the
    decode step's gather does) and the first layer's input norm (reference
    kernels.py:44). ``table [V, D]`` bf16, ``ids`` int64 of any shape; returns
    two ``[*ids.shape, D]`` bf16 tensors. D in 512, 1024, 2048, 4096."""

    if table.ndim != 2 or not table.is_contiguous() or ids.dtype != torch.int64:
        raise ValueError("embed_rms_norm takes a contiguous [V, D] table and int64 ids")
    vocab, width = table.shape
    if width not in (512, 1024, 2048, 4096) or weight.numel() != width:
        raise ValueError("embed_rms_norm supports widths 512, 1024, 2048 and 4096 with a matching weight")
    _need_bf16(table)
    w, wf = _param(weight)
    idx = ids.contiguous()
    rows = idx.numel()
    residual = torch.empty((*ids.shape, width), device=table.device, dtype=table.dtype)
    normed = torch.empty_like(residual)
    _lib.call("q35_embed_rmsnorm", table.data_ptr(), vocab, idx.data_ptr(), w.data_ptr(), wf,
              residual.data_ptr(), normed.data_ptr(), rows, width, float(eps), _stream(table))
    return residual, normed


@_device_checked
def residual_add_rms_norm(
    residual: torch.Tensor,
    update: torch.Tensor,
    weight: torch.Tensor,
    eps: float = 1e-6,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Return ``(residual + update, RMSNorm(residual + update))``. reference kernels.py:85."""

    if residual.shape != update.shape or residual.dtype != update.dtype:
        raise ValueError("residual and update must have identical shape and dtype")
    rows, width = _rows_and_width(residual)
    if not update.is_contiguous():
        raise ValueError("update must be contiguous")
    if weight.numel() != width:
        raise ValueError(f"weight has {weight.numel()} values, expected {width}")
    _need_bf16(residual)
    w, wf = _param(weight)
    residual_out = torch.empty_like(residual)
    norm_out = torch.empty_like(residual)
    _lib.call("q35_residual_rmsnorm", residual.data_ptr(), update.data_ptr(), w.data_ptr(), wf,
              residual_out.data_ptr(), norm_out.data_ptr(), rows, width, float(eps),
              _stream(residual))
    return residual_out, norm_out


@_device_checked
def gated_rms_norm(
    x: torch.Tensor,
    gate: torch.Tensor,
    weight: torch.Tensor,
    eps: float = 1e-6,
) -> torch.Tensor:
    """Gated RMSNorm with eager rounding points. reference kernels.py:139."""

    if x.shape != gate.shape:
        raise ValueError("x and gate must have identical shape")
    rows, width = _rows_and_width(x)
    if not gate.is_contiguous():
        raise ValueError("gate must be contiguous")
    if weight.numel() != width:
        raise ValueError(f"weight has {weight.numel()} values, expected {width}")
    _need_bf16(x, gate)
    w, wf = _param(weight)
    out = torch.empty_like(x)
    _lib.call("q35_gated_rmsnorm", x.data_ptr(), gate.data_ptr(), w.data_ptr(), wf, out.data_ptr(),
              rows, width, float(eps), _stream(x))
    return out


@_device_checked
def gated_rms_norm_packed(
    x: torch.Tensor,
    packed: torch.Tensor,
    gate_offset: int,
    heads: int,
    weight: torch.Tensor,
    eps: float = 1e-6,
) -> torch.Tensor:
    """Gated RMSNorm of ``x`` [tokens * heads, 128] whose gate of (token, head)
    is ``packed[token, gate_offset + head * 128 : ... + 128]``, read in place
    from the packed projection (the prefill form of reference
    integration.py:264-271, without the copy of z)."""

    rows, width = _rows_and_width(x)
    if width != 128:
        raise ValueError("the packed gated norm runs over 128-wide heads")
    if not x.is_contiguous() or not packed.is_contiguous():
        raise ValueError("x and packed must be contiguous")
    stride = packed.shape[-1]
    tokens = packed.numel() // stride
    if rows != tokens * heads or gate_offset < 0 or gate_offset + heads * 128 > stride:
        raise ValueError("gate slice does not match the packed rows")
    if weight.numel() != width:
        raise ValueError(f"weight has {weight.numel()} values, expected {width}")
    _need_bf16(x, packed)
    w, wf = _param(weight)
    out = torch.empty_like(x)
    gate = packed.reshape(-1)[gate_offset:]
    _lib.call("q35_gated_rmsnorm_grouped", x.data_ptr(), gate.data_ptr(), heads, stride,
              w.data_ptr(), wf, out.data_ptr(), rows, float(eps), _stream(x))
    return out


@_device_checked
def silu_and_mul(packed: torch.Tensor) -> torch.Tensor:
    """SiLU of the first half times the second half. reference kernels.py:170."""

    rows, packed_width = _rows_and_width(packed)
    if packed_width % 2:
        raise ValueError("packed last dimension must be even")
    _need_bf16(packed)
    width = packed_width // 2
    out = torch.empty((*packed.shape[:-1], width), device=packed.device, dtype=packed.dtype)
    _lib.call("q35_silu_mul", packed.data_ptr(), out.data_ptr(), rows, width, _stream(packed))
    return out


@_device_checked
def silu_and_mul_t(packed_t: torch.Tensor) -> torch.Tensor:
    """``silu_and_mul`` of the transposed packed projection ``[2*width,
    rows]`` (gate rows, then up rows), returned token-major ``[rows, width]``
    (reference kernels.py:170 on ``packed_t.T``). width % 64 == 0, rows % 8
    == 0."""

    if packed_t.ndim != 2 or not packed_t.is_contiguous():
        raise ValueError("transposed packed projection must be a contiguous [2*width, rows] tensor")
    two_w, rows = packed_t.shape
    width = two_w // 2
    if two_w % 2 or width % 64 or rows % 8:
        raise ValueError("transposed silu_and_mul needs width % 64 == 0 and rows % 8 == 0")
    _need_bf16(packed_t)
    out = torch.empty((rows, width), device=packed_t.device, dtype=packed_t.dtype)
    _lib.call("q35_silu_mul_t", packed_t.data_ptr(), out.data_ptr(), rows, width, _stream(packed_t))
    return out


@_device_checked
def attention_gate_mul(x: torch.Tensor, packed_qgkv: torch.Tensor, head_dim: int, *,
                       advance: torch.Tensor | None = None, amount: int = 0) -> torch.Tensor:
    """Multiply attention output by the gate inside the packed QGKV. reference kernels.py:312.

    ``advance`` (an int64 GPU scalar, e.g. a static cache's cumulative length)
    is incremented by ``amount`` in the same launch: the prefill's
    ``cumulative_length.add_`` (reference integration.py:338), deferred to
    the end of the attention so that no separate launch carries it."""

    if not x.is_contiguous() or not packed_qgkv.is_contiguous():
        raise ValueError("attention gate tensors must be contiguous")
    hidden = x.shape[-1]
    if packed_qgkv.shape[:-1] != x.shape[:-1]:
        raise ValueError("attention output and packed projection rows do not match")
    if not x.is_cuda:
        raise ValueError("fused kernels require a GPU tensor")
    if hidden % head_dim or packed_qgkv.shape[-1] < 2 * hidden:
        raise ValueError("attention gate layout does not match the packed projection")
    _need_bf16(x, packed_qgkv)
    if advance is not None and (advance.dtype != torch.int64 or advance.numel() != 1
                                or advance.device != x.device):
        raise ValueError("advance must be an int64 scalar tensor on the attention output's GPU")
    out = torch.empty_like(x)
    tokens = x.numel() // hidden
    _lib.call("q35_attn_gate_mul", x.data_ptr(), packed_qgkv.data_ptr(), out.data_ptr(), tokens,
              hidden, packed_qgkv.shape[-1], head_dim, _lib.ptr(advance), int(amount), _stream(x))
    return out


# ------------------------------------------------------------------ GEMV
def _gemv_weight(weight: torch.Tensor, weight_scale: torch.Tensor | None):
    """A fused GEMV's weight: bf16 ``[N, K]`` (scale None), or int8 ``[N, K]``
    with its fp32 per-channel scales (A8W8: the activation is quantised per
    token inside the launch). Returns ``(weight, flat scales or None)``."""

    if weight.ndim != 2 or not weight.is_contiguous():
        raise ValueError("GEMV weight must be a contiguous [N, K] tensor")
    if weight.dtype == torch.int8:
        if weight_scale is None:
            raise ValueError("int8 weights need their per-channel scales")
        scale = weight_scale.reshape(-1)
        if (scale.dtype != torch.float32 or scale.numel() != weight.shape[0]
                or not scale.is_contiguous() or scale.device != weight.device):
            raise ValueError("weight_scale must be fp32 with one value per weight row")
        return weight, scale
    if weight_scale is not None:
        raise ValueError("weight_scale is only for int8 weights")
    _need_bf16(weight)
    return weight, None


@_device_checked
def linear(x: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """Decode ``F.linear(x, W)`` for one token (bf16, fp32 accumulate).

    Replaces the vendor GEMV behind the reference's decode ``F.linear`` call
    sites (integration.py:185,245,272,298-302,359).
    """

    k = x.shape[-1]
    if x.numel() != k:
        raise ValueError("decode linear expects a single token")
    if weight.ndim != 2 or weight.shape[1] != k:
        raise ValueError("linear input and weight dimensions do not match")
    if not x.is_cuda or not weight.is_contiguous():
        raise ValueError("decode linear tensors must be contiguous GPU tensors")
    _need_bf16(x, weight)
    x = x.contiguous()
    n = weight.shape[0]
    out = torch.empty((*x.shape[:-1], n), device=x.device, dtype=x.dtype)
    _lib.call("q35_gemv_bf16", weight.data_ptr(), x.data_ptr(), None, None, 0, 0.0, None, None,
              out.data_ptr(), n, k, 0, _stream(x))
    return out


@_device_checked
def residual_norm_linear(
    residual: torch.Tensor,
    update: torch.Tensor,
    norm_weight: torch.Tensor,
    eps: float,
    weight: torch.Tensor,
    *,
    swiglu: bool = False,
    weight_scale: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """``r' = residual + update``; ``y = linear(RMSNorm(r'), W)`` in one launch.

    The residual add and RMSNorm of reference kernels.py:85 run as the GEMV
    prologue (every workgroup recomputes the 2048-wide norm from L2); with
    ``swiglu`` the epilogue of reference kernels.py:232 is applied to a packed
    [gate; up] weight. An int8 ``weight`` with ``weight_scale`` runs the A8W8
    linear on the normalised row (quantised per token in the launch).
    Returns ``(r', y)``.
    """

    k = residual.shape[-1]
    if residual.numel() != k or update.shape != residual.shape:
        raise ValueError("fused residual GEMV expects one token")
    _need_bf16(residual, update)
    weight, sw = _gemv_weight(weight, weight_scale)
    w, wf = _param(norm_weight)
    n = weight.shape[0] // 2 if swiglu else weight.shape[0]
    r_out = torch.empty_like(residual)
    out = torch.empty((*residual.shape[:-1], n), device=residual.device, dtype=residual.dtype)
    args = (residual.data_ptr(), update.data_ptr(), w.data_ptr(), wf, float(eps), r_out.data_ptr(),
            None, out.data_ptr())
    if sw is None:
        name = "q35_swiglu_gemv" if swiglu else "q35_gemv_bf16"
        _lib.call(name, weight.data_ptr(), *args, n, k, 2, _stream(residual))
    elif swiglu:
        _lib.call("q35_swiglu_gemv_i8", weight.data_ptr(), sw.data_ptr(), *args, None, n, k, 2,
                  _stream(residual))
    else:
        _lib.call("q35_gemv_i8", weight.data_ptr(), sw.data_ptr(), *args, None, None, None, n, k, 2,
                  _stream(residual))
    return r_out, out


@_device_checked
def norm_linear(
    x: torch.Tensor,
    norm_weight: torch.Tensor,
    eps: float,
    weight: torch.Tensor,
    *,
    weight_scale: torch.Tensor | None = None,
) -> torch.Tensor:
    """``linear(rms_norm(x), W)`` for one token in one launch: the RMSNorm of
    reference kernels.py:44 as the GEMV prologue (layer 0's input norm); int8
    ``weight`` + ``weight_scale``: A8W8 as residual_norm_linear."""

    k = x.shape[-1]
    if x.numel() != k or weight.ndim != 2 or weight.shape[1] != k:
        raise ValueError("fused norm GEMV expects one token matching the weight")
    _need_bf16(x)
    weight, sw = _gemv_weight(weight, weight_scale)
    w, wf = _param(norm_weight)
    n = weight.shape[0]
    out = torch.empty((*x.shape[:-1], n), device=x.device, dtype=x.dtype)
    args = (x.contiguous().data_ptr(), None, w.data_ptr(), wf, float(eps), None, None, out.data_ptr())
    if sw is None:
        _lib.call("q35_gemv_bf16", weight.data_ptr(), *args, n, k, 1, _stream(x))
    else:
        _lib.call("q35_gemv_i8", weight.data_ptr(), sw.data_ptr(), *args, None, None, None, n, k, 1,
                  _stream(x))
    return out


@_device_checked
def norm_linear_conv(
    residual: torch.Tensor,
    update: torch.Tensor | None,
    norm_weight: torch.Tensor,
    eps: float,
    weight: torch.Tensor,
    conv_weight: torch.Tensor,
    conv_state: torch.Tensor,
    *,
    token: torch.Tensor | None = None,
    weight_scale: torch.Tensor | None = None,
) -> tuple[torch.Tensor | None, torch.Tensor, torch.Tensor]:
    """DeltaNet input projection of one token in one launch.

    Prologue: ``r' = residual + update`` and its RMSNorm (or the RMSNorm of
    ``residual`` when ``update`` is None, the first layer); GEMV against the
    packed ``[qkv | z | a | b]`` weight; epilogue: for the first C rows
    (C = conv channels) the single-token causal conv update of reference
    kernels.py:622-656, which shifts ``conv_state`` in place. Returns
    ``(r' or None, packed [1,1,N], qkv [1,1,C])``.

    With ``token`` (an int64 device scalar) ``residual`` is the embedding table
    ``[V, K]``: the first layer's input is its row ``token`` (the lookup of
    integration.py:402-403, done in the prologue), returned as ``r'``. An int8
    ``weight`` with ``weight_scale`` runs the projection as A8W8.
    """

    k = residual.shape[-1]
    rows = residual.numel() // k
    if token is not None:
        if update is not None or token.dtype != torch.int64 or token.device != residual.device:
            raise ValueError("embedding gather takes an int64 GPU token and no update")
    elif rows != 1:
        raise ValueError("fused projection expects one token")
    if weight.ndim != 2 or weight.shape[1] != k:
        raise ValueError("fused projection expects one token matching the weight")
    channels, kw = conv_weight.shape
    if conv_state.shape[-2:] != (channels, kw) or conv_state.numel() != channels * kw:
        raise ValueError("conv state does not match the conv weight (batch 1)")
    if not conv_state.is_contiguous() or not conv_weight.is_contiguous():
        raise ValueError("conv tensors must be contiguous")
    _need_bf16(residual, conv_weight, conv_state)
    weight, sw = _gemv_weight(weight, weight_scale)
    w, wf = _param(norm_weight)
    n = weight.shape[0]
    dev = residual.device
    packed = torch.empty((1, 1, n), device=dev, dtype=_BF16)
    qkv = torch.empty((1, 1, channels), device=dev, dtype=_BF16)
    r_out = None
    if update is not None:
        if update.shape != residual.shape:
            raise ValueError("residual and update must have identical shape")
        r_out = torch.empty_like(residual)
    elif token is not None:
        r_out = torch.empty((1, 1, k), device=dev, dtype=_BF16)
    args = (residual.data_ptr(), _lib.ptr(update), w.data_ptr(), wf, float(eps), _lib.ptr(r_out),
            packed.data_ptr(), n, k, 2 if update is not None else 1, conv_weight.data_ptr(),
            conv_state.data_ptr(), qkv.data_ptr(), channels, kw, _lib.ptr(token), rows,
            _stream(residual))
    if sw is None:
        _lib.call("q35_gemv_conv", weight.data_ptr(), *args)
    else:
        _lib.call("q35_gemv_i8_conv", weight.data_ptr(), sw.data_ptr(), *args)
    return r_out, packed, qkv


@_device_checked
def gated_norm_linear(
    core: torch.Tensor,
    gate: torch.Tensor,
    norm_weight: torch.Tensor,
    eps: float,
    weight: torch.Tensor,
    *,
    weight_scale: torch.Tensor | None = None,
) -> torch.Tensor:
    """``linear(gated_rms_norm(core, gate), W)`` for one token in one launch:
    the gated RMSNorm of reference kernels.py:139 (heads of 128, ``w`` used
    directly) as the prologue of the DeltaNet output projection. ``gate`` may
    be a contiguous slice of the packed projection. int8 ``weight`` +
    ``weight_scale``: A8W8 on the normed row."""

    k = core.numel()
    if gate.numel() != k or weight.ndim != 2 or weight.shape[1] != k or k % 128:
        raise ValueError("gated norm GEMV expects one token of whole 128-wide heads")
    if not core.is_contiguous() or not gate.is_contiguous():
        raise ValueError("gated norm GEMV inputs must be contiguous")
    _need_bf16(core, gate)
    weight, sw = _gemv_weight(weight, weight_scale)
    w, wf = _param(norm_weight)
    n = weight.shape[0]
    out = torch.empty((1, 1, n), device=core.device, dtype=_BF16)
    args = (core.data_ptr(), gate.data_ptr(), w.data_ptr(), wf, float(eps), None, None, out.data_ptr())
    if sw is None:
        _lib.call("q35_gemv_bf16", weight.data_ptr(), *args, n, k, 3, _stream(core))
    else:
        _lib.call("q35_gemv_i8", weight.data_ptr(), sw.data_ptr(), *args, None, None, None, n, k, 3,
                  _stream(core))
    return out


# ------------------------------------------------------------------ prefill GEMM
# kinds of q35_gemm (include/q35.h)
GEMM_BF16, GEMM_SWIGLU, GEMM_I32, GEMM_DEQUANT, GEMM_DEQUANT_SWIGLU = range(5)
# Split-K workspaces, one per device, zero-filled once and kept for the life of
# the process: a captured graph holds their address, and every launch leaves
# the arrival counters at zero again. A larger request allocates a new one and
# keeps the old. Split-K GEMMs on one device therefore must not overlap in
# time (the prefill issues its GEMMs one after another).
_gemm_ws: dict[int, list[torch.Tensor]] = {}


def _gemm_workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    held = _gemm_ws.setdefault(device.index, [])
    if held and held[-1].numel() * 4 >= nbytes:
        return held[-1]
    if torch.cuda.is_current_stream_capturing():
        raise RuntimeError("the split-K GEMM workspace must exist before graph capture: "
                           "run the same shapes once outside the capture")
    ws = torch.zeros(max(nbytes, 1 << 24) // 4 + 64, device=device, dtype=torch.int32)
    held.append(ws)
    return ws


def gemm_into(a: torch.Tensor, b: torch.Tensor, c: torch.Tensor, kind: int, *,
              s_x: torch.Tensor | None = None, s_w: torch.Tensor | None = None,
              plan: tuple[int, int] | None = None) -> torch.Tensor:
    """``C = A . B^T`` of one kind on the hand-written matrix-core GEMM
    (``q35_gemm``): ``a`` [M, K], ``b`` [N, K] (SwiGLU kinds [2N, K]), ``c``
    [M, N] written in place; all contiguous on the GPU. ``plan`` = (tile 0-8,
    K splits) overrides the library's choice (for measurement)."""

    m, k = a.shape
    n = c.shape[-1]
    tile, splits = plan if plan is not None else (-1, 1)
    lib = _lib.load()
    nbytes = lib.q35_gemm_workspace(m, n, k, kind, tile, splits)
    if nbytes < 0:
        raise ValueError(f"invalid GEMM plan {plan} for kind {kind}")
    ws = _gemm_workspace(a.device, nbytes) if nbytes > 0 else None
    _lib.call("q35_gemm", a.data_ptr(), b.data_ptr(), c.data_ptr(), m, n, k, kind, _lib.ptr(s_x),
              _lib.ptr(s_w), tile, splits, _lib.ptr(ws), 0 if ws is None else ws.numel() * 4,
              _stream(a))
    return c


def _gemm_operands(x: torch.Tensor, weight: torch.Tensor, dtype: torch.dtype, swiglu: bool):
    k = x.shape[-1]
    if weight.ndim != 2 or weight.shape[1] != k:
        raise ValueError("GEMM weight must be [N, K] matching the input")
    if x.dtype != dtype or weight.dtype != dtype:
        raise ValueError(f"GEMM operands must be {dtype}")
    if k % (128 // dtype.itemsize):
        raise ValueError("the matrix-core GEMM needs K to be a multiple of 128 bytes")
    if swiglu and weight.shape[0] % 2:
        raise ValueError("packed SwiGLU weight must have an even number of rows")
    if not (x.is_cuda and weight.is_cuda and weight.is_contiguous()):
        raise ValueError("GEMM tensors must be contiguous GPU tensors")
    x2 = x.reshape(-1, k).contiguous()
    n = weight.shape[0] // 2 if swiglu else weight.shape[0]
    return x2, n


@_device_checked
def prefill_linear(x: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """``F.linear(x, W)`` for M > 1 tokens (prefill), bf16 in/out, fp32
    accumulate, on the hand-written matrix-core GEMM (the reference's prefill
    ``F.linear`` call sites, integration.py:183,245,272,298,359)."""

    return gemm_bf16(x, weight)


@_device_checked
def gemm_bf16(x: torch.Tensor, weight: torch.Tensor, *, swiglu: bool = False,
              plan: tuple[int, int] | None = None) -> torch.Tensor:
    """The hand-written matrix-core prefill GEMM: ``F.linear(x, W)`` (bf16 in
    and out, fp32 accumulate) or, with ``swiglu``, ``silu_and_mul(F.linear(x,
    W))`` for a packed ``[gate; up]`` weight in one launch (reference
    integration.py:183-185, kernels.py:158-180). K must be a multiple of 64.
    ``plan`` = (tile 0-8, K splits) overrides the library's choice."""

    x2, n = _gemm_operands(x, weight, _BF16, swiglu)
    y = torch.empty((*x.shape[:-1], n), device=x.device, dtype=_BF16)
    if x2.shape[0]:
        gemm_into(x2, weight, y.view(-1, n), GEMM_SWIGLU if swiglu else GEMM_BF16, plan=plan)
    return y


@_device_checked
def ppu_swiglu_gemv(
    x: torch.Tensor,
    packed_weight: torch.Tensor,
    *,
    block_n: int = 8,
) -> torch.Tensor:
    """Decode packed gate/up projection with fused SwiGLU. reference kernels.py:232."""

    if x.ndim != 3 or x.shape[:2] != (1, 1) or x.dtype != torch.bfloat16:
        raise ValueError("SwiGLU GEMV expects BF16 x[1,1,K]")
    if packed_weight.ndim != 2 or packed_weight.shape[0] % 2:
        raise ValueError("packed SwiGLU weight must have shape [2N,K]")
    if packed_weight.shape[1] != x.shape[-1] or packed_weight.dtype != x.dtype:
        raise ValueError("SwiGLU GEMV input and weight dimensions do not match")
    if not x.is_contiguous() or not packed_weight.is_contiguous():
        raise ValueError("SwiGLU GEMV tensors must be contiguous")
    if block_n not in (2, 4, 8):
        raise ValueError("SwiGLU GEMV block_n must be 2, 4 or 8")
    if not x.is_cuda:
        raise ValueError("fused kernels require a GPU tensor")
    n = packed_weight.shape[0] // 2
    k = x.shape[-1]
    out = torch.empty((1, 1, n), device=x.device, dtype=x.dtype)
    _lib.call("q35_swiglu_gemv", packed_weight.data_ptr(), x.data_ptr(), None, None, 0, 0.0, None,
              None, out.data_ptr(), n, k, 0, _stream(x))
    return out


@_device_checked
def lm_head_argmax(
    hidden: torch.Tensor,
    weight: torch.Tensor,
    *,
    block_n: int = 16,
    block_k: int = 128,
    out: torch.Tensor | None = None,
    mirror: torch.Tensor | None = None,
    advance: torch.Tensor | None = None,
    screen: tuple[torch.Tensor, torch.Tensor, torch.Tensor] | None = None,
    return_candidates: bool = False,
):
    """Greedy token id without materialising logits. reference kernels.py:1146.

    ``out`` (int64, one element) receives the token instead of a new tensor;
    ``mirror`` (int64, one element: a GPU tensor or pinned host memory) also
    receives it from the same launch, so a host loop can read the token of a
    captured step without a copy after it; ``advance`` (an int64 tensor, e.g.
    the decode position ids) is incremented
    by one in the same launch — the token feedback and ``position_ids += 1`` of
    reference graph.py:78-79 without extra kernels. ``screen`` (the tensors
    ``lm_head_screen_prep`` made from this ``weight``) finds the same index
    through an int8 copy of the weight and an exact recomputation of the rows
    the screen cannot exclude (about half the bytes read); with
    ``return_candidates`` it returns ``(token, rows recomputed)``, the second
    an int64 device scalar (the bf16 rows read beyond the int8 screen).
    """

    if hidden.shape != (1, weight.shape[1]) or hidden.dtype != torch.bfloat16:
        raise ValueError("lm_head_argmax supports BF16 batch=1 hidden vectors")
    if not hidden.is_contiguous() or not weight.is_contiguous():
        raise ValueError("LM head tensors must be contiguous")
    if not hidden.is_cuda:
        raise ValueError("fused kernels require a GPU tensor")
    _need_bf16(weight)
    vocab, k = weight.shape
    if screen is not None:
        wq, sw, cr = screen
        if (wq.shape != weight.shape or wq.dtype != torch.int8 or sw.shape != (vocab,)
                or cr.shape != (vocab,) or sw.dtype != torch.float32 or cr.dtype != torch.float32
                or not (wq.is_contiguous() and sw.is_contiguous() and cr.is_contiguous())):
            raise ValueError("screen must be lm_head_screen_prep(weight)")
        if k != 2048:
            raise ValueError("the screened lm_head top-1 is built for K = 2048")
        nbytes = _lib.load().q35_lm_head_top1_screened_workspace(vocab, k)
        workspace = torch.empty(nbytes, device=hidden.device, dtype=torch.uint8)
    else:
        slots = _lib.load().q35_lm_head_top1_workspace(vocab, k)
        workspace = torch.empty(slots, device=hidden.device, dtype=torch.int64)
    if out is None:
        output = torch.empty((1, 1), device=hidden.device, dtype=torch.int64)
    else:
        if out.numel() != 1 or out.dtype != torch.int64 or not out.is_contiguous():
            raise ValueError("out must be a contiguous one-element int64 tensor")
        output = out
    n_adv = 0
    if advance is not None:
        if advance.dtype != torch.int64 or not advance.is_contiguous() or advance.numel() > 64:
            raise ValueError("advance must be a contiguous int64 tensor of at most 64 elements")
        n_adv = advance.numel()
    mirror_at = None
    if mirror is not None:
        if mirror.numel() != 1 or mirror.dtype != torch.int64 or not mirror.is_contiguous():
            raise ValueError("mirror must be a contiguous one-element int64 tensor")
        if mirror.is_cuda:
            if mirror.device != hidden.device:
                raise ValueError("mirror must be on the hidden vector's GPU or in pinned host memory")
            mirror_at = mirror.data_ptr()
        else:
            mirror_at = host_device_address(mirror)
    if return_candidates and screen is None:
        raise ValueError("return_candidates needs the screened top-1")
    if screen is not None:
        _lib.call("q35_lm_head_top1_screened", weight.data_ptr(), wq.data_ptr(), sw.data_ptr(),
                  cr.data_ptr(), hidden.data_ptr(), vocab, k, workspace.data_ptr(), nbytes,
                  output.data_ptr(), mirror_at, _lib.ptr(advance), n_adv, _stream(hidden))
        if return_candidates:
            import ctypes

            n = ctypes.c_int(0)
            off = _lib.load().q35_lm_head_screened_counts(vocab, ctypes.byref(n))
            counts = workspace[off: off + 4 * n.value].view(torch.int32)
            return output, counts.to(torch.int64).sum()
    else:
        _lib.call("q35_lm_head_top1", weight.data_ptr(), hidden.data_ptr(), vocab, k,
                  workspace.data_ptr(), slots, output.data_ptr(), mirror_at, _lib.ptr(advance),
                  n_adv, _stream(hidden))
    return output


def host_device_address(t: torch.Tensor) -> int:
    """The address a kernel stores to in order to reach the pinned host
    tensor ``t`` (memory from ``pin_memory``); raises ValueError for pageable
    host memory or anything else the device cannot address."""

    import ctypes

    if t.is_cuda:
        raise ValueError("host_device_address takes a host tensor")
    dev = ctypes.c_void_p(0)
    if t.numel() == 0 or _lib.load().q35_host_device_ptr(ctypes.c_void_p(t.data_ptr()), ctypes.byref(dev)) != 0:
        raise ValueError("the tensor is not in pinned, device-mapped host memory")
    return int(dev.value)


@_device_checked
def lm_head_screen_prep(weight: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """The operands of the screened lm_head top-1 for ``weight`` [V, 2048]
    bf16: an int8 copy (per-row absmax / 127 scale) and per-row fp32 scale
    and error-bound factor. Made once per weight; 0.5 bytes per weight
    element plus 8 bytes per row."""

    if weight.ndim != 2 or weight.shape[1] != 2048 or not weight.is_contiguous():
        raise ValueError("screen operands are built for a contiguous [V, 2048] weight")
    _need_bf16(weight)
    vocab, k = weight.shape
    wq = torch.empty((vocab, k), device=weight.device, dtype=torch.int8)
    sw = torch.empty(vocab, device=weight.device, dtype=torch.float32)
    cr = torch.empty(vocab, device=weight.device, dtype=torch.float32)
    _lib.call("q35_lm_head_screen_prep", weight.data_ptr(), vocab, k, wq.data_ptr(),
              sw.data_ptr(), cr.data_ptr(), _stream(weight))
    return wq, sw, cr


# ------------------------------------------------------------------ DeltaNet
@_device_checked
def causal_conv1d_fused(x: torch.Tensor, weight: torch.Tensor, state: torch.Tensor) -> torch.Tensor:
    """Causal depthwise conv + SiLU, ``state`` updated in place. reference kernels.py:659."""

    if x.ndim != 3 or weight.ndim != 2 or state.ndim != 3:
        raise ValueError("expected x[B,L,C], weight[C,K], state[B,C,K]")
    if not x.is_contiguous() or not weight.is_contiguous() or not state.is_contiguous():
        raise ValueError("causal conv tensors must be contiguous")
    batch, seq_len, input_stride = x.shape
    channels, kernel_size = weight.shape
    if input_stride < channels or state.shape != (batch, channels, kernel_size):
        raise ValueError("causal conv shapes do not match")
    if not x.is_cuda:
        raise ValueError("fused kernels require a GPU tensor")
    _need_bf16(x, weight, state)
    out = torch.empty((batch, seq_len, channels), device=x.device, dtype=x.dtype)
    if seq_len == 1:
        _lib.call("q35_conv1d_update", x.data_ptr(), weight.data_ptr(), state.data_ptr(),
                  out.data_ptr(), batch, channels, input_stride, kernel_size, _stream(x))
    else:
        _lib.call("q35_conv1d_prefill", x.data_ptr(), weight.data_ptr(), state.data_ptr(),
                  out.data_ptr(), batch, seq_len, channels, input_stride, kernel_size, _stream(x))
    return out


def _delta_params(a_log: torch.Tensor, dt_bias: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor, int]:
    if a_log.dtype == dt_bias.dtype and a_log.dtype in (torch.float32, _BF16):
        return a_log.contiguous(), dt_bias.contiguous(), int(a_log.dtype == torch.float32)
    return a_log.float().contiguous(), dt_bias.float().contiguous(), 1


@_device_checked
def delta_recurrent_fused(
    qkv: torch.Tensor,
    packed_projection: torch.Tensor,
    a_log: torch.Tensor,
    dt_bias: torch.Tensor,
    state: torch.Tensor,
    *,
    block_v: int = 8,
    precompute_factors: bool = False,
) -> torch.Tensor:
    """Sequential gated-delta recurrence; ``state`` updated in place. reference kernels.py:854.

    ``qkv`` is ``[B,L,3*H*D]`` (after conv) and ``packed_projection`` holds
    ``[qkv,z,a,b]`` in its last dimension. L == 1 runs the one-step decode
    kernel; L > 1 the per-token factor pass and the sequential scan.
    """

    if qkv.ndim != 3 or packed_projection.ndim != 3 or state.ndim != 4:
        raise ValueError("invalid delta recurrent tensor rank")
    if not qkv.is_contiguous() or not packed_projection.is_contiguous() or not state.is_contiguous():
        raise ValueError("delta recurrent tensors must be contiguous")
    batch, seq_len, qkv_width = qkv.shape
    _, heads, dim, value_dim = state.shape
    if dim != value_dim or qkv_width != 3 * heads * dim:
        raise ValueError("delta recurrent dimensions do not match")
    packed_width = packed_projection.shape[-1]
    b_offset = qkv_width + heads * dim + heads
    if packed_width < b_offset + heads:
        raise ValueError(f"packed projection width {packed_width} is smaller than {b_offset + heads}")
    if not qkv.is_cuda:
        raise ValueError("fused kernels require a GPU tensor")
    if dim != 128:
        raise ValueError("MI355X delta kernels are built for head dim 128")
    if state.dtype != torch.float32:
        raise ValueError("delta recurrent state must be float32")
    _need_bf16(qkv, packed_projection)
    al, dt, pf = _delta_params(a_log, dt_bias)
    out = torch.empty((batch, seq_len, heads, dim), device=qkv.device, dtype=qkv.dtype)
    s = _stream(qkv)
    if seq_len == 1:
        _lib.call("q35_delta_decode", qkv.data_ptr(), qkv_width, packed_projection.data_ptr(),
                  packed_width, None, None, 0, al.data_ptr(), dt.data_ptr(), pf, state.data_ptr(),
                  None, 0, 0.0, out.data_ptr(), batch, heads, dim, 0, 0, s)
    else:
        floats = _lib.load().q35_delta_prefill_workspace(batch, seq_len, heads)
        workspace = torch.empty(floats, device=qkv.device, dtype=torch.float32)
        _lib.call("q35_delta_prefill", qkv.data_ptr(), qkv_width, packed_projection.data_ptr(),
                  packed_width, al.data_ptr(), dt.data_ptr(), pf, state.data_ptr(), out.data_ptr(),
                  workspace.data_ptr(), floats, batch, seq_len, heads, dim, s)
    return out


@_device_checked
def delta_prefill_gated(
    qkv: torch.Tensor,
    packed_projection: torch.Tensor,
    a_log: torch.Tensor,
    dt_bias: torch.Tensor,
    state: torch.Tensor,
    norm_weight: torch.Tensor,
    eps: float = 1e-6,
) -> torch.Tensor:
    """Prefill recurrence (``delta_recurrent_fused``, L > 1) followed by the
    gated RMSNorm of every (token, head) row with the gate z read in place
    from ``packed_projection`` (reference integration.py:255-271 with
    kernels.py:115-155); for 64 or more tokens the norm runs inside the
    chunked output kernel. Returns ``[B, L, H, D]`` bf16; ``state`` updated in
    place."""

    if qkv.ndim != 3 or packed_projection.ndim != 3 or state.ndim != 4:
        raise ValueError("invalid delta recurrent tensor rank")
    if not qkv.is_contiguous() or not packed_projection.is_contiguous() or not state.is_contiguous():
        raise ValueError("delta recurrent tensors must be contiguous")
    batch, seq_len, qkv_width = qkv.shape
    _, heads, dim, value_dim = state.shape
    if dim != value_dim or qkv_width != 3 * heads * dim or dim != 128 or seq_len < 2:
        raise ValueError("delta prefill dimensions do not match (head dim 128, L > 1)")
    packed_width = packed_projection.shape[-1]
    if packed_width < qkv_width + heads * dim + 2 * heads or packed_width % 8:
        raise ValueError("packed projection does not hold [qkv | z | a | b]")
    if norm_weight.numel() != dim:
        raise ValueError(f"norm weight has {norm_weight.numel()} values, expected {dim}")
    if not qkv.is_cuda:
        raise ValueError("fused kernels require a GPU tensor")
    if state.dtype != torch.float32:
        raise ValueError("delta recurrent state must be float32")
    _need_bf16(qkv, packed_projection)
    al, dt, pf = _delta_params(a_log, dt_bias)
    w, wf = _param(norm_weight)
    out = torch.empty((batch, seq_len, heads, dim), device=qkv.device, dtype=qkv.dtype)
    y = torch.empty_like(out)
    floats = _lib.load().q35_delta_prefill_workspace(batch, seq_len, heads)
    workspace = torch.empty(floats, device=qkv.device, dtype=torch.float32)
    _lib.call("q35_delta_prefill_gated", qkv.data_ptr(), qkv_width, packed_projection.data_ptr(),
              packed_width, al.data_ptr(), dt.data_ptr(), pf, state.data_ptr(), out.data_ptr(),
              workspace.data_ptr(), floats, batch, seq_len, heads, dim, w.data_ptr(), wf, float(eps),
              y.data_ptr(), _stream(qkv))
    return y


@_device_checked
def delta_prefill_gated_conv(
    packed_projection: torch.Tensor,
    conv_weight: torch.Tensor,
    conv_state: torch.Tensor,
    a_log: torch.Tensor,
    dt_bias: torch.Tensor,
    state: torch.Tensor,
    norm_weight: torch.Tensor,
    eps: float = 1e-6,
) -> torch.Tensor:
    """``causal_conv1d_fused`` (width 4, prefill) + ``delta_prefill_gated`` in
    one chain whose chunk prep applies the conv itself: the raw packed
    projection in, ``conv_state`` left as the prefill conv leaves it
    (reference integration.py:244-271). 64 or more tokens (the chunked path).
    Returns ``[B, L, H, D]`` bf16; ``state`` and ``conv_state`` updated in
    place."""

    if packed_projection.ndim != 3 or state.ndim != 4 or conv_weight.ndim != 2 or conv_state.ndim != 3:
        raise ValueError("invalid delta recurrent tensor rank")
    if not (packed_projection.is_contiguous() and state.is_contiguous() and conv_weight.is_contiguous()
            and conv_state.is_contiguous()):
        raise ValueError("delta recurrent tensors must be contiguous")
    batch, seq_len, packed_width = packed_projection.shape
    _, heads, dim, value_dim = state.shape
    channels = 3 * heads * dim
    if dim != value_dim or dim != 128 or seq_len < 64:
        raise ValueError("fused conv prefill needs head dim 128 and at least 64 tokens")
    if conv_weight.shape != (channels, 4) or conv_state.shape != (batch, channels, 4):
        raise ValueError("causal conv shapes do not match")
    if packed_width < channels + heads * dim + 2 * heads or packed_width % 8:
        raise ValueError("packed projection does not hold [qkv | z | a | b]")
    if norm_weight.numel() != dim:
        raise ValueError(f"norm weight has {norm_weight.numel()} values, expected {dim}")
    if state.dtype != torch.float32:
        raise ValueError("delta recurrent state must be float32")
    _need_bf16(packed_projection, conv_weight, conv_state)
    al, dt, pf = _delta_params(a_log, dt_bias)
    w, wf = _param(norm_weight)
    out = torch.empty((batch, seq_len, heads, dim), device=state.device, dtype=torch.bfloat16)
    y = torch.empty_like(out)
    floats = _lib.load().q35_delta_prefill_workspace(batch, seq_len, heads)
    workspace = torch.empty(floats, device=state.device, dtype=torch.float32)
    _lib.call("q35_delta_prefill_gated_conv", packed_projection.data_ptr(), packed_width,
              conv_weight.data_ptr(), conv_state.data_ptr(), al.data_ptr(), dt.data_ptr(), pf,
              state.data_ptr(), out.data_ptr(), workspace.data_ptr(), floats, batch, seq_len, heads,
              dim, w.data_ptr(), wf, float(eps), y.data_ptr(), _stream(state))
    return y


@_device_checked
def delta_decode_fused(
    packed_projection: torch.Tensor,
    conv_weight: torch.Tensor,
    conv_state: torch.Tensor,
    a_log: torch.Tensor,
    dt_bias: torch.Tensor,
    state: torch.Tensor,
    norm_weight: torch.Tensor,
    norm_eps: float,
) -> torch.Tensor:
    """One decode token of a DeltaNet layer in one launch: conv1d update, delta
    rule and gated RMSNorm (reference kernels.py:659, :854 and :139 as chained
    by integration.py:254-271). Returns the gated core ``[B*H, D]`` bf16."""

    if packed_projection.ndim != 3 or state.ndim != 4 or conv_weight.ndim != 2 or conv_state.ndim != 3:
        raise ValueError("expected packed[B,1,W], conv_weight[C,K], conv_state[B,C,K], state[B,H,D,D]")
    for name, t in (("packed_projection", packed_projection), ("conv_weight", conv_weight),
                    ("conv_state", conv_state), ("state", state)):
        if not t.is_contiguous():
            raise ValueError(f"{name} must be contiguous")
    batch, seq_len, packed_width = packed_projection.shape
    _, heads, dim, value_dim = state.shape
    if seq_len != 1:
        raise ValueError("fused DeltaNet decode takes one token")
    if state.shape[0] != batch or dim != value_dim or dim != 128 or state.dtype != torch.float32:
        raise ValueError("delta state must be float32 [B, H, 128, 128]")
    channels, kernel_size = conv_weight.shape
    if channels != 3 * heads * dim or conv_state.shape != (batch, channels, kernel_size):
        raise ValueError("conv weight/state do not match the 3*H*D convolved channels")
    if packed_width < channels + heads * dim + 2 * heads:
        raise ValueError("packed projection does not hold [qkv | z | a | b]")
    if norm_weight.numel() != dim or a_log.numel() != heads or dt_bias.numel() != heads:
        raise ValueError("norm weight, A_log and dt_bias do not match the heads")
    _need_bf16(packed_projection, conv_weight, conv_state)
    al, dt, pf = _delta_params(a_log, dt_bias)
    nw, nwf = _param(norm_weight)
    out = torch.empty((batch * heads, dim), device=packed_projection.device, dtype=_BF16)
    _lib.call("q35_delta_decode", packed_projection.data_ptr(), packed_width,
              packed_projection.data_ptr(), packed_width, conv_weight.data_ptr(),
              conv_state.data_ptr(), conv_weight.shape[1], al.data_ptr(), dt.data_ptr(), pf,
              state.data_ptr(), nw.data_ptr(), nwf, float(norm_eps), out.data_ptr(), batch, heads,
              dim, 1, 1, _stream(packed_projection))
    return out


# ------------------------------------------------------------------ attention
@_device_checked
def qgkv_norm_rope(
    packed_qgkv: torch.Tensor,
    q_weight: torch.Tensor,
    k_weight: torch.Tensor,
    cos: torch.Tensor,
    sin: torch.Tensor,
    *,
    q_heads: int,
    kv_heads: int,
    dim: int,
    rotary_dim: int,
    cache_key: torch.Tensor | None = None,
    cache_value: torch.Tensor | None = None,
    cache_start: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Packed Q+gate/K/V layout with Q/K RMSNorm and partial RoPE. reference kernels.py:507."""

    if not packed_qgkv.is_contiguous():
        raise ValueError("packed QGKV must be contiguous")
    batch, seq_len, packed_width = packed_qgkv.shape
    expected = 2 * q_heads * dim + 2 * kv_heads * dim
    if packed_width != expected:
        raise ValueError(f"packed QGKV width {packed_width}, expected {expected}")
    cos = cos.contiguous()
    sin = sin.contiguous()
    if cos.shape != (batch, seq_len, rotary_dim) or sin.shape != cos.shape:
        raise ValueError(f"RoPE shape {tuple(cos.shape)}, expected {(batch, seq_len, rotary_dim)}")
    if not packed_qgkv.is_cuda:
        raise ValueError("fused kernels require a GPU tensor")
    _need_bf16(packed_qgkv)
    if cos.dtype != _BF16:
        cos = cos.to(_BF16)
    if sin.dtype != _BF16:
        sin = sin.to(_BF16)
    qw, wf = _param(q_weight)
    kw_, kwf = _param(k_weight)
    if wf != kwf:
        qw, kw_, wf = qw.float(), kw_.float(), 1
    dev = packed_qgkv.device
    q = torch.empty((batch, q_heads, seq_len, dim), device=dev, dtype=packed_qgkv.dtype)
    write_cache = cache_key is not None
    if write_cache:
        if cache_value is None or cache_start is None:
            raise ValueError("cache key, value and start must be provided together")
        if cache_key.shape[:2] != (batch, kv_heads) or cache_key.shape[-1] != dim:
            raise ValueError("static K cache shape does not match QGKV")
        if cache_value.shape != cache_key.shape:
            raise ValueError("static K/V cache shapes must match")
        if not cache_key.is_contiguous() or not cache_value.is_contiguous():
            raise ValueError("static K/V cache must be contiguous")
        if cache_start.dtype != torch.int64 or cache_start.device != dev:
            raise ValueError("cache_start must be an int64 scalar on the GPU")
        k, v = cache_key, cache_value
        cache_len = cache_key.shape[-2]
        start_ptr = cache_start.data_ptr()
    else:
        k = torch.empty((batch, kv_heads, seq_len, dim), device=dev, dtype=packed_qgkv.dtype)
        v = torch.empty_like(k)
        cache_len = seq_len
        start_ptr = None
    _lib.call("q35_qgkv_norm_rope", packed_qgkv.data_ptr(), qw.data_ptr(), kw_.data_ptr(), wf,
              cos.data_ptr(), sin.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(), start_ptr,
              batch, seq_len, q_heads, kv_heads, dim, rotary_dim, max(cache_len, 1), _stream(q))
    return q, k, v


def _check_decode_attention(q, cache_keys, cache_values):
    if q.ndim != 4 or q.shape[0] != 1 or q.shape[2] != 1:
        raise ValueError("GQA decode attention expects q[1,H,1,D]")
    if cache_keys.ndim != 4 or cache_keys.shape[0] != 1:
        raise ValueError("static K cache must be [1,KVH,L,D]")
    if cache_values.shape != cache_keys.shape:
        raise ValueError("static K/V cache shapes must match")
    if not q.is_contiguous() or not cache_keys.is_contiguous() or not cache_values.is_contiguous():
        raise ValueError("GQA decode attention tensors must be contiguous")
    heads, head_dim = q.shape[1], q.shape[3]
    kv_heads = cache_keys.shape[1]
    if head_dim != cache_keys.shape[3] or heads % kv_heads:
        raise ValueError("GQA decode attention head layout does not match cache")
    if not q.is_cuda:
        raise ValueError("fused kernels require a GPU tensor")
    if head_dim != 256:
        raise ValueError("MI355X decode attention kernels are built for head_dim 256")
    _need_bf16(q, cache_keys, cache_values)


@_device_checked
def gqa_decode_attention(
    q: torch.Tensor,
    cache_keys: torch.Tensor,
    cache_values: torch.Tensor,
    valid_length: torch.Tensor,
    scale: float,
    *,
    splits: int = 4,
    block_n: int = 64,
    packed_gate: torch.Tensor | None = None,
) -> torch.Tensor:
    """One decode attention step over a static cache. reference kernels.py:1031.

    ``valid_length`` is a device int64 scalar that already includes the
    current token. With ``packed_gate`` (the packed QGKV row) the output gate
    of reference kernels.py:312 is fused into the combine. Returns
    ``[1, 1, H*D]`` bf16.
    """

    _check_decode_attention(q, cache_keys, cache_values)
    heads, head_dim = q.shape[1], q.shape[3]
    kv_heads, cache_len = cache_keys.shape[1], cache_keys.shape[2]
    if valid_length.dtype != torch.int64 or valid_length.device != q.device:
        raise ValueError("valid_length must be an int64 tensor on the GPU")
    floats = _lib.load().q35_gqa_decode_workspace(cache_len, heads, kv_heads, head_dim)
    workspace = torch.empty(floats, device=q.device, dtype=torch.float32)
    out = torch.empty((1, 1, heads * head_dim), device=q.device, dtype=q.dtype)
    gate_ptr = None
    if packed_gate is not None:
        if packed_gate.shape[-1] < 2 * heads * head_dim or not packed_gate.is_contiguous():
            raise ValueError("packed gate does not match the attention heads")
        gate_ptr = packed_gate.data_ptr()
    _lib.call("q35_gqa_decode", q.data_ptr(), cache_keys.data_ptr(), cache_values.data_ptr(),
              valid_length.data_ptr(), float(scale), gate_ptr, out.data_ptr(), workspace.data_ptr(),
              floats, heads, kv_heads, head_dim, cache_len, _stream(q))
    return out


@_device_checked
def gqa_decode_fused(
    packed_qgkv: torch.Tensor,
    q_weight: torch.Tensor,
    k_weight: torch.Tensor,
    inv_freq: torch.Tensor,
    positions: torch.Tensor,
    cache_keys: torch.Tensor,
    cache_values: torch.Tensor,
    cache_length: torch.Tensor,
    scale: float,
    *,
    q_heads: int,
    mrope_section: tuple[int, int, int] = (11, 11, 10),
) -> torch.Tensor:
    """A full-attention layer's decode token after its packed projection, in
    two launches: Q/K norm + RoPE (cos/sin from ``positions`` and
    ``inv_freq``), the K/V cache write at ``cache_length``, split-K attention,
    combine and sigmoid gate, then ``cache_length += 1`` — the chain
    qgkv_norm_rope -> cumulative_length.add_ -> gqa_decode_attention ->
    attention_gate_mul of reference integration.py:298-358.

    ``positions``: int64 device tensor, either one text position or the
    ``[3, ...]`` multimodal rows (temporal, height, width) of this token.
    Returns ``[1, 1, QH*D]`` bf16.
    """

    kv_heads, cache_len, dim = cache_keys.shape[1], cache_keys.shape[2], cache_keys.shape[3]
    if cache_keys.shape[0] != 1 or cache_values.shape != cache_keys.shape:
        raise ValueError("static K/V cache must be [1,KVH,L,D]")
    if packed_qgkv.numel() != 2 * q_heads * dim + 2 * kv_heads * dim or not packed_qgkv.is_contiguous():
        raise ValueError("packed QGKV does not match the cache heads")
    if dim != 256:
        raise ValueError("MI355X decode attention kernels are built for head_dim 256")
    if inv_freq.dtype != torch.float32 or positions.dtype != torch.int64:
        raise ValueError("inv_freq must be float32 and positions int64")
    if cache_length.dtype != torch.int64 or cache_length.numel() != 1:
        raise ValueError("cache_length must be an int64 scalar")
    _need_bf16(packed_qgkv, cache_keys, cache_values)
    qw, wf = _param(q_weight)
    kw_, kwf = _param(k_weight)
    if wf != kwf:
        qw, kw_, wf = qw.float(), kw_.float(), 1
    # element addresses only (no copy: the rows may be stride-0 expanded views)
    if positions.dim() >= 2 and positions.shape[0] == 3:
        p_t, p_h, p_w = (positions[i].data_ptr() for i in range(3))
    else:
        p_t = p_h = p_w = positions.data_ptr()
    floats = _lib.load().q35_gqa_decode_workspace(cache_len, q_heads, kv_heads, dim)
    workspace = torch.empty(floats, device=packed_qgkv.device, dtype=torch.float32)
    out = torch.empty((1, 1, q_heads * dim), device=packed_qgkv.device, dtype=_BF16)
    _lib.call("q35_gqa_decode_fused", packed_qgkv.data_ptr(), qw.data_ptr(), kw_.data_ptr(), wf,
              inv_freq.data_ptr(), p_t, p_h, p_w, int(mrope_section[1]), int(mrope_section[2]),
              2 * inv_freq.numel(), cache_keys.data_ptr(), cache_values.data_ptr(),
              cache_length.data_ptr(), float(scale), out.data_ptr(), workspace.data_ptr(), floats,
              q_heads, kv_heads, dim, cache_len, _stream(packed_qgkv))
    return out


@_device_checked
def gqa_prefill_attention(
    q: torch.Tensor,
    keys: torch.Tensor,
    values: torch.Tensor,
    scale: float,
    *,
    kv_start: int = 0,
    valid_length: torch.Tensor | None = None,
    length_is_start: bool = False,
) -> torch.Tensor:
    """Causal GQA prefill attention: ``q [B,QH,L,D]`` row i attends to
    ``keys/values [B,KVH,C,D]`` positions ``[0, start + i]``, with
    ``start = valid_length - L`` when the device scalar ``valid_length``
    (already including the L tokens, as a static cache's length) is given,
    ``start = valid_length`` with ``length_is_start`` (the length before the
    L tokens, when its advance comes later), else ``kv_start``. Returns
    ``[B, L, QH*D]`` bf16. Replaces the prefill attention interface call of
    reference integration.py:360-372."""

    if q.ndim != 4 or keys.ndim != 4 or keys.shape != values.shape:
        raise ValueError("prefill attention expects q[B,QH,L,D] and K/V[B,KVH,C,D]")
    batch, heads, seq_len, dim = q.shape
    kv_heads, cache_len = keys.shape[1], keys.shape[2]
    if keys.shape[0] != batch or keys.shape[3] != dim or heads % kv_heads:
        raise ValueError("prefill attention head layout does not match")
    if valid_length is None and (kv_start < 0 or kv_start + seq_len > cache_len):
        raise ValueError("prefill attention range exceeds the key/value length")
    if seq_len > cache_len:
        raise ValueError("prefill attention range exceeds the key/value length")
    if not (q.is_contiguous() and keys.is_contiguous() and values.is_contiguous()):
        raise ValueError("prefill attention tensors must be contiguous")
    if not q.is_cuda:
        raise ValueError("fused kernels require a GPU tensor")
    if dim != 256:
        raise ValueError("MI355X prefill attention kernels are built for head_dim 256")
    if valid_length is not None and (valid_length.dtype != torch.int64 or valid_length.device != q.device):
        raise ValueError("valid_length must be an int64 tensor on the GPU")
    if valid_length is not None and kv_start:
        raise ValueError("kv_start and valid_length are exclusive")
    if length_is_start and valid_length is None:
        raise ValueError("length_is_start needs valid_length")
    _need_bf16(q, keys, values)
    out = torch.empty((batch, seq_len, heads * dim), device=q.device, dtype=q.dtype)
    floats = _lib.load().q35_gqa_prefill_workspace(batch, heads, kv_heads, seq_len, cache_len)
    ws = torch.empty(max(floats, 1), device=q.device, dtype=torch.float32) if floats > 0 else None
    # with a device length, the entry's kv_start is added to it: start = *valid_len - L + kv_start
    offset = seq_len if length_is_start else 0
    _lib.call("q35_gqa_prefill", q.data_ptr(), keys.data_ptr(), values.data_ptr(), out.data_ptr(),
              batch, heads, kv_heads, dim, seq_len, cache_len,
              offset if valid_length is not None else kv_start, _lib.ptr(valid_length),
              float(scale), _lib.ptr(ws), floats, _stream(q))
    return out


# ------------------------------------------------------------------ A8W8
# Up to this many tokens the A8W8 linear runs on the dot4 GEMV kernel (weights
# read once per launch); above it, on an int8 GEMM.
_A8W8_GEMV_MAX_M = 16


@_device_checked
def quantize_weight_i8(weight: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-output-channel symmetric int8 weights and fp32 ``[N,1]`` scales.
    reference explore_runtime_quantization.py:142-155."""

    if weight.ndim != 2 or not weight.is_cuda or not weight.is_contiguous():
        raise ValueError("weight quantisation expects a contiguous GPU [N,K] tensor")
    _need_bf16(weight)
    n, k = weight.shape
    wq = torch.empty((n, k), device=weight.device, dtype=torch.int8)
    scale = torch.empty((n, 1), device=weight.device, dtype=torch.float32)
    _lib.call("q35_quant_weight_i8", weight.data_ptr(), wq.data_ptr(), scale.data_ptr(), n, k,
              _stream(weight))
    return wq, scale


@_device_checked
def attention_gate_quant(x: torch.Tensor, packed_qgkv: torch.Tensor, head_dim: int, *,
                         advance: torch.Tensor | None = None,
                         amount: int = 0) -> tuple[torch.Tensor, torch.Tensor]:
    """``quantize_act_i8(attention_gate_mul(x, packed_qgkv, head_dim))`` in
    one launch (the same bits; the gated bf16 rows are never stored): the A8W8
    o_proj input of reference kernels.py:312 + explore_runtime_quantization.py:167-172.
    ``advance`` / ``amount`` as for ``attention_gate_mul``."""

    hidden = x.shape[-1]
    if not x.is_contiguous() or not packed_qgkv.is_contiguous():
        raise ValueError("attention gate tensors must be contiguous")
    if packed_qgkv.shape[:-1] != x.shape[:-1]:
        raise ValueError("attention output and packed projection rows do not match")
    if hidden % head_dim or hidden % 8 or head_dim % 8 or hidden > 8192 or packed_qgkv.shape[-1] < 2 * hidden \
            or packed_qgkv.shape[-1] % 8:
        raise ValueError("the fused gate + quantisation needs hidden, head_dim and the packed width "
                         "multiples of 8 (hidden <= 8192) and the gate inside the packed row")
    _need_bf16(x, packed_qgkv)
    if advance is not None and (advance.dtype != torch.int64 or advance.numel() != 1):
        raise ValueError("advance must be an int64 scalar tensor")
    tokens = x.numel() // hidden
    xq = torch.empty(x.shape, device=x.device, dtype=torch.int8)
    scale = torch.empty((tokens, 1), device=x.device, dtype=torch.float32)
    _lib.call("q35_attn_gate_quant", x.data_ptr(), packed_qgkv.data_ptr(), xq.data_ptr(),
              scale.data_ptr(), tokens, hidden, packed_qgkv.shape[-1], head_dim, _lib.ptr(advance),
              int(amount), _stream(x))
    return xq, scale


@_device_checked
def quantize_act_i8(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-token dynamic symmetric int8 activations and fp32 ``[M,1]`` scales
    (the scaled_int8_quant call of reference explore_runtime_quantization.py:167-172)."""

    rows, k = _rows_and_width(x)
    _need_bf16(x)
    xq = torch.empty(x.shape, device=x.device, dtype=torch.int8)
    scale = torch.empty((rows, 1), device=x.device, dtype=torch.float32)
    _lib.call("q35_quant_act_i8", x.data_ptr(), xq.data_ptr(), scale.data_ptr(), rows, k,
              _stream(x))
    return xq, scale


@_device_checked
def a8w8_linear(
    x: torch.Tensor,
    weight_q: torch.Tensor,
    weight_scale: torch.Tensor,
    *,
    return_quant: bool = False,
    return_acc: bool = False,
):
    """A8W8 linear: per-token int8 quantisation of ``x``, int32 dot products
    against per-channel int8 weights, bf16 dequantised output
    (reference explore_runtime_quantization.py:161-181). Up to 16 tokens run
    on the int8 GEMV (for one token with the quantisation fused into the
    launch); prefill on the int8 matrix-core GEMM with the dequant fused."""

    k = x.shape[-1]
    if weight_q.ndim != 2 or weight_q.shape[1] != k or weight_q.dtype != torch.int8:
        raise ValueError("A8W8 weight must be int8 [N,K] matching the input")
    if k % 16:
        raise ValueError("A8W8 linear needs K to be a multiple of 16")
    if not x.is_cuda or not weight_q.is_contiguous():
        raise ValueError("A8W8 tensors must be contiguous GPU tensors")
    _need_bf16(x)
    x2 = x.reshape(-1, k).contiguous()
    m, n = x2.shape[0], weight_q.shape[0]
    sw = weight_scale.reshape(-1).float().contiguous()
    if sw.numel() != n:
        raise ValueError("A8W8 weight scale must have one value per output channel")
    xq = torch.empty((m, k), device=x.device, dtype=torch.int8)
    sx = torch.empty((m, 1), device=x.device, dtype=torch.float32)
    y = torch.empty((m, n), device=x.device, dtype=_BF16)
    if m > _A8W8_GEMV_MAX_M and k % 128 == 0:
        # Prefill: per-token quantisation, then the int8 matrix-core GEMM with
        # the dequant in its epilogue (exact int32 accumulators; with
        # return_acc the accumulators themselves, then the dequant kernel).
        _lib.call("q35_quant_act_i8", x2.data_ptr(), xq.data_ptr(), sx.data_ptr(), m, k, _stream(x))
        if return_acc:
            acc = torch.empty((m, n), device=x.device, dtype=torch.int32)
            gemm_into(xq, weight_q, acc, GEMM_I32)
            _lib.call("q35_dequant_i32", acc.data_ptr(), sx.data_ptr(), sw.data_ptr(), y.data_ptr(),
                      m, n, _stream(x))
        else:
            acc = None
            gemm_into(xq, weight_q, y, GEMM_DEQUANT, s_x=sx, s_w=sw)
    else:
        acc = torch.empty((m, n), device=x.device, dtype=torch.int32) if return_acc else None
        _lib.call("q35_gemv_a8w8", x2.data_ptr(), xq.data_ptr(), sx.data_ptr(), weight_q.data_ptr(),
                  sw.data_ptr(), y.data_ptr(), _lib.ptr(acc), m, n, k, _stream(x))
    y = y.reshape(*x.shape[:-1], n)
    if not (return_quant or return_acc):
        return y
    extra = []
    if return_quant:
        extra += [xq, sx]
    if return_acc:
        extra.append(acc)
    return (y, *extra)


@_device_checked
def a8w8_swiglu(x: torch.Tensor, weight_q: torch.Tensor, weight_scale: torch.Tensor) -> torch.Tensor:
    """``silu_and_mul(a8w8_linear(x, Wq, s_w))`` for a packed ``[gate; up]``
    int8 weight (reference integration.py:183-185 with PPUA8W8Linear,
    explore_runtime_quantization.py:161-181): for prefill the int32
    accumulators go straight into a fused dequant + SwiGLU kernel, so the
    dequantised gate/up rows are never written; one token or a few use the
    A8W8 GEMV and ``silu_and_mul``. Same values as the two-step form."""

    k = x.shape[-1]
    n2 = weight_q.shape[0]
    if weight_q.ndim != 2 or weight_q.shape[1] != k or weight_q.dtype != torch.int8 or n2 % 2:
        raise ValueError("packed A8W8 SwiGLU weight must be int8 [2N, K] matching the input")
    x2 = x.reshape(-1, k)
    m, n = x2.shape[0], n2 // 2
    if m <= _A8W8_GEMV_MAX_M or k % 128:
        return silu_and_mul(a8w8_linear(x, weight_q, weight_scale))
    if not x.is_cuda or not weight_q.is_contiguous():
        raise ValueError("A8W8 tensors must be contiguous GPU tensors")
    _need_bf16(x)
    x2 = x2.contiguous()
    sw = weight_scale.reshape(-1).float().contiguous()
    if sw.numel() != n2:
        raise ValueError("A8W8 weight scale must have one value per output channel")
    xq = torch.empty((m, k), device=x.device, dtype=torch.int8)
    sx = torch.empty((m, 1), device=x.device, dtype=torch.float32)
    _lib.call("q35_quant_act_i8", x2.data_ptr(), xq.data_ptr(), sx.data_ptr(), m, k, _stream(x))
    y = torch.empty((*x.shape[:-1], n), device=x.device, dtype=_BF16)
    gemm_into(xq, weight_q, y.view(m, n), GEMM_DEQUANT_SWIGLU, s_x=sx, s_w=sw)
    return y


@_device_checked
def a8w8_int_gemm(xq: torch.Tensor, weight_q: torch.Tensor) -> torch.Tensor:
    """Exact int32 ``xq . Wq^T`` for prefill int8 activations ``[..., K]`` on
    the int8 matrix-core GEMM: ``[rows, N]`` int32 (the int8 GEMM of reference
    explore_runtime_quantization.py:173-180)."""

    x2, n = _gemm_operands(xq, weight_q, torch.int8, False)
    acc = torch.empty((x2.shape[0], n), device=xq.device, dtype=torch.int32)
    if x2.shape[0]:
        gemm_into(x2, weight_q, acc, GEMM_I32)
    return acc


@_device_checked
def dequant_linear_i32(acc: torch.Tensor, x_scale: torch.Tensor, weight_scale: torch.Tensor,
                       shape: tuple[int, ...] | None = None) -> torch.Tensor:
    """``bf16(float(acc) * s_x[m] * s_w[n])`` (the A8W8 dequant of reference
    explore_runtime_quantization.py:173-180), reshaped to ``shape``."""

    m, n = acc.shape
    if acc.dtype != torch.int32 or not acc.is_contiguous() or n % 8:
        raise ValueError("dequant expects contiguous int32 [M, N] accumulators, N % 8 == 0")
    sx = x_scale.reshape(-1).float().contiguous()
    sw = weight_scale.reshape(-1).float().contiguous()
    if sx.numel() != m or sw.numel() != n:
        raise ValueError("one activation scale per row and one weight scale per column")
    y = torch.empty((m, n), device=acc.device, dtype=_BF16)
    _lib.call("q35_dequant_i32", acc.data_ptr(), sx.data_ptr(), sw.data_ptr(), y.data_ptr(), m, n,
              _stream(acc))
    return y if shape is None else y.reshape(*shape)


@_device_checked
def residual_rmsnorm_dequant_quant(residual: torch.Tensor, acc: torch.Tensor, x_scale: torch.Tensor,
                                   weight_scale: torch.Tensor, norm_weight: torch.Tensor, eps: float,
                                   *, normalized: bool = False, quant: bool = True):
    """A8W8 prefill between two int8 GEMMs: ``residual + dequant(acc)`` (the
    previous GEMM's output), RMSNorm with ``(1 + w)``, and the normalised rows
    quantised per token for the next GEMM, in one launch with the separate
    kernels' arithmetic (reference explore_runtime_quantization.py:167-180,
    integration.py:456-499). Width 2048. Returns ``(residual_out,
    normalised bf16 or None, int8 rows or None, fp32 row scales or None)``."""

    rows, width = _rows_and_width(residual)
    if width != 2048 or not (normalized or quant):
        raise ValueError("width 2048, and at least one of normalized / quant")
    if acc.dtype != torch.int32 or acc.shape != (rows, width) or not acc.is_contiguous():
        raise ValueError("acc must be contiguous int32 [rows, 2048]")
    _need_bf16(residual)
    w, wf = _param(norm_weight)
    sx = x_scale.reshape(-1).float().contiguous()
    sw = weight_scale.reshape(-1).float().contiguous()
    if sx.numel() != rows or sw.numel() != width:
        raise ValueError("one activation scale per row and one weight scale per column")
    x = residual.contiguous()
    r_out = torch.empty_like(x)
    y = torch.empty_like(x) if normalized else None
    yq = torch.empty(x.shape, device=x.device, dtype=torch.int8) if quant else None
    sy = torch.empty((rows, 1), device=x.device, dtype=torch.float32) if quant else None
    _lib.call("q35_residual_rmsnorm_dequant_quant", x.data_ptr(), acc.data_ptr(), sx.data_ptr(),
              sw.data_ptr(), w.data_ptr(), wf, r_out.data_ptr(), _lib.ptr(y), _lib.ptr(yq),
              _lib.ptr(sy), rows, width, float(eps), _stream(x))
    return r_out, y, yq, sy


@_device_checked
def dequant_swiglu_quant(acc: torch.Tensor, x_scale: torch.Tensor,
                         weight_scale: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """A8W8 prefill MLP: the SwiGLU of the packed ``[gate; up]`` accumulators
    ``acc[M, 2N]`` (dequantised as in ``a8w8_swiglu``), quantised per token
    for the down projection: ``(int8 [M, N], fp32 [M, 1])``; the bf16
    activation is never written (reference integration.py:183-187)."""

    m, n2 = acc.shape
    n = n2 // 2
    if acc.dtype != torch.int32 or not acc.is_contiguous() or n2 % 16 or n > 6144:
        raise ValueError("acc must be contiguous int32 [M, 2N], N % 8 == 0, N <= 6144")
    sx = x_scale.reshape(-1).float().contiguous()
    sw = weight_scale.reshape(-1).float().contiguous()
    if sx.numel() != m or sw.numel() != n2:
        raise ValueError("one activation scale per row and one weight scale per column")
    yq = torch.empty((m, n), device=acc.device, dtype=torch.int8)
    sy = torch.empty((m, 1), device=acc.device, dtype=torch.float32)
    _lib.call("q35_dequant_swiglu_quant", acc.data_ptr(), sx.data_ptr(), sw.data_ptr(), yq.data_ptr(),
              sy.data_ptr(), m, n, _stream(acc))
    return yq, sy


@_device_checked
def gemm_a8w8(xq: torch.Tensor, x_scale: torch.Tensor, weight_q: torch.Tensor,
              weight_scale: torch.Tensor, *, swiglu: bool = False,
              plan: tuple[int, int] | None = None) -> torch.Tensor:
    """The int8 matrix-core prefill GEMM on already quantised operands:
    ``bf16(float(xq . Wq^T) * s_x[m] * s_w[n])`` (exact int32 accumulators,
    the dequant of reference explore_runtime_quantization.py:173-180), or with
    ``swiglu`` the SwiGLU of a packed ``[gate; up]`` int8 weight on the
    dequantised bf16 gate and up. K must be a multiple of 128. ``plan`` =
    (tile 0-8, K splits) overrides the library's choice."""

    if xq.ndim != 2:
        raise ValueError("int8 GEMM activations must be [M, K]")
    x2, n = _gemm_operands(xq, weight_q, torch.int8, swiglu)
    m = x2.shape[0]
    sx = x_scale.reshape(-1).float().contiguous()
    sw = weight_scale.reshape(-1).float().contiguous()
    if sx.numel() != m or sw.numel() != weight_q.shape[0]:
        raise ValueError("int8 GEMM scales: one per token row and one per weight row")
    y = torch.empty((m, n), device=xq.device, dtype=_BF16)
    if m:
        gemm_into(x2, weight_q, y, GEMM_DEQUANT_SWIGLU if swiglu else GEMM_DEQUANT, s_x=sx, s_w=sw,
                  plan=plan)
    return y


def zero_tensors(tensors) -> None:
    """Zero a list of GPU tensors with one kernel launch (16-byte aligned
    contiguous ones; any other is cleared with ``zero_()``)."""

    fused = []
    for t in tensors:
        if t.is_cuda and t.is_contiguous() and t.data_ptr() % 16 == 0:
            fused.append(t)
        else:
            t.zero_()
    if not fused:
        return
    import ctypes

    n = len(fused)
    ptrs = (ctypes.c_void_p * n)(*[t.data_ptr() for t in fused])
    sizes = (ctypes.c_longlong * n)(*[t.numel() * t.element_size() for t in fused])
    _lib.call("q35_zero_buffers", ctypes.cast(ptrs, ctypes.c_void_p), ctypes.cast(sizes, ctypes.c_void_p),
              n, _stream(fused[0]))


@_device_checked
def stream_read(buf: torch.Tensor, one_round: bool = False) -> torch.Tensor:
    """Read every byte of a contiguous GPU tensor once with the GEMV weight
    stream's loads (one workgroup per CU) and return one int32 XOR word per
    thread. A measurement utility (no counterpart in the reference): timing
    it gives the achievable HBM read rate the decode GEMVs are compared to.
    ``one_round``: as many workgroups as request every byte at once (at most
    8 loads per lane), the read floor of a small single-launch kernel."""

    import ctypes

    if not buf.is_cuda or not buf.is_contiguous():
        raise ValueError("stream_read needs a contiguous GPU tensor")
    nbytes = buf.numel() * buf.element_size()
    if nbytes == 0 or nbytes % 16 or buf.data_ptr() % 16:
        raise ValueError("stream_read needs a 16-byte aligned size and address")
    props = torch.cuda.get_device_properties(buf.device)
    words = props.multi_processor_count * 256
    if one_round:
        words = max(words, -(-nbytes // (16 * 8)) + 256)
    out = torch.empty(words, device=buf.device, dtype=torch.int32)
    blocks = ctypes.c_int(0)
    _lib.call("q35_stream_read_round" if one_round else "q35_stream_read", buf.data_ptr(), nbytes,
              out.data_ptr(), out.numel(), ctypes.addressof(blocks), _stream(buf))
    return out[: blocks.value * 256]


# ------------------------------------------------------------------ vision
def _param_pair(a: torch.Tensor, b: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor, int]:
    """Two parameter vectors in one dtype (bf16 if both are, else fp32)."""
    if a.dtype == _BF16 and b.dtype == _BF16:
        return a.contiguous(), b.contiguous(), 0
    return a.float().contiguous(), b.float().contiguous(), 1


@_device_checked
def layer_norm(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor,
               eps: float = 1e-6) -> torch.Tensor:
    """Vision LayerNorm ``(x - mean) * rsqrt(var + eps) * w + b`` over the last
    dimension, fp32 statistics, bf16 output. reference kernels.py:1209-1218."""

    rows, width = _rows_and_width(x)
    if weight.numel() != width or bias.numel() != width:
        raise ValueError(f"layer norm parameters must have {width} values")
    _need_bf16(x)
    w, b, pf = _param_pair(weight, bias)
    out = torch.empty_like(x)
    _lib.call("q35_layernorm", x.data_ptr(), w.data_ptr(), b.data_ptr(), pf, out.data_ptr(), rows,
              width, float(eps), _stream(x))
    return out


@_device_checked
def residual_add_layer_norm(
    residual: torch.Tensor,
    update: torch.Tensor,
    weight: torch.Tensor,
    bias: torch.Tensor,
    eps: float = 1e-6,
) -> tuple[torch.Tensor, torch.Tensor]:
    """``r' = bf16(residual + update)`` and ``layer_norm(r')``; returns
    ``(r', norm)``. reference kernels.py:1249-1280."""

    if residual.shape != update.shape:
        raise ValueError("vision residual tensors must have identical shape")
    rows, width = _rows_and_width(residual)
    if not update.is_contiguous():
        raise ValueError("fused kernels require contiguous input")
    if weight.numel() != width or bias.numel() != width:
        raise ValueError(f"layer norm parameters must have {width} values")
    _need_bf16(residual, update)
    w, b, pf = _param_pair(weight, bias)
    residual_out = torch.empty_like(residual)
    norm_out = torch.empty_like(residual)
    _lib.call("q35_residual_layernorm", residual.data_ptr(), update.data_ptr(), w.data_ptr(),
              b.data_ptr(), pf, residual_out.data_ptr(), norm_out.data_ptr(), rows, width,
              float(eps), _stream(residual))
    return residual_out, norm_out


@_device_checked
def position_embed_add(
    hidden: torch.Tensor,
    embedding_table: torch.Tensor,
    indices: torch.Tensor,
    interpolation_weight: torch.Tensor,
) -> torch.Tensor:
    """``hidden + bf16(sum_n table[indices[:, n]] * weight[:, n])``: the
    interpolated vision position embedding (fp32 sum over the neighbours).
    Indices outside the table are clamped to it. reference kernels.py:1309-1336."""

    if hidden.ndim != 2 or not hidden.is_contiguous():
        raise ValueError("vision hidden tensor must be contiguous [rows,width]")
    rows, width = hidden.shape
    neighbors = indices.shape[-1]
    if indices.shape != interpolation_weight.shape or indices.shape[0] != rows:
        raise ValueError("position interpolation tensors do not match hidden rows")
    if embedding_table.ndim != 2 or embedding_table.shape[1] != width:
        raise ValueError(f"position embedding table must be [positions,{width}]")
    _need_bf16(hidden, embedding_table)
    table = embedding_table.contiguous()
    idx = indices.to(torch.int64).contiguous()
    wt, wf = _param(interpolation_weight)
    out = torch.empty_like(hidden)
    _lib.call("q35_position_embed_add", hidden.data_ptr(), table.data_ptr(), table.shape[0],
              idx.data_ptr(), wt.data_ptr(), wf, out.data_ptr(), rows, width, neighbors,
              _stream(hidden))
    return out


@_device_checked
def vision_qkv_rope(
    packed_qkv: torch.Tensor,
    cos: torch.Tensor,
    sin: torch.Tensor,
    *,
    heads: int,
    dim: int,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Packed vision QKV ``[tokens, 3*heads*dim]`` -> q, k, v ``[1, heads,
    tokens, dim]`` with rotate-half RoPE (``cos``/``sin`` ``[tokens, dim]``) on
    q and k in fp32, bf16 out. reference kernels.py:378-416."""

    if packed_qkv.ndim != 2 or not packed_qkv.is_contiguous():
        raise ValueError("packed Vision QKV must be contiguous [tokens,3*hidden]")
    tokens, packed_width = packed_qkv.shape
    if packed_width != 3 * heads * dim:
        raise ValueError(f"packed Vision QKV width {packed_width}, expected {3 * heads * dim}")
    if cos.shape != (tokens, dim) or sin.shape != cos.shape:
        raise ValueError(f"Vision RoPE shape {tuple(cos.shape)}, expected {(tokens, dim)}")
    if dim % 2:
        raise ValueError("vision head dim must be even")
    _need_bf16(packed_qkv)
    c, s, cf = _param_pair(cos, sin)
    shape = (1, heads, tokens, dim)
    q = torch.empty(shape, device=packed_qkv.device, dtype=packed_qkv.dtype)
    k = torch.empty_like(q)
    v = torch.empty_like(q)
    _lib.call("q35_vision_qkv_rope", packed_qkv.data_ptr(), c.data_ptr(), s.data_ptr(), cf,
              q.data_ptr(), k.data_ptr(), v.data_ptr(), tokens, heads, dim, _stream(packed_qkv))
    return q, k, v


@_device_checked
def vision_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float,
                     cu_seqlens: torch.Tensor | None = None) -> torch.Tensor:
    """Non-causal attention of the vision blocks: q, k, v ``[1, heads, tokens,
    dim]`` (``vision_qkv_rope``'s outputs), each query attending to the keys
    of its own image (``cu_seqlens``: image offsets ``[n + 1]``; None: one
    image). Returns ``[tokens, heads*dim]`` bf16, the output projection's
    input. No counterpart in the reference's kernel API: it replaces the
    Transformers attention-interface call of reference integration.py:671-731."""

    if q.ndim != 4 or q.shape[0] != 1 or k.shape != q.shape or v.shape != q.shape:
        raise ValueError("vision attention expects q, k, v of shape [1, heads, tokens, dim]")
    if not (q.is_contiguous() and k.is_contiguous() and v.is_contiguous()):
        raise ValueError("fused kernels require contiguous input")
    _, heads, tokens, dim = q.shape
    if dim % 8 or dim > 128:
        raise ValueError("vision attention supports head dims that are multiples of 8 up to 128")
    _need_bf16(q, k, v)
    cu, n = None, 0
    if cu_seqlens is not None:
        cu = cu_seqlens.to(torch.int32).contiguous()
        n = cu.numel() - 1
        if n < 1:
            raise ValueError("cu_seqlens needs at least two offsets")
    out = torch.empty((tokens, heads * dim), device=q.device, dtype=q.dtype)
    _lib.call("q35_vision_attention", q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
              _lib.ptr(cu), n, tokens, heads, dim, float(scale), _stream(q))
    return out


@_device_checked
def sigmoid_mul(x: torch.Tensor, gate: torch.Tensor) -> torch.Tensor:
    """``x * bf16(sigmoid(gate))`` (reference kernels.py:266-282; unused by the
    reference integration). Expressed through the attention-gate kernel with a
    packed stride of 2*width and the gate in the second half."""

    if x.shape != gate.shape or not x.is_contiguous() or not gate.is_contiguous():
        raise ValueError("x and gate must be contiguous tensors with identical shape")
    width = x.shape[-1]
    packed = torch.cat((gate, gate), dim=-1).contiguous()
    return attention_gate_mul(x, packed, width)

