"""Integer A8W8 path in numpy (test infrastructure only).

Restates reference explore_runtime_quantization.py:129-181 (PPUA8W8Linear):
  weights (closed form, :142-155): s = absmax/127 (1 when absmax == 0, fp32);
      q = clamp(round_half_even(w / s), -127, 127)
  activations (vLLM scaled_int8_quant, symmetric, dynamic per token; called
      at :167-172; vLLM is not in this image and its version is unpinned):
      s = absmax/127; q = saturate_int8(rint(x * (127/absmax))); a zero row
      gives q = 0 and s = 0
  accumulate: exact integer dot products (int32 range)
  output: bf16(float32(acc) * s_x[m] * s_w[n])

Pinning (tests/test_oracle.py): pure-Python brute force on small inputs,
hand-computed known-answer vectors (ties at .5, saturation, zero rows), and
torch.round/clamp for the weight rule. The activation rule and the dequant
order are pinned to vLLM's published kernel as restated above, not to a run of
the reference call: parity unpinned against acext/vLLM binaries.
"""

from __future__ import annotations

import numpy as np
import torch

F32 = np.float32


def bf16_to_f32(x: torch.Tensor) -> np.ndarray:
    return x.detach().to(torch.float32).cpu().numpy()


def quantize_weight(weight: torch.Tensor) -> tuple[np.ndarray, np.ndarray]:
    """-> (int8 [N,K], fp32 [N,1])."""
    w = bf16_to_f32(weight)
    absmax = np.abs(w).max(axis=1, keepdims=True).astype(F32)
    scale = np.where(absmax > 0, absmax / F32(127.0), F32(1.0)).astype(F32)
    q = np.rint(w / scale)
    return np.clip(q, -127, 127).astype(np.int8), scale


def quantize_act(x: torch.Tensor) -> tuple[np.ndarray, np.ndarray]:
    """-> (int8 [M,K], fp32 [M,1])."""
    xs = bf16_to_f32(x).reshape(-1, x.shape[-1])
    absmax = np.abs(xs).max(axis=1, keepdims=True).astype(F32)
    with np.errstate(divide="ignore", invalid="ignore"):
        inv = (F32(127.0) / absmax).astype(F32)
        v = (xs * inv).astype(F32)
    v = np.where(np.isnan(v), F32(0.0), v)
    q = np.clip(np.rint(v), -128, 127).astype(np.int8)
    scale = (absmax / F32(127.0)).astype(F32)
    return q, scale


def int_gemm(xq: np.ndarray, wq: np.ndarray) -> np.ndarray:
    """Exact int32 accumulators acc[m, n] = sum_k xq[m,k] * wq[n,k]."""
    acc = xq.astype(np.int64) @ wq.astype(np.int64).T
    assert np.abs(acc).max(initial=0) < 2**31
    return acc.astype(np.int32)


def dequant(acc: np.ndarray, sx: np.ndarray, sw: np.ndarray) -> torch.Tensor:
    y = (acc.astype(F32) * sx.reshape(-1, 1).astype(F32)).astype(F32)
    y = (y * sw.reshape(1, -1).astype(F32)).astype(F32)
    return torch.from_numpy(y).to(torch.bfloat16)


def a8w8_linear(x: torch.Tensor, wq: np.ndarray, sw: np.ndarray):
    """-> (y bf16 [M,N], xq, sx, acc)."""
    xq, sx = quantize_act(x)
    acc = int_gemm(xq, wq)
    return dequant(acc, sx, sw), xq, sx, acc
