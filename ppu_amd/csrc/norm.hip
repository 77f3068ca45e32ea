// Row-wise decode kernels: RMSNorm, residual-add + RMSNorm, gated RMSNorm,
// SiLU-and-mul and the attention output gate.
//
// One wave64 owns one row. Rows whose width is a multiple of 8 are streamed
// with 128-bit loads (8 bf16 per lane per step); other widths take a scalar
// lane-strided path. Sums of squares are reduced with the DPP/swizzle wave
// reduction from q35_common.hpp. The norm kernels make two passes over a row:
// the second pass re-reads it from L1/L2 instead of holding it in registers,
// so any width works.
#include "q35_common.hpp"

namespace {

constexpr int kWaves = 4;  // waves (rows) per 256-thread workgroup

Q35_DEV float load_w(const void* w, int i, int w_f32) {
  return w_f32 ? reinterpret_cast<const float*>(w)[i]
               : bf2f(reinterpret_cast<const uint16_t*>(w)[i]);
}

// y = bf16(x * rsqrt(mean(x^2) + eps) * (1 + w))   [reference kernels.py:24-53]
// With residual: r' = bf16(r + u) is stored and normalised instead of x
// [reference kernels.py:56-112].
template <bool RESIDUAL>
__global__ __launch_bounds__(256) void rmsnorm_rows(const uint16_t* __restrict__ x,
                                                    const uint16_t* __restrict__ u,
                                                    const void* __restrict__ w, int w_f32,
                                                    uint16_t* __restrict__ r_out,
                                                    uint16_t* __restrict__ y, int rows,
                                                    int width, float eps, int vec) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * kWaves + (threadIdx.x >> 6);
  if (row >= rows) return;
  const size_t base = (size_t)row * width;
  float ss = 0.f;
  if (vec) {
    for (int k = lane * 8; k < width; k += 512) {
      float a[8];
      unpack8(*reinterpret_cast<const uint4*>(x + base + k), a);
      if (RESIDUAL) {
        float b[8];
        unpack8(*reinterpret_cast<const uint4*>(u + base + k), b);
#pragma unroll
        for (int j = 0; j < 8; ++j) a[j] = round_bf(a[j] + b[j]);
        *reinterpret_cast<uint4*>(r_out + base + k) = pack8(a);
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) ss += a[j] * a[j];
    }
  } else {
    for (int k = lane; k < width; k += 64) {
      float a = bf2f(x[base + k]);
      if (RESIDUAL) {
        a = round_bf(a + bf2f(u[base + k]));
        r_out[base + k] = (uint16_t)f2bf(a);
      }
      ss += a * a;
    }
  }
  const float inv = rsqrt_cr(wave_sum(ss) / (float)width + eps);
  if (vec) {
    for (int k = lane * 8; k < width; k += 512) {
      float a[8];
      unpack8(*reinterpret_cast<const uint4*>(x + base + k), a);
      if (RESIDUAL) {
        float b[8];
        unpack8(*reinterpret_cast<const uint4*>(u + base + k), b);
#pragma unroll
        for (int j = 0; j < 8; ++j) a[j] = round_bf(a[j] + b[j]);
      }
      float o[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) o[j] = a[j] * inv * (1.0f + load_w(w, k + j, w_f32));
      *reinterpret_cast<uint4*>(y + base + k) = pack8(o);
    }
  } else {
    for (int k = lane; k < width; k += 64) {
      float a = bf2f(x[base + k]);
      if (RESIDUAL) a = round_bf(a + bf2f(u[base + k]));
      y[base + k] = (uint16_t)f2bf(a * inv * (1.0f + load_w(w, k, w_f32)));
    }
  }
}

// y = bf16( bf16(bf16(x * rsqrt(mean(x^2)+eps)) * bf16(w)) * silu(gate) )
// [reference kernels.py:115-155]; the weight is used directly (no 1 + w).
__global__ __launch_bounds__(256) void gated_rmsnorm_rows(const uint16_t* __restrict__ x,
                                                          const uint16_t* __restrict__ gate,
                                                          const void* __restrict__ w, int w_f32,
                                                          uint16_t* __restrict__ y, int rows,
                                                          int width, float eps) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * kWaves + (threadIdx.x >> 6);
  if (row >= rows) return;
  const size_t base = (size_t)row * width;
  float ss = 0.f;
  for (int k = lane; k < width; k += 64) {
    const float a = bf2f(x[base + k]);
    ss += a * a;
  }
  const float inv = rsqrt_cr(wave_sum(ss) / (float)width + eps);
  for (int k = lane; k < width; k += 64) {
    const float nb = round_bf(bf2f(x[base + k]) * inv);
    const float wb = round_bf(load_w(w, k, w_f32));
    const float weighted = round_bf(nb * wb);
    y[base + k] = (uint16_t)f2bf(weighted * silu_f(bf2f(gate[base + k])));
  }
}

// out[r, c] = bf16( bf16(silu(gate)) * up ), packed = [gate | up] per row
// [reference kernels.py:158-180].
__global__ __launch_bounds__(256) void silu_mul_elems(const uint16_t* __restrict__ packed,
                                                      uint16_t* __restrict__ out, long long total,
                                                      int width) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const long long row = i / width;
  const int col = (int)(i - row * width);
  const float g = bf2f(packed[row * 2 * width + col]);
  const float up = bf2f(packed[row * 2 * width + width + col]);
  out[i] = (uint16_t)f2bf(round_bf(silu_f(g)) * up);
}

// out = bf16( x * bf16(sigmoid(gate)) ); the gate of head h sits at
// packed[token, h*2*head_dim + head_dim + col] [reference kernels.py:285-333].
__global__ __launch_bounds__(256) void attn_gate_elems(const uint16_t* __restrict__ x,
                                                       const uint16_t* __restrict__ packed,
                                                       uint16_t* __restrict__ out, long long total,
                                                       int hidden, int packed_stride,
                                                       int head_dim) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const long long token = i / hidden;
  const int col = (int)(i - token * hidden);
  const int head = col / head_dim;
  const int hc = col - head * head_dim;
  const float g = bf2f(packed[token * packed_stride + head * 2 * head_dim + head_dim + hc]);
  out[i] = (uint16_t)f2bf(bf2f(x[i]) * round_bf(sigmoid_f(g)));
}

}  // namespace

extern "C" {

int q35_rmsnorm(const void* x, const void* w, int w_f32, void* y, int rows, int width, float eps,
                hipStream_t stream) {
  Q35_CHECK_ARG(rows >= 0 && width > 0);
  if (rows == 0) return 0;
  const int grid = (rows + kWaves - 1) / kWaves;
  const int vec = (width % 8 == 0) && q35_aligned16(x) && q35_aligned16(y);
  rmsnorm_rows<false><<<grid, 256, 0, stream>>>((const uint16_t*)x, nullptr, w, w_f32, nullptr,
                                                (uint16_t*)y, rows, width, eps, vec);
  return q35_last_error();
}

int q35_residual_rmsnorm(const void* residual, const void* update, const void* w, int w_f32,
                         void* residual_out, void* y, int rows, int width, float eps,
                         hipStream_t stream) {
  Q35_CHECK_ARG(rows >= 0 && width > 0);
  if (rows == 0) return 0;
  const int grid = (rows + kWaves - 1) / kWaves;
  const int vec = (width % 8 == 0) && q35_aligned16(residual) && q35_aligned16(update) &&
                  q35_aligned16(residual_out) && q35_aligned16(y);
  rmsnorm_rows<true><<<grid, 256, 0, stream>>>((const uint16_t*)residual, (const uint16_t*)update,
                                               w, w_f32, (uint16_t*)residual_out, (uint16_t*)y,
                                               rows, width, eps, vec);
  return q35_last_error();
}

int q35_gated_rmsnorm(const void* x, const void* gate, const void* w, int w_f32, void* y, int rows,
                      int width, float eps, hipStream_t stream) {
  Q35_CHECK_ARG(rows >= 0 && width > 0);
  if (rows == 0) return 0;
  const int grid = (rows + kWaves - 1) / kWaves;
  gated_rmsnorm_rows<<<grid, 256, 0, stream>>>((const uint16_t*)x, (const uint16_t*)gate, w, w_f32,
                                               (uint16_t*)y, rows, width, eps);
  return q35_last_error();
}

int q35_silu_mul(const void* packed, void* out, long long rows, int width, hipStream_t stream) {
  Q35_CHECK_ARG(rows >= 0 && width > 0);
  const long long total = rows * (long long)width;
  if (total == 0) return 0;
  const long long grid = (total + 255) / 256;
  Q35_CHECK_ARG(grid < (1ll << 31));
  silu_mul_elems<<<(unsigned)grid, 256, 0, stream>>>((const uint16_t*)packed, (uint16_t*)out, total,
                                                     width);
  return q35_last_error();
}

int q35_attn_gate_mul(const void* x, const void* packed, void* out, long long tokens, int hidden,
                      int packed_stride, int head_dim, hipStream_t stream) {
  Q35_CHECK_ARG(tokens >= 0 && hidden > 0 && head_dim > 0 && hidden % head_dim == 0);
  Q35_CHECK_ARG(packed_stride >= 2 * hidden);
  const long long total = tokens * (long long)hidden;
  if (total == 0) return 0;
  const long long grid = (total + 255) / 256;
  Q35_CHECK_ARG(grid < (1ll << 31));
  attn_gate_elems<<<(unsigned)grid, 256, 0, stream>>>((const uint16_t*)x, (const uint16_t*)packed,
                                                      (uint16_t*)out, total, hidden, packed_stride,
                                                      head_dim);
  return q35_last_error();
}

}  // extern "C"
