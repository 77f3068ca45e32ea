// Row-wise decode kernels: RMSNorm, residual-add + RMSNorm, gated RMSNorm,
// SiLU-and-mul and the attention output gate.
//
// One wave64 owns one row. Widths of 512/1024/2048/4096 keep the row in
// registers between the two passes (one memory round trip per row); other
// widths that are a multiple of 8 stream the row twice with 128-bit loads, and
// the rest take a scalar lane-strided path. Gated RMSNorm over 128-wide heads
// packs 4 rows per wave (16 lanes x 8 elements). Sums of squares are reduced
// with the DPP/swizzle reductions from q35_common.hpp.
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

// rmsnorm_rows for widths of NPER * 512: the row stays in registers between
// the two passes (lane l holds elements 512*j + 8*l .. +7), and every load
// (x, u, w) is issued before the reduction, so a row costs one round trip.
// GATHER (no RESIDUAL): x is a [table_rows, width] table and row r reads
// table row ids[r] (clamped to [0, table_rows), as the decode GEMV's gather
// does); the raw row is also stored to r_out (the embedding lookup that
// starts the residual stream).
template <bool RESIDUAL, int NPER, bool GATHER = false>
__global__ __launch_bounds__(256) void rmsnorm_rows_reg(const uint16_t* __restrict__ x,
                                                        const uint16_t* __restrict__ u,
                                                        const void* __restrict__ w, int w_f32,
                                                        uint16_t* __restrict__ r_out,
                                                        uint16_t* __restrict__ y, int rows, float eps,
                                                        const long long* __restrict__ ids = nullptr,
                                                        int table_rows = 0) {
  constexpr int width = NPER * 512;
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * kWaves + (threadIdx.x >> 6);
  if (row >= rows) return;
  const size_t base = (size_t)row * width;
  size_t xbase = base;
  if (GATHER) {
    long long r = ids[row];
    r = r < 0 ? 0 : (r >= table_rows ? table_rows - 1 : r);
    xbase = (size_t)r * width;
  }
  uint4 xa[NPER], ua[NPER], wa[NPER], wb[NPER];
#pragma unroll
  for (int j = 0; j < NPER; ++j) {
    const int k = j * 512 + lane * 8;
    xa[j] = *reinterpret_cast<const uint4*>(x + xbase + k);
    if (RESIDUAL) ua[j] = *reinterpret_cast<const uint4*>(u + base + k);
    if (w_f32) {
      wa[j] = *reinterpret_cast<const uint4*>(reinterpret_cast<const float*>(w) + k);
      wb[j] = *reinterpret_cast<const uint4*>(reinterpret_cast<const float*>(w) + k + 4);
    } else {
      wa[j] = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(w) + k);
    }
  }
  if (GATHER && r_out) {
#pragma unroll
    for (int j = 0; j < NPER; ++j) *reinterpret_cast<uint4*>(r_out + base + j * 512 + lane * 8) = xa[j];
  }
  float a[NPER][8];
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < NPER; ++j) {
    unpack8(xa[j], a[j]);
    if (RESIDUAL) {
      float b[8];
      unpack8(ua[j], b);
#pragma unroll
      for (int e = 0; e < 8; ++e) a[j][e] = round_bf(a[j][e] + b[e]);
      *reinterpret_cast<uint4*>(r_out + base + j * 512 + lane * 8) = pack8(a[j]);
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) ss += a[j][e] * a[j][e];
  }
  const float inv = rsqrt_cr(wave_sum(ss) / (float)width + eps);
#pragma unroll
  for (int j = 0; j < NPER; ++j) {
    float wf[8];
    if (w_f32) {
      wf[0] = __uint_as_float(wa[j].x); wf[1] = __uint_as_float(wa[j].y);
      wf[2] = __uint_as_float(wa[j].z); wf[3] = __uint_as_float(wa[j].w);
      wf[4] = __uint_as_float(wb[j].x); wf[5] = __uint_as_float(wb[j].y);
      wf[6] = __uint_as_float(wb[j].z); wf[7] = __uint_as_float(wb[j].w);
    } else {
      unpack8(wa[j], wf);
    }
    float o[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = a[j][e] * inv * (1.0f + wf[e]);
    *reinterpret_cast<uint4*>(y + base + j * 512 + lane * 8) = pack8(o);
  }
}

// Gated RMSNorm over rows of exactly 128 (one head): 16 lanes per row, 8
// elements per lane, 4 rows per wave; the sum of squares is a DPP row sum.
// The gate of row r is read at (r / group_rows) * group_stride +
// (r % group_rows) * 128, so a gate that sits inside a wider packed row per
// token (group_rows heads per token) is read in place.
__global__ __launch_bounds__(256) void gated_rmsnorm_rows128(const uint16_t* __restrict__ x,
                                                             const uint16_t* __restrict__ gate,
                                                             const void* __restrict__ w, int w_f32,
                                                             uint16_t* __restrict__ y, int rows,
                                                             float eps, int group_rows,
                                                             long long group_stride) {
  const int lane = threadIdx.x & 63;
  const int row = (blockIdx.x * kWaves + (threadIdx.x >> 6)) * 4 + (lane >> 4);
  const int k = (lane & 15) * 8;
  const int rc = min(row, rows - 1);
  const size_t base = (size_t)rc * 128 + k;
  const size_t gbase = (size_t)(rc / group_rows) * group_stride + (size_t)(rc % group_rows) * 128 + k;
  const uint4 xr = *reinterpret_cast<const uint4*>(x + base);
  const uint4 gr = *reinterpret_cast<const uint4*>(gate + gbase);
  float wf[8];
  if (w_f32) {
    const float4 w0 = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(w) + k);
    const float4 w1 = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(w) + k + 4);
    wf[0] = w0.x; wf[1] = w0.y; wf[2] = w0.z; wf[3] = w0.w;
    wf[4] = w1.x; wf[5] = w1.y; wf[6] = w1.z; wf[7] = w1.w;
  } else {
    unpack8(*reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(w) + k), wf);
  }
  float a[8], g[8];
  unpack8(xr, a);
  unpack8(gr, g);
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) ss += a[e] * a[e];
  const float inv = rsqrt_cr(row16_sum(ss) / 128.0f + eps);
  float o[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float nb = round_bf(a[e] * inv);
    const float weighted = round_bf(nb * round_bf(wf[e]));
    o[e] = weighted * silu_f(g[e]);
  }
  if (row < rows) *reinterpret_cast<uint4*>(y + base) = pack8(o);
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

// silu_mul_elems with 8 elements per thread (width a multiple of 8), grid
// (column blocks of 2048, rows) so no thread divides its index.
__global__ __launch_bounds__(256) void silu_mul_vec(const uint16_t* __restrict__ packed,
                                                    uint16_t* __restrict__ out, long long rows,
                                                    int width) {
  const int col = (blockIdx.x * 256 + threadIdx.x) * 8;
  if (col >= width) return;
  for (long long row = blockIdx.y; row < rows; row += gridDim.y) {
    const uint4 graw = *reinterpret_cast<const uint4*>(packed + row * 2 * width + col);
    const uint4 uraw = *reinterpret_cast<const uint4*>(packed + row * 2 * width + width + col);
    float g[8], up[8], o[8];
    unpack8(graw, g);
    unpack8(uraw, up);
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = round_bf(silu_fast(g[e])) * up[e];
    *reinterpret_cast<uint4*>(out + row * width + col) = pack8(o);
  }
}

// silu_mul on the transposed product of a packed [gate; up] projection:
// packed_t is [2 * width, rows] (channel-major: gate channels, then up
// channels, each a row of `rows` tokens), out is [rows, width] token-major,
// out[m, n] = bf16(bf16(silu(g[n, m])) * u[n, m]) as silu_mul_vec computes
// it. Tile of 64 channels x 64 tokens per workgroup: thread (n = t/4, q =
// t%4) loads 16 tokens of gate and up of channel n (16-byte loads along the
// tokens), computes them, and writes the bf16 results into an LDS tile of
// stride 33 dwords; thread (m = t/4, q) then reads the 16 channels 16q..16q+15
// of token m (conflict-free: the four q groups sit 16 banks apart) and
// stores 32 contiguous bytes. rows % 8 == 0; tokens past rows are skipped.
constexpr int kSmtS = 66;  // LDS row stride in bf16 (33 dwords)
__global__ __launch_bounds__(256) void silu_mul_t_tile(const uint16_t* __restrict__ pt,
                                                       uint16_t* __restrict__ out, int rows,
                                                       int width) {
  __shared__ alignas(16) uint16_t os[64 * kSmtS];
  const int n0 = blockIdx.x * 64, m0 = blockIdx.y * 64;
  const int t = threadIdx.x, q = t & 3;
  {
    const int n = t >> 2;
    const int m = m0 + 16 * q;
    const uint16_t* g = pt + (size_t)(n0 + n) * rows;
    const uint16_t* u = pt + (size_t)(width + n0 + n) * rows;
    uint4 graw[2], uraw[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int mm = min(m + 8 * h, rows - 8);  // rows % 8 == 0: always a whole 8-token group
      graw[h] = *reinterpret_cast<const uint4*>(g + mm);
      uraw[h] = *reinterpret_cast<const uint4*>(u + mm);
    }
    uint32_t* dst = reinterpret_cast<uint32_t*>(os + n * kSmtS + 16 * q);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      float gf[8], uf[8], o[8];
      unpack8(graw[h], gf);
      unpack8(uraw[h], uf);
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = round_bf(silu_fast(gf[e])) * uf[e];
#pragma unroll
      for (int e = 0; e < 4; ++e) dst[4 * h + e] = pack_bf2(o[2 * e], o[2 * e + 1]);
    }
  }
  __syncthreads();
  const int m = t >> 2;
  if (m0 + m >= rows) return;
  uint32_t w[8];
#pragma unroll
  for (int e = 0; e < 8; ++e)
    w[e] = (uint32_t)os[(16 * q + 2 * e) * kSmtS + m] | ((uint32_t)os[(16 * q + 2 * e + 1) * kSmtS + m] << 16);
  uint16_t* o = out + (size_t)(m0 + m) * width + n0 + 16 * q;
  *reinterpret_cast<uint4*>(o) = make_uint4(w[0], w[1], w[2], w[3]);
  *reinterpret_cast<uint4*>(o + 8) = make_uint4(w[4], w[5], w[6], w[7]);
}

// out = bf16( x * bf16(sigmoid(gate)) ); the gate of head h sits at
// packed[token, h*2*head_dim + head_dim + col] [reference kernels.py:285-333].
__global__ __launch_bounds__(256) void attn_gate_elems(const uint16_t* __restrict__ x,
                                                       const uint16_t* __restrict__ packed,
                                                       uint16_t* __restrict__ out, long long total,
                                                       int hidden, int packed_stride,
                                                       int head_dim, long long* advance,
                                                       long long amount) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (advance && i == 0) advance[0] += amount;
  if (i >= total) return;
  const long long token = i / hidden;
  const int col = (int)(i - token * hidden);
  const int head = col / head_dim;
  const int hc = col - head * head_dim;
  const float g = bf2f(packed[token * packed_stride + head * 2 * head_dim + head_dim + hc]);
  out[i] = (uint16_t)f2bf(bf2f(x[i]) * round_bf(sigmoid_f(g)));
}


// attn_gate_elems with 8 columns per thread (16-byte loads; head_dim,
// hidden and packed_stride multiples of 8), grid (column blocks, tokens).
// Both forms add `amount` to the int64 counter `advance` (when given) from
// one thread: the prefill's cache-length advance, which no kernel after the
// attention reads before this one ends.
__global__ __launch_bounds__(256) void attn_gate_vec(const uint16_t* __restrict__ x,
                                                     const uint16_t* __restrict__ packed,
                                                     uint16_t* __restrict__ out, long long tokens,
                                                     int hidden, int packed_stride, int head_dim,
                                                     long long* advance, long long amount) {
  const int col = (blockIdx.x * 256 + threadIdx.x) * 8;
  if (advance && col == 0 && blockIdx.y == 0) advance[0] += amount;
  if (col >= hidden) return;
  const int head = col / head_dim;
  const int hc = col - head * head_dim;
  for (long long t = blockIdx.y; t < tokens; t += gridDim.y) {
    const uint4 xr = *reinterpret_cast<const uint4*>(x + t * hidden + col);
    const uint4 gr = *reinterpret_cast<const uint4*>(packed + t * packed_stride + head * 2 * head_dim + head_dim + hc);
    float xv[8], gv[8], o[8];
    unpack8(xr, xv);
    unpack8(gr, gv);
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = xv[e] * round_bf(sigmoid_f(gv[e]));
    *reinterpret_cast<uint4*>(out + t * hidden + col) = pack8(o);
  }
}
}  // namespace

extern "C" {

int q35_rmsnorm(const void* x, const void* w, int w_f32, void* y, int rows, int width, float eps,
                hipStream_t stream) {
  Q35_CHECK_ARG(rows >= 0 && width > 0);
  if (rows == 0) return 0;
  const int grid = (rows + kWaves - 1) / kWaves;
  const int vec = (width % 8 == 0) && q35_aligned16(x) && q35_aligned16(y);
  if (vec && q35_aligned16(w) && (width == 512 || width == 1024 || width == 2048 || width == 4096)) {
#define Q35_RMS(NP)                                                                               \
  rmsnorm_rows_reg<false, NP><<<grid, 256, 0, stream>>>((const uint16_t*)x, nullptr, w, w_f32,  \
                                                        nullptr, (uint16_t*)y, rows, eps)
    if (width == 512) Q35_RMS(1);
    else if (width == 1024) Q35_RMS(2);
    else if (width == 2048) Q35_RMS(4);
    else Q35_RMS(8);
#undef Q35_RMS
    return q35_last_error();
  }
  rmsnorm_rows<false><<<grid, 256, 0, stream>>>((const uint16_t*)x, nullptr, w, w_f32, nullptr,
                                                (uint16_t*)y, rows, width, eps, vec);
  return q35_last_error();
}

// The embedding lookup of the prefill and the first layer's input RMSNorm
// in one launch: r_out[r] = table[clamp(ids[r])], y[r] = rms_norm(r_out[r]),
// the bits of a gather followed by q35_rmsnorm. Widths 512, 1024, 2048, 4096.
int q35_embed_rmsnorm(const void* table, int table_rows, const void* ids, const void* w, int w_f32,
                      void* r_out, void* y, int rows, int width, float eps, hipStream_t stream) {
  Q35_CHECK_ARG(rows >= 0 && table_rows > 0 && table && w && y && (rows == 0 || ids));
  Q35_CHECK_ARG(width == 512 || width == 1024 || width == 2048 || width == 4096);
  Q35_CHECK_ARG(q35_aligned16(table) && q35_aligned16(y) && q35_aligned16(w) && q35_aligned16(r_out) &&
                q35_aligned8(ids));
  if (rows == 0) return 0;
  const int grid = (rows + kWaves - 1) / kWaves;
#define Q35_ERMS(NP)                                                                              \
  rmsnorm_rows_reg<false, NP, true><<<grid, 256, 0, stream>>>(                                     \
      (const uint16_t*)table, nullptr, w, w_f32, (uint16_t*)r_out, (uint16_t*)y, rows, eps,       \
      (const long long*)ids, table_rows)
  if (width == 512) Q35_ERMS(1);
  else if (width == 1024) Q35_ERMS(2);
  else if (width == 2048) Q35_ERMS(4);
  else Q35_ERMS(8);
#undef Q35_ERMS
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
  if (vec && q35_aligned16(w) && (width == 512 || width == 1024 || width == 2048 || width == 4096)) {
#define Q35_RMS(NP)                                                                               \
  rmsnorm_rows_reg<true, NP><<<grid, 256, 0, stream>>>(                                          \
      (const uint16_t*)residual, (const uint16_t*)update, w, w_f32, (uint16_t*)residual_out,     \
      (uint16_t*)y, rows, eps)
    if (width == 512) Q35_RMS(1);
    else if (width == 1024) Q35_RMS(2);
    else if (width == 2048) Q35_RMS(4);
    else Q35_RMS(8);
#undef Q35_RMS
    return q35_last_error();
  }
  rmsnorm_rows<true><<<grid, 256, 0, stream>>>((const uint16_t*)residual, (const uint16_t*)update,
                                               w, w_f32, (uint16_t*)residual_out, (uint16_t*)y,
                                               rows, width, eps, vec);
  return q35_last_error();
}

int q35_gated_rmsnorm(const void* x, const void* gate, const void* w, int w_f32, void* y, int rows,
                      int width, float eps, hipStream_t stream) {
  Q35_CHECK_ARG(rows >= 0 && width > 0);
  if (rows == 0) return 0;
  if (width == 128 && q35_aligned16(x) && q35_aligned16(gate) && q35_aligned16(y) &&
      q35_aligned16(w)) {
    const int grid4 = (rows + 4 * kWaves - 1) / (4 * kWaves);
    gated_rmsnorm_rows128<<<grid4, 256, 0, stream>>>((const uint16_t*)x, (const uint16_t*)gate, w,
                                                     w_f32, (uint16_t*)y, rows, eps, rows,
                                                     (long long)rows * 128);
    return q35_last_error();
  }
  const int grid = (rows + kWaves - 1) / kWaves;
  gated_rmsnorm_rows<<<grid, 256, 0, stream>>>((const uint16_t*)x, (const uint16_t*)gate, w, w_f32,
                                               (uint16_t*)y, rows, width, eps);
  return q35_last_error();
}

int q35_gated_rmsnorm_grouped(const void* x, const void* gate, int group_rows,
                              long long group_stride, const void* w, int w_f32, void* y, int rows,
                              float eps, hipStream_t stream) {
  Q35_CHECK_ARG(rows >= 0 && group_rows > 0 && group_stride >= (long long)group_rows * 128);
  Q35_CHECK_ARG(group_stride % 8 == 0 && q35_aligned16(x) && q35_aligned16(gate) &&
                q35_aligned16(y) && q35_aligned16(w));
  if (rows == 0) return 0;
  const int grid4 = (rows + 4 * kWaves - 1) / (4 * kWaves);
  gated_rmsnorm_rows128<<<grid4, 256, 0, stream>>>((const uint16_t*)x, (const uint16_t*)gate, w,
                                                   w_f32, (uint16_t*)y, rows, eps, group_rows,
                                                   group_stride);
  return q35_last_error();
}

int q35_silu_mul(const void* packed, void* out, long long rows, int width, hipStream_t stream) {
  Q35_CHECK_ARG(rows >= 0 && width > 0);
  const long long total = rows * (long long)width;
  if (total == 0) return 0;
  if (width % 8 == 0 && q35_aligned16(packed) && q35_aligned16(out)) {
    const dim3 grid((unsigned)((width / 8 + 255) / 256), (unsigned)min(rows, 65535ll));
    silu_mul_vec<<<grid, 256, 0, stream>>>((const uint16_t*)packed, (uint16_t*)out, rows, width);
    return q35_last_error();
  }
  const long long grid = (total + 255) / 256;
  Q35_CHECK_ARG(grid < (1ll << 31));
  silu_mul_elems<<<(unsigned)grid, 256, 0, stream>>>((const uint16_t*)packed, (uint16_t*)out, total,
                                                     width);
  return q35_last_error();
}

int q35_silu_mul_t(const void* packed_t, void* out, int rows, int width, hipStream_t stream) {
  Q35_CHECK_ARG(rows >= 0 && width > 0 && width % 64 == 0 && rows % 8 == 0);
  Q35_CHECK_ARG(q35_aligned16(packed_t) && q35_aligned16(out));
  if (rows == 0) return 0;
  const dim3 grid((unsigned)(width / 64), (unsigned)((rows + 63) / 64));
  silu_mul_t_tile<<<grid, 256, 0, stream>>>((const uint16_t*)packed_t, (uint16_t*)out, rows, width);
  return q35_last_error();
}

int q35_attn_gate_mul(const void* x, const void* packed, void* out, long long tokens, int hidden,
                      int packed_stride, int head_dim, void* advance, long long amount,
                      hipStream_t stream) {
  Q35_CHECK_ARG(tokens >= 0 && hidden > 0 && head_dim > 0 && hidden % head_dim == 0);
  Q35_CHECK_ARG(packed_stride >= 2 * hidden);
  const long long total = tokens * (long long)hidden;
  if (total == 0 && (!advance || amount == 0)) return 0;
  if (head_dim % 8 == 0 && packed_stride % 8 == 0 && q35_aligned16(x) && q35_aligned16(packed) &&
      q35_aligned16(out)) {
    const dim3 vgrid((unsigned)((hidden / 8 + 255) / 256), (unsigned)max(1ll, min(tokens, 65535ll)));
    attn_gate_vec<<<vgrid, 256, 0, stream>>>((const uint16_t*)x, (const uint16_t*)packed,
                                             (uint16_t*)out, tokens, hidden, packed_stride, head_dim,
                                             (long long*)advance, amount);
    return q35_last_error();
  }
  const long long grid = max(1ll, (total + 255) / 256);
  Q35_CHECK_ARG(grid < (1ll << 31));
  attn_gate_elems<<<(unsigned)grid, 256, 0, stream>>>((const uint16_t*)x, (const uint16_t*)packed,
                                                      (uint16_t*)out, total, hidden, packed_stride,
                                                      head_dim, (long long*)advance, amount);
  return q35_last_error();
}

}  // extern "C"
