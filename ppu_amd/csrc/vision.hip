// Vision-encoder kernels of the image path (reference kernels.py:336-416 and
// 1188-1336): LayerNorm with and without the residual add, the interpolated
// position-embedding add, and the packed-QKV split into [1, heads, tokens,
// dim] with rotate-half RoPE on q and k.
//
//   layer_norm              y = bf16((x - mean) * rsqrt(var + eps) * w + b),
//                           mean and var over the row in fp32
//   residual_add_layer_norm r' = bf16(r + u); y = layer_norm(r')
//   position_embed_add      p = bf16(sum_n table[idx_n] * wt_n) (fp32 FMA
//                           chain over the neighbours in order);
//                           out = bf16(hidden + p)
//   vision_qkv_rope         o[c] = bf16(x[c] * cos[c] + (sign_c * x[partner c]) * sin[c]),
//                           partner = c +- dim/2, sign = -1 below dim/2;
//                           v copied
//
// Rows are independent, so every kernel runs one wave64 per row (per (token,
// head) for the RoPE split) and reduces with the DPP wave sums; widths that
// are multiples of 8 use 16-byte accesses with the row held in registers
// between the two LayerNorm passes (one memory round trip per row), other
// widths a lane-strided scalar form. Builds use -ffp-contract=off, so a*b+c
// is fused only where fmaf is written.
#include "q35_common.hpp"

namespace {

constexpr int kRowsPerBlock = 4;  // one wave per row, 4 waves per workgroup

Q35_DEV float param_at(const void* p, int k, int f32) {
  return f32 ? reinterpret_cast<const float*>(p)[k] : bf2f(reinterpret_cast<const uint16_t*>(p)[k]);
}

// 8 consecutive parameters at k (k % 8 == 0; fp32 vectors 16-byte aligned).
Q35_DEV void param8(const void* p, int k, int f32, float* o) {
  if (f32) {
    const float4 a = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(p) + k);
    const float4 b = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(p) + k + 4);
    o[0] = a.x; o[1] = a.y; o[2] = a.z; o[3] = a.w;
    o[4] = b.x; o[5] = b.y; o[6] = b.z; o[7] = b.w;
  } else {
    unpack8(*reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(p) + k), o);
  }
}

// LayerNorm of rows of width <= NJ * 512 (width % 8 == 0): lane l holds the
// 8-element groups k = 512 j + 8 l. Groups past the width read group 0 of
// the row (in bounds) and are left out of the sums and the stores.
template <bool RESIDUAL, int NJ>
__global__ __launch_bounds__(256) void layernorm_rows_vec(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ u, const void* __restrict__ w,
    const void* __restrict__ b, int p_f32, uint16_t* __restrict__ r_out, uint16_t* __restrict__ y,
    int rows, int width, float eps) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= rows) return;
  const size_t base = (size_t)row * width;
  uint4 xa[NJ], ua[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int k = j * 512 + lane * 8;
    const int kk = k < width ? k : 0;
    xa[j] = *reinterpret_cast<const uint4*>(x + base + kk);
    if (RESIDUAL) ua[j] = *reinterpret_cast<const uint4*>(u + base + kk);
  }
  float v[NJ][8];
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int k = j * 512 + lane * 8;
    const bool ok = k < width;
    unpack8(xa[j], v[j]);
    if (RESIDUAL) {
      float a[8];
      unpack8(ua[j], a);
#pragma unroll
      for (int e = 0; e < 8; ++e) v[j][e] = round_bf(v[j][e] + a[e]);
      if (ok) *reinterpret_cast<uint4*>(r_out + base + k) = pack8(v[j]);
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) s += ok ? v[j][e] : 0.f;
  }
  const float mean = wave_sum(s) / (float)width;
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const bool ok = j * 512 + lane * 8 < width;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      v[j][e] -= mean;
      ss += ok ? v[j][e] * v[j][e] : 0.f;
    }
  }
  const float inv = rsqrt_cr(wave_sum(ss) / (float)width + eps);
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int k = j * 512 + lane * 8;
    if (k < width) {
      float wv[8], bv[8], o[8];
      param8(w, k, p_f32, wv);
      param8(b, k, p_f32, bv);
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = v[j][e] * inv * wv[e] + bv[e];
      *reinterpret_cast<uint4*>(y + base + k) = pack8(o);
    }
  }
}

// Any width: lane-strided scalar passes (sum, centred sum of squares, store).
template <bool RESIDUAL>
__global__ __launch_bounds__(256) void layernorm_rows_scalar(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ u, const void* __restrict__ w,
    const void* __restrict__ b, int p_f32, uint16_t* __restrict__ r_out, uint16_t* __restrict__ y,
    int rows, int width, float eps) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= rows) return;
  const size_t base = (size_t)row * width;
  auto val = [&](int k) -> float {
    float a = bf2f(x[base + k]);
    if (RESIDUAL) a = round_bf(a + bf2f(u[base + k]));
    return a;
  };
  float s = 0.f;
  for (int k = lane; k < width; k += 64) {
    const float a = val(k);
    if (RESIDUAL) r_out[base + k] = (uint16_t)f2bf(a);
    s += a;
  }
  const float mean = wave_sum(s) / (float)width;
  float ss = 0.f;
  for (int k = lane; k < width; k += 64) {
    const float c = val(k) - mean;
    ss += c * c;
  }
  const float inv = rsqrt_cr(wave_sum(ss) / (float)width + eps);
  for (int k = lane; k < width; k += 64) {
    const float c = val(k) - mean;
    y[base + k] = (uint16_t)f2bf(c * inv * param_at(w, k, p_f32) + param_at(b, k, p_f32));
  }
}

template <bool RESIDUAL>
int layernorm_launch(const void* x, const void* u, const void* w, const void* b, int p_f32,
                     void* r_out, void* y, int rows, int width, float eps, hipStream_t stream) {
  Q35_CHECK_ARG(rows >= 0 && width > 0 && x && w && b && y && (!RESIDUAL || (u && r_out)));
  if (rows == 0) return 0;
  const unsigned grid = (unsigned)((rows + kRowsPerBlock - 1) / kRowsPerBlock);
  const bool vec = width % 8 == 0 && width <= 2048 && q35_aligned16(x) && q35_aligned16(y) &&
                   q35_aligned16(w) && q35_aligned16(b) &&
                   (!RESIDUAL || (q35_aligned16(u) && q35_aligned16(r_out)));
  const uint16_t *xs = (const uint16_t*)x, *us = (const uint16_t*)u;
  uint16_t *rs = (uint16_t*)r_out, *ys = (uint16_t*)y;
  if (vec) {
    const int nj = (width + 511) / 512;
    if (nj == 1) layernorm_rows_vec<RESIDUAL, 1><<<grid, 256, 0, stream>>>(xs, us, w, b, p_f32, rs, ys, rows, width, eps);
    else if (nj == 2) layernorm_rows_vec<RESIDUAL, 2><<<grid, 256, 0, stream>>>(xs, us, w, b, p_f32, rs, ys, rows, width, eps);
    else if (nj == 3) layernorm_rows_vec<RESIDUAL, 3><<<grid, 256, 0, stream>>>(xs, us, w, b, p_f32, rs, ys, rows, width, eps);
    else layernorm_rows_vec<RESIDUAL, 4><<<grid, 256, 0, stream>>>(xs, us, w, b, p_f32, rs, ys, rows, width, eps);
  } else {
    layernorm_rows_scalar<RESIDUAL><<<grid, 256, 0, stream>>>(xs, us, w, b, p_f32, rs, ys, rows, width, eps);
  }
  return q35_last_error();
}

// Position embedding: p = sum over the row's neighbours of table[idx] * wt
// (fp32 FMA chain in neighbour order), rounded to bf16 and added to the
// hidden row. Indices are clamped to the table, so no access leaves it.
template <bool VEC>
__global__ __launch_bounds__(256) void position_embed_add_rows(
    const uint16_t* __restrict__ hidden, const uint16_t* __restrict__ table, int table_rows,
    const long long* __restrict__ idx, const void* __restrict__ wt, int w_f32,
    uint16_t* __restrict__ out, int rows, int width, int neighbors) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= rows) return;
  const size_t base = (size_t)row * width;
  const long long* ri = idx + (size_t)row * neighbors;
  const int wbase = row * neighbors;
  if (VEC) {
    for (int k = lane * 8; k < width; k += 512) {
      float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
      for (int n = 0; n < neighbors; ++n) {
        const long long t = min(max(ri[n], 0ll), (long long)table_rows - 1);
        const float wn = param_at(wt, wbase + n, w_f32);
        float e[8];
        unpack8(*reinterpret_cast<const uint4*>(table + (size_t)t * width + k), e);
#pragma unroll
        for (int q = 0; q < 8; ++q) acc[q] = fmaf(e[q], wn, acc[q]);
      }
      float h[8], o[8];
      unpack8(*reinterpret_cast<const uint4*>(hidden + base + k), h);
#pragma unroll
      for (int q = 0; q < 8; ++q) o[q] = h[q] + round_bf(acc[q]);
      *reinterpret_cast<uint4*>(out + base + k) = pack8(o);
    }
  } else {
    for (int k = lane; k < width; k += 64) {
      float acc = 0.f;
      for (int n = 0; n < neighbors; ++n) {
        const long long t = min(max(ri[n], 0ll), (long long)table_rows - 1);
        acc = fmaf(bf2f(table[(size_t)t * width + k]), param_at(wt, wbase + n, w_f32), acc);
      }
      out[base + k] = (uint16_t)f2bf(bf2f(hidden[base + k]) + round_bf(acc));
    }
  }
}

// One wave per (token, head): lane c (+64 j) of the head's dims. q/k/v of a
// token are contiguous [q heads | k heads | v heads] in the packed row.
__global__ __launch_bounds__(256) void vision_qkv_rope_rows(
    const uint16_t* __restrict__ packed, const void* __restrict__ cos, const void* __restrict__ sin,
    int cs_f32, uint16_t* __restrict__ q_out, uint16_t* __restrict__ k_out,
    uint16_t* __restrict__ v_out, int tokens, int heads, int dim) {
  const int lane = threadIdx.x & 63;
  const long long pid = (long long)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  if (pid >= (long long)tokens * heads) return;
  const int head = (int)(pid % heads);
  const int token = (int)(pid / heads);
  const int half = dim / 2;
  const uint16_t* row = packed + (size_t)token * 3 * heads * dim;
  const uint16_t* qh = row + (size_t)head * dim;
  const uint16_t* kh = row + (size_t)(heads + head) * dim;
  const uint16_t* vh = row + (size_t)(2 * heads + head) * dim;
  const size_t ob = ((size_t)head * tokens + token) * dim;
  for (int c = lane; c < dim; c += 64) {
    const bool lo = c < half;
    const int p = lo ? c + half : c - half;
    const float cs = param_at(cos, token * dim + c, cs_f32);
    const float sn = param_at(sin, token * dim + c, cs_f32);
    const float qp = lo ? -bf2f(qh[p]) : bf2f(qh[p]);
    const float kp = lo ? -bf2f(kh[p]) : bf2f(kh[p]);
    q_out[ob + c] = (uint16_t)f2bf(bf2f(qh[c]) * cs + qp * sn);
    k_out[ob + c] = (uint16_t)f2bf(bf2f(kh[c]) * cs + kp * sn);
    v_out[ob + c] = vh[c];
  }
}

}  // namespace

extern "C" {

int q35_layernorm(const void* x, const void* w, const void* b, int p_f32, void* y, int rows,
                  int width, float eps, hipStream_t stream) {
  return layernorm_launch<false>(x, nullptr, w, b, p_f32, nullptr, y, rows, width, eps, stream);
}

int q35_residual_layernorm(const void* residual, const void* update, const void* w, const void* b,
                           int p_f32, void* residual_out, void* y, int rows, int width, float eps,
                           hipStream_t stream) {
  return layernorm_launch<true>(residual, update, w, b, p_f32, residual_out, y, rows, width, eps,
                                stream);
}

int q35_position_embed_add(const void* hidden, const void* table, int table_rows,
                           const void* indices, const void* weights, int w_f32, void* out, int rows,
                           int width, int neighbors, hipStream_t stream) {
  Q35_CHECK_ARG(rows >= 0 && width > 0 && neighbors > 0 && table_rows > 0);
  Q35_CHECK_ARG(hidden && table && indices && weights && out);
  Q35_CHECK_ARG((long long)rows * neighbors < (1ll << 31) && (long long)rows * width < (1ll << 40));
  if (rows == 0) return 0;
  const unsigned grid = (unsigned)((rows + kRowsPerBlock - 1) / kRowsPerBlock);
  const bool vec = width % 8 == 0 && q35_aligned16(hidden) && q35_aligned16(table) && q35_aligned16(out);
  if (vec)
    position_embed_add_rows<true><<<grid, 256, 0, stream>>>(
        (const uint16_t*)hidden, (const uint16_t*)table, table_rows, (const long long*)indices,
        weights, w_f32, (uint16_t*)out, rows, width, neighbors);
  else
    position_embed_add_rows<false><<<grid, 256, 0, stream>>>(
        (const uint16_t*)hidden, (const uint16_t*)table, table_rows, (const long long*)indices,
        weights, w_f32, (uint16_t*)out, rows, width, neighbors);
  return q35_last_error();
}

int q35_vision_qkv_rope(const void* packed, const void* cos, const void* sin, int cs_f32, void* q,
                        void* k, void* v, int tokens, int heads, int dim, hipStream_t stream) {
  Q35_CHECK_ARG(tokens >= 0 && heads > 0 && dim > 0 && dim % 2 == 0);
  Q35_CHECK_ARG(packed && cos && sin && q && k && v);
  Q35_CHECK_ARG((long long)tokens * 3 * heads * dim < (1ll << 31));
  if (tokens == 0) return 0;
  const long long waves = (long long)tokens * heads;
  const unsigned grid = (unsigned)((waves + kRowsPerBlock - 1) / kRowsPerBlock);
  vision_qkv_rope_rows<<<grid, 256, 0, stream>>>((const uint16_t*)packed, cos, sin, cs_f32,
                                                (uint16_t*)q, (uint16_t*)k, (uint16_t*)v, tokens,
                                                heads, dim);
  return q35_last_error();
}

}  // extern "C"
