// Vision-encoder kernels of the image path (reference kernels.py:336-416 and
// 1188-1336): LayerNorm with and without the residual add, the interpolated
// position-embedding add, the packed-QKV split into [1, heads, tokens, dim]
// with rotate-half RoPE on q and k, and the blocks' non-causal per-image
// attention on the matrix cores (the attention call of reference
// integration.py:671-731).
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
//   vision_attention        o = bf16(softmax(q k^T * scale) v) over the keys of
//                           the query's own image, P rounded to bf16
//
// The LayerNorms run one wave64 per row and reduce with the DPP wave sums;
// widths that are multiples of 8 use 16-byte accesses with the row held in
// registers between the two passes (one memory round trip per row), other
// widths a lane-strided scalar form. The RoPE split runs one thread per four
// rotation pairs (or one wave per (token, head) for other head dims). Builds
// use -ffp-contract=off, so a*b+c is fused only where fmaf is written.
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

// Native 16-byte register vector: a uint4 struct held in an array and copied
// can stay a memory copy (scratch); these stay in registers.
typedef uint32_t vz_u32x4 __attribute__((ext_vector_type(4)));

Q35_DEV vz_u32x4 ld16(const void* p) { return *reinterpret_cast<const vz_u32x4*>(p); }
Q35_DEV uint4 as_u4(vz_u32x4 v) { return __builtin_bit_cast(uint4, v); }

// LayerNorm of rows of width <= NJ * 512 (width % 8 == 0): lane l holds the
// 8-element groups k = 512 j + 8 l. Groups past the width read group 0 of
// the row (in bounds) and are left out of the sums and the stores. The
// weight and bias groups are requested together with the row, so they are in
// registers when the two reductions end (PF32: fp32 parameters).
template <bool RESIDUAL, int NJ, bool PF32>
__global__ __launch_bounds__(256) void layernorm_rows_vec(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ u, const void* __restrict__ w,
    const void* __restrict__ b, uint16_t* __restrict__ r_out, uint16_t* __restrict__ y,
    int rows, int width, float eps) {
  constexpr int PW = PF32 ? 2 : 1;  // 16-byte parameter loads per group
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= rows) return;
  const size_t base = (size_t)row * width;
  vz_u32x4 xa[NJ], ua[NJ], wa[NJ][PW], ba[NJ][PW];
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int k = j * 512 + lane * 8;
    const int kk = k < width ? k : 0;
    xa[j] = ld16(x + base + kk);
    if (RESIDUAL) ua[j] = ld16(u + base + kk);
  }
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int k = j * 512 + lane * 8;
    const int kk = k < width ? k : 0;
#pragma unroll
    for (int h = 0; h < PW; ++h) {
      if (PF32) {
        wa[j][h] = ld16(reinterpret_cast<const float*>(w) + kk + 4 * h);
        ba[j][h] = ld16(reinterpret_cast<const float*>(b) + kk + 4 * h);
      } else {
        wa[j][h] = ld16(reinterpret_cast<const uint16_t*>(w) + kk);
        ba[j][h] = ld16(reinterpret_cast<const uint16_t*>(b) + kk);
      }
    }
  }
  float v[NJ][8];
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int k = j * 512 + lane * 8;
    const bool ok = k < width;
    unpack8(as_u4(xa[j]), v[j]);
    if (RESIDUAL) {
      float a[8];
      unpack8(as_u4(ua[j]), a);
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
      if (PF32) {
        const float4 w0 = __builtin_bit_cast(float4, as_u4(wa[j][0]));
        const float4 w1 = __builtin_bit_cast(float4, as_u4(wa[j][PW - 1]));
        const float4 b0 = __builtin_bit_cast(float4, as_u4(ba[j][0]));
        const float4 b1 = __builtin_bit_cast(float4, as_u4(ba[j][PW - 1]));
        wv[0] = w0.x; wv[1] = w0.y; wv[2] = w0.z; wv[3] = w0.w;
        wv[4] = w1.x; wv[5] = w1.y; wv[6] = w1.z; wv[7] = w1.w;
        bv[0] = b0.x; bv[1] = b0.y; bv[2] = b0.z; bv[3] = b0.w;
        bv[4] = b1.x; bv[5] = b1.y; bv[6] = b1.z; bv[7] = b1.w;
      } else {
        unpack8(as_u4(wa[j][0]), wv);
        unpack8(as_u4(ba[j][0]), bv);
      }
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
#define LN_VEC(NJ_)                                                                                   \
  (p_f32 ? layernorm_rows_vec<RESIDUAL, NJ_, true><<<grid, 256, 0, stream>>>(xs, us, w, b, rs, ys, rows, width, eps) \
         : layernorm_rows_vec<RESIDUAL, NJ_, false><<<grid, 256, 0, stream>>>(xs, us, w, b, rs, ys, rows, width, eps))
    if (nj == 1) LN_VEC(1);
    else if (nj == 2) LN_VEC(2);
    else if (nj == 3) LN_VEC(3);
    else LN_VEC(4);
#undef LN_VEC
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


// Vector form for dim % 8 == 0 (16-byte aligned buffers): per token, thread
// units are the (head, 4-column group c) of q and of k, each rotating the
// pairs (c..c+3, c+half..c+half+3) with two 8-byte loads and stores, then the
// 16-byte chunks of v. Same products and sums as the per-element form
// (x * cos - partner * sin below half, x * cos + partner * sin above).
template <bool CS_F32>
__global__ __launch_bounds__(256) void vision_qkv_rope_vec(
    const uint16_t* __restrict__ packed, const void* __restrict__ cos, const void* __restrict__ sin,
    uint16_t* __restrict__ q_out, uint16_t* __restrict__ k_out, uint16_t* __restrict__ v_out,
    int tokens, int heads, int dim) {
  const int half = dim / 2, g4 = half / 4, g8 = dim / 8;
  const int nqk = heads * g4;                 // q (or k) units per token
  const int units = 2 * nqk + heads * g8;     // + v chunks
  const long long gid = (long long)blockIdx.x * 256 + threadIdx.x;
  if (gid >= (long long)tokens * units) return;
  const int token = (int)(gid / units);
  int u = (int)(gid - (long long)token * units);
  const uint16_t* row = packed + (size_t)token * 3 * heads * dim;
  if (u < 2 * nqk) {
    const int which = u >= nqk;                 // 0: q, 1: k
    u -= which * nqk;
    const int head = u / g4, c = 4 * (u - head * g4);
    const uint16_t* src = row + (size_t)(which * heads + head) * dim;
    const uint2 xl = *reinterpret_cast<const uint2*>(src + c);
    const uint2 xh = *reinterpret_cast<const uint2*>(src + c + half);
    float cl[4], ch[4], sl[4], sh[4];
    const size_t cs = (size_t)token * dim + c;
    if (CS_F32) {
      const float4 a = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(cos) + cs);
      const float4 bb = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(cos) + cs + half);
      const float4 e = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(sin) + cs);
      const float4 f = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(sin) + cs + half);
      cl[0] = a.x; cl[1] = a.y; cl[2] = a.z; cl[3] = a.w;
      ch[0] = bb.x; ch[1] = bb.y; ch[2] = bb.z; ch[3] = bb.w;
      sl[0] = e.x; sl[1] = e.y; sl[2] = e.z; sl[3] = e.w;
      sh[0] = f.x; sh[1] = f.y; sh[2] = f.z; sh[3] = f.w;
    } else {
      const uint16_t* c16 = reinterpret_cast<const uint16_t*>(cos);
      const uint16_t* s16 = reinterpret_cast<const uint16_t*>(sin);
      const uint2 a = *reinterpret_cast<const uint2*>(c16 + cs);
      const uint2 bb = *reinterpret_cast<const uint2*>(c16 + cs + half);
      const uint2 e = *reinterpret_cast<const uint2*>(s16 + cs);
      const uint2 f = *reinterpret_cast<const uint2*>(s16 + cs + half);
      cl[0] = bf_lo(a.x); cl[1] = bf_hi(a.x); cl[2] = bf_lo(a.y); cl[3] = bf_hi(a.y);
      ch[0] = bf_lo(bb.x); ch[1] = bf_hi(bb.x); ch[2] = bf_lo(bb.y); ch[3] = bf_hi(bb.y);
      sl[0] = bf_lo(e.x); sl[1] = bf_hi(e.x); sl[2] = bf_lo(e.y); sl[3] = bf_hi(e.y);
      sh[0] = bf_lo(f.x); sh[1] = bf_hi(f.x); sh[2] = bf_lo(f.y); sh[3] = bf_hi(f.y);
    }
    const float lo[4] = {bf_lo(xl.x), bf_hi(xl.x), bf_lo(xl.y), bf_hi(xl.y)};
    const float hi[4] = {bf_lo(xh.x), bf_hi(xh.x), bf_lo(xh.y), bf_hi(xh.y)};
    float ol[4], oh[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      ol[e] = lo[e] * cl[e] + (-hi[e]) * sl[e];
      oh[e] = hi[e] * ch[e] + lo[e] * sh[e];
    }
    uint16_t* dst = (which ? k_out : q_out) + ((size_t)head * tokens + token) * dim;
    *reinterpret_cast<uint2*>(dst + c) = make_uint2(pack_bf2(ol[0], ol[1]), pack_bf2(ol[2], ol[3]));
    *reinterpret_cast<uint2*>(dst + c + half) =
        make_uint2(pack_bf2(oh[0], oh[1]), pack_bf2(oh[2], oh[3]));
  } else {
    u -= 2 * nqk;
    const int head = u / g8, c = 8 * (u - head * g8);
    *reinterpret_cast<uint4*>(v_out + ((size_t)head * tokens + token) * dim + c) =
        *reinterpret_cast<const uint4*>(row + (size_t)(2 * heads + head) * dim + c);
  }
}

// ------------------------------------------------------ vision attention
// Non-causal multi-head attention of the vision blocks on the matrix cores
// (v_mfma_f32_16x16x32_bf16), one workgroup per (64 query rows, head), four
// waves of 16 rows each; keys in blocks of 64 staged once in LDS for all four
// waves (double buffered, the next block loaded into registers while the
// current one is computed). Head dims D (D % 8 == 0, D <= 128) are zero-padded
// to 32 QT (QT = ceil(D / 32)) in Q's registers and K's LDS rows; O has
// OT = ceil(D / 16) tiles of 16 dims. Both are template parameters: a tile
// count known only at run time put O behind branches, and the compiler then
// copied the whole accumulator array at each one. Per block and
// wave: S = Q K^T (4 x QT MFMAs), online softmax in fp32 (DPP row
// reductions), P rounded to bf16 and written transposed to LDS, then O += P V
// with P and V reaching the MFMA through the gfx950 transpose read
// ds_read_b64_tr_b16 (the operand layouts and lane mapping of the causal
// prefill kernel). Queries only see keys of their own image: image i holds
// tokens [cu[i], cu[i+1]). Output rows go straight to [T, H*D], the layout the
// output projection reads.
typedef short q35_i16x4v __attribute__((ext_vector_type(4)));
Q35_DEV uint2 va_read_tr16(const uint16_t* p) {
  const q35_i16x4v v =
      __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) q35_i16x4v*)(p));
  return __builtin_bit_cast(uint2, v);
}
Q35_DEV q35_f32x4 va_mfma(const uint4 a, const uint4 b, q35_f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(q35_bf16x8, a),
                                                 __builtin_bit_cast(q35_bf16x8, b), c, 0, 0, 0);
}

typedef uint32_t va_u32x4 __attribute__((ext_vector_type(4)));
constexpr int kVaKeys = 64;    // keys per block
// K / V rows in LDS: 128 elements (16 chunks of 16 bytes) per key, chunk c of
// row r stored at chunk c ^ va_swz(r % 16), a 4 x 4 transpose of the row's
// low bits. The 16 rows of a K read (one chunk each) then sit on 16 distinct
// chunks, and the 8 rows {0-3, 8-11} (or {4-7, 12-15}) of a transposed V read
// (two chunks each) on 16 distinct chunks: both without bank conflicts.
constexpr int kVaRS = 128;
Q35_DEV int va_swz(int r15) { return ((r15 & 3) << 2) | ((r15 >> 2) & 3); }
constexpr int kVaRows = 64;    // query rows per workgroup
constexpr int kVaPt = 16 + 4;  // padded P^T row (16 query rows)

// Image bounds [start, end) of token t (cu: n + 1 ascending offsets; none:
// one image of T tokens).
Q35_DEV void va_segment(const int* cu, int n, int T, int t, int& s0, int& s1) {
  s0 = 0;
  s1 = T;
  if (!cu) return;
  for (int i = 0; i < n; ++i) {
    const int a = cu[i], b = cu[i + 1];
    if (t >= a && t < b) {
      s0 = a;
      s1 = b;
    }
  }
}

// One key block of one wave: S = Q K^T for its 16 rows x 64 keys, the online
// softmax in base 2 (c = scale * log2(e) folded into one FMA per score; m is
// kept in unscaled score units), bf16 P^T through the wave's LDS tile, then
// O += P V. MASK: some key of the block lies outside a row's image (keys
// outside get p = 0). lp holds this lane's partial row sums (the row sum is
// one 16-lane reduction at the end).
template <int QT, int OT, bool MASK>
Q35_DEV void va_block(const uint16_t* __restrict__ Ks, const uint16_t* __restrict__ Vs,
                      uint16_t* __restrict__ pt, const uint4 (&qa)[QT], q35_f32x4 (&o)[OT],
                      float (&m)[4], float (&lp)[4], int kb, const int (&s0)[4],
                      const int (&s1)[4], float c, int col, int kg, int te, int tq) {
  constexpr int RS = kVaRS;
  const int gk = va_swz(col);  // K rows 16 st + col
  q35_f32x4 s[4];
#pragma unroll
  for (int st = 0; st < 4; ++st) {
    s[st] = {0.f, 0.f, 0.f, 0.f};
    const uint16_t* krow = Ks + (16 * st + col) * RS;
#pragma unroll
    for (int t = 0; t < QT; ++t)
      s[st] = va_mfma(qa[t], *reinterpret_cast<const uint4*>(krow + 8 * ((kg + 4 * t) ^ gk)), s[st]);
  }
  float corr[4], p[4][4];
  bool moved = false;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float sv[4];
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      sv[st] = s[st][i];
      if (MASK) {
        const int key = kb + 16 * st + col;
        if (key < s0[i] || key >= s1[i]) sv[st] = -INFINITY;
      }
    }
    const float m_new =
        fmaxf(m[i], row16_max(fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3]))));
    // A row with no key of its image so far keeps m = -inf: offset 0 then.
    const float mc = (MASK && m_new == -INFINITY) ? 0.f : m_new * c;
    moved |= m_new != m[i];
    corr[i] = __builtin_amdgcn_exp2f(fmaf(m[i], c, -mc));
    float ps = 0.f;
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      p[st][i] = __builtin_amdgcn_exp2f(fmaf(sv[st], c, -mc));
      ps += p[st][i];
    }
    lp[i] = fmaf(lp[i], corr[i], ps);
    m[i] = m_new;
  }
#pragma unroll
  for (int st = 0; st < 4; ++st) {
    const int off = (16 * st + col) * kVaPt + 4 * kg;
    *reinterpret_cast<uint2*>(pt + off) =
        make_uint2(pack_bf2(p[st][0], p[st][1]), pack_bf2(p[st][2], p[st][3]));
  }
  // Rescale O only when some row's maximum moved (corr == 1 otherwise).
  if (__builtin_amdgcn_ballot_w64(moved)) {
#pragma unroll
    for (int d = 0; d < OT; ++d)
#pragma unroll
      for (int i = 0; i < 4; ++i) o[d][i] *= corr[i];
  }
  // O += P V over the two 32-key halves; the wave's own LDS stores above
  // complete before its reads (LDS operations of a wave execute in order).
#pragma unroll
  for (int half = 0; half < 2; ++half) {
    const uint16_t* pth = pt + 32 * half * kVaPt;
    const uint2 a0 = va_read_tr16(pth + (8 * kg + te) * kVaPt + 4 * tq);
    const uint2 a1 = va_read_tr16(pth + (8 * kg + 4 + te) * kVaPt + 4 * tq);
    const uint4 pa = make_uint4(a0.x, a0.y, a1.x, a1.y);
    // dims 16 d + 4 tq .. +3 of rows r0 and r0 + 4: chunk 2 d + tq / 2, half tq % 2
    const int r0 = 8 * kg + te;
    const int g0 = va_swz(r0 & 15), g1 = va_swz((r0 + 4) & 15);
    const uint16_t* v0 = Vs + (32 * half + r0) * RS + 4 * (tq & 1);
    const uint16_t* v1 = Vs + (32 * half + r0 + 4) * RS + 4 * (tq & 1);
#pragma unroll
    for (int d = 0; d < OT; ++d) {
      const int cv = 2 * d + (tq >> 1);
      const uint2 b0 = va_read_tr16(v0 + 8 * (cv ^ g0)), b1 = va_read_tr16(v1 + 8 * (cv ^ g1));
      o[d] = va_mfma(pa, make_uint4(b0.x, b0.y, b1.x, b1.y), o[d]);
    }
  }
}

template <int QT, int OT, int KS>
__global__ __launch_bounds__(256 * KS) void vision_attn_fa(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
    uint16_t* __restrict__ out, const int* __restrict__ cu, int nseg, int T, int H, int D,
    float scale) {
  static_assert(QT >= 1 && QT <= 4 && (OT == 2 * QT || OT == 2 * QT - 1), "head dim tiles");
  static_assert(KS == 1 || KS == 2, "key splits");
  constexpr int NT = 256 * KS;         // threads
  constexpr int SK = kVaKeys * KS;     // keys per stage (one 64-key block per wave group)
  constexpr int DP = 32 * QT;          // padded head dim
  constexpr int RS = kVaRS;            // LDS row stride (elements), swizzled chunks
  constexpr int NLD = (SK * DP / 8 + NT - 1) / NT;  // 16-byte K (and V) chunks per thread
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int rg = wid & 3;              // 16-row group of the tile
  const int kh = wid >> 2;             // which block of a stage this wave computes
  // Workgroup -> (query tile, head): with heads a multiple of 8 the tiles of a
  // head share one residue mod 8 (one XCD, whose L2 then serves the head's
  // K/V to all of them); otherwise tiles fastest.
  const int ntiles = (T + kVaRows - 1) / kVaRows;
  int h, tile;
  if (H % 8 == 0) {
    const int slot = (int)blockIdx.x >> 3;
    h = ((int)blockIdx.x & 7) + 8 * (slot / ntiles);
    tile = slot % ntiles;
  } else {
    h = (int)blockIdx.x / ntiles;
    tile = (int)blockIdx.x % ntiles;
  }
  const int qwg = tile * kVaRows;
  const int qw0 = qwg + 16 * rg;
  const int col = lane & 15, kg = lane >> 4;
  const int te = (lane & 15) >> 2, tq = lane & 3;
  const int ch = D / 8;            // 16-byte chunks per row
  const float c = scale * 1.4426950408889634f;
  const size_t hb = (size_t)h * T * D;

  // Key range of the workgroup: images are contiguous, so the union of its
  // rows' images is [image start of its first row, image end of its last).
  int kbeg, kend, tmp;
  va_segment(cu, nseg, T, qwg, kbeg, tmp);
  va_segment(cu, nseg, T, min(qwg + kVaRows, T) - 1, tmp, kend);
  const int nst = (kend - kbeg + SK - 1) / SK;
  int s0[4], s1[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) va_segment(cu, nseg, T, min(qw0 + 4 * kg + i, T - 1), s0[i], s1[i]);
  // Keys every row of the wave may see: [latest image start, earliest end).
  int w0, w1;
  va_segment(cu, nseg, T, min(qw0 + 15, T - 1), w0, tmp);
  va_segment(cu, nseg, T, min(qw0, T - 1), tmp, w1);

  uint4 qa[QT];
  {
    const uint16_t* qrow = q + hb + (size_t)min(qw0 + col, T - 1) * D;
#pragma unroll
    for (int t = 0; t < QT; ++t) {
      const int d0 = 32 * t + 8 * kg;
      qa[t] = d0 < D ? *reinterpret_cast<const uint4*>(qrow + d0) : make_uint4(0, 0, 0, 0);
    }
  }

  __shared__ alignas(16) uint16_t kv_s[2][2][SK * RS];         // [buf][K, V][key][dim]
  __shared__ alignas(16) uint16_t pt_s[4 * KS][kVaKeys * kVaPt];  // [wave][key][row]
  // Zero the padded dims [D, 128) of every K and V row once (whole 16-byte
  // chunks, at their swizzled places): they meet the zero-padded Q dims in S
  // (0 * finite) and only unused output dims in O.
  {
    const int pc = 16 - D / 8;
    for (int i = tid; i < 2 * 2 * SK * pc; i += NT) {
      const int row = i / pc, cc = D / 8 + i % pc;
      *reinterpret_cast<uint4*>(&(&kv_s[0][0][0])[row * RS + 8 * (cc ^ va_swz(row & 15))]) =
          make_uint4(0u, 0u, 0u, 0u);
    }
  }

  // This thread's 16-byte chunks of a stage: chunk gi = tid + NT j is key
  // row gi / ch, dims 8 * (gi % ch); only chunks gi < SK * ch exist.
  int lrow[NLD], lcol[NLD];
  bool lok[NLD];
#pragma unroll
  for (int j = 0; j < NLD; ++j) {
    const int gi = tid + NT * j;
    lok[j] = gi < SK * ch;
    lrow[j] = lok[j] ? gi / ch : 0;
    lcol[j] = lok[j] ? 8 * (gi % ch) : 0;
  }
  // Native vector registers (a uint4 struct copy between global memory, the
  // arrays and LDS stays a memory copy and put the arrays in scratch).
  va_u32x4 kr0[NLD], vr0[NLD], kr1[NLD], vr1[NLD];
  // Loads are clamped into the workgroup's key range and the head's rows (a
  // range that malformed image offsets left empty reads row 0, never used).
  auto va_load = [&](va_u32x4 (&kr)[NLD], va_u32x4 (&vr)[NLD], int st) {
#pragma unroll
    for (int j = 0; j < NLD; ++j) {
      const int key = max(min(min(kbeg + st * SK + lrow[j], kend - 1), T - 1), 0);
      const size_t off = hb + (size_t)key * D + lcol[j];
      kr[j] = *reinterpret_cast<const va_u32x4*>(k + off);
      vr[j] = *reinterpret_cast<const va_u32x4*>(v + off);
    }
  };
  auto va_store = [&](const va_u32x4 (&kr)[NLD], const va_u32x4 (&vr)[NLD], int buf) {
#pragma unroll
    for (int j = 0; j < NLD; ++j) {
      if (lok[j]) {
        const int off = lrow[j] * RS + 8 * ((lcol[j] >> 3) ^ va_swz(lrow[j] & 15));
        *reinterpret_cast<va_u32x4*>(&kv_s[buf][0][off]) = kr[j];
        *reinterpret_cast<va_u32x4*>(&kv_s[buf][1][off]) = vr[j];
      }
    }
  };
  // This wave's block of stage ST (keys kb..kb+63 of LDS buffer BUF); the
  // mask is skipped when the block lies inside every row's image.
#define VA_BLOCK(BUF, ST)                                                                 \
  do {                                                                                    \
    const int kb = kbeg + (ST) * SK + kVaKeys * kh;                                       \
    const uint16_t* Ks = kv_s[BUF][0] + kVaKeys * kh * RS;                                \
    const uint16_t* Vs = kv_s[BUF][1] + kVaKeys * kh * RS;                                \
    if (kb >= w0 && kb + kVaKeys <= w1)                                                   \
      va_block<QT, OT, false>(Ks, Vs, pt, qa, o, m, lp, kb, s0, s1, c, col, kg, te, tq);  \
    else                                                                                  \
      va_block<QT, OT, true>(Ks, Vs, pt, qa, o, m, lp, kb, s0, s1, c, col, kg, te, tq);   \
  } while (0)

  q35_f32x4 o[OT];
#pragma unroll
  for (int d = 0; d < OT; ++d) o[d] = {0.f, 0.f, 0.f, 0.f};
  float m[4], lp[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    m[i] = -INFINITY;
    lp[i] = 0.f;
  }
  uint16_t* pt = pt_s[wid];

  // Two register sets and two LDS buffers: at the top of an iteration LDS
  // buffer 0 holds stage st and set 1 stage st + 1; stage st + 2 is
  // requested into set 0 while st is computed. Loads past the last stage
  // reload it (unconditional: a conditional load here made the compiler keep
  // the chunks in scratch memory). The barriers order LDS only; the loads
  // in flight stay in flight across them.
  va_load(kr0, vr0, 0);
  va_store(kr0, vr0, 0);
  va_load(kr1, vr1, min(1, nst - 1));
  lds_barrier();
  int st = 0;
  for (; st + 1 < nst; st += 2) {
    va_load(kr0, vr0, min(st + 2, nst - 1));
    VA_BLOCK(0, st);
    va_store(kr1, vr1, 1);
    lds_barrier();
    va_load(kr1, vr1, min(st + 3, nst - 1));
    VA_BLOCK(1, st + 1);
    va_store(kr0, vr0, 0);
    lds_barrier();
  }
  if (st < nst) VA_BLOCK(0, st);
#undef VA_BLOCK

  if (KS == 2) {
    // The second wave group hands its (m, partial l, O) to the first through
    // LDS ([field][row group][lane] floats, conflict-free), which merges
    // them: both groups hold the same rows and dims lane for lane.
    constexpr int NF = 4 * OT + 8;
    static_assert(NF * 4 * 64 * 4 <= (int)sizeof(kv_s), "merge area");
    float* mg = reinterpret_cast<float*>(&kv_s[0][0][0]);
    lds_barrier();  // every wave is done with the K/V buffers
    if (kh == 1) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        mg[((i) * 4 + rg) * 64 + lane] = m[i];
        mg[((4 + i) * 4 + rg) * 64 + lane] = lp[i];
#pragma unroll
        for (int d = 0; d < OT; ++d) mg[((8 + 4 * d + i) * 4 + rg) * 64 + lane] = o[d][i];
      }
    }
    lds_barrier();
    if (kh == 1) return;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float m1 = mg[((i) * 4 + rg) * 64 + lane];
      const float l1 = mg[((4 + i) * 4 + rg) * 64 + lane];
      const float mm = fmaxf(m[i], m1);
      const float msub = mm == -INFINITY ? 0.f : mm * c;
      const float f0 = __builtin_amdgcn_exp2f(fmaf(m[i], c, -msub));
      const float f1 = __builtin_amdgcn_exp2f(fmaf(m1, c, -msub));
      lp[i] = lp[i] * f0 + l1 * f1;
#pragma unroll
      for (int d = 0; d < OT; ++d)
        o[d][i] = o[d][i] * f0 + mg[((8 + 4 * d + i) * 4 + rg) * 64 + lane] * f1;
    }
  }
  const size_t ostride = (size_t)H * D;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float l = row16_sum(lp[i]);
    const int r = qw0 + 4 * kg + i;
    if (r < T) {
      const float inv = 1.0f / l;
      uint16_t* orow = out + (size_t)r * ostride + (size_t)h * D;
#pragma unroll
      for (int d = 0; d < OT; ++d) {
        const int dim = 16 * d + col;
        if (dim < D) orow[dim] = (uint16_t)f2bf(o[d][i] * inv);
      }
    }
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
  const uint16_t* ps = (const uint16_t*)packed;
  uint16_t *qs = (uint16_t*)q, *ks = (uint16_t*)k, *vs = (uint16_t*)v;
  if (dim % 8 == 0 && q35_aligned16(packed) && q35_aligned16(cos) && q35_aligned16(sin) &&
      q35_aligned16(q) && q35_aligned16(k) && q35_aligned16(v)) {
    const long long threads = (long long)tokens * (2 * heads * (dim / 8) + heads * (dim / 8));
    const unsigned grid = (unsigned)((threads + 255) / 256);
    if (cs_f32)
      vision_qkv_rope_vec<true><<<grid, 256, 0, stream>>>(ps, cos, sin, qs, ks, vs, tokens, heads, dim);
    else
      vision_qkv_rope_vec<false><<<grid, 256, 0, stream>>>(ps, cos, sin, qs, ks, vs, tokens, heads, dim);
  } else {
    const long long waves = (long long)tokens * heads;
    const unsigned grid = (unsigned)((waves + kRowsPerBlock - 1) / kRowsPerBlock);
    vision_qkv_rope_rows<<<grid, 256, 0, stream>>>(ps, cos, sin, cs_f32, qs, ks, vs, tokens, heads,
                                                  dim);
  }
  return q35_last_error();
}

int q35_vision_attention(const void* q, const void* k, const void* v, void* out,
                         const void* cu_seqlens, int n_images, int tokens, int heads, int dim,
                         float scale, hipStream_t stream) {
  Q35_CHECK_ARG(tokens >= 0 && heads > 0 && dim > 0 && dim % 8 == 0 && dim <= 128);
  Q35_CHECK_ARG(q && k && v && out && (!cu_seqlens || n_images > 0));
  Q35_CHECK_ARG(q35_aligned16(q) && q35_aligned16(k) && q35_aligned16(v));
  Q35_CHECK_ARG((long long)heads * tokens * dim < (1ll << 31));
  if (tokens == 0) return 0;
  const unsigned grid = (unsigned)((tokens + kVaRows - 1) / kVaRows) * (unsigned)heads;
  const int* cu = (const int*)cu_seqlens;
  const uint16_t *qs = (const uint16_t*)q, *ks = (const uint16_t*)k, *vs = (const uint16_t*)v;
  uint16_t* os = (uint16_t*)out;
  const int qt = (dim + 31) / 32, ot = (dim + 15) / 16;
#define VA_LAUNCH(QT_, OT_, KS_)                                                          \
  vision_attn_fa<QT_, OT_, KS_><<<grid, 256 * KS_, 0, stream>>>(qs, ks, vs, os, cu, n_images, \
                                                                tokens, heads, dim, scale)
  // Two key blocks per stage (8 waves, one workgroup per CU by LDS) while the
  // grid leaves CUs idle; one block (4 waves, two workgroups per CU) for
  // larger grids and for the 128-dim tiles, whose registers do not fit two
  // waves per SIMD.
  const bool split = grid < 512;
#define VA_PICK(QT_, OT_)        \
  if (split)                     \
    VA_LAUNCH(QT_, OT_, 2);      \
  else                           \
    VA_LAUNCH(QT_, OT_, 1);
  switch (qt * 8 + ot) {
    case 1 * 8 + 1: VA_PICK(1, 1); break;
    case 1 * 8 + 2: VA_PICK(1, 2); break;
    case 2 * 8 + 3: VA_PICK(2, 3); break;
    case 2 * 8 + 4: VA_PICK(2, 4); break;
    case 3 * 8 + 5: VA_PICK(3, 5); break;
    case 3 * 8 + 6: VA_PICK(3, 6); break;
    case 4 * 8 + 7: VA_LAUNCH(4, 7, 1); break;
    default: VA_LAUNCH(4, 8, 1); break;
  }
#undef VA_PICK
#undef VA_LAUNCH
  return q35_last_error();
}

}  // extern "C"
