// Memory-bound bf16 GEMV for batch-1 decode (M = 1), with fused prologues and
// epilogues, and the lm_head GEMV fused with a top-1 reduction.
//
//   y[n] = bf16( sum_k W[n, k] * x[k] )     W row-major [N, K] bf16, fp32 acc
//
// Work split: a workgroup of WV wave64s owns WV*R consecutive weight rows, one
// wave R rows. Lane l reads the 16-byte group k = c*512 + 8l of each of its
// rows for chunk c = 0..NCH-1, so every load instruction of a wave moves one
// contiguous 1 KiB segment of a row, and all R*NCH loads of a lane are in
// flight before the first is consumed. The activation vector is loaded once
// per workgroup (16-byte loads issued *before* the weight stream, so the
// in-order vmcnt lets the prologue run while weights are still arriving),
// transformed by the prologue and staged in LDS; the barrier between the
// prologue and the dot product orders LDS only, so the weight loads stay in
// flight across it. Row sums use the DPP wave reduction. Weights are read
// exactly once: bytes per launch = 2*N*K + activation + 2*N.
//
// Prologues:
//   RMSNORM : x = bf16(x * rsqrt(mean(x^2)+eps) * (1+w))          [kernels.py:24-53]
//   RESNORM : r' = bf16(r+u); x = RMSNorm(r'); block 0 stores r'  [kernels.py:56-112]
// Epilogues:
//   STORE   : y[n] = bf16(acc)                                    [F.linear, integration.py:185]
//   SWIGLU  : rows n and N+n of a packed [gate; up] weight:
//             y[n] = bf16(bf16(silu(bf16(g))) * bf16(u))          [kernels.py:183-263]
//   TOP1    : key = (ordered bf16(acc), inverted row); one max key per
//             workgroup into a candidate array                    [kernels.py:1093-1143]
//             (lm_head_top1_persist and the generic fallback)
#include <algorithm>
#include <mutex>

#include "q35_common.hpp"

namespace {

enum { PRO_NONE = 0, PRO_RMSNORM = 1, PRO_RESNORM = 2, PRO_GATEDNORM = 3 };
enum { EPI_STORE = 0, EPI_SWIGLU = 1, EPI_TOP1 = 2, EPI_CONV = 3 };

struct GemvArgs {
  const uint16_t* W;    // [rows_total, K]
  const uint16_t* x;    // activation (residual for RESNORM, core for GATEDNORM)
  const uint16_t* u;    // update (RESNORM) or gate z (GATEDNORM)
  const void* nw;       // norm weight
  uint16_t* r_out;      // RESNORM: r' written by block 0 (may be null)
  uint16_t* xn_out;     // normalised activation written by block 0 (may be null)
  uint16_t* y;          // output [N]
  unsigned long long* cand;  // TOP1: one key per workgroup
  int N;                // output elements (TOP1: rows)
  int K;
  int nw_f32;
  float eps;
  // EPI_CONV: rows n < conv_channels also run the depthwise conv update.
  const uint16_t* conv_w;  // [conv_channels, conv_kw]
  uint16_t* conv_state;    // [conv_channels, conv_kw], in place
  uint16_t* conv_out;      // [conv_channels]
  int conv_channels;
  int conv_kw;
  // Optional row gather: x is row *x_row (clamped to [0, x_rows)) of a
  // [x_rows, K] table (the token embedding); RMSNORM then also stores the raw
  // row to r_out (the residual stream).
  const long long* x_row;
  int x_rows;
  // int8 weights (W is int8 [rows_total, K]): per-channel scales; optional
  // int32 accumulators [N] (SwiGLU: [2N]) and the quantised activation row
  // and its scale, written by block 0.
  const float* s_w;
  int* acc_out;
  int8_t* xq_out;
  float* sx_out;
};

// Gated RMSNorm (reference kernels.py:115-155) runs over heads of this width.
constexpr int kGatedHead = 128;

// 8 norm weights from the preloaded groups: fp32 (two 16-byte groups) or bf16 (one).
Q35_DEV void nw8_from(const GemvArgs& a, const uint4 lo, const uint4 hi, float* w) {
  if (a.nw_f32) {
    w[0] = __uint_as_float(lo.x); w[1] = __uint_as_float(lo.y);
    w[2] = __uint_as_float(lo.z); w[3] = __uint_as_float(lo.w);
    w[4] = __uint_as_float(hi.x); w[5] = __uint_as_float(hi.y);
    w[6] = __uint_as_float(hi.z); w[7] = __uint_as_float(hi.w);
  } else {
    unpack8(lo, w);
  }
}

template <int WV, int R, int NCH, int PRO, int EPI, bool I8>
__global__ __launch_bounds__(WV * 64) void gemv_fused(const GemvArgs a) {
  constexpr int NT = WV * 64;
  constexpr int NV = NCH * (I8 ? 128 : 64);     // 8-element activation groups
  constexpr int PER = (NV + NT - 1) / NT;       // groups per thread
  constexpr int P = EPI == EPI_SWIGLU ? R / 2 : R;  // outputs per wave
  static_assert(NV % NT == 0 || NT % NV == 0, "activation groups must tile the workgroup");
  static_assert(EPI != EPI_TOP1, "the lm_head top-1 runs in lm_head_top1_persist");
  __shared__ uint4 xs[I8 ? 1 : NV];             // bf16 activation (8 per group)
  __shared__ uint2 xq_s[I8 ? NV : 1];           // int8 activation (8 per group)
  __shared__ float red[WV], redm[WV];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wid = tid >> 6;
  const int n0 = (blockIdx.x * WV + wid) * P;
  const bool writer = blockIdx.x == 0;
  // HALF: a gated-norm prologue on a workgroup of twice as many threads as
  // 8-element groups; each thread takes half a group (4 elements), so the
  // prologue's per-thread arithmetic, which sits between the activation
  // loads and the first dot product, is halved.
  constexpr bool HALF = PRO == PRO_GATEDNORM && NT == 2 * NV;
  // Threads past NV (when the workgroup is wider than the vector) own no
  // activation group; the test is uniform per wave (NV is a multiple of 64).
  const bool act = HALF || NV % NT == 0 || tid < NV;

  // 1. activation, update and norm-weight loads, issued before the weight
  //    stream so that the in-order vmcnt lets the prologue start while the
  //    weights are still in flight. No loads below are predicated: predicated
  //    loads split the code into branches and force a full vmcnt(0) wait.
  const uint16_t* xsrc = a.x;
  if (a.x_row) {
    long long r = a.x_row[0];
    r = r < 0 ? 0 : (r >= a.x_rows ? a.x_rows - 1 : r);
    xsrc += (size_t)r * a.K;
  }
  uint4 xa[PER], ua[PER], wa[PER], wb[PER];
  if constexpr (HALF) {
    // element offset of the thread's half group
    const int e0 = tid * 4;
    const uint2 xv = *reinterpret_cast<const uint2*>(xsrc + e0);
    const uint2 uv = *reinterpret_cast<const uint2*>(a.u + e0);
    xa[0] = make_uint4(xv.x, xv.y, 0u, 0u);
    ua[0] = make_uint4(uv.x, uv.y, 0u, 0u);
    const int kn = e0 % kGatedHead;
    if (a.nw_f32) {
      wa[0] = *reinterpret_cast<const uint4*>(reinterpret_cast<const float*>(a.nw) + kn);
    } else {
      const uint2 wv = *reinterpret_cast<const uint2*>(reinterpret_cast<const uint16_t*>(a.nw) + kn);
      wa[0] = make_uint4(wv.x, wv.y, 0u, 0u);
    }
  } else
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int i = act ? tid + j * NT : 0;
    xa[j] = *reinterpret_cast<const uint4*>(xsrc + i * 8);
    if (PRO == PRO_RESNORM || PRO == PRO_GATEDNORM)
      ua[j] = *reinterpret_cast<const uint4*>(a.u + i * 8);
    if (PRO != PRO_NONE) {
      const int kn = PRO == PRO_GATEDNORM ? (i * 8) % kGatedHead : i * 8;
      if (a.nw_f32) {
        wa[j] = *reinterpret_cast<const uint4*>(reinterpret_cast<const float*>(a.nw) + kn);
        wb[j] = *reinterpret_cast<const uint4*>(reinterpret_cast<const float*>(a.nw) + kn + 4);
      } else {
        wa[j] = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(a.nw) + kn);
      }
    }
  }
  // EPI_CONV with width-4 filters: the lane's conv state and taps (4 bf16
  // each, one 8-byte load) are requested with the activation, so the
  // epilogue's conv update has no memory round trip; without conv channels or
  // for other widths the (unused) loads read the activation instead.
  uint2 cst = make_uint2(0u, 0u), cwt = make_uint2(0u, 0u);
  if (EPI == EPI_CONV) {
    const bool fast = a.conv_channels > 0 && a.conv_kw == 4;
    const int nc = max(min(n0 + (lane < P ? lane : 0), a.conv_channels - 1), 0);
    cst = *reinterpret_cast<const uint2*>(fast ? a.conv_state + (size_t)nc * 4 : a.x);
    cwt = *reinterpret_cast<const uint2*>(fast ? a.conv_w + (size_t)nc * 4 : a.x);
  }
  // int8 weights: the per-channel scales of the lane's output rows.
  float sw_g = 0.f, sw_u = 0.f;
  if (I8) {
    const int n = min(n0 + (lane < P ? lane : 0), a.N - 1);
    sw_g = a.s_w[n];
    if (EPI == EPI_SWIGLU) sw_u = a.s_w[a.N + n];
  }

  // 2. weight stream, 16 bytes per lane per 1 KiB chunk of a row: rows past
  //    the end read row 0 (valid memory) and are never stored.
  int rows[R];
  if (EPI == EPI_SWIGLU) {
#pragma unroll
    for (int i = 0; i < P; ++i) {
      const bool ok = n0 + i < a.N;
      rows[i] = ok ? n0 + i : 0;
      rows[P + i] = ok ? a.N + n0 + i : 0;
    }
  } else {
#pragma unroll
    for (int i = 0; i < R; ++i) rows[i] = n0 + i < a.N ? n0 + i : 0;
  }
  const size_t row_bytes = (size_t)a.K * (I8 ? 1 : 2);
  uint4 w[R][NCH];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const uint8_t* wrow = reinterpret_cast<const uint8_t*>(a.W) + (size_t)rows[r] * row_bytes + lane * 16;
#pragma unroll
    for (int c = 0; c < NCH; ++c) w[r][c] = ld_stream16(wrow + c * 1024);
  }

  if (PRO == PRO_RMSNORM && writer && a.r_out && act) {
#pragma unroll
    for (int j = 0; j < PER; ++j) *reinterpret_cast<uint4*>(a.r_out + (tid + j * NT) * 8) = xa[j];
  }

  // 3. prologue: the activation values of the thread's groups (0 for idle
  //    threads); int8 weights need them rounded to bf16 before quantising.
  float o[PER][8];
  if (PRO == PRO_NONE) {
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      unpack8(xa[j], o[j]);
#pragma unroll
      for (int e = 0; e < 8; ++e) o[j][e] = act ? o[j][e] : 0.f;
    }
  } else if (HALF) {
    // Thread t holds elements 4t..4t+3: a 128-wide head is 32 consecutive
    // lanes (two DPP rows, joined by the lane ^ 16 swizzle).
    const float s4[4] = {bf_lo(xa[0].x), bf_hi(xa[0].x), bf_lo(xa[0].y), bf_hi(xa[0].y)};
    const float z4[4] = {bf_lo(ua[0].x), bf_hi(ua[0].x), bf_lo(ua[0].y), bf_hi(ua[0].y)};
    float wn[4];
    if (a.nw_f32) {
      wn[0] = __uint_as_float(wa[0].x); wn[1] = __uint_as_float(wa[0].y);
      wn[2] = __uint_as_float(wa[0].z); wn[3] = __uint_as_float(wa[0].w);
    } else {
      wn[0] = bf_lo(wa[0].x); wn[1] = bf_hi(wa[0].x); wn[2] = bf_lo(wa[0].y); wn[3] = bf_hi(wa[0].y);
    }
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) ss += s4[e] * s4[e];
    ss = row16_sum(ss);
    ss += swz_xor16_f(ss);
    const float inv = rsqrt_cr(ss * (1.0f / (float)kGatedHead) + a.eps);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float nb = round_bf(s4[e] * inv);
      const float weighted = round_bf(nb * round_bf(wn[e]));
      const float v = weighted * silu_fast(z4[e]);
      o[0][e] = I8 ? round_bf(v) : v;
      o[0][e + 4] = 0.f;
    }
  } else if (PRO == PRO_GATEDNORM) {
    // Group i holds elements 8i..8i+7, so head = i/16: the 16 groups of a head
    // sit on the 16 lanes of one DPP row (NT is a multiple of 16).
    static_assert(NT % 16 == 0, "gated norm needs whole heads per row");
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      float s[8], z[8], wn[8];
      unpack8(xa[j], s);
      unpack8(ua[j], z);
      float ss = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) ss += s[e] * s[e];
      ss = row16_sum(ss);
      // (the mean over the 128-wide head: an exact scaling by 2^-7)
      const float inv = rsqrt_cr(ss * (1.0f / (float)kGatedHead) + a.eps);
      nw8_from(a, wa[j], wb[j], wn);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float nb = round_bf(s[e] * inv);
        const float weighted = round_bf(nb * round_bf(wn[e]));
        const float v = weighted * silu_fast(z[e]);
        o[j][e] = act ? (I8 ? round_bf(v) : v) : 0.f;
      }
    }
  } else {
    float s[PER][8];
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      unpack8(xa[j], s[j]);
      if (PRO == PRO_RESNORM) {
        float b[8];
        unpack8(ua[j], b);
#pragma unroll
        for (int e = 0; e < 8; ++e) s[j][e] = round_bf(s[j][e] + b[e]);
        const int i = tid + j * NT;
        if (writer && a.r_out && act) *reinterpret_cast<uint4*>(a.r_out + i * 8) = pack8(s[j]);
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) ss += s[j][e] * s[j][e];
    }
    if (!act) ss = 0.f;  // idle threads loaded group 0; keep it out of the sum
    ss = wave_sum(ss);
    if (lane == 0) red[wid] = ss;
    lds_barrier();
    float tot = 0.f;
#pragma unroll
    for (int v = 0; v < WV; ++v) tot += red[v];
    const float inv = rsqrt_cr(tot / (float)a.K + a.eps);
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      float wn[8];
      nw8_from(a, wa[j], wb[j], wn);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float v = s[j][e] * inv * (1.0f + wn[e]);
        o[j][e] = act ? (I8 ? round_bf(v) : v) : 0.f;
      }
    }
  }
  if (PRO != PRO_NONE && writer && a.xn_out && act) {
    if constexpr (HALF) {
      *reinterpret_cast<uint2*>(a.xn_out + tid * 4) =
          make_uint2(pack_bf2(o[0][0], o[0][1]), pack_bf2(o[0][2], o[0][3]));
    } else {
#pragma unroll
      for (int j = 0; j < PER; ++j) *reinterpret_cast<uint4*>(a.xn_out + (tid + j * NT) * 8) = pack8(o[j]);
    }
  }

  // 4. stage the activation in LDS: bf16, or (int8 weights) per-token int8
  //    with s_x = absmax/127, q = sat(rint(x * 127/absmax)) over the whole row.
  float sx = 0.f;
  if (HALF && !I8) {
    reinterpret_cast<uint2*>(xs)[tid] = make_uint2(pack_bf2(o[0][0], o[0][1]), pack_bf2(o[0][2], o[0][3]));
  } else if (!I8) {
#pragma unroll
    for (int j = 0; j < PER; ++j)
      if (act) xs[tid + j * NT] = pack8(o[j]);
  } else {
    float mx = 0.f;
#pragma unroll
    for (int j = 0; j < PER; ++j)
#pragma unroll
      for (int e = 0; e < 8; ++e) mx = fmaxf(mx, fabsf(o[j][e]));
    mx = wave_max(mx);
    if (lane == 0) redm[wid] = mx;
    lds_barrier();
    mx = redm[0];
#pragma unroll
    for (int v = 1; v < WV; ++v) mx = fmaxf(mx, redm[v]);
    const float inv = 127.0f / mx;
    sx = mx / 127.0f;
    if constexpr (HALF) {
      // the thread's 4 elements: one 32-bit word of the int8 row
      const uint32_t v = quant4_i8(o[0][0], o[0][1], o[0][2], o[0][3], inv);
      reinterpret_cast<uint32_t*>(xq_s)[tid] = v;
      if (writer && a.xq_out) *reinterpret_cast<uint32_t*>(a.xq_out + tid * 4) = v;
    } else {
#pragma unroll
      for (int j = 0; j < PER; ++j) {
        const int i = tid + j * NT;
        const uint2 v = quant8_i8(o[j], inv);
        if (act) {
          xq_s[i] = v;
          if (writer && a.xq_out) *reinterpret_cast<uint2*>(a.xq_out + i * 8) = v;
        }
      }
    }
    if (writer && tid == 0 && a.sx_out) a.sx_out[0] = sx;
  }
  lds_barrier();

  // 5. dot products: fp32 FMA on bf16 pairs, or exact int32 dot4 on int8
  //    (then acc = float(acc_i32) * s_x; the row scale s_w follows per lane).
  float acc[R];
  int iacc[R];
  if (!I8) {
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.f;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      float xf[8];
      unpack8(xs[c * 64 + lane], xf);
#pragma unroll
      for (int r = 0; r < R; ++r) {
        float wf[8];
        unpack8(w[r][c], wf);
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[r] = fmaf(wf[e], xf[e], acc[r]);
      }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = wave_sum(acc[r]);
  } else {
#pragma unroll
    for (int r = 0; r < R; ++r) iacc[r] = 0;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      const uint4 xv = reinterpret_cast<const uint4*>(xq_s)[c * 64 + lane];
#pragma unroll
      for (int r = 0; r < R; ++r) iacc[r] = dot16_i8(w[r][c], xv, iacc[r]);
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
      iacc[r] = wave_sum_i32(iacc[r]);
      acc[r] = (float)iacc[r] * sx;
    }
  }

  // 6. epilogue.
  if (lane < P && n0 + lane < a.N) {
    const int n = n0 + lane;
    float v;
    if (EPI == EPI_STORE || EPI == EPI_CONV) {
      v = acc[0];
#pragma unroll
      for (int r = 1; r < R; ++r) v = lane == r ? acc[r] : v;
      if (I8) {
        v *= sw_g;
        if (a.acc_out) {
          int iv = iacc[0];
#pragma unroll
          for (int r = 1; r < R; ++r) iv = lane == r ? iacc[r] : iv;
          a.acc_out[n] = iv;
        }
      }
      if (EPI == EPI_CONV) {
        const uint32_t yb = f2bf(v);
        if (n < a.conv_channels) {
          float c;
          if (a.conv_kw == 4) {
            // window (state[1..3], y), taps oldest first, as conv_update_channel
            float cacc = fmaf(bf_hi(cst.x), bf_lo(cwt.x), 0.f);
            cacc = fmaf(bf_lo(cst.y), bf_hi(cwt.x), cacc);
            cacc = fmaf(bf_hi(cst.y), bf_lo(cwt.y), cacc);
            cacc = fmaf(bf2f(yb), bf_hi(cwt.y), cacc);
            *reinterpret_cast<uint2*>(a.conv_state + (size_t)n * 4) =
                make_uint2((cst.x >> 16) | (cst.y << 16), (cst.y >> 16) | (yb << 16));
            c = round_bf(silu_f(round_bf(cacc)));
          } else {
            c = conv_update_channel(a.conv_state + (size_t)n * a.conv_kw,
                                    a.conv_w + (size_t)n * a.conv_kw, yb, a.conv_kw);
          }
          a.conv_out[n] = (uint16_t)f2bf(c);
        }
      }
    } else {
      float g = acc[0], up = acc[P];
#pragma unroll
      for (int i = 1; i < P; ++i) {
        g = lane == i ? acc[i] : g;
        up = lane == i ? acc[P + i] : up;
      }
      if (I8) {
        g *= sw_g;
        up *= sw_u;
        if (a.acc_out) {
          int ig = iacc[0], iu = iacc[P];
#pragma unroll
          for (int i = 1; i < P; ++i) {
            ig = lane == i ? iacc[i] : ig;
            iu = lane == i ? iacc[P + i] : iu;
          }
          a.acc_out[n] = ig;
          a.acc_out[a.N + n] = iu;
        }
      }
      v = round_bf(silu_f(round_bf(g))) * round_bf(up);
    }
    a.y[n] = (uint16_t)f2bf(v);
  }
}

// Generic fallback for any K and unaligned pointers: one wave per output,
// scalar lane-strided loads. Used by small test shapes only.
template <int PRO, int EPI>
__global__ __launch_bounds__(256) void gemv_bf16_generic(const GemvArgs a) {
  const int lane = threadIdx.x & 63;
  const int wid = threadIdx.x >> 6;
  const int n = blockIdx.x * 4 + wid;
  const bool writer = blockIdx.x == 0 && wid == 0;
  __shared__ unsigned long long best_s[4];
  float inv = 1.f;
  if (PRO != PRO_NONE) {
    float ss = 0.f;
    for (int k = lane; k < a.K; k += 64) {
      float s = bf2f(a.x[k]);
      if (PRO == PRO_RESNORM) s = round_bf(s + bf2f(a.u[k]));
      ss += s * s;
    }
    inv = rsqrt_cr(wave_sum(ss) / (float)a.K + a.eps);
  }
  auto xval = [&](int k) -> float {
    if (PRO == PRO_NONE) return bf2f(a.x[k]);
    float s = bf2f(a.x[k]);
    if (PRO == PRO_RESNORM) s = round_bf(s + bf2f(a.u[k]));
    const float wk = a.nw_f32 ? reinterpret_cast<const float*>(a.nw)[k]
                              : bf2f(reinterpret_cast<const uint16_t*>(a.nw)[k]);
    return round_bf(s * inv * (1.0f + wk));
  };
  if (writer && PRO != PRO_NONE) {
    for (int k = lane; k < a.K; k += 64) {
      if (PRO == PRO_RESNORM && a.r_out) a.r_out[k] = (uint16_t)f2bf(bf2f(a.x[k]) + bf2f(a.u[k]));
      if (a.xn_out) a.xn_out[k] = (uint16_t)f2bf(xval(k));
    }
  }
  float g = 0.f, up = 0.f;
  if (n < a.N) {
    for (int k = lane; k < a.K; k += 64) {
      const float xk = xval(k);
      g = fmaf(bf2f(a.W[(size_t)n * a.K + k]), xk, g);
      if (EPI == EPI_SWIGLU) up = fmaf(bf2f(a.W[(size_t)(a.N + n) * a.K + k]), xk, up);
    }
  }
  g = wave_sum(g);
  if (EPI == EPI_SWIGLU) up = wave_sum(up);
  if (EPI == EPI_TOP1) {
    if (lane == 0) best_s[wid] = n < a.N ? top1_key(round_bf(g), (uint32_t)n) : 0ull;
    __syncthreads();
    if (threadIdx.x == 0) {
      uint64_t b = best_s[0];
      for (int i = 1; i < 4; ++i) b = u64_max(b, best_s[i]);
      a.cand[blockIdx.x] = b;
    }
    return;
  }
  if (lane == 0 && n < a.N) {
    if (EPI == EPI_STORE || EPI == EPI_CONV) {
      a.y[n] = (uint16_t)f2bf(g);
      if (EPI == EPI_CONV && n < a.conv_channels) {
        const float c = conv_update_channel(a.conv_state + (size_t)n * a.conv_kw,
                                            a.conv_w + (size_t)n * a.conv_kw, f2bf(g), a.conv_kw);
        a.conv_out[n] = (uint16_t)f2bf(c);
      }
    } else {
      a.y[n] = (uint16_t)f2bf(round_bf(silu_f(round_bf(g))) * round_bf(up));
    }
  }
}

// out[0] = the index of the largest candidate key; `mirror` (may be null)
// receives the same index with a system-scope store (a second destination
// the caller reads, e.g. the device address of pinned host memory that a
// host loop polls); every advance[i] += 1 after.
__global__ __launch_bounds__(1024) void top1_final(const unsigned long long* __restrict__ cand,
                                                   int n, long long* out, long long* mirror,
                                                   long long* advance, int n_advance) {
  __shared__ unsigned long long s[16];
  uint64_t b = 0;
#pragma unroll 8
  for (int i = threadIdx.x; i < n; i += 1024) b = u64_max(b, cand[i]);
  b = wave_max_u64(b);
  if ((threadIdx.x & 63) == 0) s[threadIdx.x >> 6] = b;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint64_t m = s[0];
    for (int i = 1; i < 16; ++i) m = u64_max(m, s[i]);
    const long long token = (long long)top1_index(m);
    out[0] = token;
    // system scope: the store is written through to memory, so a host that
    // polls a pinned mirror sees it without a release after the kernel
    if (mirror) __hip_atomic_store(mirror, token, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    for (int i = 0; i < n_advance; ++i) advance[i] += 1;
  }
}

// lm_head GEMV + top-1 as a persistent grid (a few workgroups per CU): wave w
// of the grid takes row groups w, w + G, w + 2G, ... (G = waves in the grid,
// R rows per group) and keeps its best (value, index) key in a register.
// The hidden vector is held in registers (lane l owns k = c*512 + 8l), the
// next group's rows are requested before the current group is reduced, and
// no workgroup prologue repeats per row group; one key per workgroup goes to
// top1_final. Group indices past the wave's last are clamped to it (the
// repeated rows are re-reads of lines just fetched and change no key).
template <int WV, int R, int NCH>
__global__ __launch_bounds__(WV * 64) void lm_head_top1_persist(const GemvArgs a) {
  __shared__ unsigned long long best_s[WV];
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int G = gridDim.x * WV;
  const int wg = blockIdx.x * WV + wid;
  const int ngroups = (a.N + R - 1) / R;
  const int niter = wg < ngroups ? (ngroups - 1 - wg) / G + 1 : 0;
  float xf[NCH][8];
#pragma unroll
  for (int c = 0; c < NCH; ++c) unpack8(*reinterpret_cast<const uint4*>(a.x + c * 512 + 8 * lane), xf[c]);
  const size_t row_bytes = (size_t)a.K * 2;
  const uint8_t* wbase = reinterpret_cast<const uint8_t*>(a.W) + lane * 16;
  uint64_t best = 0;
  uint4 w0[R][NCH], w1[R][NCH];
#define Q35_LM_LOAD(WB, IT)                                                           \
  do {                                                                                \
    const int grp = wg + min((IT), max(niter - 1, 0)) * G;                            \
    _Pragma("unroll") for (int r = 0; r < R; ++r) {                                   \
      const int row = min(grp * R + r, a.N - 1);                                      \
      const uint8_t* wr = wbase + (size_t)row * row_bytes;                            \
      _Pragma("unroll") for (int c = 0; c < NCH; ++c) WB[r][c] = ld_stream16(wr + c * 1024); \
    }                                                                                 \
  } while (0)
#define Q35_LM_REDUCE(WB, IT)                                                         \
  do {                                                                                \
    const int grp = wg + (IT) * G;                                                    \
    _Pragma("unroll") for (int r = 0; r < R; ++r) {                                   \
      float acc = 0.f;                                                                \
      _Pragma("unroll") for (int c = 0; c < NCH; ++c) {                               \
        float wf[8];                                                                  \
        unpack8(WB[r][c], wf);                                                        \
        _Pragma("unroll") for (int e = 0; e < 8; ++e) acc = fmaf(wf[e], xf[c][e], acc); \
      }                                                                               \
      acc = wave_sum(acc);                                                            \
      const int row = grp * R + r;                                                    \
      if (row < a.N) best = u64_max(best, top1_key(round_bf(acc), (uint32_t)row));    \
    }                                                                                 \
  } while (0)
  if (niter > 0) {
    Q35_LM_LOAD(w0, 0);
    for (int it = 0; it < niter; it += 2) {
      Q35_LM_LOAD(w1, it + 1);
      Q35_LM_REDUCE(w0, it);
      if (it + 1 >= niter) break;
      Q35_LM_LOAD(w0, it + 2);
      Q35_LM_REDUCE(w1, it + 1);
    }
  }
#undef Q35_LM_LOAD
#undef Q35_LM_REDUCE
  if (lane == 0) best_s[wid] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint64_t b = best_s[0];
#pragma unroll
    for (int v = 1; v < WV; ++v) b = u64_max(b, best_s[v]);
    a.cand[blockIdx.x] = b;
  }
}

template <int WV, int R, int NCH, int PRO, int EPI, bool I8 = false>
long long launch_fast(const GemvArgs& a, hipStream_t stream) {
  constexpr int P = EPI == EPI_SWIGLU ? R / 2 : R;
  const long long blocks = (a.N + (long long)WV * P - 1) / ((long long)WV * P);
  gemv_fused<WV, R, NCH, PRO, EPI, I8><<<(unsigned)blocks, WV * 64, 0, stream>>>(a);
  return blocks;
}

// The tiled kernel reads 16-byte groups of W, x, u, the norm weight and the
// outputs, and whole 1 KiB chunks of each weight row.
bool fast_ok(const GemvArgs& a, int PRO, bool i8 = false) {
  return (a.K % (i8 ? 1024 : 512) == 0) && q35_aligned16(a.W) && q35_aligned16(a.x) &&
         ((PRO != PRO_RESNORM && PRO != PRO_GATEDNORM) || q35_aligned16(a.u)) &&
         q35_aligned16(a.r_out) && q35_aligned16(a.xn_out) && q35_aligned16(a.xq_out) &&
         (PRO == PRO_NONE || q35_aligned16(a.nw));
}

// Shape -> tile choice (waves per workgroup, rows per wave), measured on
// MI355X with rotating weights in a captured graph.
template <int PRO, int EPI>
int dispatch(const GemvArgs& a, hipStream_t stream) {
  if (fast_ok(a, PRO)) {
    const int nch = a.K / 512;
    if constexpr (EPI == EPI_SWIGLU) {
      if (nch == 4) { launch_fast<4, 2, 4, PRO, EPI>(a, stream); return q35_last_error(); }
      if (nch == 12) { launch_fast<4, 2, 12, PRO, EPI>(a, stream); return q35_last_error(); }
    } else {
      if (PRO == PRO_GATEDNORM && nch == 4) { launch_fast<8, 1, 4, PRO, EPI>(a, stream); return q35_last_error(); }
      if (nch == 4) { launch_fast<4, 2, 4, PRO, EPI>(a, stream); return q35_last_error(); }
      if (nch == 12) { launch_fast<4, 1, 12, PRO, EPI>(a, stream); return q35_last_error(); }
      if (nch == 1) { launch_fast<4, 2, 1, PRO, EPI>(a, stream); return q35_last_error(); }
      if (nch == 2) { launch_fast<4, 2, 2, PRO, EPI>(a, stream); return q35_last_error(); }
    }
  }
  if constexpr (PRO == PRO_GATEDNORM) {
    return (int)hipErrorInvalidValue;  // gated-norm prologue: fast path only
  } else {
    const unsigned blocks = (unsigned)((a.N + 3) / 4);
    gemv_bf16_generic<PRO, EPI><<<blocks > 0 ? blocks : 1, 256, 0, stream>>>(a);
    return q35_last_error();
  }
}

// int8 weights: tiled path only (K a multiple of 1024: 1, 2, 4 or 6 chunks).
// Tiles measured on MI355X with rotating weights in a captured graph: the
// norm-prologue GEMVs do best with 4 rows per wave (more bytes in flight
// behind the two workgroup reductions), the others with 2.
template <int PRO, int EPI>
int dispatch_i8(const GemvArgs& a, hipStream_t stream) {
  if (!fast_ok(a, PRO, true) || !a.s_w) return (int)hipErrorInvalidValue;
  const int nch = a.K / 1024;
  if constexpr (EPI == EPI_SWIGLU) {
    if (nch == 2) { launch_fast<4, 4, 2, PRO, EPI, true>(a, stream); return q35_last_error(); }
    if (nch == 6) { launch_fast<4, 2, 6, PRO, EPI, true>(a, stream); return q35_last_error(); }
  } else if constexpr (PRO == PRO_RMSNORM || PRO == PRO_RESNORM) {
    if (nch == 1) { launch_fast<4, 4, 1, PRO, EPI, true>(a, stream); return q35_last_error(); }
    if (nch == 2) { launch_fast<4, 4, 2, PRO, EPI, true>(a, stream); return q35_last_error(); }
    if (nch == 4) { launch_fast<4, 2, 4, PRO, EPI, true>(a, stream); return q35_last_error(); }
    if (nch == 6) { launch_fast<4, 2, 6, PRO, EPI, true>(a, stream); return q35_last_error(); }
  } else {
    if (nch == 1) { launch_fast<4, 4, 1, PRO, EPI, true>(a, stream); return q35_last_error(); }
    if (PRO == PRO_GATEDNORM && nch == 2) { launch_fast<8, 1, 2, PRO, EPI, true>(a, stream); return q35_last_error(); }
    if (nch == 2) { launch_fast<4, 2, 2, PRO, EPI, true>(a, stream); return q35_last_error(); }
    if (nch == 4) { launch_fast<4, 2, 4, PRO, EPI, true>(a, stream); return q35_last_error(); }
    if (nch == 6) { launch_fast<4, 2, 6, PRO, EPI, true>(a, stream); return q35_last_error(); }
  }
  return (int)hipErrorInvalidValue;
}

// Persistent lm_head grid, from a sweep (MI355X, 1.017 GB of weights): 4
// waves per workgroup, one row per group, 2 workgroups per CU (512 keys for
// top1_final); 143.6 us against 160.6 us for the one-workgroup-per-16-rows
// grid of gemv_fused. 6-8 waves per CU measured best; 4 per CU or 16 per CU
// lost 5-20 %.
constexpr int kLmWV = 4, kLmR = 1, kLmBlocksPerCU = 2;
static int lm_device_cus() {
  static int cus = 0;
  if (!cus) {
    int dev = 0;
    hipDeviceProp_t prop;
    if (hipGetDevice(&dev) == hipSuccess && hipGetDeviceProperties(&prop, dev) == hipSuccess)
      cus = prop.multiProcessorCount;
    if (cus <= 0) cus = 256;
  }
  return cus;
}

// Shared by q35_lm_head_top1 and q35_lm_head_top1_noalloc: the top-1 GEMV
// writes one candidate key per workgroup to `workspace`, top1_final reduces
// them. Every slot the final reduction reads is written by the same call, so
// the workspace needs no clearing.
int lm_head_top1_launch(const void* W, const void* x, int V, int K, void* workspace,
                        long long workspace_slots, void* out, void* mirror, void* advance,
                        int n_advance, hipStream_t stream) {
  GemvArgs a{(const uint16_t*)W, (const uint16_t*)x, nullptr, nullptr, nullptr, nullptr, nullptr,
             (unsigned long long*)workspace, V, K, 0, 0.f, nullptr, nullptr, nullptr, 0, 0,
             nullptr, 0};
  long long nc;
  if (K == 2048 && fast_ok(a, PRO_NONE)) {
    nc = std::min<long long>((long long)lm_device_cus() * kLmBlocksPerCU, workspace_slots);
    lm_head_top1_persist<kLmWV, kLmR, 4><<<(unsigned)nc, kLmWV * 64, 0, stream>>>(a);
  } else {
    nc = (V + 3) / 4;
    gemv_bf16_generic<PRO_NONE, EPI_TOP1><<<(unsigned)nc, 256, 0, stream>>>(a);
  }
  const int e = q35_last_error();
  if (e) return e;
  top1_final<<<1, 1024, 0, stream>>>((const unsigned long long*)workspace, (int)nc, (long long*)out,
                                     (long long*)mirror, (long long*)advance,
                                     advance ? n_advance : 0);
  return q35_last_error();
}

// ------------------------------------------------ screened exact lm_head top-1
// The lm_head GEMV reads 1 GB of bf16 weights per token to find one index.
// The screened form reads an int8 copy of them (half the bytes) and recomputes
// exactly only the rows that can still be the answer:
//   screen    Q_r = s_r * sum_i x_i q_ri in fp32, q_r = rint(w_r / s_r), s_r =
//             absmax_r / 127, and a bound eps_r >= |B_r - Q_r|, where B_r is
//             the bf16 logit the full kernel computes for row r (its fp32 sum
//             rounded to bf16). With e_r = w_r - s_r q_r, by Cauchy-Schwarz
//             |x.w_r - Q_r| <= |x| |e_r| + (fp32 error of the screen), the
//             full kernel's fp32 sum is within n u |x| |w_r| of x.w_r
//             (n = 2048 terms, u = 2^-24), and its bf16 rounding moves it by at
//             most 2^-8 of its magnitude; with c_r = |e_r| (1 + 2^-10) +
//             2 gamma (|w_r| + |e_r|), gamma = 2.5e-4 (twice n u):
//             eps_r = |x| c_r (1 + 2^-7) + 2^-7 |Q_r|, every term at least
//             twice what it covers. U_r = Q_r + eps_r >= B_r >= Q_r - eps_r.
//   rescore   L* = max_r (Q_r - eps_r) <= max_r B_r, so every row whose B_r is
//             the maximum has U_r >= L*; only rows with !(U_r < L*) (NaN rows
//             included) are recomputed, with the full kernel's arithmetic for
//             a row (same lane layout, fmaf order and wave reduction), and the
//             usual (value, lowest index) key picks among them. The result is
//             the full kernel's, bit for bit, whatever the weights; the number
//             of recomputed rows (a few percent for random N(0, 0.02) weights,
//             where the screen's bound is about one logit standard deviation)
//             only sets the cost.
constexpr float kScreenGamma = 2.5e-4f;

// One wave per row (4 per workgroup), K = 512 * NCH: lane l holds elements
// c*512 + 8l .. +7. Writes the int8 row (natural k order), s_r and c_r.
template <int NCH>
__global__ __launch_bounds__(256) void lm_screen_prep(const uint16_t* __restrict__ W,
                                                      int8_t* __restrict__ Wq,
                                                      float* __restrict__ s_out,
                                                      float* __restrict__ c_out, int V) {
  constexpr int K = 512 * NCH;
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= V) return;
  const uint16_t* wr = W + (size_t)row * K;
  float w[NCH][8];
#pragma unroll
  for (int c = 0; c < NCH; ++c) unpack8(*reinterpret_cast<const uint4*>(wr + c * 512 + 8 * lane), w[c]);
  float am = 0.f;
#pragma unroll
  for (int c = 0; c < NCH; ++c)
#pragma unroll
    for (int e = 0; e < 8; ++e) am = fmaxf(am, fabsf(w[c][e]));
  am = wave_max(am);
  const float sc = am > 0.f ? am / 127.f : 1.f;
  const float inv = am > 0.f ? 127.f / am : 0.f;
  float se = 0.f, sw = 0.f;
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    uint32_t lo = 0, hi = 0;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float q = fminf(fmaxf(rintf(w[c][e] * inv), -127.f), 127.f);
      const float d = w[c][e] - sc * q;
      se = fmaf(d, d, se);
      sw = fmaf(w[c][e], w[c][e], sw);
      const uint32_t b = (uint32_t)((int)q & 0xff);
      if (e < 4) lo |= b << (8 * e);
      else hi |= b << (8 * (e - 4));
    }
    *reinterpret_cast<uint2*>(Wq + (size_t)row * K + c * 512 + 8 * lane) = make_uint2(lo, hi);
  }
  se = wave_sum(se);
  sw = wave_sum(sw);
  if (lane == 0) {
    const float ne = sqrtf(se), nw = sqrtf(sw);
    s_out[row] = sc;
    c_out[row] = ne * (1.0f + 0x1p-10f) + 2.0f * kScreenGamma * (nw + ne);
  }
}

// The int8 screen as a persistent grid (the lm_head top-1 layout): wave w
// takes row groups w, w + G, ... of R rows, K = 1024 * NCH8; lane l holds x
// elements c*1024 + 16l .. +15 (the bytes of its 16-byte weight load); the
// next group's rows and their s_r, c_r are requested before the current group
// is reduced. Writes U_r and one max_r (Q_r - eps_r) per workgroup.
template <int WV, int R, int NCH8>
__global__ __launch_bounds__(WV * 64) void lm_head_screen(const int8_t* __restrict__ Wq,
                                                          const float* __restrict__ s_w,
                                                          const float* __restrict__ c_r,
                                                          const uint16_t* __restrict__ x, int V,
                                                          float* __restrict__ U,
                                                          float* __restrict__ lpart) {
  constexpr int K = 1024 * NCH8;
  __shared__ float best_s[WV];
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int G = gridDim.x * WV;
  const int wg = blockIdx.x * WV + wid;
  const int ngroups = (V + R - 1) / R;
  const int niter = wg < ngroups ? (ngroups - 1 - wg) / G + 1 : 0;
  float xf[NCH8][16];
  float nx2 = 0.f;
#pragma unroll
  for (int c = 0; c < NCH8; ++c) {
    unpack8(*reinterpret_cast<const uint4*>(x + c * 1024 + 16 * lane), xf[c]);
    unpack8(*reinterpret_cast<const uint4*>(x + c * 1024 + 16 * lane + 8), xf[c] + 8);
#pragma unroll
    for (int e = 0; e < 16; ++e) nx2 = fmaf(xf[c][e], xf[c][e], nx2);
  }
  const float nx = sqrtf(wave_sum(nx2)) * (1.0f + 0x1p-10f);
  float best = -INFINITY;
  uint4 q0[R][NCH8], q1[R][NCH8];
  float s0[R], s1[R], e0[R], e1[R];
#define Q35_SC_LOAD(QB, SB, EB, IT)                                                   \
  do {                                                                                \
    const int grp = wg + min((IT), max(niter - 1, 0)) * G;                            \
    _Pragma("unroll") for (int r = 0; r < R; ++r) {                                   \
      const int row = min(grp * R + r, V - 1);                                        \
      const int8_t* wr = Wq + (size_t)row * K + 16 * lane;                            \
      _Pragma("unroll") for (int c = 0; c < NCH8; ++c) QB[r][c] = ld_stream16(wr + c * 1024); \
      SB[r] = s_w[row];                                                               \
      EB[r] = c_r[row];                                                               \
    }                                                                                 \
  } while (0)
#define Q35_SC_REDUCE(QB, SB, EB, IT)                                                 \
  do {                                                                                \
    const int grp = wg + (IT) * G;                                                    \
    _Pragma("unroll") for (int r = 0; r < R; ++r) {                                   \
      float acc = 0.f;                                                                \
      _Pragma("unroll") for (int c = 0; c < NCH8; ++c) {                              \
        const uint32_t wd[4] = {QB[r][c].x, QB[r][c].y, QB[r][c].z, QB[r][c].w};      \
        _Pragma("unroll") for (int e = 0; e < 16; ++e) {                              \
          const float q = (float)(int)(int8_t)(wd[e >> 2] >> (8 * (e & 3)));          \
          acc = fmaf(q, xf[c][e], acc);                                               \
        }                                                                             \
      }                                                                               \
      acc = wave_sum(acc);                                                            \
      const int row = grp * R + r;                                                    \
      if (row < V) {                                                                  \
        const float qv = acc * SB[r];                                                 \
        const float eps = nx * EB[r] * (1.0f + 0x1p-7f) + 0x1p-7f * fabsf(qv);        \
        if (lane == 0) U[row] = qv + eps;                                             \
        best = fmaxf(best, qv - eps);                                                 \
      }                                                                               \
    }                                                                                 \
  } while (0)
  if (niter > 0) {
    Q35_SC_LOAD(q0, s0, e0, 0);
    for (int it = 0; it < niter; it += 2) {
      Q35_SC_LOAD(q1, s1, e1, it + 1);
      Q35_SC_REDUCE(q0, s0, e0, it);
      if (it + 1 >= niter) break;
      Q35_SC_LOAD(q0, s0, e0, it + 2);
      Q35_SC_REDUCE(q1, s1, e1, it + 1);
    }
  }
#undef Q35_SC_LOAD
#undef Q35_SC_REDUCE
  if (lane == 0) best_s[wid] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    float b = best_s[0];
#pragma unroll
    for (int v = 1; v < WV; ++v) b = fmaxf(b, best_s[v]);
    lpart[blockIdx.x] = b;
  }
}

// Exact recomputation of the rows the screen left: each wave takes a
// contiguous slice of rows, tests 64 at a time (!(U_r < L*)) and recomputes
// its candidates four at a time (missing ones repeat the last candidate, so
// the loads carry no branch) with lm_head_top1_persist's arithmetic for one
// row (K = 2048: lane l holds k = c*512 + 8l, fmaf in (c, e) order,
// wave_sum, bf16 rounding). One key per workgroup for top1_final.
template <int WV>
__global__ __launch_bounds__(WV * 64) void lm_head_rescore(const uint16_t* __restrict__ W,
                                                           const uint16_t* __restrict__ x,
                                                           const float* __restrict__ U,
                                                           const float* __restrict__ lpart,
                                                           int nparts, int V,
                                                           unsigned long long* __restrict__ cand,
                                                           unsigned* __restrict__ ncand) {
  constexpr int NCH = 4, K = 2048;
  __shared__ unsigned long long best_s[WV];
  __shared__ unsigned count_s[WV];
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  float xf[NCH][8];
#pragma unroll
  for (int c = 0; c < NCH; ++c) unpack8(*reinterpret_cast<const uint4*>(x + c * 512 + 8 * lane), xf[c]);
  float lstar = -INFINITY;
  for (int i = lane; i < nparts; i += 64) lstar = fmaxf(lstar, lpart[i]);
  lstar = wave_max(lstar);
  const int nw = gridDim.x * WV;
  const int w = blockIdx.x * WV + wid;
  const int per = (V + nw - 1) / nw;
  const int r0 = min(V, w * per), r1 = min(V, r0 + per);
  uint64_t best = 0;
  unsigned count = 0;  // rows this wave recomputes (wave-uniform)
  const uint8_t* wbase = reinterpret_cast<const uint8_t*>(W) + lane * 16;
  for (int base = r0; base < r1; base += 64) {
    const int row = base + lane;
    const bool is_cand = row < r1 && !(U[min(row, V - 1)] < lstar);
    uint64_t mask = __ballot(is_cand);
    count += (unsigned)__builtin_popcountll(mask);
    while (mask) {
      int rows[4];
      int last = base;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if (mask) {
          last = base + (int)__builtin_ctzll(mask);
          mask &= mask - 1;
        }
        rows[j] = last;
      }
      uint4 wv[4][NCH];
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int c = 0; c < NCH; ++c)
          wv[j][c] = ld_stream16(wbase + (size_t)rows[j] * K * 2 + c * 1024);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float acc = 0.f;
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
          float wf[8];
          unpack8(wv[j][c], wf);
#pragma unroll
          for (int e = 0; e < 8; ++e) acc = fmaf(wf[e], xf[c][e], acc);
        }
        acc = wave_sum(acc);
        best = u64_max(best, top1_key(round_bf(acc), (uint32_t)rows[j]));
      }
    }
  }
  if (lane == 0) {
    best_s[wid] = best;
    count_s[wid] = count;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    uint64_t b = best_s[0];
    unsigned n = count_s[0];
#pragma unroll
    for (int v = 1; v < WV; ++v) {
      b = u64_max(b, best_s[v]);
      n += count_s[v];
    }
    cand[blockIdx.x] = b;
    ncand[blockIdx.x] = n;  // every workgroup writes its slot on every call
  }
}

// Screen: one workgroup of 8 waves per CU, 2 rows per group (the fastest of
// 24 shapes of waves x rows x workgroups per CU over the 248320-row int8
// copy: 75.5 us against 79.1 for two 4-wave workgroups per CU). Rescore: two
// 4-wave workgroups per CU.
constexpr int kScWV = 4, kScScreenWV = 8, kScR = 2;
// Workspace of the screened top-1: U [V] floats, then per workgroup one
// float (max lower bound), one 64-bit key and the number of rows it
// recomputed (uint32), 256-byte aligned sections.
long long screened_parts() { return (long long)lm_device_cus() * kLmBlocksPerCU; }
long long align256(long long b) { return (b + 255) / 256 * 256; }
long long screened_bytes(int V) {
  const long long nb = screened_parts();
  return align256((long long)V * 4) + align256(nb * 4) + align256(nb * 8) + nb * 4;
}

// Scratch of q35_lm_head_top1_noalloc: the candidate keys of one top-1 call
// (512 slots for the persistent 2-workgroups-per-CU grid; the one-key-per-4-
// rows fallback grid needs (V + 3) / 4). It lives in the library's device
// memory, one copy per GPU the library runs on, held until the process ends.
// All calls on one GPU share it, so calls that overlap on one GPU race.
constexpr long long kTop1ScratchSlots = 65536;  // 512 KiB
}  // namespace
static __device__ __align__(256) unsigned long long scratch[kTop1ScratchSlots];
namespace {

// Device address of this GPU's copy of `scratch`, resolved once per
// device with that device current (the array's name is only a host-side
// stand-in; kernels must receive this address).
int top1_scratch(void** out) {
  constexpr int kMaxDevices = 64;
  static std::mutex mu;
  static void* addr[kMaxDevices] = {};
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= kMaxDevices) return (int)hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(mu);
  if (!addr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return (int)e;
    addr[dev] = p;
  }
  *out = addr[dev];
  return 0;
}

}  // namespace

extern "C" {

// y[N] = W[N,K] . xa[K]; prologue: 0 none, 1 rmsnorm(x), 2 residual add + rmsnorm,
// 3 gated rmsnorm of x (heads of 128) with gate u.
int q35_gemv_bf16(const void* W, const void* x, const void* u, const void* norm_w, int norm_w_f32,
                  float eps, void* residual_out, void* x_norm_out, void* y, int N, int K,
                  int prologue, hipStream_t stream) {
  Q35_CHECK_ARG(N > 0 && K > 0 && W && x && y);
  Q35_CHECK_ARG(prologue >= 0 && prologue <= 3);
  Q35_CHECK_ARG(prologue == 0 || norm_w);
  Q35_CHECK_ARG(prologue < 2 || u);
  Q35_CHECK_ARG(prologue != 3 || K % kGatedHead == 0);
  GemvArgs a{(const uint16_t*)W, (const uint16_t*)x, (const uint16_t*)u, norm_w,
             (uint16_t*)residual_out, (uint16_t*)x_norm_out, (uint16_t*)y, nullptr, N, K,
             norm_w_f32, eps, nullptr, nullptr, nullptr, 0, 0, nullptr, 0};
  if (prologue == 0) return dispatch<PRO_NONE, EPI_STORE>(a, stream);
  if (prologue == 1) return dispatch<PRO_RMSNORM, EPI_STORE>(a, stream);
  if (prologue == 2) return dispatch<PRO_RESNORM, EPI_STORE>(a, stream);
  return dispatch<PRO_GATEDNORM, EPI_STORE>(a, stream);
}

// As q35_gemv_bf16 (prologue 0-2), and rows n < conv_channels also run the
// single-token depthwise conv update on y[n]: conv_out[n] =
// bf16(silu(bf16(sum_t w[n,t] * window[t]))), window = (state[n,1:], y[n]),
// state shifted in place. One wave owns each row, so each conv channel and its
// state are touched by exactly one wave.
int q35_gemv_conv(const void* W, const void* x, const void* u, const void* norm_w, int norm_w_f32,
                  float eps, void* residual_out, void* y, int N, int K, int prologue,
                  const void* conv_w, void* conv_state, void* conv_out, int conv_channels,
                  int conv_kw, const void* x_row, int x_rows, hipStream_t stream) {
  Q35_CHECK_ARG(N > 0 && K > 0 && W && x && y);
  Q35_CHECK_ARG(prologue >= 0 && prologue <= 2);
  Q35_CHECK_ARG(prologue == 0 || norm_w);
  Q35_CHECK_ARG(prologue != 2 || u);
  Q35_CHECK_ARG(conv_channels >= 0 && conv_channels <= N && conv_kw > 0 && conv_kw <= 16);
  Q35_CHECK_ARG(conv_channels == 0 || (conv_w && conv_state && conv_out));
  Q35_CHECK_ARG(conv_channels == 0 || conv_kw != 4 || (q35_aligned8(conv_w) && q35_aligned8(conv_state)));
  Q35_CHECK_ARG(!x_row || (prologue == 1 && x_rows > 0));
  GemvArgs a{(const uint16_t*)W, (const uint16_t*)x, (const uint16_t*)u, norm_w,
             (uint16_t*)residual_out, nullptr, (uint16_t*)y, nullptr, N, K, norm_w_f32, eps,
             (const uint16_t*)conv_w, (uint16_t*)conv_state, (uint16_t*)conv_out, conv_channels,
             conv_kw, (const long long*)x_row, x_rows};
  if (x_row && !fast_ok(a, PRO_RMSNORM)) return (int)hipErrorInvalidValue;
  if (prologue == 0) return dispatch<PRO_NONE, EPI_CONV>(a, stream);
  if (prologue == 1) return dispatch<PRO_RMSNORM, EPI_CONV>(a, stream);
  return dispatch<PRO_RESNORM, EPI_CONV>(a, stream);
}

// y[N] = bf16(silu(bf16(W[n].x))) * bf16(W[N+n].x) with W = [gate; up] of shape [2N, K].
int q35_swiglu_gemv(const void* W, const void* x, const void* u, const void* norm_w,
                    int norm_w_f32, float eps, void* residual_out, void* x_norm_out, void* y,
                    int N, int K, int prologue, hipStream_t stream) {
  Q35_CHECK_ARG(N > 0 && K > 0 && W && x && y);
  Q35_CHECK_ARG(prologue >= 0 && prologue <= 2);
  Q35_CHECK_ARG(prologue == 0 || norm_w);
  Q35_CHECK_ARG(prologue != 2 || u);
  GemvArgs a{(const uint16_t*)W, (const uint16_t*)x, (const uint16_t*)u, norm_w,
             (uint16_t*)residual_out, (uint16_t*)x_norm_out, (uint16_t*)y, nullptr, N, K,
             norm_w_f32, eps, nullptr, nullptr, nullptr, 0, 0, nullptr, 0};
  if (prologue == 0) return dispatch<PRO_NONE, EPI_SWIGLU>(a, stream);
  if (prologue == 1) return dispatch<PRO_RMSNORM, EPI_SWIGLU>(a, stream);
  return dispatch<PRO_RESNORM, EPI_SWIGLU>(a, stream);
}

// int8 weights (A8W8): y[N] = bf16(float(Wq[N,K] . xq) * s_x * s_w[n]) with the
// activation (after the prologue, rounded to bf16) quantised per token inside
// every workgroup: s_x = absmax/127, xq = sat(rint(x * 127/absmax)). Prologues
// as q35_gemv_bf16. Optional outputs: acc_out int32 [N], xq_out int8 [K] and
// sx_out fp32 [1] (the quantised activation, written by block 0).
int q35_gemv_i8(const void* Wq, const void* s_w, const void* x, const void* u, const void* norm_w,
                int norm_w_f32, float eps, void* residual_out, void* x_norm_out, void* y,
                void* acc_out, void* xq_out, void* sx_out, int N, int K, int prologue,
                hipStream_t stream) {
  Q35_CHECK_ARG(N > 0 && K > 0 && Wq && s_w && x && y);
  Q35_CHECK_ARG(prologue >= 0 && prologue <= 3);
  Q35_CHECK_ARG(prologue == 0 || norm_w);
  Q35_CHECK_ARG(prologue < 2 || u);
  Q35_CHECK_ARG(prologue != 3 || K % kGatedHead == 0);
  GemvArgs a{(const uint16_t*)Wq, (const uint16_t*)x, (const uint16_t*)u, norm_w,
             (uint16_t*)residual_out, (uint16_t*)x_norm_out, (uint16_t*)y, nullptr, N, K,
             norm_w_f32, eps, nullptr, nullptr, nullptr, 0, 0, nullptr, 0,
             (const float*)s_w, (int*)acc_out, (int8_t*)xq_out, (float*)sx_out};
  if (prologue == 0) return dispatch_i8<PRO_NONE, EPI_STORE>(a, stream);
  if (prologue == 1) return dispatch_i8<PRO_RMSNORM, EPI_STORE>(a, stream);
  if (prologue == 2) return dispatch_i8<PRO_RESNORM, EPI_STORE>(a, stream);
  return dispatch_i8<PRO_GATEDNORM, EPI_STORE>(a, stream);
}

// q35_gemv_conv with int8 weights (quantisation as q35_gemv_i8).
int q35_gemv_i8_conv(const void* Wq, const void* s_w, const void* x, const void* u,
                     const void* norm_w, int norm_w_f32, float eps, void* residual_out, void* y,
                     int N, int K, int prologue, const void* conv_w, void* conv_state,
                     void* conv_out, int conv_channels, int conv_kw, const void* x_row, int x_rows,
                     hipStream_t stream) {
  Q35_CHECK_ARG(N > 0 && K > 0 && Wq && s_w && x && y);
  Q35_CHECK_ARG(prologue >= 0 && prologue <= 2);
  Q35_CHECK_ARG(prologue == 0 || norm_w);
  Q35_CHECK_ARG(prologue != 2 || u);
  Q35_CHECK_ARG(conv_channels >= 0 && conv_channels <= N && conv_kw > 0 && conv_kw <= 16);
  Q35_CHECK_ARG(conv_channels == 0 || (conv_w && conv_state && conv_out));
  Q35_CHECK_ARG(conv_channels == 0 || conv_kw != 4 || (q35_aligned8(conv_w) && q35_aligned8(conv_state)));
  Q35_CHECK_ARG(!x_row || (prologue == 1 && x_rows > 0));
  GemvArgs a{(const uint16_t*)Wq, (const uint16_t*)x, (const uint16_t*)u, norm_w,
             (uint16_t*)residual_out, nullptr, (uint16_t*)y, nullptr, N, K, norm_w_f32, eps,
             (const uint16_t*)conv_w, (uint16_t*)conv_state, (uint16_t*)conv_out, conv_channels,
             conv_kw, (const long long*)x_row, x_rows, (const float*)s_w, nullptr, nullptr,
             nullptr};
  if (prologue == 0) return dispatch_i8<PRO_NONE, EPI_CONV>(a, stream);
  if (prologue == 1) return dispatch_i8<PRO_RMSNORM, EPI_CONV>(a, stream);
  return dispatch_i8<PRO_RESNORM, EPI_CONV>(a, stream);
}

// q35_swiglu_gemv with int8 [gate; up] weights [2N, K] and scales [2N]: gate and
// up are dequantised to bf16 before the SwiGLU. acc_out (optional) int32 [2N].
int q35_swiglu_gemv_i8(const void* Wq, const void* s_w, const void* x, const void* u,
                       const void* norm_w, int norm_w_f32, float eps, void* residual_out,
                       void* x_norm_out, void* y, void* acc_out, int N, int K, int prologue,
                       hipStream_t stream) {
  Q35_CHECK_ARG(N > 0 && K > 0 && Wq && s_w && x && y);
  Q35_CHECK_ARG(prologue >= 0 && prologue <= 2);
  Q35_CHECK_ARG(prologue == 0 || norm_w);
  Q35_CHECK_ARG(prologue != 2 || u);
  GemvArgs a{(const uint16_t*)Wq, (const uint16_t*)x, (const uint16_t*)u, norm_w,
             (uint16_t*)residual_out, (uint16_t*)x_norm_out, (uint16_t*)y, nullptr, N, K,
             norm_w_f32, eps, nullptr, nullptr, nullptr, 0, 0, nullptr, 0,
             (const float*)s_w, (int*)acc_out, nullptr, nullptr};
  if (prologue == 0) return dispatch_i8<PRO_NONE, EPI_SWIGLU>(a, stream);
  if (prologue == 1) return dispatch_i8<PRO_RMSNORM, EPI_SWIGLU>(a, stream);
  return dispatch_i8<PRO_RESNORM, EPI_SWIGLU>(a, stream);
}

// Number of 64-bit candidate slots q35_lm_head_top1 needs in its workspace.
long long q35_lm_head_top1_workspace(int V, int K) {
  if (V <= 0 || K <= 0) return 0;
  return (V + 3) / 4;  // enough for the one-row-per-wave fallback as well
}

// out[0] (int64) = argmax_v bf16(W[v].x), lowest index on ties; mirror[0]
// (optional) the same.
int q35_lm_head_top1(const void* W, const void* x, int V, int K, void* workspace,
                     long long workspace_slots, void* out, void* mirror, void* advance,
                     int n_advance, hipStream_t stream) {
  Q35_CHECK_ARG(!advance || (n_advance >= 0 && n_advance <= 64));
  Q35_CHECK_ARG(V > 0 && K > 0 && W && x && workspace && out);
  Q35_CHECK_ARG(workspace_slots >= q35_lm_head_top1_workspace(V, K) && V < (1 << 30));
  Q35_CHECK_ARG(q35_aligned8(mirror));
  return lm_head_top1_launch(W, x, V, K, workspace, workspace_slots, out, mirror, advance,
                             n_advance, stream);
}

// The device address of pinned, device-mapped host memory (hipHostMalloc):
// *dev = where a kernel stores to reach `host`. Anything else (pageable host
// memory, device memory, null) returns hipErrorInvalidValue.
int q35_host_device_ptr(const void* host, void** dev) {
  Q35_CHECK_ARG(host && dev);
  *dev = nullptr;
  hipPointerAttribute_t attr{};
  if (hipPointerGetAttributes(&attr, host) != hipSuccess) {
    (void)hipGetLastError();  // an unregistered pointer leaves an error behind
    return (int)hipErrorInvalidValue;
  }
  if (attr.type != hipMemoryTypeHost || !attr.devicePointer) return (int)hipErrorInvalidValue;
  *dev = attr.devicePointer;
  return 0;
}

// Screen operands of an lm_head weight W [V, K] (bf16, K = 2048): the int8
// copy Wq [V, K], s [V] and c [V] fp32 (see lm_head_screen).
int q35_lm_head_screen_prep(const void* W, int V, int K, void* Wq, void* s, void* c,
                            hipStream_t stream) {
  Q35_CHECK_ARG(W && Wq && s && c && V > 0 && K == 2048 && V < (1 << 30));
  Q35_CHECK_ARG(q35_aligned16(W) && q35_aligned16(Wq));
  lm_screen_prep<4><<<(unsigned)((V + 3) / 4), 256, 0, stream>>>(
      (const uint16_t*)W, (int8_t*)Wq, (float*)s, (float*)c, V);
  return q35_last_error();
}

long long q35_lm_head_top1_screened_workspace(int V, int K) {
  if (V <= 0 || K != 2048) return 0;
  return screened_bytes(V);
}

// Byte offset and count of the per-workgroup recomputed-row counts (uint32)
// in a screened top-1 workspace for vocabulary V: offset in the return
// value, count in *n.
long long q35_lm_head_screened_counts(int V, int* n) {
  const long long nb = screened_parts();
  if (n) *n = (int)nb;
  return align256((long long)V * 4) + align256(nb * 4) + align256(nb * 8);
}

// out[0] = the index q35_lm_head_top1 returns for (W, x), found through the
// int8 screen (Wq, s, c from q35_lm_head_screen_prep of this W) and the exact
// recomputation of the rows it cannot exclude; `mirror` and `advance` as there. The
// workspace's last section holds, per workgroup, how many rows it
// recomputed (q35_lm_head_screened_candidates sums them).
int q35_lm_head_top1_screened(const void* W, const void* Wq, const void* s, const void* c,
                              const void* x, int V, int K, void* workspace,
                              long long workspace_bytes, void* out, void* mirror, void* advance,
                              int n_advance, hipStream_t stream) {
  Q35_CHECK_ARG(!advance || (n_advance >= 0 && n_advance <= 64));
  Q35_CHECK_ARG(W && Wq && s && c && x && workspace && out && V > 0 && K == 2048 && V < (1 << 30));
  Q35_CHECK_ARG(q35_aligned8(mirror));
  Q35_CHECK_ARG(q35_aligned16(W) && q35_aligned16(Wq) && q35_aligned16(x) && q35_aligned16(workspace));
  Q35_CHECK_ARG(workspace_bytes >= screened_bytes(V));
  const long long nb = screened_parts();
  float* U = (float*)workspace;
  float* lpart = (float*)((char*)workspace + align256((long long)V * 4));
  unsigned long long* cand =
      (unsigned long long*)((char*)workspace + align256((long long)V * 4) + align256(nb * 4));
  unsigned* ncand = (unsigned*)((char*)cand + align256(nb * 8));
  const long long nbs = lm_device_cus();  // screen workgroups (<= nb lower-bound slots)
  lm_head_screen<kScScreenWV, kScR, 2><<<(unsigned)nbs, kScScreenWV * 64, 0, stream>>>(
      (const int8_t*)Wq, (const float*)s, (const float*)c, (const uint16_t*)x, V, U, lpart);
  int e = q35_last_error();
  if (e) return e;
  lm_head_rescore<kScWV><<<(unsigned)nb, kScWV * 64, 0, stream>>>(
      (const uint16_t*)W, (const uint16_t*)x, U, lpart, (int)nbs, V, cand, ncand);
  e = q35_last_error();
  if (e) return e;
  top1_final<<<1, 1024, 0, stream>>>(cand, (int)nb, (long long*)out, (long long*)mirror,
                                     (long long*)advance, advance ? n_advance : 0);
  return q35_last_error();
}

// Set-up for the current device: resolves this GPU's address of `scratch`
// (top1_scratch), so that no later call needs a runtime query. Once per
// device, with that device current, before the first
// q35_lm_head_top1_noalloc made under graph capture; the ppu_amd loader calls
// it for the current device.
int q35_init(void) {
  void* p = nullptr;
  return top1_scratch(&p);
}

// q35_lm_head_top1 without a workspace argument: the candidate keys go to
// this library's `scratch` array on the current device (see top1_scratch).
int q35_lm_head_top1_noalloc(const void* W, const void* x, int V, int K, void* out, void* advance,
                             int n_advance, hipStream_t stream) {
  Q35_CHECK_ARG(!advance || (n_advance >= 0 && n_advance <= 64));
  Q35_CHECK_ARG(V > 0 && K > 0 && W && x && out && V < (1 << 30));
  GemvArgs probe{(const uint16_t*)W, (const uint16_t*)x};
  const long long need = (K == 2048 && fast_ok(probe, PRO_NONE))
                             ? (long long)lm_device_cus() * kLmBlocksPerCU
                             : (long long)(V + 3) / 4;
  if (need > kTop1ScratchSlots) return (int)hipErrorInvalidValue;  // beyond the scratch array
  void* scratch = nullptr;
  const int e = top1_scratch(&scratch);
  if (e) return e;
  return lm_head_top1_launch(W, x, V, K, scratch, kTop1ScratchSlots, out, nullptr, advance,
                             n_advance, stream);
}

}  // extern "C"
