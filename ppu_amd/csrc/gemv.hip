// Memory-bound bf16 GEMV for batch-1 decode (M = 1), with fused prologues and
// epilogues, and the lm_head GEMV fused with a top-1 reduction.
//
//   y[n] = bf16( sum_k W[n, k] * x[k] )     W row-major [N, K] bf16, fp32 acc
//
// Work split: one wave64 owns R consecutive weight rows. Lane l reads the
// 16-byte group k = c*512 + 8l of every row for chunk c = 0..NCH-1, so each
// load instruction of a wave moves one contiguous 1 KiB segment of a row and
// all R*NCH loads of a lane are issued before the first one is consumed. The
// activation vector is loaded (or computed by the prologue) after the weight
// loads are in flight. Per-row partial sums are reduced with the DPP wave
// reduction. Weights are read exactly once, so the kernel is bound by HBM
// bandwidth: bytes per launch = 2*N*K (+ 2*K + 2*N).
//
// Prologues (computed redundantly by every wave from L2-resident vectors):
//   RMSNORM : x = bf16(x * rsqrt(mean(x^2)+eps) * (1+w))          [kernels.py:24-53]
//   RESNORM : r' = bf16(r+u); x = RMSNorm(r'); block 0 stores r'  [kernels.py:56-112]
// Epilogues:
//   STORE   : y[n] = bf16(acc)                                    [F.linear, integration.py:185]
//   SWIGLU  : rows n and N+n of a packed [gate; up] weight:
//             y[n] = bf16(bf16(silu(bf16(g))) * bf16(u))          [kernels.py:183-263]
#include "q35_common.hpp"

namespace {

enum { PRO_NONE = 0, PRO_RMSNORM = 1, PRO_RESNORM = 2 };
enum { EPI_STORE = 0, EPI_SWIGLU = 1 };

struct GemvArgs {
  const uint16_t* W;    // [rows_total, K]
  const uint16_t* x;    // activation (or residual for RESNORM)
  const uint16_t* u;    // update (RESNORM)
  const void* nw;       // norm weight
  uint16_t* r_out;      // RESNORM: r' written by block 0 (may be null)
  uint16_t* xn_out;     // normalised activation written by block 0 (may be null)
  uint16_t* y;          // output [N]
  int N;                // output elements
  int K;
  int nw_f32;
  float eps;
};

// Issue the loads of R rows x NCH chunks; rows at or past row_end read as 0.
template <int R, int NCH>
Q35_DEV void load_rows(const uint16_t* __restrict__ W, int K, const int* rows, int row_end,
                       int lane, uint4 (&w)[R][NCH]) {
#pragma unroll
  for (int r = 0; r < R; ++r) {
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      const int k = c * 512 + lane * 8;
      if (rows[r] < row_end && k < K) {
        w[r][c] = ld_stream16(W + (size_t)rows[r] * K + k);
      } else {
        w[r][c] = make_uint4(0, 0, 0, 0);
      }
    }
  }
}

// Activation chunk c of this lane, after the prologue; packed bf16.
template <int NCH, int PRO>
Q35_DEV void load_activation(const GemvArgs& a, int lane, bool writer, uint4 (&xv)[NCH]) {
  if (PRO == PRO_NONE) {
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      const int k = c * 512 + lane * 8;
      xv[c] = k < a.K ? *reinterpret_cast<const uint4*>(a.x + k) : make_uint4(0, 0, 0, 0);
    }
    return;
  }
  float s[NCH][8];
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int k = c * 512 + lane * 8;
    if (k < a.K) {
      unpack8(*reinterpret_cast<const uint4*>(a.x + k), s[c]);
      if (PRO == PRO_RESNORM) {
        float b[8];
        unpack8(*reinterpret_cast<const uint4*>(a.u + k), b);
#pragma unroll
        for (int j = 0; j < 8; ++j) s[c][j] = round_bf(s[c][j] + b[j]);
        if (writer && a.r_out) *reinterpret_cast<uint4*>(a.r_out + k) = pack8(s[c]);
      }
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) s[c][j] = 0.f;
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) ss += s[c][j] * s[c][j];
  }
  const float inv = rsqrt_cr(wave_sum(ss) / (float)a.K + a.eps);
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int k = c * 512 + lane * 8;
    float o[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float wj = k < a.K ? (a.nw_f32 ? reinterpret_cast<const float*>(a.nw)[k + j]
                                           : bf2f(reinterpret_cast<const uint16_t*>(a.nw)[k + j]))
                               : 0.f;
      o[j] = s[c][j] * inv * (1.0f + wj);
    }
    xv[c] = pack8(o);
    if (writer && a.xn_out && k < a.K) *reinterpret_cast<uint4*>(a.xn_out + k) = xv[c];
  }
}

template <int R, int NCH>
Q35_DEV void dot_rows(const uint4 (&w)[R][NCH], const uint4 (&xv)[NCH], float (&acc)[R]) {
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = 0.f;
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    float xf[8];
    unpack8(xv[c], xf);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      float wf[8];
      unpack8(w[r][c], wf);
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[r] = fmaf(wf[j], xf[j], acc[r]);
    }
  }
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = wave_sum(acc[r]);
}

template <int R, int NCH, int PRO, int EPI>
__global__ __launch_bounds__(256) void gemv_bf16(const GemvArgs a) {
  const int lane = threadIdx.x & 63;
  const int wave = blockIdx.x * 4 + (threadIdx.x >> 6);
  constexpr int P = EPI == EPI_SWIGLU ? R / 2 : R;  // outputs per wave
  const int n0 = wave * P;
  int rows[R];
  int row_end;
  if (EPI == EPI_SWIGLU) {
#pragma unroll
    for (int i = 0; i < P; ++i) {
      rows[i] = n0 + i < a.N ? n0 + i : 0x7fffffff;
      rows[P + i] = n0 + i < a.N ? a.N + n0 + i : 0x7fffffff;
    }
    row_end = 2 * a.N;
  } else {
#pragma unroll
    for (int i = 0; i < R; ++i) rows[i] = n0 + i;
    row_end = a.N;
  }
  const bool writer = blockIdx.x == 0 && threadIdx.x < 64;
  if (n0 >= a.N && !writer) return;

  uint4 w[R][NCH];
  load_rows<R, NCH>(a.W, a.K, rows, row_end, lane, w);
  uint4 xv[NCH];
  load_activation<NCH, PRO>(a, lane, writer, xv);
  if (n0 >= a.N) return;
  float acc[R];
  dot_rows<R, NCH>(w, xv, acc);

  if (lane == 0) {
    if (EPI == EPI_STORE) {
#pragma unroll
      for (int r = 0; r < R; ++r)
        if (n0 + r < a.N) a.y[n0 + r] = (uint16_t)f2bf(acc[r]);
    } else {
#pragma unroll
      for (int i = 0; i < P; ++i) {
        if (n0 + i < a.N) {
          const float g = round_bf(acc[i]);
          const float up = round_bf(acc[P + i]);
          a.y[n0 + i] = (uint16_t)f2bf(round_bf(silu_f(g)) * up);
        }
      }
    }
  }
}

// Generic fallback for any K (multiple of 8 or not) and unaligned pointers:
// one wave per output, scalar lane-strided loads. Used by small test shapes.
template <int PRO, int EPI>
__global__ __launch_bounds__(256) void gemv_bf16_generic(const GemvArgs a) {
  const int lane = threadIdx.x & 63;
  const int n = blockIdx.x * 4 + (threadIdx.x >> 6);
  const bool writer = blockIdx.x == 0 && threadIdx.x < 64;
  if (n >= a.N && !writer) return;
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
  if (n >= a.N) return;
  float g = 0.f, up = 0.f;
  for (int k = lane; k < a.K; k += 64) {
    const float xk = xval(k);
    g = fmaf(bf2f(a.W[(size_t)n * a.K + k]), xk, g);
    if (EPI == EPI_SWIGLU) up = fmaf(bf2f(a.W[(size_t)(a.N + n) * a.K + k]), xk, up);
  }
  g = wave_sum(g);
  if (EPI == EPI_SWIGLU) up = wave_sum(up);
  if (lane == 0) {
    if (EPI == EPI_STORE) {
      a.y[n] = (uint16_t)f2bf(g);
    } else {
      a.y[n] = (uint16_t)f2bf(round_bf(silu_f(round_bf(g))) * round_bf(up));
    }
  }
}

template <int R, int NCH, int PRO, int EPI>
int launch_fast(const GemvArgs& a, hipStream_t stream) {
  constexpr int P = EPI == EPI_SWIGLU ? R / 2 : R;
  const long long waves = (a.N + P - 1) / P;
  const long long blocks = (waves + 3) / 4;
  gemv_bf16<R, NCH, PRO, EPI><<<(unsigned)blocks, 256, 0, stream>>>(a);
  return q35_last_error();
}

template <int PRO, int EPI>
int dispatch(const GemvArgs& a, hipStream_t stream) {
  bool aligned = (a.K % 8 == 0) && q35_aligned16(a.W) && q35_aligned16(a.x) &&
                 (PRO != PRO_RESNORM || q35_aligned16(a.u)) && q35_aligned16(a.r_out) &&
                 q35_aligned16(a.xn_out);
  if (aligned) {
    const int nch = (a.K + 511) / 512;
    if constexpr (EPI == EPI_SWIGLU) {
      if (nch == 4) return launch_fast<2, 4, PRO, EPI>(a, stream);
      if (nch == 12) return launch_fast<2, 12, PRO, EPI>(a, stream);
      if (nch == 1) return launch_fast<2, 1, PRO, EPI>(a, stream);
    } else {
      const bool wide = a.N >= 8192;
      if (nch == 4) return wide ? launch_fast<2, 4, PRO, EPI>(a, stream)
                                : launch_fast<1, 4, PRO, EPI>(a, stream);
      if (nch == 12) return launch_fast<1, 12, PRO, EPI>(a, stream);
      if (nch == 1) return launch_fast<2, 1, PRO, EPI>(a, stream);
      if (nch == 2) return launch_fast<2, 2, PRO, EPI>(a, stream);
    }
  }
  const unsigned blocks = (unsigned)((a.N + 3) / 4);
  gemv_bf16_generic<PRO, EPI><<<blocks > 0 ? blocks : 1, 256, 0, stream>>>(a);
  return q35_last_error();
}

// ------------------------------------------------------------ lm_head top-1
// Each wave computes R logits, rounds them to bf16 (eager materialises bf16
// logits before argmax), and folds them into a 64-bit key (ordered bf16
// value, inverted index) so that one max reduction gives the largest value
// and, among ties, the lowest index [kernels.py:1093-1143]. Waves reduce in
// LDS; each workgroup writes one candidate key.
template <int R, int NCH>
__global__ __launch_bounds__(256) void lm_head_top1_blocks(const uint16_t* __restrict__ W,
                                                           const uint16_t* __restrict__ x, int V,
                                                           int K, unsigned long long* cand) {
  const int lane = threadIdx.x & 63;
  const int wid = threadIdx.x >> 6;
  const int n0 = (blockIdx.x * 4 + wid) * R;
  __shared__ unsigned long long best_s[4];
  uint64_t best = 0;
  if (n0 < V) {
    int rows[R];
#pragma unroll
    for (int r = 0; r < R; ++r) rows[r] = n0 + r;
    uint4 w[R][NCH];
    load_rows<R, NCH>(W, K, rows, V, lane, w);
    uint4 xv[NCH];
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      const int k = c * 512 + lane * 8;
      xv[c] = k < K ? *reinterpret_cast<const uint4*>(x + k) : make_uint4(0, 0, 0, 0);
    }
    float acc[R];
    dot_rows<R, NCH>(w, xv, acc);
#pragma unroll
    for (int r = 0; r < R; ++r)
      if (n0 + r < V) best = u64_max(best, top1_key(round_bf(acc[r]), (uint32_t)(n0 + r)));
  }
  if (lane == 0) best_s[wid] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint64_t b = best_s[0];
    for (int i = 1; i < 4; ++i) b = u64_max(b, best_s[i]);
    cand[blockIdx.x] = b;
  }
}

__global__ __launch_bounds__(256) void lm_head_top1_generic(const uint16_t* __restrict__ W,
                                                            const uint16_t* __restrict__ x, int V,
                                                            int K, unsigned long long* cand) {
  const int lane = threadIdx.x & 63;
  const int wid = threadIdx.x >> 6;
  const int n = blockIdx.x * 4 + wid;
  __shared__ unsigned long long best_s[4];
  uint64_t best = 0;
  if (n < V) {
    float acc = 0.f;
    for (int k = lane; k < K; k += 64) acc = fmaf(bf2f(W[(size_t)n * K + k]), bf2f(x[k]), acc);
    acc = wave_sum(acc);
    best = top1_key(round_bf(acc), (uint32_t)n);
  }
  if (lane == 0) best_s[wid] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint64_t b = best_s[0];
    for (int i = 1; i < 4; ++i) b = u64_max(b, best_s[i]);
    cand[blockIdx.x] = b;
  }
}

__global__ __launch_bounds__(1024) void top1_final(const unsigned long long* __restrict__ cand,
                                                   int n, long long* out) {
  __shared__ unsigned long long s[16];
  uint64_t b = 0;
  for (int i = threadIdx.x; i < n; i += 1024) b = u64_max(b, cand[i]);
  b = wave_max_u64(b);
  if ((threadIdx.x & 63) == 0) s[threadIdx.x >> 6] = b;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint64_t m = s[0];
    for (int i = 1; i < 16; ++i) m = u64_max(m, s[i]);
    out[0] = (long long)top1_index(m);
  }
}

}  // namespace

extern "C" {

// y[N] = W[N,K] . x[K]; optional prologue: mode 0 none, 1 rmsnorm(x), 2 residual add + rmsnorm.
int q35_gemv_bf16(const void* W, const void* x, const void* u, const void* norm_w, int norm_w_f32,
                  float eps, void* residual_out, void* x_norm_out, void* y, int N, int K,
                  int prologue, hipStream_t stream) {
  Q35_CHECK_ARG(N > 0 && K > 0 && W && x && y);
  Q35_CHECK_ARG(prologue >= 0 && prologue <= 2);
  Q35_CHECK_ARG(prologue == 0 || norm_w);
  Q35_CHECK_ARG(prologue != 2 || u);
  GemvArgs a{(const uint16_t*)W, (const uint16_t*)x, (const uint16_t*)u, norm_w,
             (uint16_t*)residual_out, (uint16_t*)x_norm_out, (uint16_t*)y, N, K, norm_w_f32, eps};
  if (prologue == 0) return dispatch<PRO_NONE, EPI_STORE>(a, stream);
  if (prologue == 1) return dispatch<PRO_RMSNORM, EPI_STORE>(a, stream);
  return dispatch<PRO_RESNORM, EPI_STORE>(a, stream);
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
             (uint16_t*)residual_out, (uint16_t*)x_norm_out, (uint16_t*)y, N, K, norm_w_f32, eps};
  if (prologue == 0) return dispatch<PRO_NONE, EPI_SWIGLU>(a, stream);
  if (prologue == 1) return dispatch<PRO_RMSNORM, EPI_SWIGLU>(a, stream);
  return dispatch<PRO_RESNORM, EPI_SWIGLU>(a, stream);
}

// Number of 64-bit candidate slots q35_lm_head_top1 needs in its workspace.
long long q35_lm_head_top1_workspace(int V, int K) {
  if (V <= 0 || K <= 0) return 0;
  return (V + 3) / 4;  // enough for the one-row-per-wave fallback as well
}

// out[0] (int64) = argmax_v bf16(W[v].x), lowest index on ties.
int q35_lm_head_top1(const void* W, const void* x, int V, int K, void* workspace,
                     long long workspace_slots, void* out, hipStream_t stream) {
  Q35_CHECK_ARG(V > 0 && K > 0 && W && x && workspace && out);
  const long long need = q35_lm_head_top1_workspace(V, K);
  Q35_CHECK_ARG(workspace_slots >= need && need < (1ll << 31));
  unsigned long long* cand = (unsigned long long*)workspace;
  const bool fast = K == 2048 && q35_aligned16(W) && q35_aligned16(x);
  // fast: 4 waves x 4 rows per workgroup; generic: 4 waves x 1 row.
  const long long nc = fast ? (V + 15) / 16 : (V + 3) / 4;
  if (fast) {
    lm_head_top1_blocks<4, 4><<<(unsigned)nc, 256, 0, stream>>>(
        (const uint16_t*)W, (const uint16_t*)x, V, K, cand);
  } else {
    lm_head_top1_generic<<<(unsigned)nc, 256, 0, stream>>>(
        (const uint16_t*)W, (const uint16_t*)x, V, K, cand);
  }
  const int e = q35_last_error();
  if (e) return e;
  top1_final<<<1, 1024, 0, stream>>>(cand, (int)nc, (long long*)out);
  return q35_last_error();
}

}  // extern "C"
