// A8W8 linear: per-output-channel symmetric int8 weights, per-token dynamic
// symmetric int8 activations, exact int32 accumulation with packed int8 dot
// instructions (v_dot4c_i32_i8 via __builtin_amdgcn_sdot4), dequant fused
// into the store.
//
//   weights  : s_w[n] = absmax_n/127 (1 if absmax_n == 0);
//              Wq = clamp(round_half_even(W/s_w), -127, 127)
//              [reference explore_runtime_quantization.py:142-155]
//   tokens   : s_x[m] = absmax_m/127; xq = sat_int8(rint(x * (127/absmax_m)));
//              an all-zero row gives xq = 0, s_x = 0. This is the published
//              dynamic per-token rule of vLLM's scaled_int8_quant(symmetric)
//              that the reference calls [explore_runtime_quantization.py:167-172].
//   output   : y[m, n] = bf16((float)acc[m, n] * s_x[m] * s_w[n])
//
// One token (M = 1) runs on the tiled GEMV of gemv.hip with int8 weights,
// which quantises the activation inside every workgroup (q35_gemv_i8). Here:
// weight/activation quantisation kernels, the skinny M <= 16 GEMV over
// pre-quantised activations (one wave64 owns R weight rows; lane l reads 16
// int8 at k = c*1024 + 16l, so the weight stream is read once per launch of
// MT tokens), and the dequant of a library int32 GEMM for prefill.
#include "q35_common.hpp"

// The tiled int8-weight GEMV with the activation quantisation fused (gemv.hip).
extern "C" int q35_gemv_i8(const void* Wq, const void* s_w, const void* x, const void* u,
                           const void* norm_w, int norm_w_f32, float eps, void* residual_out,
                           void* x_norm_out, void* y, void* acc_out, void* xq_out, void* sx_out,
                           int N, int K, int prologue, hipStream_t stream);

namespace {

// One wave per row: absmax, scale and round-half-even quantisation.
__global__ __launch_bounds__(256) void quant_weight_rows(const uint16_t* __restrict__ W,
                                                         int8_t* __restrict__ Wq,
                                                         float* __restrict__ scale, int N, int K) {
  const int lane = threadIdx.x & 63;
  const int n = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (n >= N) return;
  const uint16_t* row = W + (size_t)n * K;
  float mx = 0.f;
  for (int k = lane; k < K; k += 64) mx = fmaxf(mx, fabsf(bf2f(row[k])));
  mx = wave_max(mx);
  const float s = mx > 0.f ? mx / 127.0f : 1.0f;
  for (int k = lane; k < K; k += 64) {
    float q = rintf(bf2f(row[k]) / s);
    q = fminf(fmaxf(q, -127.0f), 127.0f);
    Wq[(size_t)n * K + k] = (int8_t)(int)q;
  }
  if (lane == 0) scale[n] = s;
}

// One workgroup per token row: 16-byte loads (PER groups of 8 per thread,
// K <= PER * 2048), block absmax, then q = sat(rint(x * 127/absmax)) written
// as 8-byte groups (K % 8 == 0).
template <int PER>
__global__ __launch_bounds__(256) void quant_act_rows(const uint16_t* __restrict__ x,
                                                      int8_t* __restrict__ xq,
                                                      float* __restrict__ scale, int M, int K) {
  const int m = blockIdx.x;
  const int tid = threadIdx.x;
  const uint16_t* row = x + (size_t)m * K;
  const int groups = K / 8;
  __shared__ float red[4];
  float v[PER][8];
  float mx = 0.f;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int gidx = tid + j * 256;
    const uint4 raw = *reinterpret_cast<const uint4*>(row + (size_t)min(gidx, groups - 1) * 8);
    unpack8(raw, v[j]);
#pragma unroll
    for (int e = 0; e < 8; ++e) mx = gidx < groups ? fmaxf(mx, fabsf(v[j][e])) : mx;
  }
  mx = wave_max(mx);
  if ((tid & 63) == 0) red[tid >> 6] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const float inv = 127.0f / mx;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int gidx = tid + j * 256;
    if (gidx < groups) {
      uint32_t q[2] = {0u, 0u};
#pragma unroll
      for (int e = 0; e < 8; ++e) q[e >> 2] |= (uint32_t)(uint8_t)sat_i8(v[j][e] * inv) << (8 * (e & 3));
      *reinterpret_cast<uint2*>(xq + (size_t)m * K + gidx * 8) = make_uint2(q[0], q[1]);
    }
  }
  if (tid == 0) scale[m] = mx / 127.0f;
}

struct A8Args {
  const int8_t* Wq;       // [N, K]
  const float* s_w;       // [N]
  const int8_t* xq;       // [M, K] (input, or written by block 0 when quantising)
  const float* s_x;       // [M]
  const uint16_t* x;      // bf16 [1, K] when the M=1 quantisation is fused
  int8_t* xq_out;         // fused quant: block 0 stores xq (may be null)
  float* s_x_out;         // fused quant: block 0 stores s_x (may be null)
  uint16_t* y;            // [M, N] bf16
  int* acc_out;           // optional int32 [M, N]
  int M, N, K;
};

// General M (pre-quantised activations), any K multiple of 16.
template <int R, int MT>
__global__ __launch_bounds__(256) void a8w8_gemv_mt(const A8Args a, int m0) {
  const int lane = threadIdx.x & 63;
  const int n0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * R;
  if (n0 >= a.N) return;
  const int mcount = min(MT, a.M - m0);
  int acc[R][MT];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int m = 0; m < MT; ++m) acc[r][m] = 0;
  for (int k = lane * 16; k < a.K; k += 1024) {
    uint4 w[R];
#pragma unroll
    for (int r = 0; r < R; ++r)
      w[r] = n0 + r < a.N ? ld_stream16(a.Wq + (size_t)(n0 + r) * a.K + k) : make_uint4(0, 0, 0, 0);
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      if (m < mcount) {
        const uint4 xv = *reinterpret_cast<const uint4*>(a.xq + (size_t)(m0 + m) * a.K + k);
#pragma unroll
        for (int r = 0; r < R; ++r) acc[r][m] = dot16_i8(w[r], xv, acc[r][m]);
      }
    }
  }
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int m = 0; m < MT; ++m) acc[r][m] = wave_sum_i32(acc[r][m]);
  if (lane == 0) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      if (n0 + r >= a.N) continue;
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        if (m < mcount) {
          const size_t o = (size_t)(m0 + m) * a.N + n0 + r;
          a.y[o] = (uint16_t)f2bf((float)acc[r][m] * a.s_x[m0 + m] * a.s_w[n0 + r]);
          if (a.acc_out) a.acc_out[o] = acc[r][m];
        }
      }
    }
  }
}

// One step of the halving butterfly and the rest by recursion (all indices
// compile-time, so the values stay in registers): H values are exchanged
// across lane bit S, or, once one value is left, plain xor-adds finish.
template <int H, int S, int N>
Q35_DEV void bfly_reduce(int (&acc)[N], int lane) {
  if constexpr (S >= 1) {
    if constexpr (H >= 1) {
      const bool upper = (lane & S) != 0;
#pragma unroll
      for (int j = 0; j < H; ++j) {
        const int send = upper ? acc[j] : acc[j + H];
        const int keep = upper ? acc[j + H] : acc[j];
        acc[j] = keep + __shfl_xor(send, S, 64);
      }
      bfly_reduce<H / 2, S / 2, N>(acc, lane);
    } else {
      acc[0] += __shfl_xor(acc[0], S, 64);
      bfly_reduce<0, S / 2, N>(acc, lane);
    }
  }
}

// Skinny A8W8 for 2..MT tokens in one pass over the weights (K = NCH KiB).
// The workgroup stages the MT pre-quantised rows in LDS (requested before the
// weight stream, so both are in flight together); lane l owns bytes
// c*1024 + 16l of each of its R rows and forms R*MT int32 partial sums with
// v_dot4. The R*MT sums are reduced across the wave by a halving butterfly:
// at step s (32, 16, ..., 1) each lane keeps the half of its values selected
// by lane bit s and adds the partner's copy, so after log2(R*MT) steps lane
// i holds value i summed over the lanes that share its high bits (remaining
// steps add the rest) -- R*MT - 1 shuffles instead of R*MT full reductions.
template <int R, int NCH, int MT>
__global__ __launch_bounds__(256) void a8w8_gemv_skinny(const A8Args a) {
  constexpr int V = R * MT;  // partial sums per lane (power of two, <= 64)
  static_assert((V & (V - 1)) == 0 && V <= 64 && V >= 2, "R*MT must be a power of two <= 64");
  constexpr int KV = NCH * 64;  // uint4 per activation row
  __shared__ uint4 xs[MT * KV];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int n0 = (blockIdx.x * 4 + (tid >> 6)) * R;

  // 1. activation rows (rows past M read row M-1 and are zeroed), then weights.
  constexpr int PER = (MT * KV + 255) / 256;
  uint4 xr[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int i = min(tid + j * 256, MT * KV - 1);
    const int m = i / KV;
    xr[j] = *reinterpret_cast<const uint4*>(a.xq + (size_t)min(m, a.M - 1) * a.K + (i - m * KV) * 16);
  }
  uint4 w[R][NCH];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int8_t* wrow = a.Wq + (size_t)min(n0 + r, a.N - 1) * a.K + lane * 16;
#pragma unroll
    for (int c = 0; c < NCH; ++c) w[r][c] = ld_stream16(wrow + c * 1024);
  }
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int i = tid + j * 256;
    if (i < MT * KV) xs[i] = i / KV < a.M ? xr[j] : make_uint4(0, 0, 0, 0);
  }
  __syncthreads();

  // 2. int32 partial sums, value index v = r * MT + m.
  int acc[V];
#pragma unroll
  for (int v = 0; v < V; ++v) acc[v] = 0;
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      const uint4 xv = xs[m * KV + c * 64 + lane];
#pragma unroll
      for (int r = 0; r < R; ++r) acc[r * MT + m] = dot16_i8(w[r][c], xv, acc[r * MT + m]);
    }
  }

  // 3. butterfly reduce-scatter over the wave (integer adds: exact).
  bfly_reduce<V / 2, 32, V>(acc, lane);
  // Lane l holds value index l >> (6 - log2 V).
  constexpr int LOGV = V >= 64 ? 6 : V >= 32 ? 5 : V >= 16 ? 4 : V >= 8 ? 3 : V >= 4 ? 2 : 1;
  if ((lane & ((1 << (6 - LOGV)) - 1)) == 0) {
    const int v = lane >> (6 - LOGV);
    const int r = v / MT, m = v % MT;
    const int n = n0 + r;
    if (n < a.N && m < a.M) {
      const size_t o = (size_t)m * a.N + n;
      a.y[o] = (uint16_t)f2bf((float)acc[0] * a.s_x[m] * a.s_w[n]);
      if (a.acc_out) a.acc_out[o] = acc[0];
    }
  }
}

// y[m, n] = bf16((float)acc[m, n] * s_x[m] * s_w[n]); 8 outputs per thread.
// y[m, n..n+7] = bf16(acc * s_x[m] * s_w[n..]) (that multiplication order):
// grid (column blocks of 2048, rows), every load issued before use.
__global__ __launch_bounds__(256) void dequant_rows(const int* __restrict__ acc,
                                                    const float* __restrict__ s_x,
                                                    const float* __restrict__ s_w,
                                                    uint16_t* __restrict__ y, int M, int N) {
  const int n = (blockIdx.x * 256 + threadIdx.x) * 8;
  if (n >= N) return;
  const float4 w0 = *reinterpret_cast<const float4*>(s_w + n);
  const float4 w1 = *reinterpret_cast<const float4*>(s_w + n + 4);
  const float w[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
  for (int m = blockIdx.y; m < M; m += gridDim.y) {
    const size_t i = (size_t)m * N + n;
    const int4 a0 = *reinterpret_cast<const int4*>(acc + i);
    const int4 a1 = *reinterpret_cast<const int4*>(acc + i + 4);
    const float sx = s_x[m];
    const int av[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
    float o[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = (float)av[e] * sx * w[e];
    *reinterpret_cast<uint4*>(y + i) = pack8(o);
  }
}

}  // namespace

extern "C" {

// y[M,N] = bf16(acc * s_x[m] * s_w[n]) for int32 accumulators from any int8 GEMM.
int q35_dequant_i32(const void* acc, const void* s_x, const void* s_w, void* y, int M, int N,
                    hipStream_t stream) {
  Q35_CHECK_ARG(M > 0 && N > 0 && N % 8 == 0 && acc && s_x && s_w && y);
  Q35_CHECK_ARG(q35_aligned16(acc) && q35_aligned16(y) && q35_aligned16(s_w));
  const dim3 grid((unsigned)((N / 8 + 255) / 256), (unsigned)min(M, 65535));
  dequant_rows<<<grid, 256, 0, stream>>>((const int*)acc, (const float*)s_x, (const float*)s_w,
                                         (uint16_t*)y, M, N);
  return q35_last_error();
}

int q35_quant_weight_i8(const void* W, void* Wq, void* scale, int N, int K, hipStream_t stream) {
  Q35_CHECK_ARG(N > 0 && K > 0 && W && Wq && scale);
  quant_weight_rows<<<(N + 3) / 4, 256, 0, stream>>>((const uint16_t*)W, (int8_t*)Wq,
                                                    (float*)scale, N, K);
  return q35_last_error();
}

int q35_quant_act_i8(const void* x, void* xq, void* scale, int M, int K, hipStream_t stream) {
  // One workgroup per row holds the row in registers: K a multiple of 8, at most 8192.
  Q35_CHECK_ARG(M >= 0 && K > 0 && K % 8 == 0 && K <= 8192);
  Q35_CHECK_ARG(q35_aligned16(x) && q35_aligned8(xq));
  if (M == 0) return 0;
  const int per = (K / 8 + 255) / 256;
  if (per == 1)
    quant_act_rows<1><<<M, 256, 0, stream>>>((const uint16_t*)x, (int8_t*)xq, (float*)scale, M, K);
  else if (per == 2)
    quant_act_rows<2><<<M, 256, 0, stream>>>((const uint16_t*)x, (int8_t*)xq, (float*)scale, M, K);
  else if (per == 3)
    quant_act_rows<3><<<M, 256, 0, stream>>>((const uint16_t*)x, (int8_t*)xq, (float*)scale, M, K);
  else
    quant_act_rows<4><<<M, 256, 0, stream>>>((const uint16_t*)x, (int8_t*)xq, (float*)scale, M, K);
  return q35_last_error();
}

// y[M,N] = bf16(acc * s_x[m] * s_w[n]). When x (bf16) is given and M == 1 the
// activation quantisation is fused and xq/s_x receive its result (optional);
// otherwise xq/s_x are inputs. acc_out (optional) receives the int32 sums.
int q35_gemv_a8w8(const void* x, void* xq, void* s_x, const void* Wq, const void* s_w, void* y,
                  void* acc_out, int M, int N, int K, hipStream_t stream) {
  Q35_CHECK_ARG(M > 0 && N > 0 && K > 0 && K % 16 == 0 && Wq && s_w && y);
  Q35_CHECK_ARG(q35_aligned16(Wq) && q35_aligned16(xq) && q35_aligned16(x));
  A8Args a{(const int8_t*)Wq, (const float*)s_w, (const int8_t*)xq, (const float*)s_x,
           (const uint16_t*)x, (int8_t*)xq, (float*)s_x, (uint16_t*)y, (int*)acc_out, M, N, K};
  if (x && M == 1 && (K == 1024 || K == 2048 || K == 4096 || K == 6144)) {
    // One token: the tiled int8-weight GEMV quantises x in every workgroup.
    return q35_gemv_i8(Wq, s_w, x, nullptr, nullptr, 0, 0.f, nullptr, nullptr, y, acc_out, xq, s_x,
                       N, K, 0, stream);
  }
  if (x) {
    Q35_CHECK_ARG(xq && s_x);
    const int e = q35_quant_act_i8(x, xq, s_x, M, K, stream);
    if (e) return e;
  }
  Q35_CHECK_ARG(xq && s_x);
  a.x = nullptr;
  // 2..16 tokens with K = 2 or 6 KiB: one pass over the weights.
  if (M <= 16 && (K == 2048 || K == 6144) && q35_aligned16(xq)) {
    const unsigned grid2 = (unsigned)((N + 15) / 16), grid6 = (unsigned)((N + 7) / 8);
#define Q35_SKINNY(MT)                                                                      \
  {                                                                                         \
    if (K == 2048) a8w8_gemv_skinny<4, 2, MT><<<grid2, 256, 0, stream>>>(a);                \
    else a8w8_gemv_skinny<2, 6, MT><<<grid6, 256, 0, stream>>>(a);                          \
    return q35_last_error();                                                                \
  }
    if (M <= 4) Q35_SKINNY(4)
    if (M <= 8) Q35_SKINNY(8)
    Q35_SKINNY(16)
#undef Q35_SKINNY
  }
  constexpr int R = 2, MT = 4;
  const unsigned grid = (unsigned)((N + 4 * R - 1) / (4 * R));
  for (int m0 = 0; m0 < M; m0 += MT) {
    a8w8_gemv_mt<R, MT><<<grid, 256, 0, stream>>>(a, m0);
    const int e = q35_last_error();
    if (e) return e;
  }
  return 0;
}

}  // extern "C"
