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

// One wave per token row.
__global__ __launch_bounds__(256) void quant_act_rows(const uint16_t* __restrict__ x,
                                                      int8_t* __restrict__ xq,
                                                      float* __restrict__ scale, int M, int K) {
  const int lane = threadIdx.x & 63;
  const int m = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (m >= M) return;
  const uint16_t* row = x + (size_t)m * K;
  float mx = 0.f;
  for (int k = lane; k < K; k += 64) mx = fmaxf(mx, fabsf(bf2f(row[k])));
  mx = wave_max(mx);
  const float inv = 127.0f / mx;
  for (int k = lane; k < K; k += 64) xq[(size_t)m * K + k] = sat_i8(bf2f(row[k]) * inv);
  if (lane == 0) scale[m] = mx / 127.0f;
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

// y[m, n] = bf16((float)acc[m, n] * s_x[m] * s_w[n]); 8 outputs per thread.
__global__ __launch_bounds__(256) void dequant_rows(const int* __restrict__ acc,
                                                    const float* __restrict__ s_x,
                                                    const float* __restrict__ s_w,
                                                    uint16_t* __restrict__ y, int M, int N) {
  const long long i = ((long long)blockIdx.x * blockDim.x + threadIdx.x) * 8;
  if (i >= (long long)M * N) return;
  const int m = (int)(i / N);
  const int n = (int)(i - (long long)m * N);
  const float sx = s_x[m];
  const int4 a0 = *reinterpret_cast<const int4*>(acc + i);
  const int4 a1 = *reinterpret_cast<const int4*>(acc + i + 4);
  const int av[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
  float o[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = (float)av[e] * sx * s_w[n + e];
  *reinterpret_cast<uint4*>(y + i) = pack8(o);
}

}  // namespace

extern "C" {

// y[M,N] = bf16(acc * s_x[m] * s_w[n]) for int32 accumulators from any int8 GEMM.
int q35_dequant_i32(const void* acc, const void* s_x, const void* s_w, void* y, int M, int N,
                    hipStream_t stream) {
  Q35_CHECK_ARG(M > 0 && N > 0 && N % 8 == 0 && acc && s_x && s_w && y);
  Q35_CHECK_ARG(q35_aligned16(acc) && q35_aligned16(y));
  const long long groups = (long long)M * N / 8;
  const long long grid = (groups + 255) / 256;
  Q35_CHECK_ARG(grid < (1ll << 31));
  dequant_rows<<<(unsigned)grid, 256, 0, stream>>>((const int*)acc, (const float*)s_x,
                                                  (const float*)s_w, (uint16_t*)y, M, N);
  return q35_last_error();
}

int q35_quant_weight_i8(const void* W, void* Wq, void* scale, int N, int K, hipStream_t stream) {
  Q35_CHECK_ARG(N > 0 && K > 0 && W && Wq && scale);
  quant_weight_rows<<<(N + 3) / 4, 256, 0, stream>>>((const uint16_t*)W, (int8_t*)Wq,
                                                    (float*)scale, N, K);
  return q35_last_error();
}

int q35_quant_act_i8(const void* x, void* xq, void* scale, int M, int K, hipStream_t stream) {
  Q35_CHECK_ARG(M >= 0 && K > 0);
  if (M == 0) return 0;
  quant_act_rows<<<(M + 3) / 4, 256, 0, stream>>>((const uint16_t*)x, (int8_t*)xq, (float*)scale,
                                                  M, K);
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
