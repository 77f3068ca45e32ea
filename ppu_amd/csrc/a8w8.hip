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
// weight/activation quantisation kernels, the skinny 2..16-token GEMM on the
// int8 matrix cores (the weight stream is read once per launch; the per-token
// quantisation fused while M*K is small), a dot4 GEMV for other shapes, and
// the dequant of a library int32 GEMM for prefill.
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

// The attention output gate applied before the quantisation (GATE): the
// row's values become bf16(x * bf16(sigmoid(gate))) with the gate of head h
// at packed[token, h*2*head_dim + head_dim + c] (attn_gate_vec's arithmetic),
// and block 0 adds `amount` to the int64 counter `advance` when given.
struct GateIn {
  const uint16_t* packed;
  int stride, head_dim;
  long long* advance;
  long long amount;
};

// One workgroup per token row: 16-byte loads (PER groups of 8 per thread,
// K <= PER * 2048), block absmax, then q = sat(rint(x * 127/absmax)) written
// as 8-byte groups (K % 8 == 0).
template <int PER, bool GATE = false>
__global__ __launch_bounds__(256) void quant_act_rows(const uint16_t* __restrict__ x,
                                                      int8_t* __restrict__ xq,
                                                      float* __restrict__ scale, int M, int K,
                                                      const GateIn gt = GateIn{}) {
  const int m = blockIdx.x;
  const int tid = threadIdx.x;
  const uint16_t* row = x + (size_t)m * K;
  const int groups = K / 8;
  __shared__ float red[4];
  if (GATE && gt.advance && m == 0 && tid == 0) gt.advance[0] += gt.amount;
  if (m >= M) return;  // the advance-only launch (no rows): nothing is read
  float v[PER][8];
  float mx = 0.f;
  uint4 graw[PER];
  if (GATE) {
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const int col = min(tid + j * 256, groups - 1) * 8;
      const int head = col / gt.head_dim;
      graw[j] = *reinterpret_cast<const uint4*>(gt.packed + (size_t)m * gt.stride +
                                                (size_t)head * 2 * gt.head_dim + gt.head_dim +
                                                (col - head * gt.head_dim));
    }
  }
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int gidx = tid + j * 256;
    const uint4 raw = *reinterpret_cast<const uint4*>(row + (size_t)min(gidx, groups - 1) * 8);
    unpack8(raw, v[j]);
    if (GATE) {
      float gv[8];
      unpack8(graw[j], gv);
#pragma unroll
      for (int e = 0; e < 8; ++e) v[j][e] = round_bf(v[j][e] * round_bf(sigmoid_f(gv[e])));
    }
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
      *reinterpret_cast<uint2*>(xq + (size_t)m * K + gidx * 8) = quant8_i8(v[j], inv);
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

// Skinny A8W8 for 2..MT tokens (MT = 4, 8 or 16) in one pass over the
// weights, on the int8 matrix cores (v_mfma_i32_16x16x64_i8): the tokens fill
// the 16 columns of the B operand, 16 weight rows the A operand, so a wave
// forms a 16 x 16 int32 tile per 64 k with one instruction and the dot4 work
// of the M tokens (the VALU bound of a dot4 skinny GEMV at M = 16) vanishes.
// Operand layout (wave64): lane l supplies row l%16 of A and column l%16 of
// B, 16 consecutive k at 16*(l/16) of the 64-k block; lane l receives C rows
// 4*(l/16)+e, column l%16. Both operands use the same k order, and integer
// sums are exact in any order, so any such k assignment gives the same acc.
//
// Workgroup: RT row tiles of 16 weight rows x KS slices of K, one wave per
// (tile, slice); lane l of a wave streams 16 bytes at k = k0 + 64c + 16(l/16)
// of row l%16, KB = K/(KS*64) loads, all in flight before the first MFMA.
// QUANT: the MT bf16 activation rows are read by every workgroup (requested
// before the weight stream: loads retire in order, so the quantisation runs
// while the weights arrive) and quantised per token in LDS with the rule of
// quant_act_rows; workgroup 0 stores xq and s_x when asked. Otherwise the
// int8 rows and s_x are inputs. Rows past M read row M-1 and are never
// stored; B columns past MT repeat a staged row and are dropped. The KS
// partial tiles are summed in LDS, then one thread per output dequantises.
// R8: tiles of 8 weight rows (A rows 8..15 repeat rows 0..7 and their outputs
// are dropped), for N = 2048: 256 workgroups instead of 128, so twice the CUs
// stream the weights (the matrix-core time of the wasted half is small).
template <int MT, int RT, int KS, int K, bool QUANT, bool R8 = false>
__global__ __launch_bounds__(RT * KS * 64) void a8w8_skinny_mfma(const A8Args a) {
  constexpr int TR = R8 ? 8 : 16;  // weight rows per tile
  constexpr int NW = RT * KS;
  constexpr int KB = K / (KS * 64);          // MFMAs (16-byte loads) per lane
  constexpr int XS = K + 16;                 // LDS row stride: rows 16 bytes apart in the banks
  constexpr int RPW = (MT + NW - 1) / NW;    // activation rows per wave
  constexpr int XV = QUANT ? K / 512 : K / 1024;  // 16-byte activation loads per lane and row
  static_assert(K % (KS * 64) == 0 && KS >= 4 && (MT & (MT - 1)) == 0 && MT <= 16, "tile shape");
  static_assert(XV >= 1, "K too small for the activation tiling");
  // MT staged rows plus one discard row for waves whose row index passes MT.
  __shared__ __attribute__((aligned(16))) int8_t xq_s[(MT + 1) * XS];
  __shared__ float sx_s[MT + 1];
  __shared__ int4 red[NW][64];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wid = tid >> 6;
  const int nb = blockIdx.x * RT * TR;

  // 1. activation rows (bf16 or int8), the output thread's weight scale, then
  //    the weight stream (unpredicated: rows past N read row N-1).
  uint4 xr[RPW][XV];
#pragma unroll
  for (int j = 0; j < RPW; ++j) {
    const int m = min(wid + NW * j, a.M - 1);
#pragma unroll
    for (int t = 0; t < XV; ++t) {
      const int q = lane + 64 * t;
      xr[j][t] = QUANT ? *reinterpret_cast<const uint4*>(a.x + (size_t)m * K + q * 8)
                       : *reinterpret_cast<const uint4*>(a.xq + (size_t)m * K + q * 16);
    }
  }
  // Output thread t < RT*256: tile t/256, token m = (t%256)/16, row n = t%16.
  const int o_rt = tid >> 8, o_m = (tid >> 4) & 15, o_n = tid & 15;
  const int o_row = nb + o_rt * TR + o_n;
  const float sw = a.s_w[min(o_row, a.N - 1)];
  const float sx_in = QUANT ? 0.f : a.s_x[min(o_m, a.M - 1)];
  __builtin_amdgcn_sched_barrier(0);
  const int rt = wid / KS, ks = wid % KS;
  const int wrow = min(nb + rt * TR + (lane & (TR - 1)), a.N - 1);
  const int8_t* wp = a.Wq + (size_t)wrow * K + ks * (K / KS) + 16 * (lane >> 4);
  uint4 w[KB];
#pragma unroll
  for (int c = 0; c < KB; ++c) w[c] = ld_stream16(wp + 64 * c);
  __builtin_amdgcn_sched_barrier(0);

  // 2. stage the int8 rows in LDS (quantising bf16 rows per token).
  const bool writer = blockIdx.x == 0;
#pragma unroll
  for (int j = 0; j < RPW; ++j) {
    const int m = min(wid + NW * j, MT);  // MT: the discard row (no branch around the loads)
    if (QUANT) {
      float v[XV][8];
      float mx = 0.f;
#pragma unroll
      for (int t = 0; t < XV; ++t) {
        unpack8(xr[j][t], v[t]);
#pragma unroll
        for (int e = 0; e < 8; ++e) mx = fmaxf(mx, fabsf(v[t][e]));
      }
      mx = wave_max(mx);
      const float inv = 127.0f / mx;
#pragma unroll
      for (int t = 0; t < XV; ++t) {
        const int q = lane + 64 * t;
        const uint2 pv = quant8_i8(v[t], inv);
        *reinterpret_cast<uint2*>(xq_s + m * XS + q * 8) = pv;
        if (writer && a.xq_out && m < a.M) *reinterpret_cast<uint2*>(a.xq_out + (size_t)m * K + q * 8) = pv;
      }
      if (lane == 0) {
        sx_s[m] = mx / 127.0f;
        if (writer && a.s_x_out && m < a.M) a.s_x_out[m] = mx / 127.0f;
      }
    } else {
#pragma unroll
      for (int t = 0; t < XV; ++t) {
        // Field-wise vector store (a struct copy here becomes a private-memory memcpy).
        const q35_u32x4 v = {xr[j][t].x, xr[j][t].y, xr[j][t].z, xr[j][t].w};
        *reinterpret_cast<q35_u32x4*>(xq_s + m * XS + (lane + 64 * t) * 16) = v;
      }
    }
  }
  lds_barrier();

  // 3. KB int8 MFMAs over the wave's k slice.
  typedef int q35_i32x4 __attribute__((ext_vector_type(4)));
  q35_i32x4 acc = {0, 0, 0, 0};
  const int8_t* bp = xq_s + (lane & 15 & (MT - 1)) * XS + ks * (K / KS) + 16 * (lane >> 4);
#pragma unroll
  for (int c = 0; c < KB; ++c) {
    const q35_i32x4 bv = *reinterpret_cast<const q35_i32x4*>(bp + 64 * c);
    const q35_i32x4 av = {(int)w[c].x, (int)w[c].y, (int)w[c].z, (int)w[c].w};
    acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, bv, acc, 0, 0, 0);
  }

  // 4. sum the KS slices of each tile; output (m, n) sits at lane 16(n/4)+m, element n%4.
  red[wid][lane] = make_int4(acc[0], acc[1], acc[2], acc[3]);
  lds_barrier();
  if (tid < RT * 256) {
    const int* rp = reinterpret_cast<const int*>(&red[o_rt * KS][0]) + (16 * (o_n >> 2) + o_m) * 4 + (o_n & 3);
    int s = 0;
#pragma unroll
    for (int k2 = 0; k2 < KS; ++k2) s += rp[k2 * 256];
    if (o_m < a.M && o_n < TR && o_row < a.N) {
      const size_t o = (size_t)o_m * a.N + o_row;
      const float sx = QUANT ? sx_s[o_m] : sx_in;
      a.y[o] = (uint16_t)f2bf((float)s * sx * sw);
      if (a.acc_out) a.acc_out[o] = s;
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

template <int MT, int RT, int KS, int K, bool QUANT, bool R8 = false>
int launch_skinny(const A8Args& a, hipStream_t stream) {
  // QUANT needs the bf16 rows; otherwise the int8 rows and their scales.
  if (QUANT ? !a.x : (!a.xq || !a.s_x)) return (int)hipErrorInvalidValue;
  constexpr int TR = R8 ? 8 : 16;
  const unsigned grid = (unsigned)((a.N + TR * RT - 1) / (TR * RT));
  a8w8_skinny_mfma<MT, RT, KS, K, QUANT, R8><<<grid, RT * KS * 64, 0, stream>>>(a);
  return q35_last_error();
}

// Prefill SwiGLU on the int32 accumulators of the packed [gate; up] int8
// GEMM: g = bf16(acc[m, n] * s_x[m] * s_w[n]), u = bf16(acc[m, N+n] * s_x[m] *
// s_w[N+n]) (the dequant of q35_dequant_i32), y[m, n] = bf16(bf16(silu(g)) *
// u) (silu_and_mul's rounding points, the hardware exp/reciprocal SiLU of the
// prefill SiLU-mul) -- the dequantised gate/up rows are never stored. Grid
// (column blocks of 2048 outputs, rows); 8 outputs per thread.
__global__ __launch_bounds__(256) void dequant_swiglu_rows(const int* __restrict__ acc,
                                                           const float* __restrict__ s_x,
                                                           const float* __restrict__ s_w,
                                                           uint16_t* __restrict__ y, int M, int N) {
  const int n = (blockIdx.x * 256 + threadIdx.x) * 8;
  if (n >= N) return;
  const float4 g0 = *reinterpret_cast<const float4*>(s_w + n);
  const float4 g1 = *reinterpret_cast<const float4*>(s_w + n + 4);
  const float4 u0 = *reinterpret_cast<const float4*>(s_w + N + n);
  const float4 u1 = *reinterpret_cast<const float4*>(s_w + N + n + 4);
  const float wg[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
  const float wu[8] = {u0.x, u0.y, u0.z, u0.w, u1.x, u1.y, u1.z, u1.w};
  for (int m = blockIdx.y; m < M; m += gridDim.y) {
    const int* row = acc + (size_t)m * 2 * N;
    const int4 a0 = *reinterpret_cast<const int4*>(row + n);
    const int4 a1 = *reinterpret_cast<const int4*>(row + n + 4);
    const int4 b0 = *reinterpret_cast<const int4*>(row + N + n);
    const int4 b1 = *reinterpret_cast<const int4*>(row + N + n + 4);
    const float sx = s_x[m];
    const int ag[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
    const int au[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
    float o[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float g = round_bf((float)ag[e] * sx * wg[e]);
      const float u = round_bf((float)au[e] * sx * wu[e]);
      o[e] = round_bf(silu_fast(g)) * u;
    }
    *reinterpret_cast<uint4*>(y + (size_t)m * N + n) = pack8(o);
  }
}

// ---------------------------------------------------------- A8W8 prefill rows
// The prefill of an A8W8 layer hands int8 activations and int32 accumulators
// between its GEMMs. These kernels fuse the steps around them, each with the
// arithmetic of the separate kernels it replaces, so the values are the same
// bits:
//   resnorm_dequant_quant_rows  update = bf16(float(acc) * s_x[m] * s_w[k])
//     (q35_dequant_i32), r = bf16(x + update), y = bf16(r * rsqrt(mean(r^2) +
//     eps) * (1 + w)) (q35_residual_rmsnorm, width 2048), and optionally y
//     quantised per token (q35_quant_act_i8: s = absmax/127, q = sat(rint(y *
//     127/absmax))). One wave per row; lane l holds k = 512j + 8l .. +7; every
//     load is issued before the reduction.
//   swiglu_quant_rows  act = bf16(bf16(silu(g)) * u) from the [gate; up]
//     accumulators (q35_dequant_swiglu_i32), quantised per token; the bf16
//     act is never stored. One workgroup per row (N / 8 <= 3 * 256).
template <bool QUANT, bool YOUT>
__global__ __launch_bounds__(256) void resnorm_dequant_quant_rows(
    const uint16_t* __restrict__ x, const int* __restrict__ acc, const float* __restrict__ s_x,
    const float* __restrict__ s_w, const void* __restrict__ w, int w_f32,
    uint16_t* __restrict__ r_out, uint16_t* __restrict__ y, int8_t* __restrict__ yq,
    float* __restrict__ s_y, int rows, float eps) {
  constexpr int NPER = 4, width = 2048;
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const size_t base = (size_t)row * width;
  uint4 xa[NPER], wa[NPER], wb[NPER];
  int4 c0[NPER], c1[NPER];
  float4 s0[NPER], s1[NPER];
  const float sx = s_x[row];
#pragma unroll
  for (int j = 0; j < NPER; ++j) {
    const int k = j * 512 + lane * 8;
    xa[j] = *reinterpret_cast<const uint4*>(x + base + k);
    c0[j] = *reinterpret_cast<const int4*>(acc + base + k);
    c1[j] = *reinterpret_cast<const int4*>(acc + base + k + 4);
    s0[j] = *reinterpret_cast<const float4*>(s_w + k);
    s1[j] = *reinterpret_cast<const float4*>(s_w + k + 4);
    if (w_f32) {
      wa[j] = *reinterpret_cast<const uint4*>(reinterpret_cast<const float*>(w) + k);
      wb[j] = *reinterpret_cast<const uint4*>(reinterpret_cast<const float*>(w) + k + 4);
    } else {
      wa[j] = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(w) + k);
    }
  }
  float a[NPER][8];
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < NPER; ++j) {
    unpack8(xa[j], a[j]);
    const int av[8] = {c0[j].x, c0[j].y, c0[j].z, c0[j].w, c1[j].x, c1[j].y, c1[j].z, c1[j].w};
    const float sv[8] = {s0[j].x, s0[j].y, s0[j].z, s0[j].w, s1[j].x, s1[j].y, s1[j].z, s1[j].w};
#pragma unroll
    for (int e = 0; e < 8; ++e) a[j][e] = round_bf(a[j][e] + round_bf((float)av[e] * sx * sv[e]));
    *reinterpret_cast<uint4*>(r_out + base + j * 512 + lane * 8) = pack8(a[j]);
#pragma unroll
    for (int e = 0; e < 8; ++e) ss += a[j][e] * a[j][e];
  }
  const float inv = rsqrt_cr(wave_sum(ss) / (float)width + eps);
  float o[NPER][8];
  float mx = 0.f;
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
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      o[j][e] = round_bf(a[j][e] * inv * (1.0f + wf[e]));
      mx = fmaxf(mx, fabsf(o[j][e]));
    }
    if (YOUT) *reinterpret_cast<uint4*>(y + base + j * 512 + lane * 8) = pack8(o[j]);
  }
  if (QUANT) {
    mx = wave_max(mx);
    const float qinv = 127.0f / mx;
#pragma unroll
    for (int j = 0; j < NPER; ++j)
      *reinterpret_cast<uint2*>(yq + base + j * 512 + lane * 8) = quant8_i8(o[j], qinv);
    if (lane == 0) s_y[row] = mx / 127.0f;
  }
}

__global__ __launch_bounds__(256) void swiglu_quant_rows(const int* __restrict__ acc,
                                                         const float* __restrict__ s_x,
                                                         const float* __restrict__ s_w,
                                                         int8_t* __restrict__ yq,
                                                         float* __restrict__ s_y, int N) {
  constexpr int PER = 3;
  const int m = blockIdx.x;
  const int tid = threadIdx.x;
  const int groups = N / 8;
  const int* row = acc + (size_t)m * 2 * N;
  const float sx = s_x[m];
  __shared__ float red[4];
  float o[PER][8];
  float mx = 0.f;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int gi = min(tid + 256 * j, groups - 1);
    const int n = gi * 8;
    const int4 a0 = *reinterpret_cast<const int4*>(row + n);
    const int4 a1 = *reinterpret_cast<const int4*>(row + n + 4);
    const int4 b0 = *reinterpret_cast<const int4*>(row + N + n);
    const int4 b1 = *reinterpret_cast<const int4*>(row + N + n + 4);
    const float4 g0 = *reinterpret_cast<const float4*>(s_w + n);
    const float4 g1 = *reinterpret_cast<const float4*>(s_w + n + 4);
    const float4 u0 = *reinterpret_cast<const float4*>(s_w + N + n);
    const float4 u1 = *reinterpret_cast<const float4*>(s_w + N + n + 4);
    const int ag[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
    const int au[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
    const float wg[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
    const float wu[8] = {u0.x, u0.y, u0.z, u0.w, u1.x, u1.y, u1.z, u1.w};
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float g = round_bf((float)ag[e] * sx * wg[e]);
      const float u = round_bf((float)au[e] * sx * wu[e]);
      o[j][e] = round_bf(round_bf(silu_fast(g)) * u);
      mx = tid + 256 * j < groups ? fmaxf(mx, fabsf(o[j][e])) : mx;
    }
  }
  mx = wave_max(mx);
  if ((tid & 63) == 0) red[tid >> 6] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const float qinv = 127.0f / mx;
#pragma unroll
  for (int j = 0; j < PER; ++j)
    if (tid + 256 * j < groups)
      *reinterpret_cast<uint2*>(yq + (size_t)m * N + (tid + 256 * j) * 8) = quant8_i8(o[j], qinv);
  if (tid == 0) s_y[m] = mx / 127.0f;
}

}  // namespace

extern "C" {

// y[M,N] = bf16(bf16(silu(g)) * u) with g, u the dequantised columns n and
// N + n of the int32 accumulators acc[M, 2N] of a packed [gate; up] A8W8
// GEMM (N % 8 == 0, 16-byte aligned acc, s_w and y).
int q35_dequant_swiglu_i32(const void* acc, const void* s_x, const void* s_w, void* y, int M, int N,
                           hipStream_t stream) {
  Q35_CHECK_ARG(M > 0 && N > 0 && N % 8 == 0 && acc && s_x && s_w && y);
  Q35_CHECK_ARG(q35_aligned16(acc) && q35_aligned16(y) && q35_aligned16(s_w));
  const dim3 grid((unsigned)((N / 8 + 255) / 256), (unsigned)min(M, 65535));
  dequant_swiglu_rows<<<grid, 256, 0, stream>>>((const int*)acc, (const float*)s_x,
                                                (const float*)s_w, (uint16_t*)y, M, N);
  return q35_last_error();
}


// A8W8 prefill: residual add of a dequantised int8-GEMM output + RMSNorm
// (width 2048) with the normalised rows optionally quantised per token; the
// same bits as q35_dequant_i32 -> q35_residual_rmsnorm -> q35_quant_act_i8.
// y and (yq, s_y) may each be null (not both); acc, x, r_out, y, s_w, w
// 16-byte aligned.
int q35_residual_rmsnorm_dequant_quant(const void* x, const void* acc, const void* s_x,
                                       const void* s_w, const void* w, int w_f32, void* r_out,
                                       void* y, void* yq, void* s_y, int rows, int width, float eps,
                                       hipStream_t stream) {
  Q35_CHECK_ARG(rows > 0 && width == 2048 && x && acc && s_x && s_w && w && r_out);
  Q35_CHECK_ARG((y || yq) && (!yq || s_y));
  Q35_CHECK_ARG(q35_aligned16(x) && q35_aligned16(acc) && q35_aligned16(s_w) && q35_aligned16(w) &&
                q35_aligned16(r_out) && (!y || q35_aligned16(y)) && (!yq || q35_aligned8(yq)));
  const unsigned grid = (unsigned)((rows + 3) / 4);
#define Q35_RDQ(Q, Y)                                                                               \
  resnorm_dequant_quant_rows<Q, Y><<<grid, 256, 0, stream>>>(                                      \
      (const uint16_t*)x, (const int*)acc, (const float*)s_x, (const float*)s_w, w, w_f32,          \
      (uint16_t*)r_out, (uint16_t*)y, (int8_t*)yq, (float*)s_y, rows, eps)
  if (yq && y) Q35_RDQ(true, true);
  else if (yq) Q35_RDQ(true, false);
  else Q35_RDQ(false, true);
#undef Q35_RDQ
  return q35_last_error();
}

// A8W8 prefill: the SwiGLU of a packed [gate; up] int8 GEMM's accumulators
// acc[M, 2N] (q35_dequant_swiglu_i32's values) quantised per token into
// yq[M, N] int8 and s_y[M] (q35_quant_act_i8's rule); N % 8 == 0, N <= 6144.
int q35_dequant_swiglu_quant(const void* acc, const void* s_x, const void* s_w, void* yq, void* s_y,
                             int M, int N, hipStream_t stream) {
  Q35_CHECK_ARG(M > 0 && N > 0 && N % 8 == 0 && N <= 3 * 256 * 8 && acc && s_x && s_w && yq && s_y);
  Q35_CHECK_ARG(q35_aligned16(acc) && q35_aligned16(s_w) && q35_aligned8(yq));
  swiglu_quant_rows<<<(unsigned)M, 256, 0, stream>>>((const int*)acc, (const float*)s_x,
                                                     (const float*)s_w, (int8_t*)yq, (float*)s_y, N);
  return q35_last_error();
}

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

// attention_gate_mul then the per-token int8 quantisation in one launch; the
// same bits as q35_attn_gate_mul -> q35_quant_act_i8, the gated bf16 rows
// never stored. advance / amount as for q35_attn_gate_mul.
int q35_attn_gate_quant(const void* x, const void* packed, void* xq, void* scale, long long tokens,
                        int hidden, int packed_stride, int head_dim, void* advance, long long amount,
                        hipStream_t stream) {
  Q35_CHECK_ARG(tokens >= 0 && tokens < (1ll << 31) && hidden > 0 && hidden % 8 == 0 && hidden <= 8192);
  Q35_CHECK_ARG(head_dim > 0 && head_dim % 8 == 0 && hidden % head_dim == 0);
  Q35_CHECK_ARG(packed_stride >= 2 * hidden && packed_stride % 8 == 0);
  Q35_CHECK_ARG(tokens == 0 || (x && packed && xq && scale));  // empty tensors may be null
  Q35_CHECK_ARG(q35_aligned16(x) && q35_aligned16(packed) && q35_aligned8(xq));
  if (tokens == 0 && (!advance || amount == 0)) return 0;
  const GateIn gt{(const uint16_t*)packed, packed_stride, head_dim, (long long*)advance, amount};
  const unsigned grid = (unsigned)(tokens > 0 ? tokens : 1);
  const int M = (int)tokens;
  const int per = (hidden / 8 + 255) / 256;
  if (tokens == 0) {
    // only the advance: one workgroup whose rows are all past the end
    quant_act_rows<1, true><<<1, 256, 0, stream>>>((const uint16_t*)x, (int8_t*)xq, (float*)scale,
                                                   0, hidden, GateIn{nullptr, 0, head_dim,
                                                                     (long long*)advance, amount});
    return q35_last_error();
  }
#define Q35_GQ(P)                                                                                  \
  quant_act_rows<P, true><<<grid, 256, 0, stream>>>((const uint16_t*)x, (int8_t*)xq, (float*)scale, \
                                                    M, hidden, gt)
  if (per == 1) Q35_GQ(1);
  else if (per == 2) Q35_GQ(2);
  else if (per == 3) Q35_GQ(3);
  else Q35_GQ(4);
#undef Q35_GQ
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
  // 2..16 tokens with K = 2 or 6 KiB: one pass over the weights on the int8
  // matrix cores. Tiles and the fused quantisation per (K, MT) from a measured
  // sweep (MI355X, rotating 640 MB of weights): every workgroup of the fused
  // form quantises all MT rows itself, which stops paying at MT*K = 96 Ki.
  if (M <= 16 && (K == 2048 || K == 6144)) {
    const int mt = M <= 4 ? 4 : M <= 8 ? 8 : 16;
    const bool fuse = x && mt * K <= 49152;
    if (x && !fuse) {
      Q35_CHECK_ARG(xq && s_x);
      const int e = q35_quant_act_i8(x, xq, s_x, M, K, stream);
      if (e) return e;
    }
    if (!fuse) Q35_CHECK_ARG(xq && s_x);
    a.x = fuse ? (const uint16_t*)x : nullptr;
    a.xq_out = fuse ? (int8_t*)xq : nullptr;
    a.s_x_out = fuse ? (float*)s_x : nullptr;
    if (K == 2048) {  // 48 rows x 4 K slices per workgroup (256 workgroups at N = 12288)
      if (mt == 4) return fuse ? launch_skinny<4, 3, 4, 2048, true>(a, stream)
                               : launch_skinny<4, 3, 4, 2048, false>(a, stream);
      if (mt == 8) return fuse ? launch_skinny<8, 3, 4, 2048, true>(a, stream)
                               : launch_skinny<8, 3, 4, 2048, false>(a, stream);
      return fuse ? launch_skinny<16, 3, 4, 2048, true>(a, stream)
                  : launch_skinny<16, 3, 4, 2048, false>(a, stream);
    }
    // K = 6 KiB: 8-row tiles when N leaves fewer than 256 workgroups of 16 rows
    if (a.N <= 2048) {
      if (mt == 4) return fuse ? launch_skinny<4, 1, 4, 6144, true, true>(a, stream)
                               : launch_skinny<4, 1, 4, 6144, false, true>(a, stream);
      if (mt == 8) return fuse ? launch_skinny<8, 1, 8, 6144, true, true>(a, stream)
                               : launch_skinny<8, 1, 8, 6144, false, true>(a, stream);
      return launch_skinny<16, 1, 4, 6144, false, true>(a, stream);
    }
    if (mt == 4) return fuse ? launch_skinny<4, 1, 4, 6144, true>(a, stream)
                             : launch_skinny<4, 1, 4, 6144, false>(a, stream);
    if (mt == 8) return fuse ? launch_skinny<8, 1, 8, 6144, true>(a, stream)
                             : launch_skinny<8, 1, 8, 6144, false>(a, stream);
    return launch_skinny<16, 1, 4, 6144, false>(a, stream);
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
