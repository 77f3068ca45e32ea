// Gated DeltaNet decode and prefill kernels: depthwise causal conv1d (+SiLU)
// with its rolling state, the gated delta-rule recurrence and the gated
// RMSNorm epilogue.
//
// Layouts (batch b, head h, token t; H heads of dim D = 128):
//   packed projection  [B, L, P]  = [q (H*D) | k (H*D) | v (H*D) | z (H*D) | a (H) | b (H) | pad]
//   qkv after conv     [B, L, 3*H*D]
//   conv weight        [C, KW] bf16, conv state [B, C, KW] bf16 (last KW inputs)
//   recurrent state    [B, H, D(k), D(v)] fp32, v contiguous, updated in place
//   core output        [B, L, H, D] bf16
//
// Per token and head (reference kernels.py:768-851, restating the fp32 rule):
//   q^ = q * rsqrt(sum q^2 + 1e-6) * (1/sqrt(D)),  k^ = k * rsqrt(sum k^2 + 1e-6)
//   alpha = exp(-exp(A_log) * softplus(a + dt_bias)),  beta = sigmoid(b)
//   S = alpha*S;  m = S^T k^;  d = beta*(v - m);  S += k^ d^T;  o = S^T q^
#include "q35_common.hpp"

namespace {

Q35_DEV float ld_param(const void* p, int i, int is_f32) {
  return is_f32 ? reinterpret_cast<const float*>(p)[i] : bf2f(reinterpret_cast<const uint16_t*>(p)[i]);
}

Q35_DEV float softplus20(float x) { return x > 20.0f ? x : logf(1.0f + expf(x)); }

// ------------------------------------------------------------------ conv1d
__global__ __launch_bounds__(256) void conv1d_update(const uint16_t* __restrict__ x,
                                                     const uint16_t* __restrict__ w,
                                                     uint16_t* __restrict__ state,
                                                     uint16_t* __restrict__ out, int B, int C,
                                                     int in_stride, int kw) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= B * C) return;
  const int b = i / C, c = i - b * C;
  const float o = conv_update_channel(state + (size_t)i * kw, w + (size_t)c * kw,
                                      x[(size_t)b * in_stride + c], kw);
  out[i] = (uint16_t)f2bf(o);
}

// Prefill conv: zero history before token 0 (the stored state is not read),
// and the last KW inputs are written to the state [reference kernels.py:576-619].
__global__ __launch_bounds__(256) void conv1d_prefill(const uint16_t* __restrict__ x,
                                                      const uint16_t* __restrict__ w,
                                                      uint16_t* __restrict__ state,
                                                      uint16_t* __restrict__ out, int B, int L,
                                                      int C, int in_stride, int kw) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (long long)B * L * C) return;
  const int c = (int)(i % C);
  const long long tf = i / C;
  const int t = (int)(tf % L);
  const int b = (int)(tf / L);
  float acc = 0.f;
  for (int tap = 0; tap < kw; ++tap) {
    const int src = t - (kw - 1 - tap);
    if (src >= 0)
      acc = fmaf(bf2f(x[((size_t)b * L + src) * in_stride + c]), bf2f(w[(size_t)c * kw + tap]), acc);
  }
  out[i] = (uint16_t)f2bf(silu_f(round_bf(acc)));
  const int pos = t - (L - kw);
  if (pos >= 0 && pos < kw)
    state[((size_t)b * C + c) * kw + pos] = x[((size_t)b * L + t) * in_stride + c];
}

// ------------------------------------------------------------- decode step
// One 256-thread workgroup per (batch, head); D = 128 fixed. Thread t owns
// v-columns 4*(t%32)..+3 of k-rows (t/32) + 8*i, i = 0..15: each k-row of the
// fp32 state is 512 contiguous bytes read by 32 lanes with 16-byte loads, and
// the state is read once and written once per step.
constexpr int kD = 128;

struct DeltaArgs {
  const uint16_t* src;     // FUSE_CONV: packed projection; else post-conv qkv
  int src_stride;          // elements per token row of src
  const uint16_t* packed;  // packed projection (a, b, z)
  int packed_stride;
  const uint16_t* conv_w;  // [C, kw]
  uint16_t* conv_state;    // [B, C, kw]
  int conv_channels;       // C = 3*H*D
  int kw;
  const void* a_log;
  const void* dt_bias;
  int params_f32;
  float* state;            // [B, H, D, D]
  const void* norm_w;      // gated norm weight [D]
  int norm_w_f32;
  float norm_eps;
  uint16_t* out;           // [B, H, D]
  int H;
  int z_off, a_off, b_off;
};

template <bool FUSE_CONV, bool FUSE_GNORM>
__global__ __launch_bounds__(256) void delta_decode(const DeltaArgs p) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wid = tid >> 6;
  const int bh = blockIdx.x;
  const int b = bh / p.H, h = bh - b * p.H;
  const int vq = tid & 31;   // v columns 4*vq .. 4*vq+3
  const int kg = tid >> 5;   // k rows kg + 8*i

  __shared__ float qs[kD], ks[kD], vs[kD];
  __shared__ float red[4][kD];
  __shared__ float sc[4];

  // Issue the state loads first: 16 x 16 B per thread, 64 KiB per head.
  float* S = p.state + (size_t)bh * kD * kD;
  float4 st[16];
#pragma unroll
  for (int i = 0; i < 16; ++i)
    st[i] = *reinterpret_cast<const float4*>(S + (size_t)(kg + 8 * i) * kD + 4 * vq);

  // q, k, v for this head (after conv).
  const uint16_t* srow = p.src + (size_t)b * p.src_stride;
  for (int j = tid; j < 3 * kD; j += 256) {
    const int part = j / kD, i = j - part * kD;
    const int ch = part * p.H * kD + h * kD + i;
    float val;
    if (FUSE_CONV) {
      val = conv_update_channel(p.conv_state + ((size_t)b * p.conv_channels + ch) * p.kw,
                                p.conv_w + (size_t)ch * p.kw, srow[ch], p.kw);
    } else {
      val = bf2f(srow[ch]);
    }
    (part == 0 ? qs : part == 1 ? ks : vs)[i] = val;
  }
  __syncthreads();

  // Norm factors (wave 0: q, wave 1: k) and the gates.
  if (wid < 2) {
    const float* src = wid == 0 ? qs : ks;
    const float a0 = src[lane], a1 = src[lane + 64];
    const float tot = wave_sum(a0 * a0 + a1 * a1);
    if (lane == 0) sc[wid] = rsqrt_cr(tot + 1e-6f);
  } else if (tid == 128) {
    const uint16_t* prow = p.packed + (size_t)b * p.packed_stride;
    const float a = bf2f(prow[p.a_off + h]) + ld_param(p.dt_bias, h, p.params_f32);
    const float g = -expf(ld_param(p.a_log, h, p.params_f32)) * softplus20(a);
    sc[2] = expf(g);
    sc[3] = 1.0f / (1.0f + expf(-bf2f(prow[p.b_off + h])));
  }
  __syncthreads();
  const float q_inv = sc[0], k_inv = sc[1], alpha = sc[2], beta = sc[3];
  const float qscale = 0.08838834764831845f;  // fp32(1/sqrt(128))

  // S = alpha*S; partial m = S^T k^ over this thread's rows.
  float4 m = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const float kh = ks[kg + 8 * i] * k_inv;
    st[i].x *= alpha; st[i].y *= alpha; st[i].z *= alpha; st[i].w *= alpha;
    m.x = fmaf(st[i].x, kh, m.x); m.y = fmaf(st[i].y, kh, m.y);
    m.z = fmaf(st[i].z, kh, m.z); m.w = fmaf(st[i].w, kh, m.w);
  }
  // Reduce over the 8 k-groups: lanes l and l^32 of a wave, then the 4 waves.
  m.x += __shfl_xor(m.x, 32); m.y += __shfl_xor(m.y, 32);
  m.z += __shfl_xor(m.z, 32); m.w += __shfl_xor(m.w, 32);
  if (lane < 32) *reinterpret_cast<float4*>(&red[wid][4 * vq]) = m;
  __syncthreads();
  if (tid < kD) {
    const float mem = (red[0][tid] + red[1][tid]) + (red[2][tid] + red[3][tid]);
    vs[tid] = beta * (vs[tid] - mem);   // delta
  }
  __syncthreads();
  const float4 d = *reinterpret_cast<const float4*>(&vs[4 * vq]);
  float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const float kh = ks[kg + 8 * i] * k_inv;
    const float qh = qs[kg + 8 * i] * q_inv * qscale;
    st[i].x += kh * d.x; st[i].y += kh * d.y; st[i].z += kh * d.z; st[i].w += kh * d.w;
    o.x = fmaf(st[i].x, qh, o.x); o.y = fmaf(st[i].y, qh, o.y);
    o.z = fmaf(st[i].z, qh, o.z); o.w = fmaf(st[i].w, qh, o.w);
    *reinterpret_cast<float4*>(S + (size_t)(kg + 8 * i) * kD + 4 * vq) = st[i];
  }
  o.x += __shfl_xor(o.x, 32); o.y += __shfl_xor(o.y, 32);
  o.z += __shfl_xor(o.z, 32); o.w += __shfl_xor(o.w, 32);
  __syncthreads();  // red[] reuse
  if (lane < 32) *reinterpret_cast<float4*>(&red[wid][4 * vq]) = o;
  __syncthreads();
  float core = 0.f;
  if (tid < kD) core = round_bf((red[0][tid] + red[1][tid]) + (red[2][tid] + red[3][tid]));
  uint16_t* orow = p.out + (size_t)bh * kD;
  if (!FUSE_GNORM) {
    if (tid < kD) orow[tid] = (uint16_t)f2bf(core);
    return;
  }
  // Gated RMSNorm over the head [reference kernels.py:115-155].
  if (wid < 2) {
    const float ss = wave_sum(core * core);
    if (lane == 0) sc[wid] = ss;
  }
  __syncthreads();
  if (tid < kD) {
    const float inv = rsqrt_cr((sc[0] + sc[1]) / (float)kD + p.norm_eps);
    const float nb = round_bf(core * inv);
    const float wb = round_bf(ld_param(p.norm_w, tid, p.norm_w_f32));
    const float weighted = round_bf(nb * wb);
    const float z = bf2f(p.packed[(size_t)b * p.packed_stride + p.z_off + h * kD + tid]);
    orow[tid] = (uint16_t)f2bf(weighted * silu_f(z));
  }
}

// Delta rule only (input already convolved), one wave64 per (batch, head,
// 8-column v tile): 16 waves per head, 256 for the 2B shape, so the whole chip
// streams the state. Lane (rg = lane/2, cq = lane%2) owns state rows rg + 32i
// (i < 4), columns 8*tile + 4cq .. +3 (16-byte loads; a row segment of the
// tile is 32 contiguous bytes). Every reduction over the 128 k rows is
// in-thread (4 rows) plus the 32 lanes of equal cq (xor shuffles over lane
// bits 1..5), so the kernel has no barrier and no LDS. Each wave recomputes
// the head's norm factors and gates (q, k are 512 bytes from L2); the state
// is read once and written once.
// Tile placement: four tiles share each 128-byte line of a state row, and
// workgroups are dispatched to the 8 XCDs (each with its own L2) round-robin
// by linear id, so with tile = id % 16 every line was fetched by four L2s
// (FETCH_SIZE 2.6x the state). When B*H is a multiple of 8 the 16 tiles of
// a head are given ids of one residue mod 8 (one XCD): id = xcd + 8*slot,
// head = xcd + 8*(slot / 16), tile = slot % 16.
constexpr int kWT = 8;  // v columns per wave

// Sum over the 32 lanes of equal lane % 2 (every lane gets its class's sum):
// inside each 16-lane row by DPP (xor 2, then rotations by 4 and 8, which
// keep the parity and together cover the row's 8 lanes of one parity), then
// across rows by a swizzle (lane ^ 16) and one permute (lane ^ 32): two LDS-
// unit exchanges per value instead of five.
constexpr int kDppRowRor4 = 0x124, kDppRowRor8 = 0x128;
Q35_DEV float parity_sum(float v) {
  v += dpp_f<Q35_DPP_QUAD_XOR2>(v);
  v += dpp_f<kDppRowRor4>(v);
  v += dpp_f<kDppRowRor8>(v);
  v += swz_xor16_f(v);
  v += __shfl_xor(v, 32);
  return v;
}
Q35_DEV float4 xor_sum_rows(float4 v) {
  return make_float4(parity_sum(v.x), parity_sum(v.y), parity_sum(v.z), parity_sum(v.w));
}

template <bool PF32>  // gate parameters (A_log, dt_bias) fp32, else bf16
__global__ __launch_bounds__(64) void delta_decode_wave(const DeltaArgs p) {
  const int lane = threadIdx.x;
  constexpr int tiles = kD / kWT;
  const int id = blockIdx.x;
  int tile, bh;
  if ((gridDim.x / tiles) % 8 == 0) {
    const int slot = id >> 3;
    tile = slot % tiles;
    bh = (id & 7) + 8 * (slot / tiles);
  } else {
    tile = id % tiles;
    bh = id / tiles;
  }
  const int b = bh / p.H, h = bh - b * p.H;
  const int rg = lane >> 1, cq = lane & 1;
  const int c0 = tile * kWT + 4 * cq;

  // The small loads (q, k, v, gate inputs) are issued before the state: loads
  // retire in order, so the norms and gates are computed while the state is
  // still in flight.
  const uint16_t* srow = p.src + (size_t)b * p.src_stride;
  const float q0 = bf2f(srow[h * kD + lane]), q1 = bf2f(srow[h * kD + 64 + lane]);
  const float k0 = bf2f(srow[p.H * kD + h * kD + lane]), k1 = bf2f(srow[p.H * kD + h * kD + 64 + lane]);
  const uint16_t* vsrc = srow + 2 * p.H * kD + h * kD + c0;
  const float v0 = bf2f(vsrc[0]), v1 = bf2f(vsrc[1]), v2 = bf2f(vsrc[2]), v3 = bf2f(vsrc[3]);
  const uint16_t* prow = p.packed + (size_t)b * p.packed_stride;
  const float a_in = bf2f(prow[p.a_off + h]), b_in = bf2f(prow[p.b_off + h]);
  const float a_log = ld_param(p.a_log, h, PF32), dt_b = ld_param(p.dt_bias, h, PF32);
  float* S = p.state + (size_t)bh * kD * kD;
  float4 st[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const q35_f32x4 v = __builtin_nontemporal_load(reinterpret_cast<const q35_f32x4*>(S + (size_t)(rg + 32 * i) * kD + c0));
    st[i] = make_float4(v.x, v.y, v.z, v.w);
  }
  __builtin_amdgcn_sched_barrier(0);  // keep every load above the math below
  const float g = -expf(a_log) * softplus20(a_in + dt_b);
  const float alpha = expf(g);
  const float beta = 1.0f / (1.0f + expf(-b_in));
  const float q_inv = rsqrt_cr(wave_sum(q0 * q0 + q1 * q1) + 1e-6f);
  const float k_inv = rsqrt_cr(wave_sum(k0 * k0 + k1 * k1) + 1e-6f);
  const float qscale = 0.08838834764831845f;  // fp32(1/sqrt(128))
  // row r of q / k sits in lane r % 64, element r / 64
  float kh[4], qh[4];
  kh[0] = __shfl(k0, rg) * k_inv;
  kh[1] = __shfl(k0, rg + 32) * k_inv;
  kh[2] = __shfl(k1, rg) * k_inv;
  kh[3] = __shfl(k1, rg + 32) * k_inv;
  qh[0] = __shfl(q0, rg) * q_inv * qscale;
  qh[1] = __shfl(q0, rg + 32) * q_inv * qscale;
  qh[2] = __shfl(q1, rg) * q_inv * qscale;
  qh[3] = __shfl(q1, rg + 32) * q_inv * qscale;

  // decay, then m = (alpha S)^T k_hat over the 128 rows
  float4 m = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    st[i].x *= alpha; st[i].y *= alpha; st[i].z *= alpha; st[i].w *= alpha;
    m.x = fmaf(st[i].x, kh[i], m.x); m.y = fmaf(st[i].y, kh[i], m.y);
    m.z = fmaf(st[i].z, kh[i], m.z); m.w = fmaf(st[i].w, kh[i], m.w);
  }
  m = xor_sum_rows(m);
  const float4 d = make_float4(beta * (v0 - m.x), beta * (v1 - m.y), beta * (v2 - m.z), beta * (v3 - m.w));
  // S += k_hat delta^T, o = S^T q_hat
  float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    st[i].x += kh[i] * d.x; st[i].y += kh[i] * d.y; st[i].z += kh[i] * d.z; st[i].w += kh[i] * d.w;
    o.x = fmaf(st[i].x, qh[i], o.x); o.y = fmaf(st[i].y, qh[i], o.y);
    o.z = fmaf(st[i].z, qh[i], o.z); o.w = fmaf(st[i].w, qh[i], o.w);
    __builtin_nontemporal_store(q35_f32x4{st[i].x, st[i].y, st[i].z, st[i].w},
                                reinterpret_cast<q35_f32x4*>(S + (size_t)(rg + 32 * i) * kD + c0));
  }
  o = xor_sum_rows(o);
  if (rg == 0)
    *reinterpret_cast<uint2*>(p.out + (size_t)bh * kD + c0) = make_uint2(pack_bf2(o.x, o.y), pack_bf2(o.z, o.w));
}

// ------------------------------------------------------------- prefill scan
// conv1d_prefill for width-4 filters, 8 channels x 4 tokens per thread: the
// 7 input rows t0-3 .. t0+3 (16-byte loads, rows before 0 are zero) feed the
// 4 outputs; taps are summed oldest first as in conv1d_prefill.
__global__ __launch_bounds__(256) void conv1d_prefill_vec4(const uint16_t* __restrict__ x,
                                                           const uint16_t* __restrict__ w,
                                                           uint16_t* __restrict__ state,
                                                           uint16_t* __restrict__ out, int B, int L,
                                                           int C, int in_stride) {
  constexpr int KW = 4, TOK = 4;
  // 32-bit index arithmetic: the host limits the grid to fewer than 2^31 threads.
  const unsigned idx = blockIdx.x * blockDim.x + threadIdx.x;
  const unsigned cgs = C / 8;
  const unsigned tgs = (L + TOK - 1) / TOK;
  if (idx >= (unsigned)B * tgs * cgs) return;
  const int cg = (int)(idx % cgs);
  const unsigned rest = idx / cgs;
  const int tg = (int)(rest % tgs);
  const int b = (int)(rest / tgs);
  const int c = cg * 8;
  const int t0 = tg * TOK;
  // Every row and tap load is issued before any is used (rows before token 0
  // are read at row 0 and zeroed by a select): a branch per row would make
  // the compiler wait for each load in turn.
  uint4 raw[TOK + KW - 1], wraw[4];
#pragma unroll
  for (int r = 0; r < TOK + KW - 1; ++r) {
    const int sc = min(max(t0 - (KW - 1) + r, 0), L - 1);
    raw[r] = *reinterpret_cast<const uint4*>(x + ((size_t)b * L + sc) * in_stride + c);
  }
#pragma unroll
  for (int q = 0; q < 4; ++q) wraw[q] = *reinterpret_cast<const uint4*>(w + (size_t)c * KW + q * 8);
  __builtin_amdgcn_sched_barrier(0);  // keep every load above the arithmetic
  float xin[TOK + KW - 1][8];
#pragma unroll
  for (int r = 0; r < TOK + KW - 1; ++r) {
    const bool before = t0 - (KW - 1) + r < 0;
    unpack8(raw[r], xin[r]);
#pragma unroll
    for (int e = 0; e < 8; ++e) xin[r][e] = before ? 0.f : xin[r][e];
  }
  float wt[8][KW];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    float f[8];
    unpack8(wraw[q], f);
#pragma unroll
    for (int e = 0; e < 8; ++e) wt[2 * q + e / 4][e % 4] = f[e];
  }
#pragma unroll
  for (int j = 0; j < TOK; ++j) {
    const int t = t0 + j;
    if (t >= L) break;
    float o[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float acc = 0.f;
#pragma unroll
      for (int tap = 0; tap < KW; ++tap) acc = fmaf(xin[j + tap][e], wt[e][tap], acc);
      o[e] = silu_fast(round_bf(acc));
    }
    *reinterpret_cast<uint4*>(out + ((size_t)b * L + t) * C + c) = pack8(o);
    const int pos = t - (L - KW);
    if (pos >= 0) {
#pragma unroll
      for (int e = 0; e < 8; ++e)
        state[((size_t)b * C + c + e) * KW + pos] = (uint16_t)f2bf(xin[j + KW - 1][e]);
    }
  }
}

// Per (token, head) scalars (q_inv, k_inv, g = log alpha, beta) [reference
// kernels.py:713-765], 16 lanes per (token, head) row: 4 rows per wave,
// 16-byte loads of q and k, DPP row sums of squares.
__global__ __launch_bounds__(256) void delta_factors16(const uint16_t* __restrict__ qkv,
                                                       int qkv_stride,
                                                       const uint16_t* __restrict__ packed,
                                                       int packed_stride, const void* a_log,
                                                       const void* dt_bias, int params_f32,
                                                       float* __restrict__ factors, int rows, int H,
                                                       int a_off, int b_off) {
  const int lane = threadIdx.x & 63;
  const int r = (blockIdx.x * 4 + (threadIdx.x >> 6)) * 4 + (lane >> 4);
  const int rc = min(r, rows - 1);
  const int h = rc % H;
  const long long tf = rc / H;
  const int k8 = (lane & 15) * 8;
  const uint16_t* row = qkv + (size_t)tf * qkv_stride;
  float q[8], k[8];
  unpack8(*reinterpret_cast<const uint4*>(row + h * kD + k8), q);
  unpack8(*reinterpret_cast<const uint4*>(row + H * kD + h * kD + k8), k);
  float qs = 0.f, ks = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    qs += q[e] * q[e];
    ks += k[e] * k[e];
  }
  qs = row16_sum(qs);
  ks = row16_sum(ks);
  if ((lane & 15) == 0 && r < rows) {
    const uint16_t* prow = packed + (size_t)tf * packed_stride;
    const float a = bf2f(prow[a_off + h]) + ld_param(dt_bias, h, params_f32);
    const float g = -expf(ld_param(a_log, h, params_f32)) * softplus20(a);
    const float beta = 1.0f / (1.0f + expf(-bf2f(prow[b_off + h])));
    *reinterpret_cast<float4*>(factors + (size_t)r * 4) =
        make_float4(rsqrt_cr(qs + 1e-6f), rsqrt_cr(ks + 1e-6f), g, beta);
  }
}

// Sequential scan over L tokens. One wave per (batch, head, 8-column v tile);
// lane = (v pair vp = lane/16, k-group kg = lane%16 of 8 rows), so the
// [128 x 8] fp32 state tile lives in registers (16 per lane) for the whole
// sequence and every reduction over k is a 16-lane DPP row sum. Tokens are
// processed in groups of kScanAhead; the next group's inputs (q, k, v,
// factors) are requested before the current group is processed, so the loop
// runs at the latency of its arithmetic chain, not of memory. Steps past L
// read the last token and are no-ops (alpha = 1, beta = 0, no store).
constexpr int kScanAhead = 8;

struct ScanIn {
  uint4 q, k;
  uint32_t v;
  float4 f;
};

Q35_DEV ScanIn scan_load(const uint16_t* __restrict__ qkv, int qkv_stride,
                         const float* __restrict__ factors, int b, int L, int H, int h, int t,
                         int kg, int v0) {
  ScanIn in;
  const uint16_t* row = qkv + ((size_t)b * L + t) * qkv_stride;
  in.q = *reinterpret_cast<const uint4*>(row + h * kD + kg * 8);
  in.k = *reinterpret_cast<const uint4*>(row + H * kD + h * kD + kg * 8);
  in.v = *reinterpret_cast<const uint32_t*>(row + 2 * H * kD + h * kD + v0);
  in.f = *reinterpret_cast<const float4*>(factors + (((size_t)b * L + t) * H + h) * 4);
  return in;
}

__global__ __launch_bounds__(64) void delta_scan(const uint16_t* __restrict__ qkv, int qkv_stride,
                                                 const float* __restrict__ factors,
                                                 float* __restrict__ state,
                                                 uint16_t* __restrict__ out, int L, int H) {
  const int lane = threadIdx.x;
  const int tiles = kD / 8;
  const int tile = blockIdx.x % tiles;
  const int bh = blockIdx.x / tiles;
  const int b = bh / H, h = bh - b * H;
  const int kg = lane & 15, vp = lane >> 4;
  const int v0 = tile * 8 + 2 * vp;
  float* S = state + (size_t)bh * kD * kD;
  float s[8][2];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float2 t2 = *reinterpret_cast<const float2*>(S + (size_t)(kg * 8 + i) * kD + v0);
    s[i][0] = t2.x; s[i][1] = t2.y;
  }
  const float qscale = 0.08838834764831845f;
  ScanIn cur[kScanAhead];
#pragma unroll
  for (int j = 0; j < kScanAhead; ++j)
    cur[j] = scan_load(qkv, qkv_stride, factors, b, L, H, h, min(j, L - 1), kg, v0);
  for (int t0 = 0; t0 < L; t0 += kScanAhead) {
    // The next group's inputs are all requested before this group is
    // processed, so they have landed by the copy at the end of the group.
    ScanIn nxt[kScanAhead];
#pragma unroll
    for (int j = 0; j < kScanAhead; ++j)
      nxt[j] = scan_load(qkv, qkv_stride, factors, b, L, H, h, min(t0 + kScanAhead + j, L - 1),
                         kg, v0);
#pragma unroll
    for (int j = 0; j < kScanAhead; ++j) {
      const int t = t0 + j;
      const ScanIn in = cur[j];
      const bool live = t < L;
      float q[8], k[8];
      unpack8(in.q, q);
      unpack8(in.k, k);
      const float4 f = in.f;
      const float alpha = live ? expf(f.z) : 1.0f;
      const float beta = live ? f.w : 0.0f;
      float ma0 = 0.f, ma1 = 0.f, mb0 = 0.f, mb1 = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        k[i] *= f.y;
        q[i] = q[i] * f.x * qscale;
        s[i][0] *= alpha; s[i][1] *= alpha;
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        ma0 = fmaf(s[i][0], k[i], ma0);
        ma1 = fmaf(s[i][1], k[i], ma1);
        mb0 = fmaf(s[i + 4][0], k[i + 4], mb0);
        mb1 = fmaf(s[i + 4][1], k[i + 4], mb1);
      }
      const float m0 = row16_sum(ma0 + mb0), m1 = row16_sum(ma1 + mb1);
      const float d0 = beta * (bf_lo(in.v) - m0), d1 = beta * (bf_hi(in.v) - m1);
      float oa0 = 0.f, oa1 = 0.f, ob0 = 0.f, ob1 = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        s[i][0] += k[i] * d0;
        s[i][1] += k[i] * d1;
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        oa0 = fmaf(s[i][0], q[i], oa0);
        oa1 = fmaf(s[i][1], q[i], oa1);
        ob0 = fmaf(s[i + 4][0], q[i + 4], ob0);
        ob1 = fmaf(s[i + 4][1], q[i + 4], ob1);
      }
      const float o0 = row16_sum(oa0 + ob0), o1 = row16_sum(oa1 + ob1);
      if (live && kg == 0)
        *reinterpret_cast<uint32_t*>(out + (((size_t)b * L + t) * H + h) * kD + v0) = pack_bf2(o0, o1);
    }
#pragma unroll
    for (int j = 0; j < kScanAhead; ++j) cur[j] = nxt[j];
  }
#pragma unroll
  for (int i = 0; i < 8; ++i)
    *reinterpret_cast<float2*>(S + (size_t)(kg * 8 + i) * kD + v0) = make_float2(s[i][0], s[i][1]);
}

// ------------------------------------------------------- chunked prefill
// The recurrence over a chunk of C = 64 tokens in closed form (the UT / WY
// representation of the delta rule), so that the sequential dependence is
// over L/64 chunks instead of L tokens and the work is matrix products. Per
// head, with q, k, v the raw (bf16) conv outputs of the chunk, q_inv, k_inv
// their norm factors, K = diag(k_inv) k and Q = diag(q_inv / sqrt(D)) q the
// scaled vectors of the recurrence, G_i the cumulative log-decay inside the
// chunk and gamma_i = e^{G_i}:
//   A[i][j] = beta_i e^{G_i-G_j} (K_i . K_j)  (j < i),   T = (I + A)^{-1}
//   W = T diag(beta gamma) K,   U0 = T diag(beta) V      (independent of S)
//   U = U0 - W S                                           (the delta vectors)
//   O = diag(gamma) Q S + P U,  P[i][j] = e^{G_i-G_j} (Q_i . K_j)  (j <= i)
//   S <- gamma_C S + K''^T U,   K''[j] = e^{G_C-G_j} K_j
// which is the token loop unrolled exactly (every decay factor is e^{a-b}
// with a <= b, so nothing overflows). Padding tokens past L carry q = k = v =
// 0, g = 0, beta = 0 and leave S unchanged.
//
// The products run on the bf16 matrix cores (v_mfma_f32_16x16x32_bf16, fp32
// accumulation). q, k and v are bf16 values, so a product with one of them
// as an operand is exact in the MFMA; the scale factors are applied outside:
// K K^T and Q K^T are products of the raw rows, W = (T diag(beta gamma
// k_inv)) k, U0 = (T diag(beta)) v, diag(gamma) Q S = diag(sc) (q S) with sc =
// gamma q_inv / sqrt(D), and K''^T U = k^T (diag(f) U) with f_j = e^{G_C-G_j}
// k_inv_j. An fp32 operand x is split into x_hi = bf16(x) and x_lo = bf16(x -
// x_hi), |x - x_hi - x_lo| <= 2^-18 |x|: its product with a bf16 operand b is
// x_hi b + x_lo b (two MFMAs), a product of two fp32 operands x_hi y_hi +
// x_hi y_lo + x_lo y_hi (three; the dropped x_lo y_lo is below 2^-16 of the
// product). The operands whose rounding reaches the state directly, the
// scaled rows of T (into W and U0) and diag(f) U (into S), are split in three
// (x_mid = bf16(x - x_hi), x_lo = bf16(x - x_hi - x_mid), within 2^-27 |x|):
// with that the state stays within the fp32 token loop's own rounding of an
// exact evaluation, where two-part splits of these operands left errors ~40x
// larger. The triangular solve for T stays in fp32 (v_mfma_f32_16x16x4f32).
//   delta_chunk_prep : one workgroup per (chunk, head): conv, factors, A and
//     P, T by 16 x 16 blocks (diagonal blocks by forward substitution, the
//     rest as MFMA products), W and U0, and every operand of the two later
//     kernels, written in their per-lane MFMA operand order (coalesced 1 KiB
//     rows of 16-byte lane entries).
//   delta_chunk_scan : one workgroup per (16-column v tile, head): the
//     [128 x 16] state tile in LDS and only the recurrence (U = U0 - W S,
//     S <- gamma_C S + K''^T U) per chunk; the state entering each chunk and
//     U are stored as split operands of the output kernel.
//   delta_chunk_out  : one workgroup per (chunk, head), all in parallel:
//     O = diag(sc) (q S) + P U from the snapshots.
// MFMA 16x16x32 bf16 (wave64): A[16 x 32]: lane l holds row l%16, 8
// consecutive k at 8*(l/16); B[32 x 16]: column l%16, the same 8 k; C[16 x
// 16]: rows 4*(l/16) + e (e < 4) of column l%16. The fp32 16x16x4 form has
// A: row l%16, k l/16; B: k l/16, column l%16; the same C.
constexpr int kChunk = 64;
constexpr int kRS = 136;  // bf16 row stride of the raw q / k / v tiles in LDS
constexpr int kAS = 68;   // fp32 row stride of A and of T
constexpr int kXS = 36;   // fp32 row stride of the per-wave transpose tiles
constexpr float kQScale = 0.08838834764831845f;  // 1 / sqrt(D)
// Workspace floats per (batch, head, chunk); every operand is a row of 64
// lane entries of 16 bytes (8 bf16, or a float4 for U0):
//   W   [row tile 4][k step 4][hi, lo]   A operand of W S
//   U0  [row tile 4][v tile 8]           C layout
//   kT  [k tile 8][t step 2]             A operand of k^T (diag(f) U)
//   q   [row tile 4][k step 4]           A operand of q S
//   P   [row tile 4][t step 2][hi, lo]   A operand of P U (zero above the diagonal)
//   f [64], sc [64]
constexpr int kOffW = 0, kOffU0 = 8192, kOffKT = 16384, kOffQ = 20480, kOffP = 24576,
              kOffF = 28672, kOffSc = 28736;
constexpr int kChunkFloats = 28800;
// Snapshot floats per (batch, head, chunk): the state entering the chunk as
// the B operand of q S, [v tile][k step 4][hi, lo] (2048 floats per v tile),
// then U as the B operand of P U, [v tile][t step 2][hi, lo] (1024 floats per
// v tile) from kSnapU.
constexpr int kSnapSTile = 2048, kSnapU = 8 * kSnapSTile, kSnapUTile = 1024;
constexpr int kSnapFloats = kSnapU + 8 * kSnapUTile;

Q35_DEV q35_f32x4 mfma4(float a, float b, q35_f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

Q35_DEV q35_f32x4 mfma_bf(const uint4 a, const uint4 b, q35_f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(q35_bf16x8, a),
                                                 __builtin_bit_cast(q35_bf16x8, b), c, 0, 0, 0);
}

// x = hi + lo (+ a remainder below 2^-18 |x|) for 8 fp32 values: hi = bf16(x)
// (round to nearest even), lo = bf16(x - hi) (x - hi is exact in fp32).
struct Split8 {
  uint4 hi, lo;
};
Q35_DEV Split8 split8(const float4 a, const float4 b) {
  const float x[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
  uint32_t h[4], l[4];
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    h[p] = pack_bf2(x[2 * p], x[2 * p + 1]);
    l[p] = pack_bf2(x[2 * p] - bf_lo(h[p]), x[2 * p + 1] - bf_hi(h[p]));
  }
  return Split8{make_uint4(h[0], h[1], h[2], h[3]), make_uint4(l[0], l[1], l[2], l[3])};
}

// The same in three parts: x = hi + mid + lo within 2^-27 |x|.
struct Split8x3 {
  uint4 hi, mid, lo;
};
Q35_DEV Split8x3 split8x3(const float4 a, const float4 b) {
  const float x[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
  uint32_t h[4], m[4], l[4];
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    h[p] = pack_bf2(x[2 * p], x[2 * p + 1]);
    const float r0 = x[2 * p] - bf_lo(h[p]), r1 = x[2 * p + 1] - bf_hi(h[p]);
    m[p] = pack_bf2(r0, r1);
    l[p] = pack_bf2(r0 - bf_lo(m[p]), r1 - bf_hi(m[p]));
  }
  return Split8x3{make_uint4(h[0], h[1], h[2], h[3]), make_uint4(m[0], m[1], m[2], m[3]),
                  make_uint4(l[0], l[1], l[2], l[3])};
}

Q35_DEV float4 mul4(const float4 a, const float4 b) {
  return make_float4(a.x * b.x, a.y * b.y, a.z * b.z, a.w * b.w);
}

// Optional inputs of chunk prep: with CONV, qkv is the raw packed projection
// and the width-4 causal conv + SiLU of conv1d_prefill_vec4 is applied here
// (the conv output is never stored); the conv state receives the last four
// input rows, as conv1d_prefill writes it.
struct ConvIn {
  const uint16_t* w;  // [3*H*D, 4] taps
  uint16_t* state;    // [B, 3*H*D, 4]
};

// PF32: A_log and dt_bias are fp32 (else bf16); a template parameter, since a
// run-time branch between two load forms makes the compiler wait for each.
template <bool PF32, bool CONV>
__global__ __launch_bounds__(256) void delta_chunk_prep(const uint16_t* __restrict__ qkv,
                                                        int qkv_stride,
                                                        const uint16_t* __restrict__ packed,
                                                        int packed_stride, const void* a_log,
                                                        const void* dt_bias, int params_f32,
                                                        int a_off, int b_off,
                                                        float* __restrict__ ws,
                                                        float* __restrict__ gc_out, int L, int H,
                                                        int nC, ConvIn conv) {
  const int c = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wid = tid >> 6;
  const int col = lane & 15, g4 = lane >> 4;
  const size_t bhc = ((size_t)b * H + h) * nC + c;
  float* wsb = ws + bhc * kChunkFloats;
  __shared__ alignas(16) uint16_t Qr[kChunk * kRS];  // raw q, k, v rows (bf16)
  __shared__ alignas(16) uint16_t Kr[kChunk * kRS];
  __shared__ alignas(16) uint16_t Vr[kChunk * kRS];
  __shared__ alignas(16) float Am[kChunk * kAS];     // A (strictly lower)
  __shared__ alignas(16) float Tm[kChunk * kAS];     // T = (I + A)^{-1} (lower)
  __shared__ alignas(16) float Xs[4][kChunk * kXS];  // per-wave transpose tiles
  __shared__ alignas(16) float G_s[kChunk], b_s[kChunk], qinv_s[kChunk], kinv_s[kChunk], wsc_s[kChunk];

  // The token's gate inputs and the head's parameters, requested first (with
  // CONV they are then in flight during the conv below).
  const int ti = tid >> 2;
  const int tcg = min(c * kChunk + ti, L - 1);
  const uint16_t* prow0 = packed + ((size_t)b * L + tcg) * packed_stride;
  const float a_raw = bf2f(prow0[a_off + h]), b_raw = bf2f(prow0[b_off + h]);
  const float alog = ld_param(a_log, h, PF32), dtb = ld_param(dt_bias, h, PF32);
  if (CONV) {
    // 0. the conv of this chunk and head into Qr / Kr / Vr. Thread items are
    //    (8-channel group g of q, k or v; 4 tokens), 768 of them (48 groups x
    //    16 token blocks), three per thread, each with its 7 input rows (4 + 3
    //    before; rows before token 0 are zero) and 4 x 8 taps; every load of
    //    the three items is issued before any is used. The bf16 rounding of
    //    the conv sums takes one conversion per pair of values.
    {
      constexpr int NI = 3;
      uint4 raw[NI][7], wr[NI][4];
#pragma unroll
      for (int it = 0; it < NI; ++it) {
        const int item = tid + 256 * it;
        const int g = item % 48, t0 = (item / 48) * 4;
        const int ch = (g >> 4) * H * kD + h * kD + (g & 15) * 8;  // conv channel of the group
#pragma unroll
        for (int r = 0; r < 7; ++r) {
          const int tr = min(max(c * kChunk + t0 - 3 + r, 0), L - 1);
          raw[it][r] = *reinterpret_cast<const uint4*>(qkv + ((size_t)b * L + tr) * qkv_stride + ch);
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) wr[it][q] = *reinterpret_cast<const uint4*>(conv.w + (size_t)ch * 4 + q * 8);
      }
#pragma unroll
      for (int it = 0; it < NI; ++it) {
        const int item = tid + 256 * it;
        const int g = item % 48, t0 = (item / 48) * 4;
        const int arr = g >> 4, d = (g & 15) * 8;
        const int ch = arr * H * kD + h * kD + d;
        uint16_t* dst = arr == 0 ? Qr : (arr == 1 ? Kr : Vr);
        float wt[8][4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          float f[8];
          unpack8(wr[it][q], f);
#pragma unroll
          for (int e = 0; e < 8; ++e) wt[2 * q + e / 4][e % 4] = f[e];
        }
        float xr[7][8];
#pragma unroll
        for (int r = 0; r < 7; ++r) {
          const bool before = c * kChunk + t0 - 3 + r < 0;
          unpack8(before ? make_uint4(0u, 0u, 0u, 0u) : raw[it][r], xr[r]);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int t = c * kChunk + t0 + j;
          float acc[8], o[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            acc[e] = 0.f;
#pragma unroll
            for (int tap = 0; tap < 4; ++tap) acc[e] = fmaf(xr[j + tap][e], wt[e][tap], acc[e]);
          }
#pragma unroll
          for (int p2 = 0; p2 < 4; ++p2) {
            const uint32_t hb = pack_bf2(acc[2 * p2], acc[2 * p2 + 1]);
            o[2 * p2] = silu_fast(bf_lo(hb));
            o[2 * p2 + 1] = silu_fast(bf_hi(hb));
          }
          *reinterpret_cast<uint4*>(dst + (t0 + j) * kRS + d) = pack8(o);  // the conv output is bf16
          const int pos = t - (L - 4);
          if (t < L && pos >= 0) {
#pragma unroll
            for (int e = 0; e < 8; ++e)
              conv.state[((size_t)b * 3 * H * kD + ch + e) * 4 + pos] = (uint16_t)f2bf(xr[j + 3][e]);
          }
        }
      }
    }
    __syncthreads();
  }

  // 1. per token (4 threads, 32 dims each): q_inv, k_inv = rsqrt(sum of
  //    squares + 1e-6) over the head (quad sum), g = -e^{A_log} softplus(a +
  //    dt_bias), beta = sigmoid(b) [reference kernels.py:713-765]. The raw
  //    rows of tokens past L become zeros; the q rows are also the output
  //    kernel's A operand (row tile i/16, k step = the thread's quarter,
  //    lane (i%16) + 16u for its 8-dim group u).
  {
    const int i = tid >> 2, qq = tid & 3;
    const int t = c * kChunk + i;
    const bool live = t < L;
    uint4 rq[4], rk[4], rv[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int d = qq * 32 + u * 8;
      if (CONV) {
        rq[u] = *reinterpret_cast<const uint4*>(&Qr[i * kRS + d]);
        rk[u] = *reinterpret_cast<const uint4*>(&Kr[i * kRS + d]);
        rv[u] = *reinterpret_cast<const uint4*>(&Vr[i * kRS + d]);
      } else {
        const uint16_t* row = qkv + ((size_t)b * L + min(t, L - 1)) * qkv_stride;
        rq[u] = *reinterpret_cast<const uint4*>(row + h * kD + d);
        rk[u] = *reinterpret_cast<const uint4*>(row + H * kD + h * kD + d);
        rv[u] = *reinterpret_cast<const uint4*>(row + 2 * H * kD + h * kD + d);
      }
    }
    float qs = 0.f, ks = 0.f;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      float fq[8], fk[8];
      unpack8(rq[u], fq);
      unpack8(rk[u], fk);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        qs += fq[e] * fq[e];
        ks += fk[e] * fk[e];
      }
    }
    qs += __shfl_xor(qs, 1, 64);
    ks += __shfl_xor(ks, 1, 64);
    qs += __shfl_xor(qs, 2, 64);
    ks += __shfl_xor(ks, 2, 64);
    if (!live) {
#pragma unroll
      for (int u = 0; u < 4; ++u) rq[u] = rk[u] = rv[u] = make_uint4(0u, 0u, 0u, 0u);
    }
    if (!CONV || !live) {
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int d = qq * 32 + u * 8;
        *reinterpret_cast<uint4*>(&Qr[i * kRS + d]) = rq[u];
        *reinterpret_cast<uint4*>(&Kr[i * kRS + d]) = rk[u];
        *reinterpret_cast<uint4*>(&Vr[i * kRS + d]) = rv[u];
      }
    }
#pragma unroll
    for (int u = 0; u < 4; ++u)
      *reinterpret_cast<uint4*>(wsb + kOffQ + (((i >> 4) * 4 + qq) * 64 + (i & 15) + 16 * u) * 4) = rq[u];
    if (qq == 0) {
      qinv_s[i] = rsqrt_cr(qs + 1e-6f);
      kinv_s[i] = rsqrt_cr(ks + 1e-6f);
      G_s[i] = live ? -expf(alog) * softplus20(a_raw + dtb) : 0.f;  // g = log alpha, summed below
      b_s[i] = live ? 1.0f / (1.0f + expf(-b_raw)) : 0.f;
    }
  }
  __syncthreads();

  // 2. cumulative log-decay G (inclusive scan over the chunk, wave 0) and the
  //    per-token scales: f, sc (to the workspace) and beta gamma k_inv (W).
  if (wid == 0) {
    float gs = G_s[lane];
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const float up = __shfl_up(gs, o, 64);
      if (lane >= o) gs += up;
    }
    const float glast = __shfl(gs, 63, 64);
    const float gam = expf(gs), ki = kinv_s[lane];
    G_s[lane] = gs;
    wsc_s[lane] = b_s[lane] * gam * ki;
    wsb[kOffF + lane] = expf(glast - gs) * ki;
    wsb[kOffSc + lane] = gam * qinv_s[lane] * kQScale;
    if (lane == 0) gc_out[bhc] = expf(glast);
  }
  __syncthreads();

  // 3. A (into LDS) and P (split, to the workspace) on the lower block
  //    triangle. P is exported by (row tile rt, t step s) groups of two tiles
  //    (jt = 2s, 2s + 1; a tile above the diagonal is zero), each group on one
  //    wave, so its transpose goes through the wave's own tile: wave 0 takes
  //    (3, 0) and (0, 0), wave 1 (3, 1) and (2, 1), wave 2 (1, 0), wave 3
  //    (2, 0): 3/3/2/2 tiles. Operands are raw rows of 16 bytes.
  {
    const unsigned groups = wid == 0 ? 0x0300u : (wid == 1 ? 0x0607u : (wid == 2 ? 0x01u : 0x02u));
    const int ng = wid < 2 ? 2 : 1;
    float* xs = Xs[wid];
    for (int n = 0; n < ng; ++n) {
      const int gi = (groups >> (8 * n)) & 0xff;
      const int rt = gi & 3, s = gi >> 2;
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) {
        const int jt = 2 * s + jj;
        q35_f32x4 kk = {0.f, 0.f, 0.f, 0.f}, qk = kk;
        if (jt <= rt) {
          const uint16_t* ki = &Kr[(16 * rt + col) * kRS + 8 * g4];
          const uint16_t* kj = &Kr[(16 * jt + col) * kRS + 8 * g4];
          const uint16_t* qi = &Qr[(16 * rt + col) * kRS + 8 * g4];
#pragma unroll
          for (int st = 0; st < 4; ++st) {
            const uint4 x = *reinterpret_cast<const uint4*>(ki + 32 * st);
            const uint4 y = *reinterpret_cast<const uint4*>(kj + 32 * st);
            const uint4 z = *reinterpret_cast<const uint4*>(qi + 32 * st);
            kk = mfma_bf(x, y, kk);  // (k k^T)[i][j]
            qk = mfma_bf(z, y, qk);  // (q k^T)[i][j]
          }
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int i = 16 * rt + 4 * g4 + e, j = 16 * jt + col;
          const float dec = j <= i ? expf(G_s[i] - G_s[j]) : 0.f;
          if (jt <= rt) Am[i * kAS + j] = j < i ? b_s[i] * (kinv_s[i] * kinv_s[j]) * dec * kk[e] : 0.f;
          xs[(4 * g4 + e) * kXS + 16 * jj + col] = qinv_s[i] * kQScale * kinv_s[j] * dec * qk[e];
        }
      }
      // the group as the A operand (row 16 rt + l%16, columns 32 s + 8(l/16)
      // .. +7); the wave's own LDS stores complete before its later reads
      const float* pr = &xs[col * kXS + 8 * g4];
      const Split8 sp = split8(*reinterpret_cast<const float4*>(pr), *reinterpret_cast<const float4*>(pr + 4));
      uint4* dp = reinterpret_cast<uint4*>(wsb + kOffP) + (rt * 2 + s) * 128 + lane;
      dp[0] = sp.hi;
      dp[64] = sp.lo;
    }
  }
  __syncthreads();

  // 4. T = (I + A)^{-1} by 16 x 16 blocks (A strictly lower triangular):
  //    T_II = (I + A_II)^{-1} by forward substitution (wave I, lane = column),
  //    then T_IJ = -T_II sum_{K=J}^{I-1} A_IK T_KJ level by level (I - J =
  //    1, 2, 3) as 16 x 16 x 16 fp32 MFMA products, one block per wave.
  {
    const int I = wid, j = lane & 15;
    float t[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      float a0 = 0.f, a1 = 0.f;
#pragma unroll
      for (int k = 0; k + 1 < i; k += 2) {
        a0 = fmaf(Am[(16 * I + i) * kAS + 16 * I + k], t[k], a0);
        a1 = fmaf(Am[(16 * I + i) * kAS + 16 * I + k + 1], t[k + 1], a1);
      }
      if (i & 1) a0 = fmaf(Am[(16 * I + i) * kAS + 16 * I + i - 1], t[i - 1], a0);
      t[i] = (i == j ? 1.f : 0.f) - (a0 + a1);
    }
    if (lane < 16) {
#pragma unroll
      for (int i = 0; i < 16; ++i) Tm[(16 * I + i) * kAS + 16 * I + j] = t[i];
    }
  }
  __syncthreads();
  // C += A B for 16 x 16 tiles in LDS (A row stride kAS, B row stride sb).
  auto mm16 = [&](const float* at, const float* bt, int sb, q35_f32x4 c) {
#pragma unroll
    for (int st = 0; st < 4; ++st) c = mfma4(at[col * kAS + 4 * st + g4], bt[(4 * st + g4) * sb + col], c);
    return c;
  };
  for (int d = 1; d < 4; ++d) {
    if (wid < 4 - d) {
      const int J = wid, I = wid + d;
      q35_f32x4 x = {0.f, 0.f, 0.f, 0.f};
      for (int K = J; K < I; ++K) x = mm16(&Am[16 * I * kAS + 16 * K], &Tm[16 * K * kAS + 16 * J], kAS, x);
      float* xs = Xs[wid];
#pragma unroll
      for (int e = 0; e < 4; ++e) xs[(4 * g4 + e) * 17 + col] = x[e];
      // the wave's own LDS stores complete before its later reads (in-order LDS)
      const q35_f32x4 tt = mm16(&Tm[16 * I * kAS + 16 * I], xs, 17, q35_f32x4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
      for (int e = 0; e < 4; ++e) Tm[(16 * I + 4 * g4 + e) * kAS + 16 * J + col] = -tt[e];
    }
    __syncthreads();
  }

  // 5. W = (T diag(beta gamma k_inv)) k and U0 = (T diag(beta)) v for the
  //    wave's two dim (v) tiles dt = 2 wid + dd and every row tile: the T rows
  //    are split, the k / v columns (8 consecutive tokens of one dim; the kT
  //    operand of the scan) are exact. T is lower triangular: row tile rt
  //    needs the t steps s <= rt/2, and the lane's 8 columns of block
  //    2s + (l/16)/2 are zero when that block is above the diagonal.
  {
    uint4 kop[2][2], vop[2][2];
#pragma unroll
    for (int dd = 0; dd < 2; ++dd)
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const int dim = 16 * (2 * wid + dd) + col;
        const uint16_t* kc = &Kr[(32 * s + 8 * g4) * kRS + dim];
        const uint16_t* vc = &Vr[(32 * s + 8 * g4) * kRS + dim];
        uint32_t kw[4], vw[4];
#pragma unroll
        for (int p = 0; p < 4; ++p) {
          kw[p] = (uint32_t)kc[2 * p * kRS] | ((uint32_t)kc[(2 * p + 1) * kRS] << 16);
          vw[p] = (uint32_t)vc[2 * p * kRS] | ((uint32_t)vc[(2 * p + 1) * kRS] << 16);
        }
        kop[dd][s] = make_uint4(kw[0], kw[1], kw[2], kw[3]);
        vop[dd][s] = make_uint4(vw[0], vw[1], vw[2], vw[3]);
        *reinterpret_cast<uint4*>(wsb + kOffKT + (((2 * wid + dd) * 2 + s) * 64 + lane) * 4) = kop[dd][s];
      }
    float* xw = Xs[wid];  // W rows 0..63, columns 32 wid .. +31
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) {
      q35_f32x4 w[2], u[2];
#pragma unroll
      for (int dd = 0; dd < 2; ++dd) w[dd] = u[dd] = q35_f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s <= rt / 2; ++s) {
        const int j0 = 32 * s + 8 * g4;
        float4 t0 = make_float4(0.f, 0.f, 0.f, 0.f), t1 = t0;
        if (2 * s + (g4 >> 1) <= rt) {
          t0 = *reinterpret_cast<const float4*>(&Tm[(16 * rt + col) * kAS + j0]);
          t1 = *reinterpret_cast<const float4*>(&Tm[(16 * rt + col) * kAS + j0 + 4]);
        }
        const Split8x3 sw = split8x3(mul4(t0, *reinterpret_cast<const float4*>(&wsc_s[j0])),
                                     mul4(t1, *reinterpret_cast<const float4*>(&wsc_s[j0 + 4])));
        const Split8x3 su = split8x3(mul4(t0, *reinterpret_cast<const float4*>(&b_s[j0])),
                                     mul4(t1, *reinterpret_cast<const float4*>(&b_s[j0 + 4])));
#pragma unroll
        for (int dd = 0; dd < 2; ++dd) {
          w[dd] = mfma_bf(sw.hi, kop[dd][s], w[dd]);
          u[dd] = mfma_bf(su.hi, vop[dd][s], u[dd]);
        }
#pragma unroll
        for (int dd = 0; dd < 2; ++dd) {
          w[dd] = mfma_bf(sw.mid, kop[dd][s], w[dd]);
          u[dd] = mfma_bf(su.mid, vop[dd][s], u[dd]);
        }
#pragma unroll
        for (int dd = 0; dd < 2; ++dd) {
          w[dd] = mfma_bf(sw.lo, kop[dd][s], w[dd]);
          u[dd] = mfma_bf(su.lo, vop[dd][s], u[dd]);
        }
      }
#pragma unroll
      for (int dd = 0; dd < 2; ++dd) {
        *reinterpret_cast<float4*>(wsb + kOffU0 + ((rt * 8 + 2 * wid + dd) * 64 + lane) * 4) =
            make_float4(u[dd][0], u[dd][1], u[dd][2], u[dd][3]);
#pragma unroll
        for (int e = 0; e < 4; ++e) xw[(16 * rt + 4 * g4 + e) * kXS + 16 * dd + col] = w[dd][e];
      }
    }
    // W as the scan's A operand: row 16 rt + l%16, dims 32 wid + 8(l/16) .. +7
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) {
      const float* wr = &xw[(16 * rt + col) * kXS + 8 * g4];
      const Split8 sp = split8(*reinterpret_cast<const float4*>(wr), *reinterpret_cast<const float4*>(wr + 4));
      uint4* dp = reinterpret_cast<uint4*>(wsb + kOffW) + (rt * 4 + wid) * 128 + lane;
      dp[0] = sp.hi;
      dp[64] = sp.lo;
    }
  }
}

// The fp32 state tile lives in registers, in the C layout of the state update
// (wave w owns k tiles 2w and 2w + 1: rows 16 kt + 4(l/16) + e of column
// l%16). LDS holds only its bf16 hi / lo parts, transposed ([column][k]) and
// double-buffered, as the B operand of W S (8 consecutive k of one column:
// one 16-byte read per part); each wave splits only its own rows. U likewise:
// the wave that computes rows of U splits them (diag(f) U in three parts for
// the state update, U in two for the snapshot) into transposed LDS tiles.
constexpr int kSB = kD + 8;      // bf16 per transposed state column
constexpr int kUB = kChunk + 8;  // bf16 per transposed U column

// hi / lo (two parts) of 4 values as bf16 pairs
Q35_DEV void split4(const float* x, uint2& hi, uint2& lo) {
  const uint32_t h0 = pack_bf2(x[0], x[1]), h1 = pack_bf2(x[2], x[3]);
  hi = make_uint2(h0, h1);
  lo = make_uint2(pack_bf2(x[0] - bf_lo(h0), x[1] - bf_hi(h0)), pack_bf2(x[2] - bf_lo(h1), x[3] - bf_hi(h1)));
}

__global__ __launch_bounds__(256) void delta_chunk_scan(const float* __restrict__ ws,
                                                        const float* __restrict__ gc,
                                                        float* __restrict__ state,
                                                        float* __restrict__ snap, int H, int nC) {
  // Workgroups are dispatched to the 8 XCDs round-robin by linear id; the 8
  // v tiles of a head read the same chunk operands, so they are placed on one
  // XCD (one L2 fill serves all 8): id = xcd + 8*slot, head = xcd + 8*(slot/8).
  const int id = blockIdx.x, b = blockIdx.y;
  int tile, h;
  if (H % 8 == 0) {
    const int slot = id >> 3;
    h = (id & 7) + 8 * (slot >> 3);
    tile = slot & 7;
  } else {
    tile = id & 7;
    h = id >> 3;
  }
  const int tid = threadIdx.x;
  const int lane = tid & 63, wid = tid >> 6;
  const int col = lane & 15, g4 = lane >> 4;
  const size_t bh = (size_t)b * H + h;
  __shared__ alignas(16) uint16_t Sp[2][2][16 * kSB];  // [buffer][hi, lo][column][k]
  // diag(f) U hi, mid, lo and U hi, lo, each [column][t]
  __shared__ alignas(16) uint16_t Up[5][16 * kUB];
  float* Sg = state + bh * kD * kD + tile * 16;
  float sr[2][4];
#pragma unroll
  for (int dd = 0; dd < 2; ++dd)
#pragma unroll
    for (int e = 0; e < 4; ++e) sr[dd][e] = Sg[(size_t)(16 * (2 * wid + dd) + 4 * g4 + e) * kD + col];
  auto split_state = [&](int buf) {
#pragma unroll
    for (int dd = 0; dd < 2; ++dd) {
      uint2 hi, lo;
      split4(sr[dd], hi, lo);
      const int k0 = 16 * (2 * wid + dd) + 4 * g4;
      *reinterpret_cast<uint2*>(&Sp[buf][0][col * kSB + k0]) = hi;
      *reinterpret_cast<uint2*>(&Sp[buf][1][col * kSB + k0]) = lo;
    }
  };
  // This wave's operands of one chunk: row tile wid of W (4 k steps, hi and
  // lo) and of U0, f of the lane's 4 rows of U, k tiles 2 wid and 2 wid + 1
  // of kT (2 t steps). Chunk c + 1 is requested in two halves between the
  // MFMAs of chunk c (the kT half during the U phase, the W half during the
  // state update).
  struct ChunkOps {
    uint4 w[4][2], kt[2][2];
    float4 f, u0;
    float gC;
  };
  auto load_k = [&](int c, ChunkOps& op) {
    const float* wsb = ws + (bh * nC + c) * kChunkFloats;
#pragma unroll
    for (int dd = 0; dd < 2; ++dd)
#pragma unroll
      for (int s = 0; s < 2; ++s)
        op.kt[dd][s] = *reinterpret_cast<const uint4*>(wsb + kOffKT + (((2 * wid + dd) * 2 + s) * 64 + lane) * 4);
    op.gC = gc[bh * nC + c];
  };
  auto load_w = [&](int c, ChunkOps& op) {
    const float* wsb = ws + (bh * nC + c) * kChunkFloats;
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int hl = 0; hl < 2; ++hl)
        op.w[s][hl] = *reinterpret_cast<const uint4*>(wsb + kOffW + (((wid * 4 + s) * 2 + hl) * 64 + lane) * 4);
    op.u0 = *reinterpret_cast<const float4*>(wsb + kOffU0 + ((wid * 8 + tile) * 64 + lane) * 4);
    op.f = *reinterpret_cast<const float4*>(wsb + kOffF + 16 * wid + 4 * g4);
  };
  // Two operand sets alternate (chunk c computes from one while chunk c + 1
  // loads into the other): copying a set whose loads are still in flight
  // would wait for them.
  ChunkOps opa, opb;
  load_k(0, opa);
  load_w(0, opa);
  split_state(0);
  __syncthreads();
#define Q35_SCAN_CHUNK(CUR, NXT, C)                                                           \
  do {                                                                                        \
    const int ci = (C); /* not named c: the argument is an expression in the loop's c */     \
    const int cn = min(ci + 1, nC - 1);                                                       \
    const uint16_t* sh = Sp[ci & 1][0];                                                       \
    const uint16_t* sl = Sp[ci & 1][1];                                                       \
    float* sp = snap + (bh * nC + ci) * kSnapFloats;                                          \
    /* snapshot of the entering state: wave wid stores k step wid (hi, lo) */                \
    {                                                                                         \
      uint4* dp = reinterpret_cast<uint4*>(sp + tile * kSnapSTile) + wid * 128 + lane;        \
      dp[0] = *reinterpret_cast<const uint4*>(&sh[col * kSB + 32 * wid + 8 * g4]);            \
      dp[64] = *reinterpret_cast<const uint4*>(&sl[col * kSB + 32 * wid + 8 * g4]);           \
    }                                                                                         \
    /* U = U0 - W S (rows 16 wid .., this v tile): W_hi S_hi, W_hi S_lo, W_lo S_hi */        \
    q35_f32x4 a0 = {0.f, 0.f, 0.f, 0.f}, a1 = a0, a2 = a0;                                    \
    _Pragma("unroll") for (int s = 0; s < 4; ++s) {                                           \
      const uint4 bh_ = *reinterpret_cast<const uint4*>(&sh[col * kSB + 32 * s + 8 * g4]);    \
      const uint4 bl_ = *reinterpret_cast<const uint4*>(&sl[col * kSB + 32 * s + 8 * g4]);    \
      a0 = mfma_bf(CUR.w[s][0], bh_, a0);                                                     \
      a1 = mfma_bf(CUR.w[s][0], bl_, a1);                                                     \
      a2 = mfma_bf(CUR.w[s][1], bh_, a2);                                                     \
    }                                                                                         \
    {                                                                                         \
      const float u0v[4] = {CUR.u0.x, CUR.u0.y, CUR.u0.z, CUR.u0.w};                          \
      const float fv[4] = {CUR.f.x, CUR.f.y, CUR.f.z, CUR.f.w};                               \
      float u[4], fu[4];                                                                      \
      _Pragma("unroll") for (int e = 0; e < 4; ++e) {                                         \
        u[e] = u0v[e] - ((a0[e] + a1[e]) + a2[e]);                                            \
        fu[e] = u[e] * fv[e];                                                                 \
      }                                                                                       \
      /* diag(f) U in three parts, U in two, into the transposed tiles */                    \
      uint2 h3, m3, l3, h2, l2;                                                               \
      split4(fu, h3, m3);                                                                     \
      {                                                                                       \
        const float r[4] = {fu[0] - bf_lo(h3.x) - bf_lo(m3.x), fu[1] - bf_hi(h3.x) - bf_hi(m3.x), \
                            fu[2] - bf_lo(h3.y) - bf_lo(m3.y), fu[3] - bf_hi(h3.y) - bf_hi(m3.y)}; \
        l3 = make_uint2(pack_bf2(r[0], r[1]), pack_bf2(r[2], r[3]));                          \
      }                                                                                       \
      split4(u, h2, l2);                                                                      \
      const int o = col * kUB + 16 * wid + 4 * g4;                                            \
      *reinterpret_cast<uint2*>(&Up[0][o]) = h3;                                              \
      *reinterpret_cast<uint2*>(&Up[1][o]) = m3;                                              \
      *reinterpret_cast<uint2*>(&Up[2][o]) = l3;                                              \
      *reinterpret_cast<uint2*>(&Up[3][o]) = h2;                                              \
      *reinterpret_cast<uint2*>(&Up[4][o]) = l2;                                              \
    }                                                                                         \
    load_k(cn, NXT);                                                                          \
    __syncthreads();                                                                          \
    /* snapshot of U: waves 0 and 1 store t step wid (hi, lo) */                             \
    if (wid < 2) {                                                                            \
      uint4* dp = reinterpret_cast<uint4*>(sp + kSnapU + tile * kSnapUTile) + wid * 128 + lane; \
      dp[0] = *reinterpret_cast<const uint4*>(&Up[3][col * kUB + 32 * wid + 8 * g4]);         \
      dp[64] = *reinterpret_cast<const uint4*>(&Up[4][col * kUB + 32 * wid + 8 * g4]);        \
    }                                                                                         \
    /* S <- gamma_C S + k^T (diag(f) U) (k tiles 2 wid, 2 wid + 1) */                        \
    q35_f32x4 ah[2], am[2], al[2];                                                            \
    _Pragma("unroll") for (int dd = 0; dd < 2; ++dd) {                                        \
      ah[dd] = q35_f32x4{CUR.gC * sr[dd][0], CUR.gC * sr[dd][1], CUR.gC * sr[dd][2], CUR.gC * sr[dd][3]}; \
      am[dd] = al[dd] = q35_f32x4{0.f, 0.f, 0.f, 0.f};                                        \
    }                                                                                         \
    _Pragma("unroll") for (int s = 0; s < 2; ++s) {                                           \
      const int o = col * kUB + 32 * s + 8 * g4;                                              \
      const uint4 bh_ = *reinterpret_cast<const uint4*>(&Up[0][o]);                           \
      const uint4 bm_ = *reinterpret_cast<const uint4*>(&Up[1][o]);                           \
      const uint4 bl_ = *reinterpret_cast<const uint4*>(&Up[2][o]);                           \
      _Pragma("unroll") for (int dd = 0; dd < 2; ++dd) {                                      \
        ah[dd] = mfma_bf(CUR.kt[dd][s], bh_, ah[dd]);                                         \
        am[dd] = mfma_bf(CUR.kt[dd][s], bm_, am[dd]);                                         \
        al[dd] = mfma_bf(CUR.kt[dd][s], bl_, al[dd]);                                         \
      }                                                                                       \
    }                                                                                         \
    _Pragma("unroll") for (int dd = 0; dd < 2; ++dd)                                          \
      _Pragma("unroll") for (int e = 0; e < 4; ++e) sr[dd][e] = ah[dd][e] + (am[dd][e] + al[dd][e]); \
    split_state((ci & 1) ^ 1);                                                                \
    load_w(cn, NXT);                                                                          \
    __syncthreads(); /* the new state is complete; U and the old state are free */            \
  } while (0)
  // Pairs of chunks with no branch between them (a conditional second half
  // let the compiler sink the prefetch into it, next to its use).
  int c = 0;
  for (; c + 1 < nC; c += 2) {
    Q35_SCAN_CHUNK(opa, opb, c);
    Q35_SCAN_CHUNK(opb, opa, c + 1);
  }
  if (c < nC) Q35_SCAN_CHUNK(opa, opb, c);
#undef Q35_SCAN_CHUNK
#pragma unroll
  for (int dd = 0; dd < 2; ++dd)
#pragma unroll
    for (int e = 0; e < 4; ++e) Sg[(size_t)(16 * (2 * wid + dd) + 4 * g4 + e) * kD + col] = sr[dd][e];
}

// Gated RMSNorm fused into the output kernel (optional): with the core row
// of a token spread over the lanes of two waves, y = bf16(bf16(bf16(o *
// rsqrt(mean(o^2) + eps)) * bf16(w)) * silu(z)) with o the bf16 core output
// and z the gate slice of the packed projection [reference kernels.py:115-155].
struct GatedNormArgs {
  const uint16_t* z;   // packed + z offset; gate of (token, head) at z + token*stride + head*128
  long long z_stride;  // elements per token row of the packed projection
  const void* w;       // [128] bf16 or fp32
  int w_f32;
  float eps;
  uint16_t* y;         // [B, L, H, 128]
};

// O = diag(sc) (q S) + P U for one (chunk, head) from the snapshots, which
// the scan stores in this kernel's B-operand order: nothing is staged in LDS,
// every operand is one coalesced 1 KiB read per wave. Wave w (8 per
// workgroup, two per SIMD) takes a row tile of 16 tokens (w for w < 4, 7 - w
// above) and column tiles 4 (w / 4) .. +3, with q and P loaded once; the S
// and U operands of column tile t + 1 are requested before tile t is
// computed (two register sets alternate). q S is exact in the bf16 products
// (q_hi S_hi... : q S_hi + q S_lo), P U takes P_hi U_hi + P_hi U_lo + P_lo
// U_hi over the t steps at or below the diagonal. GN: the gated RMSNorm of
// each token row is applied before the store (the two column halves of a
// row meet in LDS for the sum of squares; WF32: the norm weight is fp32, else
// bf16); otherwise the core output is stored.
template <bool GN, bool WF32>
__global__ __launch_bounds__(512) void delta_chunk_out(const float* __restrict__ ws,
                                                       const float* __restrict__ snap,
                                                       uint16_t* __restrict__ out, int L, int H,
                                                       int nC, const GatedNormArgs gn) {
  const int c = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  // Waves w and w + 4 share a SIMD: pairing row tile w with row tile 3 - w
  // gives every SIMD the same causal P U work.
  const int tid = threadIdx.x, lane = tid & 63, half = tid >> 8;
  // wave-uniform (readfirstlane): the causal P U tests below are scalar
  // branches, not exec-mask branches that would drain the loads in flight
  const int wid = __builtin_amdgcn_readfirstlane(half ? 3 - ((tid >> 6) & 3) : (tid >> 6) & 3);
  const int ns = wid / 2 + 1;  // t steps of P U at or below the diagonal
  const int col = lane & 15, g4 = lane >> 4;
  const size_t bhc = ((size_t)b * H + h) * nC + c;
  const float* wsb = ws + bhc * kChunkFloats;
  const float* sp = snap + bhc * kSnapFloats;
  __shared__ float ss_s[GN ? 2 : 1][kChunk];
  constexpr int kYS = kD + 8;  // bf16 row stride of the gated norm's output tile
  __shared__ alignas(16) uint16_t yt[GN ? kChunk * kYS : 8];
  struct TileOps {
    uint4 s[4][2], u[2][2];
  };
  // U steps past the diagonal are never used: they re-read step 0.
  auto load_tile = [&](int tile, TileOps& t) {
    const uint4* st = reinterpret_cast<const uint4*>(sp + tile * kSnapSTile) + lane;
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int hl = 0; hl < 2; ++hl) t.s[s][hl] = st[(2 * s + hl) * 64];
    const uint4* ut = reinterpret_cast<const uint4*>(sp + kSnapU + tile * kSnapUTile) + lane;
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int hl = 0; hl < 2; ++hl) t.u[s][hl] = ut[(2 * (s < ns ? s : 0) + hl) * 64];
  };
  uint4 qo[4], po[2][2];
#pragma unroll
  for (int s = 0; s < 4; ++s)
    qo[s] = *reinterpret_cast<const uint4*>(wsb + kOffQ + ((wid * 4 + s) * 64 + lane) * 4);
#pragma unroll
  for (int s = 0; s < 2; ++s)
#pragma unroll
    for (int hl = 0; hl < 2; ++hl)
      po[s][hl] = *reinterpret_cast<const uint4*>(
          wsb + kOffP + (((wid * 2 + (s < ns ? s : 0)) * 2 + hl) * 64 + lane) * 4);
  const float4 scv = *reinterpret_cast<const float4*>(wsb + kOffSc + 16 * wid + 4 * g4);
  TileOps ta, tb;
  load_tile(4 * half, ta);
  load_tile(4 * half + 1, tb);
  // GN: this thread's part of the gated norm, by 16-byte rows: token row
  // tid / 8 of the chunk, columns 16 (tid % 8) .. +15 (its gate values and
  // norm weights, requested with the operands).
  const int gr = tid >> 3, gc0 = 16 * (tid & 7);
  uint4 zv[2] = {make_uint4(0u, 0u, 0u, 0u), make_uint4(0u, 0u, 0u, 0u)};
  float wv[16];
  if (GN) {
    const int t = min(c * kChunk + gr, L - 1);
    const uint16_t* zp = gn.z + ((size_t)b * L + t) * gn.z_stride + (size_t)h * kD + gc0;
    zv[0] = *reinterpret_cast<const uint4*>(zp);
    zv[1] = *reinterpret_cast<const uint4*>(zp + 8);
    // The weight type is a template parameter: a run-time branch between
    // two load forms would make the compiler drain every load in flight.
    if (WF32) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float4 w4 = reinterpret_cast<const float4*>(gn.w)[gc0 / 4 + q];
        wv[4 * q] = w4.x; wv[4 * q + 1] = w4.y; wv[4 * q + 2] = w4.z; wv[4 * q + 3] = w4.w;
      }
    } else {
      unpack8(reinterpret_cast<const uint4*>(gn.w)[gc0 / 8], wv);
      unpack8(reinterpret_cast<const uint4*>(gn.w)[gc0 / 8 + 1], wv + 8);
    }
  }
  // Every load above the first MFMA (the scheduler would otherwise start the
  // chains after the first few loads and wait on each in turn).
  __builtin_amdgcn_sched_barrier(0);
  float ob[4][4];
  auto compute = [&](int tt, const TileOps& t) {
    q35_f32x4 qa = {0.f, 0.f, 0.f, 0.f}, qb = qa, pa = qa, pb = qa, pc = qa;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      qa = mfma_bf(qo[s], t.s[s][0], qa);
      qb = mfma_bf(qo[s], t.s[s][1], qb);
    }
#pragma unroll
    for (int s = 0; s < 2; ++s)
      if (s < ns) {
        pa = mfma_bf(po[s][0], t.u[s][0], pa);
        pb = mfma_bf(po[s][0], t.u[s][1], pb);
        pc = mfma_bf(po[s][1], t.u[s][0], pc);
      }
    const float sc[4] = {scv.x, scv.y, scv.z, scv.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float o = sc[e] * (qa[e] + qb[e]) + ((pa[e] + pb[e]) + pc[e]);
      if (GN) {
        ob[tt][e] = round_bf(o);
      } else {
        const int tok = c * kChunk + 16 * wid + 4 * g4 + e;
        if (tok < L) out[(((size_t)b * L + tok) * H + h) * kD + (4 * half + tt) * 16 + col] = (uint16_t)f2bf(o);
      }
    }
  };
  compute(0, ta);
  load_tile(4 * half + 2, ta);
  compute(1, tb);
  load_tile(4 * half + 3, tb);
  compute(2, ta);
  compute(3, tb);
  if (GN) {
    // Sum of squares of each row: 4 tiles in the lane, the 16 column lanes
    // (one DPP row), then the two halves through LDS.
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float ss = 0.f;
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) ss += ob[tt][e] * ob[tt][e];
      ss = row16_sum(ss);
      if (col == 0) ss_s[half][16 * wid + 4 * g4 + e] = ss;
    }
    __syncthreads();
    // the normalised core (bf16) into the chunk's [64 x 128] output tile
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int r = 16 * wid + 4 * g4 + e;
      const float inv = rsqrt_cr((ss_s[0][r] + ss_s[1][r]) / (float)kD + gn.eps);
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) yt[r * kYS + (4 * half + tt) * 16 + col] = (uint16_t)f2bf(ob[tt][e] * inv);
    }
    __syncthreads();
    const int t = c * kChunk + gr;
    if (t < L) {
      float nb[16], zf[16], v[16];
      unpack8(*reinterpret_cast<const uint4*>(&yt[gr * kYS + gc0]), nb);
      unpack8(*reinterpret_cast<const uint4*>(&yt[gr * kYS + gc0 + 8]), nb + 8);
      unpack8(zv[0], zf);
      unpack8(zv[1], zf + 8);
#pragma unroll
      for (int e = 0; e < 16; ++e) v[e] = round_bf(nb[e] * round_bf(wv[e])) * silu_f(zf[e]);
      uint16_t* yp = gn.y + (((size_t)b * L + t) * H + h) * kD + gc0;
      *reinterpret_cast<uint4*>(yp) = pack8(v);
      *reinterpret_cast<uint4*>(yp + 8) = pack8(v + 8);
    }
  }
}
}  // namespace

extern "C" {

int q35_conv1d_update(const void* x, const void* w, void* state, void* out, int B, int C,
                      int in_stride, int kw, hipStream_t stream) {
  Q35_CHECK_ARG(B >= 0 && C > 0 && kw > 0 && kw <= 16 && in_stride >= C);
  if (B == 0) return 0;
  const int total = B * C;
  conv1d_update<<<(total + 255) / 256, 256, 0, stream>>>((const uint16_t*)x, (const uint16_t*)w,
                                                        (uint16_t*)state, (uint16_t*)out, B, C,
                                                        in_stride, kw);
  return q35_last_error();
}

int q35_conv1d_prefill(const void* x, const void* w, void* state, void* out, int B, int L, int C,
                       int in_stride, int kw, hipStream_t stream) {
  Q35_CHECK_ARG(B >= 0 && L > 0 && C > 0 && kw > 0 && kw <= 16 && in_stride >= C);
  const long long total = (long long)B * L * C;
  if (total == 0) return 0;
  const long long vthreads = (long long)B * ((L + 3) / 4) * (C / 8);
  if (kw == 4 && C % 8 == 0 && in_stride % 8 == 0 && q35_aligned16(x) && q35_aligned16(w) &&
      q35_aligned16(out) && vthreads < (1ll << 31) - 256) {
    const long long g = (vthreads + 255) / 256;
    conv1d_prefill_vec4<<<(unsigned)g, 256, 0, stream>>>((const uint16_t*)x, (const uint16_t*)w,
                                                         (uint16_t*)state, (uint16_t*)out, B, L, C,
                                                         in_stride);
    return q35_last_error();
  }
  const long long grid = (total + 255) / 256;
  Q35_CHECK_ARG(grid < (1ll << 31));
  conv1d_prefill<<<(unsigned)grid, 256, 0, stream>>>((const uint16_t*)x, (const uint16_t*)w,
                                                     (uint16_t*)state, (uint16_t*)out, B, L, C,
                                                     in_stride, kw);
  return q35_last_error();
}

// One decode step of the recurrence for all heads. With fuse_conv the input
// is the raw packed projection and the conv state/weight are applied first;
// with fuse_gnorm the output is the gated RMSNorm of the core output.
int q35_delta_decode(const void* src, int src_stride, const void* packed, int packed_stride,
                     const void* conv_w, void* conv_state, int kw, const void* a_log,
                     const void* dt_bias, int params_f32, void* state, const void* norm_w,
                     int norm_w_f32, float norm_eps, void* out, int B, int H, int D,
                     int fuse_conv, int fuse_gnorm, hipStream_t stream) {
  Q35_CHECK_ARG(B >= 0 && H > 0 && D == kD);
  Q35_CHECK_ARG(src_stride >= 3 * H * D && packed_stride >= 4 * H * D + 2 * H);
  Q35_CHECK_ARG(!fuse_conv || (conv_w && conv_state && kw > 0 && kw <= 16));
  Q35_CHECK_ARG(!fuse_gnorm || norm_w);
  Q35_CHECK_ARG(q35_aligned16(state));
  if (B == 0) return 0;
  DeltaArgs p;
  p.src = (const uint16_t*)src;
  p.src_stride = src_stride;
  p.packed = (const uint16_t*)packed;
  p.packed_stride = packed_stride;
  p.conv_w = (const uint16_t*)conv_w;
  p.conv_state = (uint16_t*)conv_state;
  p.conv_channels = 3 * H * D;
  p.kw = kw;
  p.a_log = a_log;
  p.dt_bias = dt_bias;
  p.params_f32 = params_f32;
  p.state = (float*)state;
  p.norm_w = norm_w;
  p.norm_w_f32 = norm_w_f32;
  p.norm_eps = norm_eps;
  p.out = (uint16_t*)out;
  p.H = H;
  p.z_off = 3 * H * D;
  p.a_off = 4 * H * D;
  p.b_off = 4 * H * D + H;
  const unsigned grid = (unsigned)(B * H);
  if (fuse_conv && fuse_gnorm) delta_decode<true, true><<<grid, 256, 0, stream>>>(p);
  else if (fuse_conv) delta_decode<true, false><<<grid, 256, 0, stream>>>(p);
  else if (fuse_gnorm) delta_decode<false, true><<<grid, 256, 0, stream>>>(p);
  else {
    Q35_CHECK_ARG(q35_aligned8(out));
    if (params_f32) delta_decode_wave<true><<<grid * (kD / kWT), 64, 0, stream>>>(p);
    else delta_decode_wave<false><<<grid * (kD / kWT), 64, 0, stream>>>(p);
  }
  return q35_last_error();
}

// Prefill runs the chunked form for L >= 64 tokens, the token scan below that.
constexpr int kChunkMinL = 64;

// Floats of workspace q35_delta_prefill needs: 4 factors per (batch, token,
// head), and for the chunked form 28800 operand floats, 1 decay and 24576
// snapshot floats per (batch, head, chunk).
long long q35_delta_prefill_workspace(int B, int L, int H) {
  long long n = 4ll * B * L * H;
  if (L >= kChunkMinL)  // + 3: the snapshots start at the next 16-byte boundary
    n += (long long)B * H * ((L + kChunk - 1) / kChunk) * (kChunkFloats + 1 + kSnapFloats) + 3;
  return n;
}

}  // extern "C"

namespace {

// The prefill recurrence (token scan below 64 tokens, chunked form above);
// with gn the chunked output kernel also applies the gated RMSNorm into gn->y.
int delta_prefill(const void* qkv, int qkv_stride, const void* packed, int packed_stride,
                  const void* a_log, const void* dt_bias, int params_f32, void* state, void* out,
                  void* workspace, long long workspace_floats, int B, int L, int H, int D,
                  const GatedNormArgs* gn, hipStream_t stream, const ConvIn* conv = nullptr) {
  Q35_CHECK_ARG(B >= 0 && L > 0 && H > 0 && D == kD);
  Q35_CHECK_ARG(qkv_stride >= 3 * H * D && qkv_stride % 8 == 0);
  Q35_CHECK_ARG(packed_stride >= 4 * H * D + 2 * H);
  Q35_CHECK_ARG(workspace_floats >= q35_delta_prefill_workspace(B, L, H));
  Q35_CHECK_ARG(q35_aligned16(qkv) && q35_aligned16(workspace) && q35_aligned16(state));
  if (B == 0) return 0;
  const long long rows = (long long)B * L * H;
  Q35_CHECK_ARG(rows < (1ll << 30));
  int e = 0;
  if (L < kChunkMinL) {
    delta_factors16<<<(unsigned)((rows + 15) / 16), 256, 0, stream>>>(
        (const uint16_t*)qkv, qkv_stride, (const uint16_t*)packed, packed_stride, a_log, dt_bias,
        params_f32, (float*)workspace, (int)rows, H, 4 * H * D, 4 * H * D + H);
    e = q35_last_error();
    if (e) return e;
    delta_scan<<<(unsigned)(B * H * (kD / 8)), 64, 0, stream>>>(
        (const uint16_t*)qkv, qkv_stride, (const float*)workspace, (float*)state, (uint16_t*)out, L,
        H);
    return q35_last_error();
  }
  const int nC = (L + kChunk - 1) / kChunk;
  Q35_CHECK_ARG(B < 65536 && H < 65536);
  float* chunk_ws = (float*)workspace + 4ll * B * L * H;
  float* gc = chunk_ws + (size_t)B * H * nC * kChunkFloats;
  // Snapshots start 16-byte aligned after the B*H*nC chunk decays.
  float* snap = gc + (((size_t)B * H * nC + 3) & ~(size_t)3);
  const ConvIn cv = conv ? *conv : ConvIn{nullptr, nullptr};
#define PREP(PF, CV)                                                                              \
  delta_chunk_prep<PF, CV><<<dim3(nC, H, B), 256, 0, stream>>>(                                   \
      (const uint16_t*)qkv, qkv_stride, (const uint16_t*)packed, packed_stride, a_log, dt_bias,   \
      params_f32, 4 * H * D, 4 * H * D + H, chunk_ws, gc, L, H, nC, cv)
  if (params_f32) {
    if (conv) PREP(true, true); else PREP(true, false);
  } else {
    if (conv) PREP(false, true); else PREP(false, false);
  }
#undef PREP
  e = q35_last_error();
  if (e) return e;
  delta_chunk_scan<<<dim3((kD / 16) * H, B), 256, 0, stream>>>(chunk_ws, gc, (float*)state, snap,
                                                              H, nC);
  e = q35_last_error();
  if (e) return e;
  if (gn && gn->y && gn->w_f32)
    delta_chunk_out<true, true><<<dim3(nC, H, B), 512, 0, stream>>>(chunk_ws, snap, (uint16_t*)out, L,
                                                                   H, nC, *gn);
  else if (gn && gn->y)
    delta_chunk_out<true, false><<<dim3(nC, H, B), 512, 0, stream>>>(chunk_ws, snap, (uint16_t*)out, L,
                                                                    H, nC, *gn);
  else
    delta_chunk_out<false, false><<<dim3(nC, H, B), 512, 0, stream>>>(chunk_ws, snap, (uint16_t*)out, L,
                                                                     H, nC, GatedNormArgs{});
  return q35_last_error();
}

}  // namespace

// gated_rmsnorm of norm.hip, for the token-scan path of the fused entry point.
extern "C" int q35_gated_rmsnorm_grouped(const void* x, const void* gate, int group_rows,
                                         long long group_stride, const void* w, int w_f32, void* y,
                                         int rows, float eps, hipStream_t stream);

extern "C" {

// Sequential recurrence over L tokens (input: post-conv qkv), state in place.
int q35_delta_prefill(const void* qkv, int qkv_stride, const void* packed, int packed_stride,
                      const void* a_log, const void* dt_bias, int params_f32, void* state,
                      void* out, void* workspace, long long workspace_floats, int B, int L, int H,
                      int D, hipStream_t stream) {
  return delta_prefill(qkv, qkv_stride, packed, packed_stride, a_log, dt_bias, params_f32, state,
                       out, workspace, workspace_floats, B, L, H, D, nullptr, stream);
}

// The same recurrence followed by the gated RMSNorm of every (token, head)
// row with the gate z = packed[token, 3*H*D + h*D ...] and weight norm_w:
// y receives the normalised output ([B, L, H, D] bf16); out is the core
// output (written by the token-scan path only).
int q35_delta_prefill_gated(const void* qkv, int qkv_stride, const void* packed, int packed_stride,
                            const void* a_log, const void* dt_bias, int params_f32, void* state,
                            void* out, void* workspace, long long workspace_floats, int B, int L,
                            int H, int D, const void* norm_w, int norm_w_f32, float eps, void* y,
                            hipStream_t stream) {
  Q35_CHECK_ARG(norm_w && y && out && D == kD && packed_stride % 8 == 0);
  Q35_CHECK_ARG(q35_aligned16(norm_w) && q35_aligned16(y) && q35_aligned16(packed));
  const GatedNormArgs gn{(const uint16_t*)packed + 3ll * H * D, packed_stride, norm_w, norm_w_f32,
                         eps, (uint16_t*)y};
  const int e = delta_prefill(qkv, qkv_stride, packed, packed_stride, a_log, dt_bias, params_f32,
                              state, out, workspace, workspace_floats, B, L, H, D,
                              L >= kChunkMinL ? &gn : nullptr, stream);
  if (e || L >= kChunkMinL) return e;
  return q35_gated_rmsnorm_grouped(out, (const uint16_t*)packed + 3ll * H * D, H, packed_stride,
                                   norm_w, norm_w_f32, y, B * L * H, eps, stream);
}


// q35_delta_prefill_gated with the causal conv folded into the chunk prep:
// the input is the raw packed projection (conv channels [0, 3*H*D), then z,
// a, b as for q35_delta_prefill_gated), conv_w the [3*H*D, 4] taps and
// conv_state receives the last four input rows of every conv channel (what
// q35_conv1d_prefill writes). Chunked path only: L >= 64 (else error 1).
int q35_delta_prefill_gated_conv(const void* packed, int packed_stride, const void* conv_w,
                                 void* conv_state, const void* a_log, const void* dt_bias,
                                 int params_f32, void* state, void* out, void* workspace,
                                 long long workspace_floats, int B, int L, int H, int D,
                                 const void* norm_w, int norm_w_f32, float eps, void* y,
                                 hipStream_t stream) {
  Q35_CHECK_ARG(L >= kChunkMinL && conv_w && conv_state && q35_aligned16(conv_w));
  Q35_CHECK_ARG(norm_w && y && out && D == kD && packed_stride % 8 == 0);
  Q35_CHECK_ARG(q35_aligned16(norm_w) && q35_aligned16(y) && q35_aligned16(packed));
  const GatedNormArgs gn{(const uint16_t*)packed + 3ll * H * D, packed_stride, norm_w, norm_w_f32,
                         eps, (uint16_t*)y};
  const ConvIn cv{(const uint16_t*)conv_w, (uint16_t*)conv_state};
  return delta_prefill(packed, packed_stride, packed, packed_stride, a_log, dt_bias, params_f32,
                       state, out, workspace, workspace_floats, B, L, H, D, &gn, stream, &cv);
}

}  // extern "C"
