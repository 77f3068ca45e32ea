// Shared device helpers for the gfx950 (CDNA4) decode kernels.
//
// bf16 values travel as raw 16-bit patterns (uint16_t) so no host or device
// header type sits in the C ABI. Conversions are explicit: fp32 -> bf16 is
// round-to-nearest-even, the rounding torch (CPU and GPU) and Triton's
// `.to(tl.bfloat16)` use, so every rounding point of the reference kernels is
// reproduced at the same place.
//
// Reductions are wave64: quad_perm / row_half_mirror / row_mirror DPP moves
// reduce each 16-lane row, ds_swizzle (xor 16) joins the two rows of each
// 32-lane half and v_readlane joins the halves. No LDS allocation is needed.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define Q35_DEV __device__ __forceinline__

typedef uint16_t bf16_t;

// ---------------------------------------------------------------- bf16 <-> f32
Q35_DEV float bf2f(uint32_t h16) { return __uint_as_float(h16 << 16); }
Q35_DEV float bf_lo(uint32_t pair) { return __uint_as_float(pair << 16); }
Q35_DEV float bf_hi(uint32_t pair) { return __uint_as_float(pair & 0xffff0000u); }

// fp32 -> bf16 with gfx950's v_cvt_pk_bf16_f32: round to nearest even, NaN
// stays NaN (the rounding torch's .to(bfloat16) and Triton's casts use).
typedef float q35_f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 q35_bf16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 q35_bf16x8 __attribute__((ext_vector_type(8)));
typedef float q35_f32x4 __attribute__((ext_vector_type(4)));
Q35_DEV uint32_t f2bf(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }
Q35_DEV float round_bf(float f) { return bf2f(f2bf(f)); }
Q35_DEV uint32_t pack_bf2(float lo, float hi) {
  const q35_f32x2 v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, q35_bf16x2));
}

// Unpack 8 bf16 held in a uint4 into fp32.
Q35_DEV void unpack8(const uint4 v, float* f) {
  f[0] = bf_lo(v.x); f[1] = bf_hi(v.x);
  f[2] = bf_lo(v.y); f[3] = bf_hi(v.y);
  f[4] = bf_lo(v.z); f[5] = bf_hi(v.z);
  f[6] = bf_lo(v.w); f[7] = bf_hi(v.w);
}
Q35_DEV uint4 pack8(const float* f) {
  uint4 v;
  v.x = pack_bf2(f[0], f[1]);
  v.y = pack_bf2(f[2], f[3]);
  v.z = pack_bf2(f[4], f[5]);
  v.w = pack_bf2(f[6], f[7]);
  return v;
}

// 128-bit streaming load of data read exactly once (weights): non-temporal
// hint so it does not displace reused lines (activations, KV) from L2/MALL.
typedef uint32_t q35_u32x4 __attribute__((ext_vector_type(4)));
Q35_DEV uint4 ld_stream16(const void* p) {
  const q35_u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const q35_u32x4*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

// ---------------------------------------------------------------- math
// 1/sqrt with two correctly rounded steps (sqrt, then divide): the same
// arithmetic torch's CPU rsqrt performs, so norm factors match the oracle.
Q35_DEV float rsqrt_cr(float x) { return 1.0f / sqrtf(x); }
Q35_DEV float silu_f(float x) { return x / (1.0f + expf(-x)); }
// SiLU from the hardware exp2 and reciprocal (a few fp32 ulp from silu_f), for
// the VALU-bound prefill elementwise kernels whose result is rounded to bf16
// immediately: the fp32 difference moves that rounding only for values within
// a few ulp of a bf16 rounding boundary.
Q35_DEV float silu_fast(float x) { return x * __builtin_amdgcn_rcpf(1.0f + __expf(-x)); }
Q35_DEV float sigmoid_f(float x) { return 1.0f / (1.0f + expf(-x)); }
// ---------------------------------------------------------------- DPP moves
template <int CTRL>
Q35_DEV float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
template <int CTRL>
Q35_DEV int dpp_i(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}
#define Q35_DPP_QUAD_XOR1 0xB1   // quad_perm [1,0,3,2]
#define Q35_DPP_QUAD_XOR2 0x4E   // quad_perm [2,3,0,1]
#define Q35_DPP_ROW_HALF_MIRROR 0x141
#define Q35_DPP_ROW_MIRROR 0x140
#define Q35_SWZ_XOR16 0x401F     // ds_swizzle bitmask mode: and 0x1f, xor 0x10

Q35_DEV float swz_xor16_f(float v) {
  return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), Q35_SWZ_XOR16));
}

// Sum over each aligned group of 16 lanes; every lane of the row gets it.
Q35_DEV float row16_sum(float v) {
  v += dpp_f<Q35_DPP_QUAD_XOR1>(v);
  v += dpp_f<Q35_DPP_QUAD_XOR2>(v);
  v += dpp_f<Q35_DPP_ROW_HALF_MIRROR>(v);
  v += dpp_f<Q35_DPP_ROW_MIRROR>(v);
  return v;
}

// Max over the 16 lanes of a DPP row (same exchange pattern as row16_sum).
Q35_DEV float row16_max(float v) {
  v = fmaxf(v, dpp_f<Q35_DPP_QUAD_XOR1>(v));
  v = fmaxf(v, dpp_f<Q35_DPP_QUAD_XOR2>(v));
  v = fmaxf(v, dpp_f<Q35_DPP_ROW_HALF_MIRROR>(v));
  v = fmaxf(v, dpp_f<Q35_DPP_ROW_MIRROR>(v));
  return v;
}

// Sum over the whole wave64; the result is wave-uniform.
Q35_DEV float wave_sum(float v) {
  v = row16_sum(v);
  v += swz_xor16_f(v);
  const float lo = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float hi = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  return lo + hi;
}

Q35_DEV float wave_max(float v) {
  v = fmaxf(v, dpp_f<Q35_DPP_QUAD_XOR1>(v));
  v = fmaxf(v, dpp_f<Q35_DPP_QUAD_XOR2>(v));
  v = fmaxf(v, dpp_f<Q35_DPP_ROW_HALF_MIRROR>(v));
  v = fmaxf(v, dpp_f<Q35_DPP_ROW_MIRROR>(v));
  v = fmaxf(v, swz_xor16_f(v));
  const float lo = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float hi = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  return fmaxf(lo, hi);
}

// 64-bit max over the wave (used for packed value/index argmax keys).
Q35_DEV uint64_t u64_max(uint64_t a, uint64_t b) { return a > b ? a : b; }
Q35_DEV uint64_t wave_max_u64(uint64_t v) {
  for (int off = 1; off < 64; off <<= 1) {
    const uint32_t lo = (uint32_t)__shfl_xor((int)(uint32_t)v, off, 64);
    const uint32_t hi = (uint32_t)__shfl_xor((int)(uint32_t)(v >> 32), off, 64);
    v = u64_max(v, ((uint64_t)hi << 32) | lo);
  }
  return v;
}

// Order-preserving key for a bf16 value (as fp32 with zero low half) and an
// index: larger value wins, then the lower index. -0 and +0 compare equal,
// as float comparison does.
Q35_DEV uint64_t top1_key(float v_bf16, uint32_t index) {
  uint32_t b = __float_as_uint(v_bf16) >> 16;
  if ((b & 0x7fffu) == 0) b = 0;                 // fold -0 onto +0
  const uint32_t ord = (b & 0x8000u) ? (~b & 0xffffu) : (b | 0x8000u);
  return ((uint64_t)ord << 32) | (uint64_t)(0xffffffffu - index);
}
Q35_DEV uint32_t top1_index(uint64_t key) { return 0xffffffffu - (uint32_t)(key & 0xffffffffu); }

// ---------------------------------------------------------------- launch checks
#define Q35_CHECK_ARG(cond)                    \
  do {                                         \
    if (!(cond)) return (int)hipErrorInvalidValue; \
  } while (0)

static inline int q35_last_error() { return (int)hipGetLastError(); }

static inline bool q35_aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }
static inline bool q35_aligned8(const void* p) { return ((uintptr_t)p & 7u) == 0; }
static inline bool q35_aligned4(const void* p) { return ((uintptr_t)p & 3u) == 0; }

// Workgroup barrier that orders LDS only: outstanding global loads (e.g. a
// weight stream issued before the barrier) stay in flight across it.
Q35_DEV void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Single-token depthwise causal conv for one channel (reference
// kernels.py:622-656): window = (state[1..kw-1], x); the state is shifted in
// place; returns bf16(silu(bf16(sum_t w[t]*window[t]))) as fp32.
Q35_DEV float conv_update_channel(uint16_t* __restrict__ st, const uint16_t* __restrict__ w,
                                  uint32_t xin, int kw) {
  float acc = 0.f;
  for (int t = 0; t < kw - 1; ++t) {
    const uint16_t s = st[t + 1];
    st[t] = s;
    acc = fmaf(bf2f(s), bf2f(w[t]), acc);
  }
  st[kw - 1] = (uint16_t)xin;
  acc = fmaf(bf2f(xin), bf2f(w[kw - 1]), acc);
  return round_bf(silu_f(round_bf(acc)));
}

// ------------------------------------------------------------------ int8
// Four quantised bytes packed little-endian: q = sat_int8(rint(v * inv)) with
// NaN -> 0 (the same map as sat_i8, in fewer instructions): v_rndne_f32, then
// v_cvt_i32_f32 (NaN -> 0, +-inf saturate to the int32 range), v_med3_i32 to
// [-128, 127], and two byte permutes per pair.
Q35_DEV int cvt_i32_sat(float r) {
  int i;
  asm("v_cvt_i32_f32 %0, %1" : "=v"(i) : "v"(r));
  return i;
}
Q35_DEV uint32_t quant4_i8(float a, float b, float c, float d, float inv) {
  const int ia = min(max(cvt_i32_sat(__builtin_rintf(a * inv)), -128), 127);
  const int ib = min(max(cvt_i32_sat(__builtin_rintf(b * inv)), -128), 127);
  const int ic = min(max(cvt_i32_sat(__builtin_rintf(c * inv)), -128), 127);
  const int id = min(max(cvt_i32_sat(__builtin_rintf(d * inv)), -128), 127);
  // perm(S0, S1, sel): selector byte 0-3 picks a byte of S1, 4-7 of S0, 0x0c gives 0.
  const uint32_t lo = __builtin_amdgcn_perm((uint32_t)ib, (uint32_t)ia, 0x0c0c0400u);
  const uint32_t hi = __builtin_amdgcn_perm((uint32_t)id, (uint32_t)ic, 0x0c0c0400u);
  return __builtin_amdgcn_perm(hi, lo, 0x05040100u);
}
// Eight consecutive values into two packed words.
Q35_DEV uint2 quant8_i8(const float* v, float inv) {
  return make_uint2(quant4_i8(v[0], v[1], v[2], v[3], inv), quant4_i8(v[4], v[5], v[6], v[7], inv));
}

// 16 int8 pairs into an int32 accumulator (v_dot4c_i32_i8).
Q35_DEV int dot16_i8(const uint4 a, const uint4 b, int acc) {
  acc = __builtin_amdgcn_sdot4((int)a.x, (int)b.x, acc, false);
  acc = __builtin_amdgcn_sdot4((int)a.y, (int)b.y, acc, false);
  acc = __builtin_amdgcn_sdot4((int)a.z, (int)b.z, acc, false);
  acc = __builtin_amdgcn_sdot4((int)a.w, (int)b.w, acc, false);
  return acc;
}

Q35_DEV int wave_sum_i32(int v) {
  v += dpp_i<Q35_DPP_QUAD_XOR1>(v);
  v += dpp_i<Q35_DPP_QUAD_XOR2>(v);
  v += dpp_i<Q35_DPP_ROW_HALF_MIRROR>(v);
  v += dpp_i<Q35_DPP_ROW_MIRROR>(v);
  v += __builtin_amdgcn_ds_swizzle(v, Q35_SWZ_XOR16);
  return __builtin_amdgcn_readlane(v, 0) + __builtin_amdgcn_readlane(v, 32);
}

