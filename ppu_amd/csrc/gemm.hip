// Prefill GEMMs on the gfx950 matrix cores: C[M, N] = A[M, K] . B[N, K]^T
// with both operands K-contiguous (activations x weights^T, as F.linear).
//
//   kind 0  bf16 A, B -> bf16 C = bf16(acc)                        [F.linear, integration.py:183,245,298]
//   kind 1  bf16, B = [gate; up] (2N rows) -> C[m, n] = bf16(bf16(silu(bf16 g)) * bf16 u)
//                                                                   [integration.py:183-185 + kernels.py:158-180]
//   kind 2  int8 A, B -> int32 C = acc (exact)                     [the int8 GEMM of explore_runtime_quantization.py:173-180]
//   kind 3  int8 -> bf16 C = bf16(float(acc) * s_x[m] * s_w[n])    [the same with its dequant]
//   kind 4  int8, B = [gate; up] -> SwiGLU of the dequantised gate and up (kind 1's rounding points)
//
// bf16 runs on v_mfma_f32_32x32x16_bf16 (fp32 accumulators), int8 on
// v_mfma_i32_32x32x32_i8 (exact int32). Both take 16 bytes per lane and
// operand: lane l holds row l % 32 of its 32-row block and bytes
// [16 (l / 32), +16) of a 32-byte k window, so one LDS layout and one
// fragment read serve both.
//
// Workgroup: 4 waves as 2 x 2 over a TM x TN tile; each wave holds FM x FN
// accumulator blocks of 32 x 32 (tile 0: 256 x 192, the wave 128 x 96, 12
// blocks = 192 accumulator registers).
//
// Operand staging. K advances in stages of RB bytes per row. A stage of the
// A and B tiles goes straight from memory into LDS with
// global_load_lds_dwordx4 (each wave instruction writes 1 KiB of LDS: 1024 /
// RB rows, 16 bytes per lane) into a ring of NS stage buffers, so no register
// holds a fetched stage and NS - 1 stages are in flight. The loads are issued
// from inline asm, so the only waits on them are the ring's explicit vmcnt
// waits. Each lane's global source is chosen so that the LDS image is
// swizzled: 16-byte chunk c of tile row r sits at slot c ^ swz(r), which
// makes the fragment reads (16 consecutive rows, one logical chunk, per 16
// lanes) hit 16 distinct bank groups of the 256-byte LDS bank window.
// Measured on the 2B prefill shapes (timing copies with parts switched off):
//  * the operand stream is the bound; stages of 128-byte rows (every request
//    a whole L2 line) move twice the bytes per second of 64-byte rows, whose
//    requests each pull a 128-byte line for 64 useful bytes;
//  * workgroups that share operand rows (the M tiles of one weight tile, the
//    N tiles of one activation tile) run on one XCD; when they walk K in
//    lockstep every one of them waits for the same L2 misses, so each
//    workgroup starts its K walk at its own stage offset (K rotation) and the
//    later readers of a line find it in L2 (DMA-only time -15 to -30 %);
//  * a wave issues in order, so a run of fragment reads ahead of the MFMAs
//    stalls them behind the LDS queue; one read (and one DMA) per MFMA, in
//    the order the next k step consumes them, hides the reads completely.
//
// Ring schedule (one barrier per stage): in stage kt the fragments of k step
// t + 1 are read under the MFMAs of step t, and the buffer of stage kt - 1
// (free since the last barrier) is refilled with stage kt + NS - 1 under the
// MFMAs of the first steps; in the last step, after half of its MFMAs, each
// wave waits for its part of stage kt + 1 (vmcnt) and all waves meet at
// s_barrier, then the first fragments of stage kt + 1 are read under the
// second half.
//
// Split K (for outputs with fewer tiles than CUs): `splits` workgroups per
// tile each take kps stages. Each stores its partial tile (fp32 / int32 bit
// patterns, in accumulator-register order so every wave store is 512
// contiguous bytes) with agent-scope stores, every thread waits until its
// stores have completed (s_waitcnt vmcnt(0)), and one thread counts the
// workgroup's arrival on the tile's counter (agent-scope atomic add). The
// workgroup that arrives last resets the counter and sums the partials in
// split order, its own from registers, so the result does not depend on
// arrival order; it reads them with agent-scope loads issued only after it
// has seen the count. Agent-scope stores and loads (sc1) are coherent across
// the XCDs' L2s by themselves; completed stores before the count and loads
// after it give the ordering. (Agent-scope release / acquire fences would
// add an L2 write-back per arriving workgroup and an L2 invalidate per last
// one, which discards the operands the XCD's other workgroups are streaming:
// measured 2-3x slower on the split plans.) The counters (a fixed region of
// kMaxSplitTiles at the start of the workspace) and the partials live in the
// caller's workspace, which must be zero-filled once before its first use;
// every launch leaves the counters at zero again (a launch aborted part way
// can leave them non-zero: zero the workspace again after such an error).
// Two launches that overlap in time must not share a workspace.
//
// Tile order: units (tile, split) are grouped so that the units sharing B
// rows and a K range (consecutive M tiles) run on one XCD and read the
// weights into one L2: with U units and U % 8 == 0, workgroup b (XCD b % 8)
// takes unit (b % 8) * U / 8 + b / 8, M tile fastest.
#include "q35_common.hpp"

namespace {

enum { KIND_BF16 = 0, KIND_SWIGLU = 1, KIND_I32 = 2, KIND_DEQ = 3, KIND_DEQ_SWIGLU = 4 };
constexpr int kNumKinds = 5;
constexpr int kMaxSplitTiles = 8192;  // counters at the start of a split-K workspace
constexpr int kCounterBytes = kMaxSplitTiles * 4;

struct GemmArgs {
  const uint8_t* A;  // [M, K]
  const uint8_t* B;  // [N, K] (SwiGLU kinds: [2N, K])
  void* C;           // [M, N] bf16 or int32
  int M, N, K;       // K in elements
  const float* s_x;  // int8 kinds 3, 4: per-row scales of A
  const float* s_w;  // per-row scales of B
  unsigned* cnt;     // split-K arrival counters, one per tile
  uint8_t* part;     // split-K partial tiles
  int splits, kps;   // splits per tile, stages per split
};

typedef __attribute__((address_space(3))) uint8_t lds_u8;
Q35_DEV uint32_t lds_offset(const void* p) { return (uint32_t)(uintptr_t)(const lds_u8*)p; }

// One wave instruction of the stage ring: lane i copies the 16 bytes at
// sbase + voff to LDS bytes [lds + 16 i, +16) (the LDS base goes in m0).
Q35_DEV void dma16(uint32_t lds, const uint8_t* sbase, uint32_t voff) {
  asm volatile("global_load_lds_dwordx4 %0, %1" : : "v"(voff), "s"(sbase), "{m0}"(lds) : "memory");
}
// s_waitcnt vmcnt(N) (gfx9 encoding: vmcnt in bits 3:0 and 15:14, expcnt
// and lgkmcnt at their "no wait" maxima). As a builtin the compiler's wait
// pass sees it and keeps it; it does not know of the asm loads it waits for.
template <int N>
Q35_DEV void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}
// This wave's LDS reads complete (s_waitcnt lgkmcnt(0)).
Q35_DEV void wait_lds() { __builtin_amdgcn_s_waitcnt(15 | (7 << 4) | (3 << 14)); }
// Workgroup barrier; the empty asm statements keep the compiler from moving
// memory accesses across it (the builtin barrier alone does not order them).
Q35_DEV void ring_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}
// Keeps the compiler's scheduler from moving any instruction across it, so
// the MFMA / read / DMA interleave below is issued as written.
#define Q35_PIN() __builtin_amdgcn_sched_barrier(0)

typedef float q35_f32x16 __attribute__((ext_vector_type(16)));
typedef int q35_i32x16 __attribute__((ext_vector_type(16)));
typedef int q35_i32x4 __attribute__((ext_vector_type(4)));
Q35_DEV q35_f32x16 mfma32(const q35_u32x4 a, const q35_u32x4 b, q35_f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(q35_bf16x8, a),
                                                 __builtin_bit_cast(q35_bf16x8, b), c, 0, 0, 0);
}
Q35_DEV q35_i32x16 mfma32(const q35_u32x4 a, const q35_u32x4 b, q35_i32x16 c) {
  return __builtin_amdgcn_mfma_i32_32x32x32_i8(__builtin_bit_cast(q35_i32x4, a),
                                               __builtin_bit_cast(q35_i32x4, b), c, 0, 0, 0);
}
template <bool I8> struct GemmAcc { using T = q35_f32x16; using E = float; };
template <> struct GemmAcc<true> { using T = q35_i32x16; using E = int; };
Q35_DEV uint32_t acc_bits(float v) { return __float_as_uint(v); }
Q35_DEV uint32_t acc_bits(int v) { return (uint32_t)v; }
Q35_DEV float acc_from(uint32_t b, float) { return __uint_as_float(b); }
Q35_DEV int acc_from(uint32_t b, int) { return (int)b; }

constexpr bool kind_i8(int kind) { return kind >= KIND_I32; }
constexpr bool kind_swiglu(int kind) { return kind == KIND_SWIGLU || kind == KIND_DEQ_SWIGLU; }

template <bool V> struct BoolTag { static constexpr bool value = V; };

// Slot of 16-byte chunk c of tile row r in the swizzled LDS image.
template <int RB>
Q35_DEV int swz(int r) {
  return RB == 64 ? (r >> 2) & 3 : (r >> 1) & 7;
}

template <int WM, int WN, int FM, int FN, int RB, int NSA, int NSB, bool ROT, int KIND, bool SPLIT, bool STAGED>
__global__ __launch_bounds__(256, 1) void gemm_ring(const GemmArgs a) {
  constexpr bool I8 = kind_i8(KIND);
  constexpr bool SWIGLU = kind_swiglu(KIND);
  constexpr int ES = I8 ? 1 : 2;
  constexpr int TM = WM * FM * 32, TN = WN * FN * 32;
  constexpr int NC = SWIGLU ? TN / 2 : TN;  // output columns per tile
  constexpr int RPG = 1024 / RB;             // tile rows per 1 KiB DMA group
  constexpr int CPR = RB / 16;               // 16-byte chunks per row and stage
  constexpr int GA = TM / RPG, GB = TN / RPG;
  constexpr int LA = GA / 4, LB = GB / 4;    // DMA instructions per wave and stage (A, B)
  constexpr int LPW = LA + LB;
  constexpr int ASTAGE = TM * RB, BSTAGE = TN * RB;  // LDS bytes per stage of A and of B
  constexpr int ABYTES = NSA * ASTAGE;       // the A ring, then the B ring
  constexpr int LDSB = ABYTES + NSB * BSTAGE;
  constexpr int T = RB / 32;                 // MFMA k steps per stage
  constexpr int NMF = FM * FN;               // MFMAs per k step
  constexpr int NR = FM + FN;                // fragment reads per k step
  constexpr int H = NMF / 2;                 // MFMAs of the last step before the barrier
  static_assert(WM * WN == 4, "4 waves");
  static_assert(GA % 4 == 0 && GB % 4 == 0, "every wave issues the same DMA groups of A and B");
  static_assert(T % 2 == 0, "fragment register sets alternate between k steps");
  static_assert(!SWIGLU || WN == 2, "SwiGLU pairs the gate waves with the up waves");
  static_assert(NSA >= 2 && NSB >= NSA && LDSB <= 160 * 1024, "the stage rings fit the LDS");
  static_assert(LPW <= (T - 1) * NMF, "the refill fits the MFMA slots of the first steps");
  static_assert(STAGED || KIND == KIND_BF16 || KIND == KIND_I32, "direct stores: bf16 and int32 kinds");
  using AccT = typename GemmAcc<I8>::T;
  using EltT = typename GemmAcc<I8>::E;
  __shared__ __attribute__((aligned(1024))) uint8_t lds[LDSB];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = tid >> 6;
  const int wm = w % WM, wn = w / WM;

  // ---- unit of this workgroup: (tile, split)
  const int mt = (a.M + TM - 1) / TM;
  const int nt = (a.N + NC - 1) / NC;
  const int ntiles = mt * nt;
  const int S = SPLIT ? a.splits : 1;
  const int U = ntiles * S;
  int u = (int)blockIdx.x;
  if ((U & 7) == 0) u = (u & 7) * (U >> 3) + (u >> 3);
  const int tm = u % mt;
  const int rest = u / mt;
  const int ks = SPLIT ? rest % S : 0;
  const int tn = SPLIT ? rest / S : rest;
  const int tile = tn * mt + tm;
  const int m0 = tm * TM, n0 = tn * NC;
  const int nk = a.kps;  // stages of this workgroup
  // K rotation (ROT): the workgroups sharing rows start at different stages
  const int krot = ROT ? ((tm % 4) * nk / 4 + (tn & 7) * nk / 32) % nk : 0;
  const uint32_t rowb = (uint32_t)a.K * ES;
  // dequant kinds: the tile's row scales s_x[m0 ..] and column scales s_w[..]
  // (SwiGLU: gate then up columns), loaded now and published through LDS in
  // the epilogue (NSC <= 512: two per thread)
  constexpr bool DEQ = KIND == KIND_DEQ || KIND == KIND_DEQ_SWIGLU;
  constexpr int NSC = DEQ ? TM + (SWIGLU ? 2 * NC : NC) : 0;
  static_assert(NSC <= 512, "two scales per thread");
  float scl[2] = {0.f, 0.f};
  if constexpr (DEQ) {
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int x = tid + 256 * q;
      if (x < TM) {
        scl[q] = a.s_x[min(m0 + x, a.M - 1)];
      } else if (x < NSC) {
        const int y = x - TM;
        scl[q] = y < NC ? a.s_w[min(n0 + y, a.N - 1)] : a.s_w[a.N + min(n0 + y - NC, a.N - 1)];
      }
    }
  }

  // ---- DMA sources: wave w issues groups g = w + 4 i (A groups first)
  uint32_t voff[LPW];
#pragma unroll
  for (int i = 0; i < LPW; ++i) {
    const int g = w + 4 * i;
    const bool isA = i < GA / 4;
    const int r = (isA ? g : g - GA) * RPG + lane / CPR;  // tile row
    const int c = (lane % CPR) ^ swz<RB>(r);
    int grow;
    if (isA) {
      grow = min(m0 + r, a.M - 1);
    } else if (SWIGLU) {
      grow = r < TN / 2 ? min(n0 + r, a.N - 1) : a.N + min(n0 + r - TN / 2, a.N - 1);
    } else {
      grow = min(n0 + r, a.N - 1);
    }
    voff[i] = (uint32_t)grow * rowb + (uint32_t)(ks * nk) * RB + 16u * c;
  }
  const uint32_t lds0 = __builtin_amdgcn_readfirstlane(lds_offset(lds) + (uint32_t)w * 1024u);
  // instruction i of the DMA of stage kt: A (i < LA) into A buffer abuf, B into B buffer bbuf
  auto dma = [&](int kt, int abuf, int bbuf, int i) {
    int ksr = kt + krot;
    if (ksr >= nk) ksr -= nk;
    if (i < LA)
      dma16(lds0 + (uint32_t)abuf * ASTAGE + 4096u * i, a.A + (size_t)ksr * RB, voff[i]);
    else
      dma16(lds0 + ABYTES + (uint32_t)bbuf * BSTAGE + 4096u * (i - LA), a.B + (size_t)ksr * RB, voff[i]);
  };

  // ---- fragment sources: row l32 of each 32-row block, logical chunk 2t + kh
  const int l32 = lane & 31, kh = lane >> 5;
  uint32_t fa[T], fb[T];
#pragma unroll
  for (int t = 0; t < T; ++t) {
    const uint32_t co = 16u * (uint32_t)((2 * t + kh) ^ swz<RB>(l32));
    fa[t] = (uint32_t)(wm * FM * 32 + l32) * RB + co;
    fb[t] = (uint32_t)(wn * FN * 32 + l32) * RB + co;
  }
  q35_u32x4 ra[2][FM], rb[2][FN];
  // fragment r of step t in the order the MFMAs consume them: A0, B0 .. B(FN-1), A1 ..
  auto read1 = [&](int abuf, int bbuf, int t, int set, int r) {
    const uint8_t* pa = lds + abuf * ASTAGE;
    const uint8_t* pb = lds + ABYTES + bbuf * BSTAGE;
    if (r == 0) {
      ra[set][0] = *reinterpret_cast<const q35_u32x4*>(pa + fa[t]);
    } else if (r <= FN) {
      rb[set][r - 1] = *reinterpret_cast<const q35_u32x4*>(pb + fb[t] + (r - 1) * 32 * RB);
    } else {
      ra[set][r - FN] = *reinterpret_cast<const q35_u32x4*>(pa + fa[t] + (r - FN) * 32 * RB);
    }
  };

  AccT acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0;
  auto mfma = [&](int set, int q) {
    acc[q / FN][q % FN] = mfma32(ra[set][q / FN], rb[set][q % FN], acc[q / FN][q % FN]);
  };

  // ---- prologue: A stages 0 .. NSA-2 and B stages 0 .. NSB-2 in flight (A
  // before B of the same stage, as in the loop), stage 0 landed, its first
  // fragments read
#pragma unroll
  for (int s = 0; s < NSB - 1; ++s) {
    if (s < NSA - 1 && s < nk)
#pragma unroll
      for (int i = 0; i < LA; ++i) dma(s, s, 0, i);
    if (s < nk)
#pragma unroll
      for (int i = LA; i < LPW; ++i) dma(s, 0, s, i);
  }
  // issued after stage 0's B: (NSB - 2) later B stages and (NSA - 2) later A stages
  if (nk >= NSB - 1) wait_vm<(NSB - 2) * LB + (NSA - 2) * LA>();
  else wait_vm<0>();
  ring_barrier();
#pragma unroll
  for (int r = 0; r < NR; ++r) read1(0, 0, 0, 0, r);

  // One stage. RA / RB: the A / B buffer of stage kt - 1 is refilled with
  // stage kt + NSA - 1 / kt + NSB - 1 (A refills stop NSA - 1 stages before
  // the end, B refills NSB - 1).
  // Wait before the barrier, steady state: stage kt + 1's last load is its A
  // (issued at stage kt + 2 - NSA) when NSA < NSB, else its B; the loads
  // issued after it are then LB + (NSA - 2) (LA + LB), or (NSA - 2) (LA + LB).
  constexpr int WAITN = (NSA < NSB ? LB : 0) + (NSA - 2) * LPW;
  int abuf = 0, bbuf = 0;
  auto stage = [&](int kt, auto ra_tag, auto rb_tag) {
    constexpr bool RA = decltype(ra_tag)::value, RB_ = decltype(rb_tag)::value;
    const int rabuf = abuf == 0 ? NSA - 1 : abuf - 1;  // buffers of stage kt - 1
    const int rbbuf = bbuf == 0 ? NSB - 1 : bbuf - 1;
    // steps 0 .. T-2: one MFMA, one fragment read of the next step, and
    // (first steps) the DMA refills, per slot
#pragma unroll
    for (int t = 0; t < T - 1; ++t) {
#pragma unroll
      for (int q = 0; q < NMF; ++q) {
        mfma(t & 1, q);
        if constexpr (NR <= NMF) {
          if (q < NR) read1(abuf, bbuf, t + 1, (t + 1) & 1, q);
        } else {  // more fragments than MFMAs per step: spread them over the slots
#pragma unroll
          for (int r = q * NR / NMF; r < (q + 1) * NR / NMF; ++r) read1(abuf, bbuf, t + 1, (t + 1) & 1, r);
        }
        const int slot = t * NMF + q;
        if (RA && slot < LA) dma(kt + NSA - 1, rabuf, 0, slot);
        if (RB_ && slot >= LA && slot < LPW) dma(kt + NSB - 1, 0, rbbuf, slot);
        Q35_PIN();
      }
    }
    // last step: half the MFMAs, the ring barrier, the other half with the
    // first fragments of stage kt + 1
    constexpr int cur = (T - 1) & 1;
#pragma unroll
    for (int q = 0; q < H; ++q) {
      mfma(cur, q);
      Q35_PIN();
    }
    const int nabuf = abuf + 1 == NSA ? 0 : abuf + 1;
    const int nbbuf = bbuf + 1 == NSB ? 0 : bbuf + 1;
    const bool more = kt + 1 < nk;
    wait_lds();  // on both paths, so the second half waits for nothing
    if (more) {
      // stage kt + 1 landed: this wave's part (vmcnt), then every wave's
      if (RA && RB_) wait_vm<WAITN>();
      else wait_vm<0>();
      ring_barrier();
    }
    Q35_PIN();
#pragma unroll
    for (int q = H; q < NMF; ++q) {
      mfma(cur, q);
      if (more) {
        const int s = q - H;
#pragma unroll
        for (int r = s * NR / (NMF - H); r < (s + 1) * NR / (NMF - H); ++r) read1(nabuf, nbbuf, 0, cur ^ 1, r);
      }
      Q35_PIN();
    }
    abuf = nabuf;
    bbuf = nbbuf;
  };
  int kt = 0;
  for (; kt + NSB - 1 < nk; ++kt) stage(kt, BoolTag<true>{}, BoolTag<true>{});
  for (; kt + NSA - 1 < nk; ++kt) stage(kt, BoolTag<true>{}, BoolTag<false>{});
  for (; kt < nk; ++kt) stage(kt, BoolTag<false>{}, BoolTag<false>{});

  // ---- split K: partial tiles, arrival count, the last workgroup sums
  if constexpr (SPLIT) {
    constexpr int NP = NMF * 8;  // 8-byte pairs per thread
    uint64_t* mine = reinterpret_cast<uint64_t*>(a.part) + ((size_t)ks * ntiles + tile) * NP * 256 + tid;
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int e = 0; e < 16; e += 2) {
          const uint64_t v = (uint64_t)acc_bits(acc[i][j][e]) | ((uint64_t)acc_bits(acc[i][j][e + 1]) << 32);
          __hip_atomic_store(mine + (size_t)(((i * FN + j) * 16 + e) / 2) * 256, v, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
        }
    // Every thread waits for its own partial stores to complete (the
    // workgroup barrier does not wait for memory), then one arrival is counted.
    wait_vm<0>();
    // (the count is shared through the first word of the stage ring, which
    // no wave reads any more after this barrier)
    unsigned* arrived = reinterpret_cast<unsigned*>(lds);
    __syncthreads();
    if (tid == 0) {
      const unsigned n = __hip_atomic_fetch_add(a.cnt + tile, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (n == (unsigned)S - 1)
        __hip_atomic_store(a.cnt + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      *arrived = n;
    }
    __syncthreads();
    if (*arrived != (unsigned)S - 1) return;
    AccT own[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j) own[i][j] = acc[i][j];
    for (int sp = 0; sp < S; ++sp) {
      const uint64_t* src = reinterpret_cast<const uint64_t*>(a.part) + ((size_t)sp * ntiles + tile) * NP * 256 + tid;
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
          for (int e = 0; e < 16; e += 2) {
            EltT lo, hi;
            if (sp == ks) {
              lo = own[i][j][e];
              hi = own[i][j][e + 1];
            } else {
              const uint64_t v = __hip_atomic_load(
                  const_cast<uint64_t*>(src + (size_t)(((i * FN + j) * 16 + e) / 2) * 256),
                  __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
              lo = acc_from((uint32_t)v, EltT{});
              hi = acc_from((uint32_t)(v >> 32), EltT{});
            }
            acc[i][j][e] = sp == 0 ? lo : acc[i][j][e] + lo;
            acc[i][j][e + 1] = sp == 0 ? hi : acc[i][j][e + 1] + hi;
          }
    }
  }

  // ---- epilogue. Element r of a 32x32 block sits at row 8 (r / 4) + 4 kh +
  // r % 4, column l32.
  if constexpr (!STAGED) {
    // Direct: each lane stores its elements (bf16: 64-byte row segments per
    // half wave; int32: 128-byte); tiles inside C store without checks.
    const int rbase = m0 + wm * FM * 32 + 4 * kh;
    const int cbase = n0 + wn * FN * 32 + l32;
    const bool full = m0 + TM <= a.M && n0 + TN <= a.N;
    auto store = [&](int i, int r, int j, bool check) {
      const int row = rbase + 32 * i + 8 * (r >> 2) + (r & 3);
      const int col = cbase + 32 * j;
      if (check && (row >= a.M || col >= a.N)) return;
      const size_t at = (size_t)row * a.N + col;
      if constexpr (KIND == KIND_I32) reinterpret_cast<int*>(a.C)[at] = acc[i][j][r];
      else reinterpret_cast<uint16_t*>(a.C)[at] = (uint16_t)f2bf(acc[i][j][r]);
    };
    if (full) {
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r)
#pragma unroll
          for (int j = 0; j < FN; ++j) store(i, r, j, false);
    } else {
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r)
#pragma unroll
          for (int j = 0; j < FN; ++j) store(i, r, j, true);
    }
    return;
  }
  // Staged through LDS. bf16 kinds and the int8 dequant kinds stage the
  // whole tile as bf16: the values they store, or the rounded gate / up; the
  // dequant kinds first publish the tile's scales in LDS and dequantise each
  // accumulator in registers, float(acc) * s_x * s_w rounded to bf16 (the
  // int32 tile would not fit the LDS in one pass, and staging it in two half
  // tiles left half the waves idle in each: the dequant epilogue of the
  // 256x192 tile took 11.2 us, now 5.9; with SwiGLU 11.6, now 8.5). The
  // int32 kind stages its accumulators one half tile (one wave row) at a
  // time. Rows are staged at a stride of TN elements + 16 bytes (the two
  // halves of each write instruction, rows r and r + 4, fall on different
  // banks). Then every thread takes ITER chunks of 16 staged bytes along the
  // rows, all read before any is converted, and stores each chunk's outputs
  // with one 16-byte store (a copy, or SwiGLU of the gate and up columns, the
  // two halves of a staged row).
  {
    constexpr bool W16 = !I8 || DEQ;           // staged as bf16
    constexpr int EB = W16 ? 2 : 4;            // staged bytes per element
    constexpr int PH = W16 ? 1 : WM;           // phases (half tiles for int8)
    constexpr int PR = TM / PH;                // staged rows per phase
    constexpr int SB = TN * EB + 16;           // staged row stride in bytes
    constexpr int VPC = 16 / EB;               // values per 16-byte chunk
    constexpr int CPRW = NC / VPC;             // output chunks per row
    constexpr int ITER = PR * CPRW / 256;      // chunks per thread and phase
    constexpr int SCO = PR * SB;               // LDS offset of the scales
    static_assert(PR * CPRW % 256 == 0, "the chunks divide over the workgroup");
    static_assert(SCO + NSC * 4 <= LDSB, "the staged tile and scales fit the rings");
    const bool vec = (a.N & 7) == 0;
    float* sc = reinterpret_cast<float*>(lds + SCO);
    wait_lds();
    __syncthreads();  // every wave is done with the stage ring
    if constexpr (DEQ) {
#pragma unroll
      for (int q = 0; q < 2; ++q)
        if (tid + 256 * q < NSC) sc[tid + 256 * q] = scl[q];
      __syncthreads();  // the scales, before the dequant below reads them
    }
#pragma unroll
    for (int h = 0; h < PH; ++h) {
      if (PH == 1 || wm == h) {
        const int rb0 = PH == 1 ? wm * FM * 32 : 0;
        // dequant kinds: s_w of staged column c at sc[TM + c] (SwiGLU: the up
        // columns follow the gate columns), read once per column block; s_x
        // of the block row's 16 rows (4 runs of 4) as four 16-byte reads
        float swr[FN];
        if constexpr (DEQ) {
#pragma unroll
          for (int j = 0; j < FN; ++j) swr[j] = sc[TM + wn * FN * 32 + j * 32 + l32];
        }
#pragma unroll
        for (int i = 0; i < FM; ++i) {
          q35_f32x4 sxr[4];
          if constexpr (DEQ) {
#pragma unroll
            for (int q = 0; q < 4; ++q)
              sxr[q] = *reinterpret_cast<const q35_f32x4*>(sc + rb0 + i * 32 + 8 * q + 4 * kh);
          }
#pragma unroll
          for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const int off = (rb0 + i * 32 + 8 * (r >> 2) + 4 * kh + (r & 3)) * SB +
                              (wn * FN * 32 + j * 32 + l32) * EB;
              if constexpr (DEQ) {
                const float d = (float)acc[i][j][r] * sxr[r >> 2][r & 3] * swr[j];
                *reinterpret_cast<uint16_t*>(lds + off) = (uint16_t)f2bf(d);
              } else if constexpr (W16)
                *reinterpret_cast<uint16_t*>(lds + off) = (uint16_t)f2bf(acc[i][j][r]);
              else
                *reinterpret_cast<uint32_t*>(lds + off) = acc_bits(acc[i][j][r]);
            }
        }
      }
      __syncthreads();
      q35_u32x4 v[ITER], u[ITER];
#pragma unroll
      for (int it = 0; it < ITER; ++it) {
        const int c = tid + 256 * it;
        const uint8_t* src = lds + (c / CPRW) * SB + (c % CPRW) * 16;
        v[it] = *reinterpret_cast<const q35_u32x4*>(src);
        if constexpr (SWIGLU) u[it] = *reinterpret_cast<const q35_u32x4*>(src + TN / 2 * EB);
      }
#pragma unroll
      for (int it = 0; it < ITER; ++it) {
        const int c = tid + 256 * it;
        const int lrow = h * PR + c / CPRW, lcol = (c % CPRW) * VPC;
        const int grow = m0 + lrow;
        const int col = n0 + lcol;
        if (grow >= a.M || col >= a.N) continue;
        const int ncol = min(VPC, a.N - col);
        const size_t at = (size_t)grow * a.N + col;
        if constexpr (KIND == KIND_I32) {
          int* C = reinterpret_cast<int*>(a.C) + at;
          if (vec && ncol == VPC) *reinterpret_cast<q35_u32x4*>(C) = v[it];
          else for (int e = 0; e < ncol; ++e) C[e] = (int)v[it][e];
        } else if constexpr (KIND == KIND_BF16 || KIND == KIND_DEQ) {
          uint16_t* C = reinterpret_cast<uint16_t*>(a.C) + at;
          if (vec && ncol == VPC) *reinterpret_cast<q35_u32x4*>(C) = v[it];
          else for (int e = 0; e < ncol; ++e) C[e] = (uint16_t)(v[it][e >> 1] >> (16 * (e & 1)));
        } else {  // SwiGLU of the staged bf16 gate and up
          static_assert(VPC == 8, "SwiGLU kinds stage bf16");
          float o[VPC];
#pragma unroll
          for (int e = 0; e < VPC; ++e) {
            const uint32_t gw = v[it][e >> 1], uw = u[it][e >> 1];
            const float g = (e & 1) ? bf_hi(gw) : bf_lo(gw);
            const float uu = (e & 1) ? bf_hi(uw) : bf_lo(uw);
            o[e] = round_bf(silu_fast(g)) * uu;
          }
          uint16_t* C = reinterpret_cast<uint16_t*>(a.C) + at;
          if (vec && ncol == 8) *reinterpret_cast<uint4*>(C) = pack8(o);
          else for (int e = 0; e < ncol; ++e) C[e] = (uint16_t)f2bf(o[e]);
        }
      }
      if (h + 1 < PH) __syncthreads();
    }
  }
}

// ---------------------------------------------------------------- plans
// Tile shapes (waves 2 x 2; FM x FN blocks of 32 x 32 per wave; RB bytes per
// row and stage; NSA / NSB stages in the A / B rings; LDS = NSA TM RB + NSB
// TN RB; K rotation; epilogue staged through LDS, or direct stores for the
// bf16 / int32 kinds):
//   0: 256 x 192 (4 x 3), RB 128, NSA 2, NSB 4,       staged  (160 KiB)
//   1: 128 x 128 (2 x 2), RB 128, NSA 4, NSB 6, rot,  staged  (160 KiB)
//   2: 256 x 128 (4 x 2), RB 128, NSA 2, NSB 4,       staged  (128 KiB)
//   3: 128 x 192 (2 x 3), RB 128, NSA 4, NSB 4, rot,  staged  (160 KiB)
//   4: 256 x 192 (4 x 3), RB 128, NSA 2, NSB 2,       staged  (112 KiB)
//   5: tile 0 with direct stores; 6: tile 1 with direct stores; 7: tile 6
//   without K rotation
//   8: 128 x 64 (2 x 1), RB 128, NSA 6, NSB 8, rot, direct   (160 KiB)
#define Q35_GEMM_TILES(X)                     \
  X(0, 2, 2, 4, 3, 128, 2, 4, false, true)    \
  X(1, 2, 2, 2, 2, 128, 4, 6, true, true)     \
  X(2, 2, 2, 4, 2, 128, 2, 4, false, true)    \
  X(3, 2, 2, 2, 3, 128, 4, 4, true, true)     \
  X(4, 2, 2, 4, 3, 128, 2, 2, false, true)    \
  X(5, 2, 2, 4, 3, 128, 2, 4, false, false)   \
  X(6, 2, 2, 2, 2, 128, 4, 6, true, false)    \
  X(7, 2, 2, 2, 2, 128, 4, 6, false, false)   \
  X(8, 2, 2, 2, 1, 128, 6, 8, true, false)
constexpr int kTiles = 9;
constexpr int kTM[kTiles] = {256, 128, 256, 128, 256, 256, 128, 128, 128};
constexpr int kTN[kTiles] = {192, 128, 128, 192, 192, 192, 128, 128, 64};
constexpr int kRB[kTiles] = {128, 128, 128, 128, 128, 128, 128, 128, 128};
constexpr bool kStaged[kTiles] = {true, true, true, true, true, false, false, false, false};
constexpr bool kSplitOk[kTiles] = {false, true, true, true, false, false, true, true, true};  // up to 8 blocks per wave
constexpr int kMaxSplits = 8;

long long tiles_of(int tile, int M, int N, int kind) {
  const int nc = kind_swiglu(kind) ? kTN[tile] / 2 : kTN[tile];
  return (long long)((M + kTM[tile] - 1) / kTM[tile]) * ((N + nc - 1) / nc);
}

long long workspace_bytes(int tile, int M, int N, int kind, int splits) {
  if (splits <= 1) return 0;
  return kCounterBytes + tiles_of(tile, M, N, kind) * splits * kTM[tile] * kTN[tile] * 4ll;
}

// Default plan by output shape (measured at M = 1024 on the 2B prefill
// shapes, profiles/prefill_gemm_sweep.txt): the widest tile that still gives
// most CUs a workgroup, with direct stores for the bf16 / int32 kinds and the
// staged epilogue for SwiGLU and dequant; outputs with fewer tiles than CUs
// split K only when each split keeps at least 40 stages (the partial-tile
// exchange costs more than the idle CUs below that).
void plan(int M, int N, int K, int kind, int* tile, int* splits) {
  const int es = kind_i8(kind) ? 1 : 2;
  const bool direct = kind == KIND_BF16 || kind == KIND_I32;
  *splits = 1;
  if (kind_swiglu(kind)) {
    *tile = tiles_of(0, M, N, kind) >= 192 ? 0 : 3;
    return;
  }
  if (tiles_of(0, M, N, kind) >= 160) {
    *tile = direct ? 5 : 0;
  } else if (tiles_of(3, M, N, kind) >= 160) {
    *tile = 3;
  } else if (direct && tiles_of(8, M, N, kind) <= 256) {
    // one round of 128x64 tiles: at M = 1024, N = 2048 all 256 CUs without a
    // K split (o_proj 18.4 -> 14.8 us, down 44.9 -> 37.9 us against 128x128
    // tiles on 128 CUs, split 2 for the down projection)
    *tile = 8;
  } else {
    *tile = direct ? 6 : 1;
    const long long t = tiles_of(1, M, N, kind);
    const int nk = K * es / kRB[1];
    while (*splits < kMaxSplits && t * *splits * 2 <= 256 && nk % (*splits * 2) == 0 &&
           nk / (*splits * 2) >= 40 && t <= kMaxSplitTiles)
      *splits *= 2;
  }
}

template <int WM, int WN, int FM, int FN, int RB, int NSA, int NSB, bool ROT, int KIND, bool STAGED>
int launch_one(const GemmArgs& a, hipStream_t stream) {
  if constexpr (!STAGED && KIND != KIND_BF16 && KIND != KIND_I32) {
    return (int)hipErrorInvalidValue;  // direct stores: bf16 and int32 kinds
  } else {
  constexpr int TM = WM * FM * 32, TN = WN * FN * 32;
  constexpr int NC = kind_swiglu(KIND) ? TN / 2 : TN;
  const long long units = (long long)((a.M + TM - 1) / TM) * ((a.N + NC - 1) / NC) * a.splits;
  Q35_CHECK_ARG(units < (1ll << 31));
  if (a.splits > 1) {
    if constexpr (kind_swiglu(KIND) || FM * FN > 8) {
      return (int)hipErrorInvalidValue;  // split K: tiles of up to 8 blocks per wave, no SwiGLU
    } else {
      gemm_ring<WM, WN, FM, FN, RB, NSA, NSB, ROT, KIND, true, STAGED><<<(unsigned)units, 256, 0, stream>>>(a);
    }
  } else {
    gemm_ring<WM, WN, FM, FN, RB, NSA, NSB, ROT, KIND, false, STAGED><<<(unsigned)units, 256, 0, stream>>>(a);
  }
  return q35_last_error();
  }
}

template <int KIND>
int launch_tile(int tile, const GemmArgs& a, hipStream_t stream) {
  switch (tile) {
#define Q35_GEMM_CASE(id, wm, wn, fm, fn, rb, nsa, nsb, rot, staged) \
  case id: return launch_one<wm, wn, fm, fn, rb, nsa, nsb, rot, KIND, staged>(a, stream);
    Q35_GEMM_TILES(Q35_GEMM_CASE)
#undef Q35_GEMM_CASE
    default: return (int)hipErrorInvalidValue;
  }
}

int gemm_run(const void* A, const void* B, void* C, int M, int N, int K, int kind, const float* s_x,
             const float* s_w, int tile, int splits, void* ws, long long ws_bytes, hipStream_t stream) {
  Q35_CHECK_ARG(kind >= 0 && kind < kNumKinds);
  if (tile < 0) plan(M, N, K, kind, &tile, &splits);
  const int es = kind_i8(kind) ? 1 : 2;
  Q35_CHECK_ARG(A && B && C && M > 0 && N > 0 && K > 0);
  Q35_CHECK_ARG(tile >= 0 && tile < kTiles && splits >= 1 && splits <= kMaxSplits);
  Q35_CHECK_ARG(kStaged[tile] || kind == KIND_BF16 || kind == KIND_I32);
  Q35_CHECK_ARG(q35_aligned16(A) && q35_aligned16(B) && ((long long)K * es) % kRB[tile] == 0);
  Q35_CHECK_ARG((kind != KIND_DEQ && kind != KIND_DEQ_SWIGLU) || (s_x && s_w));
  // 32-bit byte offsets of every operand row
  Q35_CHECK_ARG((long long)M * K * es < (1ll << 32) && (kind_swiglu(kind) ? 2ll : 1ll) * N * K * es < (1ll << 32));
  const int nk = (int)((long long)K * es / kRB[tile]);
  Q35_CHECK_ARG(nk % splits == 0);
  if (splits > 1) {
    Q35_CHECK_ARG(kSplitOk[tile] && !kind_swiglu(kind) && tiles_of(tile, M, N, kind) <= kMaxSplitTiles);
    Q35_CHECK_ARG(ws && q35_aligned16(ws) && ws_bytes >= workspace_bytes(tile, M, N, kind, splits));
  }
  GemmArgs a{(const uint8_t*)A, (const uint8_t*)B, C, M, N, K, s_x, s_w, nullptr, nullptr, splits, nk / splits};
  if (splits > 1) {
    a.cnt = (unsigned*)ws;
    a.part = (uint8_t*)ws + kCounterBytes;
  }
  switch (kind) {
    case KIND_BF16: return launch_tile<KIND_BF16>(tile, a, stream);
    case KIND_SWIGLU: return launch_tile<KIND_SWIGLU>(tile, a, stream);
    case KIND_I32: return launch_tile<KIND_I32>(tile, a, stream);
    case KIND_DEQ: return launch_tile<KIND_DEQ>(tile, a, stream);
    default: return launch_tile<KIND_DEQ_SWIGLU>(tile, a, stream);
  }
}

}  // namespace

extern "C" {

// Workspace bytes of q35_gemm for (M, N, K, kind) and a plan (tile < 0: the
// default plan); 0 when the plan does not split K, -1 for an invalid plan.
long long q35_gemm_workspace(int M, int N, int K, int kind, int tile, int splits) {
  if (M <= 0 || N <= 0 || K <= 0 || kind < 0 || kind >= kNumKinds) return -1;
  if (tile < 0) plan(M, N, K, kind, &tile, &splits);
  if (tile >= kTiles || splits < 1 || splits > kMaxSplits) return -1;
  if (!kStaged[tile] && kind != KIND_BF16 && kind != KIND_I32) return -1;
  if (splits > 1 && (!kSplitOk[tile] || kind_swiglu(kind) || tiles_of(tile, M, N, kind) > kMaxSplitTiles))
    return -1;
  return workspace_bytes(tile, M, N, kind, splits);
}

// Prefill GEMM C = A . B^T of the given kind (0 bf16, 1 bf16 SwiGLU, 2 int8 ->
// int32, 3 int8 -> bf16 dequant, 4 int8 SwiGLU; see gemm.hip's header).
// K * element bytes a multiple of 128 (the stage width); A and B 16-byte
// aligned; every operand below 2^32 bytes. tile < 0 picks the default plan,
// otherwise tile 0-8 with `splits` K splits (the stage count divisible by
// splits). A split plan needs a workspace of q35_gemm_workspace bytes,
// zero-filled before its first use.
int q35_gemm(const void* A, const void* B, void* C, int M, int N, int K, int kind, const void* s_x,
             const void* s_w, int tile, int splits, void* workspace, long long workspace_bytes,
             hipStream_t stream) {
  return gemm_run(A, B, C, M, N, K, kind, (const float*)s_x, (const float*)s_w, tile, splits,
                  workspace, workspace_bytes, stream);
}

}  // extern "C"
