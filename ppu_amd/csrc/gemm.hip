// Prefill GEMMs on the gfx950 matrix cores: C[M, N] = A[M, K] . B[N, K]^T,
// bf16 in, fp32 accumulate (v_mfma_f32_32x32x16_bf16), bf16 out, with the
// SwiGLU of the packed gate/up projection fused into the epilogue; and the
// same kernel on int8 operands (v_mfma_i32_32x32x32_i8, exact int32
// accumulators) with the A8W8 dequant bf16(float(acc) * s_x[m] * s_w[n])
// in the epilogue.
//
//   STORE  : C[m, n] = bf16(acc)                                 [F.linear, integration.py:183,245,298]
//   SWIGLU : B = [gate; up] (2N rows); C[m, n] = bf16(bf16(silu(bf16 g)) * bf16 u)
//            with g, u the accumulators of rows n and N + n     [integration.py:183-185 + kernels.py:158-180]
//
// Tiling: a workgroup of 4 waves owns a TM x TN tile of (M rows, B rows);
// the waves are stacked along M and each holds FM x FN accumulator tiles of
// 32 x 32 (v_mfma_f32_32x32x16_bf16; SWIGLU: the first FN/2 column tiles are
// gate rows, the last FN/2 the up rows of the same outputs, so the epilogue
// pairs them in registers). K runs in stages of 64: each stage of A and B is
// fetched with 16-byte loads (8 consecutive lanes read one 128-byte row
// segment) two stages ahead into registers, written to one of two LDS
// buffers and read back as MFMA fragments (lane l: row l%32, 8 consecutive
// k at 8*(l/32) of a 16-k step). LDS rows are 128 bytes and the banks span
// 256 bytes (two rows); 16-byte chunk c of row r is stored at chunk
// c ^ ((r >> 1) & 7), so the 16 lanes of one 128-bit access phase hit 16
// different 16-byte bank groups both when reading fragments (16 consecutive
// rows, same logical chunk) and when storing a stage (two rows, 8 chunks
// each). (Swizzling by r & 7 alone left rows r and r + 8 on the same banks:
// measured as SQ_LDS_BANK_CONFLICT.) One barrier per stage.
// (The 32x32 form keeps each accumulator in place; with 16x16 tiles this
// compiler rotated the accumulators through copies every iteration.)
//
// Status (MI355X, M = 1024, the 2B prefill shapes, graph-timed): correct,
// but slower than the ROCm library GEMMs, so the prefill path keeps the
// library. bf16: N x K = 8320x2048 57.8 us vs 48.9, 2048x2048 21.4 vs 18.1,
// 12288x2048 60 vs 50.6, 2048x6144 41.9 vs 43.3 (split K, the one win);
// SwiGLU 61 vs ~57 for library GEMM + silu_mul. int8 (vs torch._int_mm +
// dequant kernel): 46.1 vs 41.3, 21.2 vs 12.0, 30.4 vs 22.6, 52.3 vs 48.1,
// 36.0 vs 28.3. Measured split of the bf16 12288x2048 time: 34 us with the
// MFMAs alone, +10 us for the fragment reads from LDS, +17 us for the global
// fetches (two stages ahead is not enough latency cover at one workgroup per
// CU; a third register set does not fit beside 192 accumulator registers);
// the int8 form halves the MFMA share and keeps the rest. Staging the
// stages straight into LDS (global_load_lds_dwordx4, a 3-4 deep ring) was
// no faster and was dropped.
//
// Tile order: tiles that share B rows (the weights, read once from HBM) run
// on one XCD: with T tiles and T % 8 == 0, workgroup b (dispatched to XCD
// b % 8) takes tile (b % 8) * T/8 + b / 8, M-tile index fastest.
#include "q35_common.hpp"

namespace {

enum { GEMM_STORE = 0, GEMM_SWIGLU = 1 };
constexpr int kBK = 64;        // k per stage: 8 chunks of 16 bytes per row
constexpr int kRowB = 128;     // LDS bytes per tile row and stage

struct GemmArgs {
  const uint16_t* A;  // [M, K]
  const uint16_t* B;  // [N, K], SWIGLU [2N, K]
  uint16_t* C;        // [M, N]
  int M, N, K;
  // split-K: `splits` workgroups per tile each take `kps` stages of K; their
  // fp32 partial tiles go to `ws` and the last one to finish a tile sums them.
  float* ws;
  int splits, kps;
  // A8W8: A and B are int8, C = bf16(float(acc) * s_x[m] * s_w[n]).
  const float* s_x;
  const float* s_w;
};

// Arrival counters of the split-K tiles (one per output tile, at most
// kMaxSplitTiles), in the library's device memory: zero at load, and every
// tile's last workgroup resets its counter, so each launch finds them zero.
// Split-K launches that run at the same time on one GPU (two streams) would
// share them: the prefill path issues its GEMMs on one stream.
constexpr int kMaxSplitTiles = 8192;
__device__ unsigned split_tile_count[kMaxSplitTiles];

typedef float q35_f32x16 __attribute__((ext_vector_type(16)));
typedef int q35_i32x16 __attribute__((ext_vector_type(16)));
typedef int q35_i32x4 __attribute__((ext_vector_type(4)));
Q35_DEV q35_f32x16 mfma32_bf16(const uint4 a, const uint4 b, q35_f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(q35_bf16x8, a),
                                                 __builtin_bit_cast(q35_bf16x8, b), c, 0, 0, 0);
}
// int8 x int8 -> exact int32 (A8W8): 16 bytes per lane and operand, 32 k per
// instruction, the same lane layout in bytes as the bf16 form.
Q35_DEV q35_i32x16 mfma32_bf16(const uint4 a, const uint4 b, q35_i32x16 c) {
  return __builtin_amdgcn_mfma_i32_32x32x32_i8(__builtin_bit_cast(q35_i32x4, a),
                                               __builtin_bit_cast(q35_i32x4, b), c, 0, 0, 0);
}
template <bool I8> struct GemmAcc { using T = q35_f32x16; };
template <> struct GemmAcc<true> { using T = q35_i32x16; };
Q35_DEV uint32_t acc_bits(float v) { return __float_as_uint(v); }
Q35_DEV uint32_t acc_bits(int v) { return (uint32_t)v; }
Q35_DEV float acc_from(uint32_t b, float) { return __uint_as_float(b); }
Q35_DEV int acc_from(uint32_t b, int) { return (int)b; }

// Instruction groups of one GEMM stage in issue order (LLVM sched_group_barrier
// masks: 0x8 MFMA, 0x100 LDS read, 0x200 LDS write, 0x20 global read).
#define Q35_SGB(mask, n) __builtin_amdgcn_sched_group_barrier(mask, n, 0)
template <int FM, int FN>
Q35_DEV void gemm_stage_schedule() {
  constexpr int NF = FM + FN, NMF = FM * FN;  // fragment reads and MFMAs per 16-k step
  Q35_SGB(0x100, NF);                         // step 0 fragments
  _Pragma("unroll") for (int s = 0; s < 3; ++s) {
    _Pragma("unroll") for (int i = 0; i < NF; ++i) { Q35_SGB(0x8, 1); Q35_SGB(0x100, 1); }
    if (s == 0) Q35_SGB(0x8, NMF - NF);
    if (s == 1) {
      _Pragma("unroll") for (int i = 0; i < NMF - NF; ++i) Q35_SGB(0x8, 1), Q35_SGB(0x200, 4);
    }
    if (s == 2) {
      _Pragma("unroll") for (int i = 0; i < NMF - NF; ++i) Q35_SGB(0x8, 1), Q35_SGB(0x20, 4);
    }
  }
  Q35_SGB(0x8, NMF);
}

// The end of every GEMM workgroup: (split-K) the partial-tile exchange and
// sum, then the bf16 (or SwiGLU) store of the tile.
template <int WM, int FM, int FN, int EPI, bool SPLIT, bool I8 = false>
Q35_DEV void gemm_finish(const GemmArgs& a, typename GemmAcc<I8>::T (&acc)[FM][FN], int T, int tile,
                         int ks, int m0, int n0) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wm = (tid >> 6) % WM, wn = (tid >> 6) / WM;
  const int l32 = lane & 31, kh = lane >> 5;
  if (SPLIT) {
    // Partial tiles are stored in accumulator-register order, so the summing
    // workgroup reads back exactly the elements of its own registers. Stores and loads are agent-scope (they bypass the non-
    // coherent per-XCD L2), the stores are complete (vmcnt 0) before the
    // workgroup's arrival is counted, and the partials are summed in split
    // order whichever workgroup arrives last, so the result is deterministic.
    constexpr int NE = FM * FN * 16;
    constexpr int NP = NE / 2;  // 8-byte pairs per thread
    // pair p of thread tid sits at p * 256 + tid: every store and load
    // instruction of a wave covers 512 contiguous bytes
    uint64_t* mine = reinterpret_cast<uint64_t*>(a.ws) + ((size_t)ks * T + tile) * NP * 256 + tid;
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int e = 0; e < 16; e += 2) {
          const uint64_t v = (uint64_t)acc_bits(acc[i][j][e]) |
                             ((uint64_t)acc_bits(acc[i][j][e + 1]) << 32);
          __hip_atomic_store(mine + (size_t)(((i * FN + j) * 16 + e) / 2) * 256, v,
                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __shared__ unsigned arrived;
    lds_barrier();
    if (tid == 0)
      arrived = __hip_atomic_fetch_add(&split_tile_count[tile], 1u, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
    lds_barrier();
    if (arrived != (unsigned)a.splits - 1) return;  // not the last: done
    // The last workgroup reads every partial, its own included, in split
    // order, straight into the accumulators.
    for (int sp = 0; sp < a.splits; ++sp) {
      const uint64_t* src = reinterpret_cast<const uint64_t*>(a.ws) + ((size_t)sp * T + tile) * NP * 256 + tid;
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
          for (int e = 0; e < 16; e += 2) {
            const uint64_t w = __hip_atomic_load(
                const_cast<uint64_t*>(src + (size_t)(((i * FN + j) * 16 + e) / 2) * 256),
                __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const auto lo = acc_from((uint32_t)w, acc[i][j][e]);
            const auto hi = acc_from((uint32_t)(w >> 32), acc[i][j][e]);
            acc[i][j][e] = sp == 0 ? lo : acc[i][j][e] + lo;
            acc[i][j][e + 1] = sp == 0 ? hi : acc[i][j][e + 1] + hi;
          }
    }
    if (tid == 0)
      __hip_atomic_store(&split_tile_count[tile], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }

  // Epilogue: element r of a 32x32 tile sits at row 8*(r/4) + 4*(lane/32) +
  // r%4, column lane%32.
  const int row0 = m0 + wm * FM * 32 + 4 * kh;
#pragma unroll
  for (int i = 0; i < FM; ++i) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = row0 + 32 * i + 8 * (r >> 2) + (r & 3);
      if (row >= a.M) continue;
      uint16_t* crow = a.C + (size_t)row * a.N;
      const float sx = I8 ? a.s_x[row] : 1.f;
      if (EPI == GEMM_SWIGLU) {
#pragma unroll
        for (int j = 0; j < FN / 2; ++j) {
          const int col = n0 + wn * (FN / 2) * 32 + 32 * j + l32;
          float g, u;
          if (I8) {  // dequantise gate and up to bf16 first, as the separate kernels do
            const int cc = min(col, a.N - 1);
            g = round_bf((float)acc[i][j][r] * sx * a.s_w[cc]);
            u = round_bf((float)acc[i][j + FN / 2][r] * sx * a.s_w[a.N + cc]);
          } else {
            g = round_bf(acc[i][j][r]);
            u = round_bf(acc[i][j + FN / 2][r]);
          }
          if (col < a.N) crow[col] = (uint16_t)f2bf(round_bf(silu_fast(g)) * u);
        }
      } else {
#pragma unroll
        for (int j = 0; j < FN; ++j) {
          const int col = n0 + wn * FN * 32 + 32 * j + l32;
          const float v = I8 ? (float)acc[i][j][r] * sx * a.s_w[min(col, a.N - 1)] : (float)acc[i][j][r];
          if (col < a.N) crow[col] = (uint16_t)f2bf(v);
        }
      }
    }
  }
}

template <int WM, int FM, int FN, int EPI, bool SPLIT, bool I8>
__global__ __launch_bounds__(256) void gemm_tn(const GemmArgs a) {
  constexpr int ES = I8 ? 1 : 2;  // bytes per element; a stage is 128 bytes of every row
  static_assert(EPI != GEMM_SWIGLU || FN % 2 == 0, "SwiGLU pairs gate and up tiles");
  static_assert(WM == 1 || WM == 2 || WM == 4, "waves along M");
  constexpr int WN = 4 / WM;
  constexpr int TM = WM * FM * 32, TN = WN * FN * 32;
  constexpr int LA = TM / 32, LB = TN / 32;        // 16-byte chunks per thread and stage
  constexpr int SA = TM * kRowB, SB = TN * kRowB;  // stage bytes of A and B
  constexpr int NC = EPI == GEMM_SWIGLU ? TN / 2 : TN;  // output columns per tile
  __shared__ __attribute__((aligned(16))) uint8_t lds[2 * (SA + SB)];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wm = (tid >> 6) % WM, wn = (tid >> 6) / WM;

  // Tile of this workgroup.
  const int mtiles = (a.M + TM - 1) / TM;
  const int ntiles = (a.N + NC - 1) / NC;
  const int T = mtiles * ntiles;
  // split s of every tile is the s-th run of T workgroups
  const int ks = SPLIT ? (int)blockIdx.x / T : 0;
  int t = SPLIT ? (int)blockIdx.x - ks * T : (int)blockIdx.x;
  const int tile = t;
  if (T % 8 == 0) t = (t & 7) * (T >> 3) + (t >> 3);
  const int m0 = (t % mtiles) * TM;
  const int n0 = (t / mtiles) * NC;
  const int K = a.K;
  const int kbeg = SPLIT ? ks * a.kps : 0;
  const int nk = SPLIT ? kbeg + a.kps : K * ES / kRowB;  // one past this workgroup's last stage

  // Global chunk sources: thread row r0 + 32i, chunk c (rows past the end
  // repeat the last row and are never stored).
  const int r0 = tid >> 3, c = tid & 7;
  const int st_off = r0 * kRowB + 16 * (c ^ ((r0 >> 1) & 7));
  uint32_t offA[LA], offB[LB];
#pragma unroll
  for (int i = 0; i < LA; ++i) offA[i] = (uint32_t)min(m0 + r0 + 32 * i, a.M - 1) * (uint32_t)(K * ES) + 16 * c;
#pragma unroll
  for (int i = 0; i < LB; ++i) {
    const int row = r0 + 32 * i;
    int brow;
    if (EPI == GEMM_SWIGLU)
      brow = row < TN / 2 ? min(n0 + row, a.N - 1) : a.N + min(n0 + row - TN / 2, a.N - 1);
    else
      brow = min(n0 + row, a.N - 1);
    offB[i] = (uint32_t)brow * (uint32_t)(K * ES) + 16 * c;
  }

  // Fragment sources in a stage: lane row l32 of a 32-row tile, logical
  // chunk 2s + kh of the 16-k step s.
  const int l32 = lane & 31, kh = lane >> 5;
  int swz[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) swz[s] = 16 * ((2 * s + kh) ^ ((l32 >> 1) & 7));
  const int a_row = (wm * FM * 32 + l32) * kRowB;
  // B rows of column tile j: STORE, the wave's FN tiles; SWIGLU, its FN/2
  // gate tiles in the first half of the stage and the matching up tiles in
  // the second half.
  int b_row[FN];
#pragma unroll
  for (int j = 0; j < FN; ++j) {
    const int r = EPI == GEMM_SWIGLU
                      ? (j < FN / 2 ? wn * (FN / 2) * 32 + 32 * j : TN / 2 + wn * (FN / 2) * 32 + 32 * (j - FN / 2))
                      : wn * FN * 32 + 32 * j;
    b_row[j] = SA + (r + l32) * kRowB;
  }

  typename GemmAcc<I8>::T acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0;

  uint4 ra0[LA], rb0[LB], ra1[LA], rb1[LB];
#define Q35_GLOAD(RA, RB, KT)                                                            \
  do {                                                                                   \
    const uint32_t kk = (uint32_t)(KT) * kRowB;                                          \
    _Pragma("unroll") for (int i = 0; i < LA; ++i) RA[i] = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint8_t*>(a.A) + offA[i] + kk); \
    _Pragma("unroll") for (int i = 0; i < LB; ++i) RB[i] = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint8_t*>(a.B) + offB[i] + kk); \
  } while (0)
#define Q35_SSTORE(RA, RB, ST)                                                           \
  do {                                                                                   \
    uint8_t* sb = lds + (ST) * (SA + SB) + st_off;                                       \
    _Pragma("unroll") for (int i = 0; i < LA; ++i) {                                     \
      const q35_u32x4 v = {RA[i].x, RA[i].y, RA[i].z, RA[i].w};                          \
      *reinterpret_cast<q35_u32x4*>(sb + i * 32 * kRowB) = v;                            \
    }                                                                                    \
    _Pragma("unroll") for (int i = 0; i < LB; ++i) {                                     \
      const q35_u32x4 v = {RB[i].x, RB[i].y, RB[i].z, RB[i].w};                          \
      *reinterpret_cast<q35_u32x4*>(sb + SA + i * 32 * kRowB) = v;                       \
    }                                                                                    \
  } while (0)
#define Q35_READ(FA, FB, SB, S)                                                          \
  do {                                                                                   \
    _Pragma("unroll") for (int i = 0; i < FM; ++i)                                       \
      FA[i] = *reinterpret_cast<const uint4*>((SB) + a_row + i * 32 * kRowB + swz[S]);   \
    _Pragma("unroll") for (int j = 0; j < FN; ++j)                                       \
      FB[j] = *reinterpret_cast<const uint4*>((SB) + b_row[j] + swz[S]);                 \
  } while (0)
#define Q35_MFMA(FA, FB)                                                                 \
  do {                                                                                   \
    _Pragma("unroll") for (int i = 0; i < FM; ++i)                                       \
      _Pragma("unroll") for (int j = 0; j < FN; ++j) acc[i][j] = mfma32_bf16(FA[i], FB[j], acc[i][j]); \
  } while (0)
  // One stage: the fragments of 16-k step s + 1 are read while the MFMAs of
  // step s run, the next stage's registers go to the other LDS buffer after
  // step 1 and the fetch two stages ahead is issued after step 2; the group
  // barriers keep the scheduler from clustering the LDS and memory traffic
  // away from the MFMAs.
#define Q35_SCHED() gemm_stage_schedule<FM, FN>()
#define Q35_STAGE(ST, RAS, RBS, NST, RAL, RBL, KTL)                                      \
  do {                                                                                   \
    const uint8_t* sb = lds + (ST) * (SA + SB);                                          \
    uint4 fa0[FM], fb0[FN], fa1[FM], fb1[FN];                                            \
    Q35_READ(fa0, fb0, sb, 0);                                                           \
    Q35_READ(fa1, fb1, sb, 1);                                                           \
    Q35_MFMA(fa0, fb0);                                                                  \
    Q35_READ(fa0, fb0, sb, 2);                                                           \
    Q35_MFMA(fa1, fb1);                                                                  \
    Q35_SSTORE(RAS, RBS, NST);                                                           \
    Q35_READ(fa1, fb1, sb, 3);                                                           \
    Q35_MFMA(fa0, fb0);                                                                  \
    Q35_GLOAD(RAL, RBL, KTL);                                                            \
    Q35_MFMA(fa1, fb1);                                                                  \
    Q35_SCHED();                                                                         \
  } while (0)

  // Stage 0 in LDS, stages 1 and 2 in flight; every later stage is fetched
  // two steps before use. Fetch indices are clamped (the extra fetches at
  // the end are never used), so no load sits behind a branch.
  Q35_GLOAD(ra0, rb0, kbeg);
  Q35_SSTORE(ra0, rb0, 0);
  Q35_GLOAD(ra1, rb1, min(kbeg + 1, nk - 1));
  Q35_GLOAD(ra0, rb0, min(kbeg + 2, nk - 1));
  lds_barrier();
  for (int kt = kbeg; kt < nk; kt += 2) {
    Q35_STAGE(0, ra1, rb1, 1, ra1, rb1, min(kt + 3, nk - 1));
    lds_barrier();
    Q35_STAGE(1, ra0, rb0, 0, ra0, rb0, min(kt + 4, nk - 1));
    lds_barrier();
  }
#undef Q35_READ
#undef Q35_MFMA
#undef Q35_STAGE
#undef Q35_SCHED
#undef Q35_GLOAD
#undef Q35_SSTORE

  gemm_finish<WM, FM, FN, EPI, SPLIT, I8>(a, acc, T, tile, ks, m0, n0);
}

// Tile shapes (waves along M, 32x32 MFMA tiles per wave along M and N):
// 0: 256x192 (4x1 waves, 2x6 tiles); 1: 128x128 (2x2 waves, 2x2);
// 2: 256x128 (4x1 waves, 2x4); 3: 128x256 (2x2 waves, 2x4).
constexpr int kTiles = 4;
constexpr int kTileTM[kTiles] = {256, 128, 256, 128};
constexpr int kTileTN[kTiles] = {192, 128, 128, 256};
constexpr int kTileRegs[kTiles] = {12 * 16, 4 * 16, 8 * 16, 8 * 16};  // accumulators per thread

template <int WM, int FM, int FN, int EPI, bool I8>
int launch_gemm(const GemmArgs& a, hipStream_t stream) {
  constexpr int TM = WM * FM * 32, TN = (4 / WM) * FN * 32;
  constexpr int NC = EPI == GEMM_SWIGLU ? TN / 2 : TN;
  const long long tiles = (long long)((a.M + TM - 1) / TM) * ((a.N + NC - 1) / NC);
  Q35_CHECK_ARG(tiles * a.splits < (1ll << 31));
  if (a.splits > 1) {
    if constexpr (FM * FN <= 8) {
      Q35_CHECK_ARG(tiles <= kMaxSplitTiles && a.ws);
      gemm_tn<WM, FM, FN, EPI, true, I8><<<(unsigned)(tiles * a.splits), 256, 0, stream>>>(a);
    } else {
      return (int)hipErrorInvalidValue;  // split-K for the tiles of up to 8 MFMA blocks per wave
    }
  } else {
    gemm_tn<WM, FM, FN, EPI, false, I8><<<(unsigned)tiles, 256, 0, stream>>>(a);
  }
  return q35_last_error();
}

template <int EPI, bool I8>
int launch_tile(int tile, const GemmArgs& a, hipStream_t stream) {
  switch (tile) {
    case 0: return launch_gemm<4, 2, 6, EPI, I8>(a, stream);
    case 1: return launch_gemm<2, 2, 2, EPI, I8>(a, stream);
    case 2: return launch_gemm<4, 2, 4, EPI, I8>(a, stream);
    case 3: return launch_gemm<2, 2, 4, EPI, I8>(a, stream);
    default: return (int)hipErrorInvalidValue;
  }
}

long long tiles_of(int tile, int M, int N, int swiglu) {
  const int nc = swiglu ? kTileTN[tile] / 2 : kTileTN[tile];
  return (long long)((M + kTileTM[tile] - 1) / kTileTM[tile]) * ((N + nc - 1) / nc);
}

// Tile shape and split count by output shape (measured at M = 1024 on the 2B
// prefill shapes): 128x128 tiles unless the output is wide enough for
// 256x192 (N >= 12288); outputs that leave fewer tiles than CUs (N = 2048)
// split K over 2 workgroups per tile.
void plan(int M, int N, int K, int es, int swiglu, int* tile, int* splits) {
  *tile = (swiglu ? 2 * N : N) >= 12288 ? 0 : 1;
  *splits = 1;
  if (swiglu) return;
  const int nk = K * es / kRowB;
  if (*tile == 1 && tiles_of(1, M, N, 0) < 256 && nk % 4 == 0 && tiles_of(1, M, N, 0) <= kMaxSplitTiles)
    *splits = 2;
}

long long workspace_bytes(int tile, int M, int N, int splits, int swiglu) {
  if (splits <= 1) return 0;
  return tiles_of(tile, M, N, swiglu) * splits * 256ll * kTileRegs[tile] * 4;
}

int gemm_run(const void* A, const void* B, void* C, int M, int N, int K, int tile, int splits,
             int swiglu, bool i8, const float* s_x, const float* s_w, void* ws, long long ws_bytes,
             hipStream_t stream) {
  const int es = i8 ? 1 : 2;
  Q35_CHECK_ARG(A && B && C && M > 0 && N > 0 && K > 0 && (K * es) % (2 * kRowB) == 0);
  Q35_CHECK_ARG(q35_aligned16(A) && q35_aligned16(B));
  Q35_CHECK_ARG(!i8 || (s_x && s_w));
  Q35_CHECK_ARG((long long)M * K * es < (1ll << 32) && (swiglu ? 2ll : 1ll) * N * K * es < (1ll << 32));
  Q35_CHECK_ARG(tile >= 0 && tile < kTiles && splits >= 1 && splits <= 16);
  const int nk = K * es / kRowB;
  Q35_CHECK_ARG(nk % (2 * splits) == 0);  // every split runs whole pairs of stages
  Q35_CHECK_ARG(splits == 1 || ws_bytes >= workspace_bytes(tile, M, N, splits, swiglu));
  const GemmArgs a{(const uint16_t*)A, (const uint16_t*)B, (uint16_t*)C, M, N, K,
                   (float*)ws, splits, nk / splits, s_x, s_w};
  if (i8)
    return swiglu ? launch_tile<GEMM_SWIGLU, true>(tile, a, stream)
                  : launch_tile<GEMM_STORE, true>(tile, a, stream);
  return swiglu ? launch_tile<GEMM_SWIGLU, false>(tile, a, stream)
                : launch_tile<GEMM_STORE, false>(tile, a, stream);
}

}  // namespace

extern "C" {

// Workspace bytes q35_gemm_bf16 / q35_gemm_swiglu_bf16 need for this shape.
long long q35_gemm_workspace(int M, int N, int K, int swiglu) {
  if (M <= 0 || N <= 0 || K <= 0) return 0;
  int tile, splits;
  plan(M, N, K, 2, swiglu, &tile, &splits);
  return workspace_bytes(tile, M, N, splits, swiglu);
}

// C[M,N] = bf16(A[M,K] . B[N,K]^T). K a multiple of 128, A/B 16-byte aligned,
// M*K and N*K below 2^31 elements; workspace of q35_gemm_workspace bytes.
int q35_gemm_bf16(const void* A, const void* B, void* C, int M, int N, int K, void* workspace,
                  long long workspace_bytes, hipStream_t stream) {
  int tile, splits;
  plan(M, N, K, 2, 0, &tile, &splits);
  return gemm_run(A, B, C, M, N, K, tile, splits, 0, false, nullptr, nullptr, workspace,
                  workspace_bytes, stream);
}

// C[M,N] = bf16(bf16(silu(bf16(A.Bg^T))) * bf16(A.Bu^T)) with B = [Bg; Bu]
// ([2N, K]): the packed gate/up projection and silu_and_mul in one launch.
int q35_gemm_swiglu_bf16(const void* A, const void* B, void* C, int M, int N, int K,
                         void* workspace, long long workspace_bytes, hipStream_t stream) {
  int tile, splits;
  plan(M, N, K, 2, 1, &tile, &splits);
  return gemm_run(A, B, C, M, N, K, tile, splits, 1, false, nullptr, nullptr, workspace,
                  workspace_bytes, stream);
}

// Explicit tile shape (0-3) and split count (K / 64 divisible by 2 * splits),
// for measurement and tests; workspace_bytes as returned for that plan by
// q35_gemm_plan_workspace.
int q35_gemm_bf16_plan(const void* A, const void* B, void* C, int M, int N, int K, int tile,
                       int splits, int swiglu, void* workspace, long long workspace_bytes,
                       hipStream_t stream) {
  return gemm_run(A, B, C, M, N, K, tile, splits, swiglu, false, nullptr, nullptr, workspace,
                  workspace_bytes, stream);
}

long long q35_gemm_plan_workspace(int M, int N, int tile, int splits, int swiglu) {
  if (M <= 0 || N <= 0 || tile < 0 || tile >= kTiles || splits < 1) return -1;
  return workspace_bytes(tile, M, N, splits, swiglu);
}

// A8W8 prefill GEMM: int8 A[M,K] (per-token quantised, scales s_x[M]) times
// int8 B[N,K]^T (per-channel, scales s_w[N]; swiglu: B = [gate; up] [2N, K],
// s_w [2N]) on the int8 matrix cores, exact int32 accumulators, dequantised
// in the epilogue: C = bf16(float(acc) * s_x[m] * s_w[n]) (swiglu: gate and up
// dequantised to bf16, then bf16(silu(g)) * u). K a multiple of 256. tile < 0
// picks the plan; workspace of q35_gemm_a8w8_workspace bytes for that plan.
long long q35_gemm_a8w8_workspace(int M, int N, int K, int swiglu, int tile, int splits) {
  if (M <= 0 || N <= 0 || K <= 0) return 0;
  if (tile < 0) plan(M, N, K, 1, swiglu, &tile, &splits);
  if (tile >= kTiles || splits < 1) return -1;
  return workspace_bytes(tile, M, N, splits, swiglu);
}

int q35_gemm_a8w8(const void* Aq, const void* s_x, const void* Bq, const void* s_w, void* C, int M,
                  int N, int K, int swiglu, int tile, int splits, void* workspace,
                  long long workspace_bytes, hipStream_t stream) {
  if (tile < 0) plan(M, N, K, 1, swiglu, &tile, &splits);
  return gemm_run(Aq, Bq, C, M, N, K, tile, splits, swiglu, true, (const float*)s_x,
                  (const float*)s_w, workspace, workspace_bytes, stream);
}

}  // extern "C"
