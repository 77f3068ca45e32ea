// Prefill GEMMs on the gfx950 matrix cores: C[M, N] = A[M, K] . B[N, K]^T,
// bf16 in, fp32 accumulate (v_mfma_f32_32x32x16_bf16), bf16 out, with the
// SwiGLU of the packed gate/up projection fused into the epilogue.
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
// Status (MI355X, M = 1024, K = 2048): correct, but slower than the ROCm
// library GEMM that F.linear runs (N = 12288: 60 vs 48 us; SwiGLU 63-67 us vs
// ~55 us for library GEMM + silu_mul), so the prefill path keeps the library.
// Measured split of the 60 us: 34 us with the MFMAs alone, +10 us for the
// fragment reads from LDS, +17 us for the global fetches (two stages ahead
// is not enough latency cover at one workgroup per CU; a third register set
// does not fit beside 192 accumulator registers).
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
};

typedef float q35_f32x16 __attribute__((ext_vector_type(16)));
Q35_DEV q35_f32x16 mfma32_bf16(const uint4 a, const uint4 b, q35_f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(q35_bf16x8, a),
                                                 __builtin_bit_cast(q35_bf16x8, b), c, 0, 0, 0);
}

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

template <int WM, int FM, int FN, int EPI>
__global__ __launch_bounds__(256) void gemm_tn(const GemmArgs a) {
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
  int t = blockIdx.x;
  if (T % 8 == 0) t = (t & 7) * (T >> 3) + (t >> 3);
  const int m0 = (t % mtiles) * TM;
  const int n0 = (t / mtiles) * NC;
  const int K = a.K;
  const int nk = K / kBK;

  // Global chunk sources: thread row r0 + 32i, chunk c (rows past the end
  // repeat the last row and are never stored).
  const int r0 = tid >> 3, c = tid & 7;
  const int st_off = r0 * kRowB + 16 * (c ^ ((r0 >> 1) & 7));
  uint32_t offA[LA], offB[LB];
#pragma unroll
  for (int i = 0; i < LA; ++i) offA[i] = (uint32_t)min(m0 + r0 + 32 * i, a.M - 1) * (uint32_t)K + 8 * c;
#pragma unroll
  for (int i = 0; i < LB; ++i) {
    const int row = r0 + 32 * i;
    int brow;
    if (EPI == GEMM_SWIGLU)
      brow = row < TN / 2 ? min(n0 + row, a.N - 1) : a.N + min(n0 + row - TN / 2, a.N - 1);
    else
      brow = min(n0 + row, a.N - 1);
    offB[i] = (uint32_t)brow * (uint32_t)K + 8 * c;
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

  q35_f32x16 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  uint4 ra0[LA], rb0[LB], ra1[LA], rb1[LB];
#define Q35_GLOAD(RA, RB, KT)                                                            \
  do {                                                                                   \
    const uint32_t kk = (uint32_t)(KT) * kBK;                                            \
    _Pragma("unroll") for (int i = 0; i < LA; ++i) RA[i] = *reinterpret_cast<const uint4*>(a.A + offA[i] + kk); \
    _Pragma("unroll") for (int i = 0; i < LB; ++i) RB[i] = *reinterpret_cast<const uint4*>(a.B + offB[i] + kk); \
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
  Q35_GLOAD(ra0, rb0, 0);
  Q35_SSTORE(ra0, rb0, 0);
  Q35_GLOAD(ra1, rb1, min(1, nk - 1));
  Q35_GLOAD(ra0, rb0, min(2, nk - 1));
  lds_barrier();
  for (int kt = 0; kt < nk; kt += 2) {
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
      if (EPI == GEMM_SWIGLU) {
#pragma unroll
        for (int j = 0; j < FN / 2; ++j) {
          const int col = n0 + wn * (FN / 2) * 32 + 32 * j + l32;
          const float g = round_bf(acc[i][j][r]);
          const float u = round_bf(acc[i][j + FN / 2][r]);
          if (col < a.N) crow[col] = (uint16_t)f2bf(round_bf(silu_fast(g)) * u);
        }
      } else {
#pragma unroll
        for (int j = 0; j < FN; ++j) {
          const int col = n0 + wn * FN * 32 + 32 * j + l32;
          if (col < a.N) crow[col] = (uint16_t)f2bf(acc[i][j][r]);
        }
      }
    }
  }
}

template <int WM, int FM, int FN, int EPI>
int launch_gemm(const GemmArgs& a, hipStream_t stream) {
  constexpr int TM = WM * FM * 32, TN = (4 / WM) * FN * 32;
  constexpr int NC = EPI == GEMM_SWIGLU ? TN / 2 : TN;
  const long long tiles = (long long)((a.M + TM - 1) / TM) * ((a.N + NC - 1) / NC);
  Q35_CHECK_ARG(tiles < (1ll << 31));
  gemm_tn<WM, FM, FN, EPI><<<(unsigned)tiles, 256, 0, stream>>>(a);
  return q35_last_error();
}

}  // namespace

extern "C" {

// C[M,N] = bf16(A[M,K] . B[N,K]^T). K a multiple of 128, A/B 16-byte aligned,
// M*K and N*K below 2^32 elements.
int q35_gemm_bf16(const void* A, const void* B, void* C, int M, int N, int K, hipStream_t stream) {
  Q35_CHECK_ARG(A && B && C && M > 0 && N > 0 && K > 0 && K % 128 == 0);
  Q35_CHECK_ARG(q35_aligned16(A) && q35_aligned16(B));
  Q35_CHECK_ARG((long long)M * K < (1ll << 32) && (long long)N * K < (1ll << 32));
  const GemmArgs a{(const uint16_t*)A, (const uint16_t*)B, (uint16_t*)C, M, N, K};
  return launch_gemm<4, 2, 6, GEMM_STORE>(a, stream);
}

// C[M,N] = bf16(bf16(silu(bf16(A.Bg^T))) * bf16(A.Bu^T)) with B = [Bg; Bu]
// ([2N, K]): the packed gate/up projection and silu_and_mul in one launch.
int q35_gemm_swiglu_bf16(const void* A, const void* B, void* C, int M, int N, int K,
                         hipStream_t stream) {
  Q35_CHECK_ARG(A && B && C && M > 0 && N > 0 && K > 0 && K % 128 == 0);
  Q35_CHECK_ARG(q35_aligned16(A) && q35_aligned16(B));
  Q35_CHECK_ARG((long long)M * K < (1ll << 32) && 2ll * N * K < (1ll << 32));
  const GemmArgs a{(const uint16_t*)A, (const uint16_t*)B, (uint16_t*)C, M, N, K};
  return launch_gemm<4, 2, 6, GEMM_SWIGLU>(a, stream);
}

}  // extern "C"
