// Full-attention layer kernels: Q/K RMSNorm + partial RoPE with the static
// KV-cache write, split-K GQA decode attention with a log-sum-exp combine
// (optionally fused with the sigmoid output gate), and causal GQA prefill
// attention.
//
// Layouts:
//   packed QGKV [B, L, 2*QH*D + 2*KVH*D] = per q head [q (D) | gate (D)], then k (KVH*D), v (KVH*D)
//   q           [B, QH, L, D] bf16
//   K/V cache   [B, KVH, cache_len, D] bf16; the valid length / write offset is
//               an int64 device scalar, so no launch depends on host state.
#include "q35_common.hpp"

namespace {

// ------------------------------------------------------------ QGKV norm + RoPE
// One wave per (token, q head); lane owns E = D/64 consecutive dims.
// Rounding points follow the reference kernel (kernels.py:419-573):
//   n = bf16(x * rsqrt(mean(x^2) + 1e-6) * (1 + w))
//   rot = bf16(bf16(n*cos) + bf16(bf16(+-n_partner) * sin)) for dims < rotary_dim
template <int E>
Q35_DEV void norm_head(const uint16_t* __restrict__ src, const void* w, int w_f32, int lane, int D,
                       float (&n)[E]) {
  float x[E];
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    x[e] = bf2f(src[lane * E + e]);
    ss += x[e] * x[e];
  }
  const float inv = rsqrt_cr(wave_sum(ss) / (float)D + 1.0e-6f);
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int c = lane * E + e;
    const float wc = w_f32 ? reinterpret_cast<const float*>(w)[c] : bf2f(reinterpret_cast<const uint16_t*>(w)[c]);
    n[e] = round_bf(x[e] * inv * (1.0f + wc));
  }
}

template <int E>
Q35_DEV void rope_head(const float (&n)[E], const uint16_t* __restrict__ cos,
                       const uint16_t* __restrict__ sin, int lane, int rot, float (&o)[E]) {
  const int half = rot / 2;
  const int shift = half / E;  // partner lane distance (half is a multiple of E)
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int c = lane * E + e;
    const int partner_lane = c < half ? lane + shift : lane - shift;
    const float pn = __shfl(n[e], partner_lane & 63, 64);
    if (c < rot) {
      const float cs = bf2f(cos[c]), sn = bf2f(sin[c]);
      const float qc = round_bf(n[e] * cs);
      const float rh = c < half ? -pn : pn;
      const float qs = round_bf(rh * sn);
      o[e] = round_bf(qc + qs);
    } else {
      o[e] = n[e];
    }
  }
}

template <int E>
__global__ __launch_bounds__(256) void qgkv_norm_rope_k(
    const uint16_t* __restrict__ packed, const void* qw, const void* kw, int w_f32,
    const uint16_t* __restrict__ cos, const uint16_t* __restrict__ sin, uint16_t* __restrict__ q_out,
    uint16_t* __restrict__ k_out, uint16_t* __restrict__ v_out, const long long* cache_start,
    int B, int L, int QH, int KVH, int D, int rot, int cache_len) {
  const int lane = threadIdx.x & 63;
  const int pid = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (pid >= B * L * QH) return;
  const int head = pid % QH;
  const int tf = pid / QH;  // b*L + t
  const int t = tf % L, b = tf / L;
  const int P = 2 * QH * D + 2 * KVH * D;
  const uint16_t* row = packed + (size_t)tf * P;
  const uint16_t* cs = cos + (size_t)tf * rot;
  const uint16_t* sn = sin + (size_t)tf * rot;

  float n[E], o[E];
  norm_head<E>(row + head * 2 * D, qw, w_f32, lane, D, n);
  rope_head<E>(n, cs, sn, lane, rot, o);
  uint16_t* qo = q_out + (((size_t)b * QH + head) * L + t) * D;
#pragma unroll
  for (int e = 0; e < E; ++e) qo[lane * E + e] = (uint16_t)f2bf(o[e]);

  if (head < KVH) {
    const uint16_t* krow = row + 2 * QH * D + head * D;
    const uint16_t* vrow = row + 2 * QH * D + KVH * D + head * D;
    norm_head<E>(krow, kw, w_f32, lane, D, n);
    rope_head<E>(n, cs, sn, lane, rot, o);
    long long pos = t;
    int len = L;
    if (cache_start) {
      pos += cache_start[0];
      len = cache_len;
    }
    if (pos >= 0 && pos < len) {  // never write outside the cache
      const size_t off = (((size_t)b * KVH + head) * len + pos) * D;
#pragma unroll
      for (int e = 0; e < E; ++e) {
        k_out[off + lane * E + e] = (uint16_t)f2bf(o[e]);
        v_out[off + lane * E + e] = vrow[lane * E + e];
      }
    }
  }
}

// ------------------------------------------------------- GQA split-K decode
// Grid (KVH, splits): a workgroup reads one contiguous chunk of one KV head
// once and serves all G = QH/KVH query heads of that head, so K/V bytes are
// read from HBM exactly once per step. D = 256. A workgroup of 4 waves covers
// 32 tokens per iteration, 8 per wave in two groups of 4 (8 waves, two per
// SIMD, measured no faster: the per-workgroup latency chain dominates):
//   QK: lane = (token row lane/16 of a group, dims 8*(lane%16) and
//       128 + 8*(lane%16)); bf16 pair dot products (v_dot2) reduced over the
//       16-lane DPP row, then times the softmax scale.
//   PV: lane owns dims 4*lane..4*lane+3; p values are broadcast by readlane.
// The loads that the Q/K norm + RoPE prologue needs are issued first and the
// K/V rows of the first iteration right after, so the prologue runs while
// K/V are in flight (loads retire in order); later iterations are prefetched
// one ahead. Each wave runs an online softmax over its tokens, the waves are
// merged in LDS and the workgroup writes (acc[D], m, l) per query head and
// split; gqa_decode_combine merges the splits.
constexpr int kAD = 256;
constexpr int kMaxG = 8;
constexpr int kSplitWaves = 4;                // waves per split workgroup
constexpr int kWaveTok = 32 / kSplitWaves;    // tokens per wave per iteration
constexpr int kWaveGroups = kWaveTok / 4;     // K row groups of 4 tokens per wave
static_assert(kWaveTok % 4 == 0 && kWaveGroups >= 1, "4-token K row groups per wave");
constexpr int kIterTok = kSplitWaves * kWaveTok;  // tokens per workgroup iteration
constexpr int kMaxSplits = 128;            // splits per KV head

// Extra inputs of the fused decode step: the packed QGKV row of the current
// token, the Q/K norm weights, the rotary frequencies and positions. The
// kernel then normalises and rotates q itself (every workgroup, its own G
// heads), and the workgroup whose chunk holds the new token also computes
// k, writes k and v into the cache and attends to the new token from LDS.
struct FusedQ {
  const uint16_t* packed;      // [2*QH*D + 2*KVH*D]
  const void* q_w;
  const void* k_w;
  int w_f32;
  const float* inv_freq;       // [rot/2] fp32
  const long long* pos_t;      // text/temporal position
  const long long* pos_h;      // multimodal rope rows (may equal pos_t)
  const long long* pos_w;
  int sec_h, sec_w;            // interleaved mrope: frequencies taken from H / W rows
  int rot;                     // rotary dims (64)
  uint16_t* k_cache;           // written at the new token's position
  uint16_t* v_cache;
};

// Global loads of one 256-wide head (lane: dims 4*lane..+3) and its norm
// weights (bf16 in w0, or fp32 in w0:w1).
struct HeadLoads {
  uint2 x, w0, w1;
};
Q35_DEV HeadLoads load_head(const uint16_t* __restrict__ src, const void* w, int w_f32, int lane) {
  HeadLoads h;
  h.x = *reinterpret_cast<const uint2*>(src + 4 * lane);
  const char* wb = reinterpret_cast<const char*>(w) + (w_f32 ? 16 * lane : 8 * lane);
  h.w0 = *reinterpret_cast<const uint2*>(wb);
  h.w1 = *reinterpret_cast<const uint2*>(wb + (w_f32 ? 8 : 0));
  return h;
}

// Rotary inputs: lane j owns frequency i = j mod rot/2 (rot/2 <= 64).
struct RopeLoads {
  float invf;
  long long pt, ph, pw;
};
Q35_DEV RopeLoads load_rope(const FusedQ& f, int lane) {
  // The positions are vector loads (nontemporal): issued in program order
  // with the other prologue loads, they return before the K/V stream instead
  // of waiting on the scalar cache.
  RopeLoads r;
  r.invf = f.inv_freq[lane % (f.rot / 2)];
  r.pt = __builtin_nontemporal_load(f.pos_t);
  r.ph = __builtin_nontemporal_load(f.pos_h);
  r.pw = __builtin_nontemporal_load(f.pos_w);
  return r;
}

// cos/sin of the lane's 4 dims (bf16-rounded), shared by every head of the
// token: freq_i = pos * inv_freq[i] in fp32, the position row of frequency i
// chosen by the interleaved multimodal sections, cos/sin in fp32 rounded to
// bf16, exactly as Transformers' rotary table; dims c and c + rot/2 share
// frequency c mod rot/2. Lane j computes frequency j mod rot/2 once and the
// lanes gather theirs by shuffle.
struct RopeTable {
  float cs[4], sn[4];
};
Q35_DEV RopeTable rope_table(const RopeLoads& r, const FusedQ& f, int lane) {
  const int half = f.rot / 2;
  const int i = lane % half;
  long long p = r.pt;
  if (i % 3 == 1 && i < 3 * f.sec_h) p = r.ph;
  if (i % 3 == 2 && i < 3 * f.sec_w) p = r.pw;
  float sn, cs;
  sincosf((float)p * r.invf, &sn, &cs);
  cs = round_bf(cs);
  sn = round_bf(sn);
  RopeTable t;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int src = (lane * 4 + e) % half;
    t.cs[e] = __shfl(cs, src, 64);
    t.sn[e] = __shfl(sn, src, 64);
  }
  return t;
}

// Q/K RMSNorm (1 + w) + partial RoPE of one head from its loads. Rounding
// points follow the reference kernel (kernels.py:419-573):
//   n = bf16(x * rsqrt(mean(x^2) + 1e-6) * (1 + w))
//   rot = bf16(bf16(n*cos) + bf16(bf16(+-n_partner) * sin)) for dims < rot
Q35_DEV void norm_rope(const HeadLoads& h, int w_f32, const RopeTable& t, int rot, int lane,
                       float (&o)[4]) {
  const float x[4] = {bf_lo(h.x.x), bf_hi(h.x.x), bf_lo(h.x.y), bf_hi(h.x.y)};
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < 4; ++e) ss += x[e] * x[e];
  const float inv = rsqrt_cr(wave_sum(ss) / (float)kAD + 1.0e-6f);
  float wc[4];
  if (w_f32) {
    wc[0] = __uint_as_float(h.w0.x); wc[1] = __uint_as_float(h.w0.y);
    wc[2] = __uint_as_float(h.w1.x); wc[3] = __uint_as_float(h.w1.y);
  } else {
    wc[0] = bf_lo(h.w0.x); wc[1] = bf_hi(h.w0.x); wc[2] = bf_lo(h.w0.y); wc[3] = bf_hi(h.w0.y);
  }
  float n[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) n[e] = round_bf(x[e] * inv * (1.0f + wc[e]));
  const int half = rot / 2;
  const int shift = half / 4;
  // Partner of dim c is c + half (first half) or c - half: lane +- half/4.
  const bool first = lane * 4 < half;
  const int partner_lane = (first ? lane + shift : lane - shift) & 63;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float pn = __shfl(n[e], partner_lane, 64);
    const float qc = round_bf(n[e] * t.cs[e]);
    const float rh = first ? -pn : pn;
    const float r = round_bf(qc + round_bf(rh * t.sn[e]));
    o[e] = lane * 4 < rot ? r : n[e];
  }
}

// Prefill Q/K norm + RoPE for 256-wide heads (the qgkv_norm_rope_k contract,
// same arithmetic as norm_rope): one wave per (token, query head), lane dims
// 4*lane .. +3. Every load (the q head and its norm weights, the token's
// cos/sin, and the k and v heads with the k weights, read by every wave and
// used by waves of heads < KVH) is an 8-byte vector load issued before any
// arithmetic; the weight type is chosen by address, so no branch separates
// the loads. rot > 0, rot % 8 == 0 (checked on the host).
__global__ __launch_bounds__(256) void qgkv_norm_rope_256(
    const uint16_t* __restrict__ packed, const void* qw, const void* kw, int w_f32,
    const uint16_t* __restrict__ cos, const uint16_t* __restrict__ sin, uint16_t* __restrict__ q_out,
    uint16_t* __restrict__ k_out, uint16_t* __restrict__ v_out, const long long* cache_start,
    int B, int L, int QH, int KVH, int rot, int cache_len) {
  const int lane = threadIdx.x & 63;
  const int pid = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (pid >= B * L * QH) return;
  const int head = pid % QH;
  const int tf = pid / QH;  // b*L + t
  const int t = tf % L, b = tf / L;
  const uint16_t* row = packed + (size_t)tf * (2 * QH * kAD + 2 * KVH * kAD);
  const int kh = min(head, KVH - 1);
  const HeadLoads hq = load_head(row + head * 2 * kAD, qw, w_f32, lane);
  const HeadLoads hk = load_head(row + 2 * QH * kAD + kh * kAD, kw, w_f32, lane);
  const uint2 vv = *reinterpret_cast<const uint2*>(row + 2 * QH * kAD + KVH * kAD + kh * kAD + 4 * lane);
  const int rc = (4 * lane) % rot;  // lanes past rot/4 read valid, unused entries
  const uint2 cr = *reinterpret_cast<const uint2*>(cos + (size_t)tf * rot + rc);
  const uint2 sr = *reinterpret_cast<const uint2*>(sin + (size_t)tf * rot + rc);
  const long long start = cache_start ? cache_start[0] : 0;
  RopeTable tab;
  tab.cs[0] = bf_lo(cr.x); tab.cs[1] = bf_hi(cr.x); tab.cs[2] = bf_lo(cr.y); tab.cs[3] = bf_hi(cr.y);
  tab.sn[0] = bf_lo(sr.x); tab.sn[1] = bf_hi(sr.x); tab.sn[2] = bf_lo(sr.y); tab.sn[3] = bf_hi(sr.y);
  float o[4];
  norm_rope(hq, w_f32, tab, rot, lane, o);
  uint16_t* qo = q_out + (((size_t)b * QH + head) * L + t) * kAD + 4 * lane;
  *reinterpret_cast<uint2*>(qo) = make_uint2(pack_bf2(o[0], o[1]), pack_bf2(o[2], o[3]));
  if (head < KVH) {
    norm_rope(hk, w_f32, tab, rot, lane, o);
    const long long pos = t + start;
    const int len = cache_start ? cache_len : L;
    if (pos >= 0 && pos < len) {  // never write outside the cache
      const size_t off = (((size_t)b * KVH + head) * len + pos) * kAD + 4 * lane;
      *reinterpret_cast<uint2*>(k_out + off) = make_uint2(pack_bf2(o[0], o[1]), pack_bf2(o[2], o[3]));
      *reinterpret_cast<uint2*>(v_out + off) = vv;
    }
  }
}

// Max of a value that is uniform within each 16-lane row, over the 4 rows.
Q35_DEV float rows4_max(float v) {
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

Q35_DEV float dot2_bf16(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(q35_bf16x2, a),
                                         __builtin_bit_cast(q35_bf16x2, b), c, false);
}

template <int G, bool FUSED>
__global__ __launch_bounds__(kSplitWaves * 64) void gqa_decode_split(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ Kc, const uint16_t* __restrict__ Vc,
    const long long* __restrict__ valid_len, float* __restrict__ acc_out, float* __restrict__ ml_out,
    int cache_len, int chunk, int splits, float scale, const FusedQ fq) {
  constexpr int NW = kSplitWaves;
  constexpr int HPW = (G + NW - 1) / NW;  // query heads per wave in the prologue
  const int lane = threadIdx.x & 63;
  const int wid = threadIdx.x >> 6;
  const int kvh = blockIdx.x;
  const int split = blockIdx.y;
  const int KVH = gridDim.x;
  const int QH = G * KVH;
  // FUSED: valid_len counts the tokens before this one; the new token sits at
  // index n_old and is attended from LDS by the workgroup that owns it.
  const long long n_old = FUSED ? valid_len[0] : 0;
  const int n_cached = FUSED ? (int)min((long long)cache_len, n_old)
                             : (int)min((long long)cache_len, valid_len[0]);
  const int start = split * chunk;
  const int end = min(start + chunk, n_cached);
  const bool owns_new = FUSED && n_old >= start && n_old < start + chunk;
  const int n_iter = end > start ? (end - start + kIterTok - 1) / kIterTok : 0;

  // 1. prologue loads: the wave's query heads, and (FUSED) the new token's k
  //    and v rows, the norm weights and the rotary inputs.
  HeadLoads hq[HPW], hk;
  uint2 vnew = make_uint2(0, 0);
  RopeLoads rl;
#pragma unroll
  for (int j = 0; j < HPW; ++j) {
    const int g = (wid + NW * j) % G;
    if (FUSED) {
      hq[j] = load_head(fq.packed + (size_t)(kvh * G + g) * 2 * kAD, fq.q_w, fq.w_f32, lane);
    } else {
      hq[j].x = *reinterpret_cast<const uint2*>(q + (size_t)(kvh * G + g) * kAD + 4 * lane);
    }
  }
  if (FUSED) {
    const uint16_t* krow = fq.packed + (size_t)2 * QH * kAD + (size_t)kvh * kAD;
    hk = load_head(krow, fq.k_w, fq.w_f32, lane);
    vnew = *reinterpret_cast<const uint2*>(krow + (size_t)KVH * kAD + 4 * lane);
    rl = load_rope(fq, lane);
  }

  // 2. K/V rows of the first iteration. Group gi of a wave holds tokens
  //    tb + 4*gi + row (K, the lane's 16 dims), V rows tb + i (dims 4*lane..).
  //    The row indices do not depend on the valid length (a device scalar
  //    whose load would otherwise delay every K/V request by a round trip):
  //    they are clamped to the chunk's last row inside the cache capacity,
  //    and rows at or past the valid end (whatever bits they hold) are
  //    masked out of the softmax and their V values replaced by zeros.
  const uint16_t* Kh = Kc + (size_t)kvh * cache_len * kAD;
  const uint16_t* Vh = Vc + (size_t)kvh * cache_len * kAD;
  const int rw = lane >> 4;
  const int ds = lane & 15;
  const int tmax = min(start + chunk, cache_len) - 1;
  uint4 kr[kWaveGroups][2];
  uint2 vr[kWaveTok];
  auto load_kv = [&](int it, uint4 (&kd)[kWaveGroups][2], uint2 (&vd)[kWaveTok]) {
    const int tb = start + it * kIterTok + wid * kWaveTok;
#pragma unroll
    for (int gi = 0; gi < kWaveGroups; ++gi) {
      const int t = min(tb + 4 * gi + rw, tmax);
      kd[gi][0] = *reinterpret_cast<const uint4*>(Kh + (size_t)t * kAD + ds * 8);
      kd[gi][1] = *reinterpret_cast<const uint4*>(Kh + (size_t)t * kAD + 128 + ds * 8);
    }
#pragma unroll
    for (int i = 0; i < kWaveTok; ++i) {
      const int t = min(tb + i, tmax);
      vd[i] = *reinterpret_cast<const uint2*>(Vh + (size_t)t * kAD + 4 * lane);
    }
  };
  load_kv(0, kr, vr);

  // 3. prologue: q heads (bf16 pairs, unscaled) into LDS; FUSED also the new
  //    token's k and v, written into the cache by the owning workgroup.
  __shared__ uint2 q_s[G][kAD / 4];
  __shared__ float kn_s[FUSED ? kAD : 1], vn_s[FUSED ? kAD : 1];
  RopeTable rt;
  if (FUSED) rt = rope_table(rl, fq, lane);
#pragma unroll
  for (int j = 0; j < HPW; ++j) {
    const int g = wid + NW * j;
    if (g < G) {
      if (FUSED) {
        float o[4];
        norm_rope(hq[j], fq.w_f32, rt, fq.rot, lane, o);
        q_s[g][lane] = make_uint2(pack_bf2(o[0], o[1]), pack_bf2(o[2], o[3]));
      } else {
        q_s[g][lane] = hq[j].x;
      }
    }
  }
  // The new token's k is normalised by the first wave without a q head.
  constexpr int KW = G % NW;
  if (owns_new && wid == KW) {
    float o[4];
    norm_rope(hk, fq.w_f32, rt, fq.rot, lane, o);
    *reinterpret_cast<float4*>(&kn_s[4 * lane]) = make_float4(o[0], o[1], o[2], o[3]);
    *reinterpret_cast<float4*>(&vn_s[4 * lane]) =
        make_float4(bf_lo(vnew.x), bf_hi(vnew.x), bf_lo(vnew.y), bf_hi(vnew.y));
    if (n_old < cache_len) {
      const size_t off = ((size_t)kvh * cache_len + (size_t)n_old) * kAD + 4 * lane;
      *reinterpret_cast<uint2*>(fq.k_cache + off) = make_uint2(pack_bf2(o[0], o[1]), pack_bf2(o[2], o[3]));
      *reinterpret_cast<uint2*>(fq.v_cache + off) = vnew;
    }
  }
  __syncthreads();

  // The lane's q slices as bf16 pairs: dims 8*ds.. and 128 + 8*ds...
  uint32_t qp[G][8];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const uint2 a = q_s[g][2 * ds], b = q_s[g][2 * ds + 1];
    const uint2 c = q_s[g][32 + 2 * ds], d = q_s[g][32 + 2 * ds + 1];
    qp[g][0] = a.x; qp[g][1] = a.y; qp[g][2] = b.x; qp[g][3] = b.y;
    qp[g][4] = c.x; qp[g][5] = c.y; qp[g][6] = d.x; qp[g][7] = d.y;
  }

  // 4. online softmax over the wave's tokens (m and l wave-uniform).
  float m[G], l[G], acc[G][4];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = -INFINITY;
    l[g] = 0.f;
    acc[g][0] = acc[g][1] = acc[g][2] = acc[g][3] = 0.f;
  }
  // One 32-token step of the workgroup from the registers KR / VR.
#define Q35_ATT_STEP(KR, VR, IT)                                                                \
  do {                                                                                          \
    const int tb = start + (IT) * kIterTok + wid * kWaveTok;                                    \
    float vf[kWaveTok][4];                                                                      \
    _Pragma("unroll") for (int i = 0; i < kWaveTok; ++i) {                                      \
      const bool in = tb + i < end;                                                             \
      vf[i][0] = in ? bf_lo(VR[i].x) : 0.f;                                                     \
      vf[i][1] = in ? bf_hi(VR[i].x) : 0.f;                                                     \
      vf[i][2] = in ? bf_lo(VR[i].y) : 0.f;                                                     \
      vf[i][3] = in ? bf_hi(VR[i].y) : 0.f;                                                     \
    }                                                                                           \
    _Pragma("unroll") for (int g = 0; g < G; ++g) {                                             \
      float s[kWaveGroups];                                                                     \
      _Pragma("unroll") for (int gi = 0; gi < kWaveGroups; ++gi) {                              \
        const uint4 k0 = KR[gi][0], k1 = KR[gi][1];                                             \
        float d = dot2_bf16(qp[g][0], k0.x, 0.f);                                               \
        d = dot2_bf16(qp[g][1], k0.y, d);                                                       \
        d = dot2_bf16(qp[g][2], k0.z, d);                                                       \
        d = dot2_bf16(qp[g][3], k0.w, d);                                                       \
        d = dot2_bf16(qp[g][4], k1.x, d);                                                       \
        d = dot2_bf16(qp[g][5], k1.y, d);                                                       \
        d = dot2_bf16(qp[g][6], k1.z, d);                                                       \
        d = dot2_bf16(qp[g][7], k1.w, d);                                                       \
        d = row16_sum(d) * scale;                                                               \
        s[gi] = tb + 4 * gi + rw < end ? d : -INFINITY;                                         \
      }                                                                                         \
      float smax = s[0];                                                                        \
      _Pragma("unroll") for (int gi = 1; gi < kWaveGroups; ++gi) smax = fmaxf(smax, s[gi]);     \
      const float m_new = fmaxf(m[g], rows4_max(smax));                                         \
      /* A wave whose tokens so far all lie past the valid end keeps m = -inf:              */  \
      /* subtract 0 then, so that corr and p are 0 instead of NaN.                          */  \
      const float m_sub = m_new == -INFINITY ? 0.f : m_new;                                     \
      const float corr = expf(m[g] - m_sub);                                                    \
      float pg[kWaveGroups];                                                                    \
      _Pragma("unroll") for (int gi = 0; gi < kWaveGroups; ++gi) pg[gi] = expf(s[gi] - m_sub);  \
      _Pragma("unroll") for (int e = 0; e < 4; ++e) acc[g][e] *= corr;                          \
      float psum = 0.f;                                                                         \
      _Pragma("unroll") for (int i = 0; i < kWaveTok; ++i) {                                    \
        const float pi = __int_as_float(                                                        \
            __builtin_amdgcn_readlane(__float_as_int(pg[i / 4]), 16 * (i & 3)));                \
        psum += pi;                                                                             \
        _Pragma("unroll") for (int e = 0; e < 4; ++e) acc[g][e] = fmaf(pi, vf[i][e], acc[g][e]); \
      }                                                                                         \
      l[g] = l[g] * corr + psum;                                                                \
      m[g] = m_new;                                                                             \
    }                                                                                           \
  } while (0)
  // Two register sets alternate over pairs of steps, the next step's rows
  // requested before the current one is reduced; nothing copies a set whose
  // loads are in flight, and a single step (the decode shape) issues no
  // prefetch at all.
  uint4 kb[kWaveGroups][2];
  uint2 vb[kWaveTok];
  int it = 0;
  for (; it + 1 < n_iter; it += 2) {
    load_kv(it + 1, kb, vb);
    Q35_ATT_STEP(kr, vr, it);
    if (it + 2 < n_iter) load_kv(it + 2, kr, vr);
    Q35_ATT_STEP(kb, vb, it + 1);
  }
  if (it < n_iter) Q35_ATT_STEP(kr, vr, it);
#undef Q35_ATT_STEP

  // The new token (FUSED): the owning workgroup folds it in, head g by wave
  // g % NW (into that wave's state), so the heads are folded in parallel.
  if (owns_new) {
    const float4 kv = *reinterpret_cast<const float4*>(&kn_s[4 * lane]);
    const float4 vv = *reinterpret_cast<const float4*>(&vn_s[4 * lane]);
#pragma unroll
    for (int g = 0; g < G; ++g) {
      if (g % NW != wid) continue;
      const uint2 qv = q_s[g][lane];
      float sdot = bf_lo(qv.x) * kv.x;
      sdot = fmaf(bf_hi(qv.x), kv.y, sdot);
      sdot = fmaf(bf_lo(qv.y), kv.z, sdot);
      sdot = fmaf(bf_hi(qv.y), kv.w, sdot);
      const float sc = wave_sum(sdot) * scale;
      const float m_new = fmaxf(m[g], sc);
      const float corr = expf(m[g] - m_new);
      const float p = expf(sc - m_new);
      l[g] = l[g] * corr + p;
      acc[g][0] = fmaf(p, vv.x, acc[g][0] * corr);
      acc[g][1] = fmaf(p, vv.y, acc[g][1] * corr);
      acc[g][2] = fmaf(p, vv.z, acc[g][2] * corr);
      acc[g][3] = fmaf(p, vv.w, acc[g][3] * corr);
      m[g] = m_new;
    }
  }

  // 5. merge the waves in LDS (one barrier: every thread derives the wave
  //    factors e^(m_w - max_w m_w), 0 for a wave without tokens, of its
  //    head itself); write this split's (acc, m, l) per head.
  __shared__ float m_s[NW][G], l_s[NW][G];
  __shared__ float a_s[NW][G][kAD];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    if (lane == 0) {
      m_s[wid][g] = m[g];
      l_s[wid][g] = l[g];
    }
    *reinterpret_cast<float4*>(&a_s[wid][g][4 * lane]) = make_float4(acc[g][0], acc[g][1], acc[g][2], acc[g][3]);
  }
  __syncthreads();
  for (int idx = threadIdx.x; idx < G * kAD / 4; idx += NW * 64) {
    const int g = idx / (kAD / 4), d = (idx % (kAD / 4)) * 4;
    float mm = -INFINITY;
#pragma unroll
    for (int v = 0; v < NW; ++v) mm = fmaxf(mm, m_s[v][g]);
    float f[NW];
#pragma unroll
    for (int w = 0; w < NW; ++w) f[w] = m_s[w][g] == -INFINITY ? 0.f : expf(m_s[w][g] - mm);
    float4 a = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const float4 v = *reinterpret_cast<const float4*>(&a_s[w][g][d]);
      a.x += v.x * f[w];
      a.y += v.y * f[w];
      a.z += v.z * f[w];
      a.w += v.w * f[w];
    }
    const int slot = (kvh * G + g) * splits + split;
    *reinterpret_cast<float4*>(acc_out + (size_t)slot * kAD + d) = a;
    if (d == 0) {
      float ll = 0.f;
#pragma unroll
      for (int v = 0; v < NW; ++v) ll += l_s[v][g] * f[v];
      *reinterpret_cast<float2*>(ml_out + slot * 2) = make_float2(mm, ll);
    }
  }
}

// Log-sum-exp merge of the splits -> bf16, optionally times bf16(sigmoid(gate))
// [reference kernels.py:1007-1028 and 285-333]. Grid (query head, quarter of
// the 256 dims): thread (part = t/16, col = t%16) owns dims 64*quarter +
// 4*col .. +3 of splits part, part + 16, ... (up to 16*B splits). Every
// thread requests its partials (clamped indices) before wave 0 reads the
// (m, l) pairs and turns them into weights in LDS, so the merge is one
// memory round trip; the 16 parts are summed in LDS. Four workgroups per
// head keep each thread's share of a 128-split merge at 8 loads.
template <int B>
__global__ __launch_bounds__(256) void gqa_decode_combine(const float* __restrict__ acc,
                                                          const float* __restrict__ ml,
                                                          const uint16_t* __restrict__ packed_gate,
                                                          uint16_t* __restrict__ out, int splits,
                                                          long long* advance_len) {
  const int h = blockIdx.x >> 2, qd = blockIdx.x & 3;
  const int t = threadIdx.x;
  const int col = t & 15;
  const int part = t >> 4;
  const int d0 = 64 * qd + 4 * col;
  // The split kernel that read the length has completed (stream order).
  if (advance_len && blockIdx.x == 0 && t == 0) advance_len[0] += 1;
  const float* mlh = ml + (size_t)h * splits * 2;
  const float* acch = acc + (size_t)h * splits * kAD + d0;
  __shared__ float w_s[kMaxSplits];
  __shared__ float lt_s;
  __shared__ float4 red_s[16][16];
  const uint2 graw = packed_gate && part == 0
                         ? *reinterpret_cast<const uint2*>(packed_gate + h * 2 * kAD + kAD + d0)
                         : make_uint2(0, 0);
  float4 a[B];
#pragma unroll
  for (int j = 0; j < B; ++j)
    a[j] = *reinterpret_cast<const float4*>(acch + (size_t)min(part + 16 * j, splits - 1) * kAD);
  if (t < 64) {
    float mx = -INFINITY;
    for (int s = t; s < splits; s += 64) mx = fmaxf(mx, mlh[2 * s]);
    mx = wave_max(mx);
    float lt = 0.f;
    for (int s = t; s < splits; s += 64) {
      const float ms = mlh[2 * s];
      const float w = ms == -INFINITY ? 0.f : expf(ms - mx);
      w_s[s] = w;
      lt += mlh[2 * s + 1] * w;
    }
    lt = wave_sum(lt);
    if (t == 0) lt_s = lt;
  }
  __syncthreads();
  float4 tot = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int j = 0; j < B; ++j) {
    const int s = part + 16 * j;
    const float w = s < splits ? w_s[s] : 0.f;
    tot.x = fmaf(a[j].x, w, tot.x);
    tot.y = fmaf(a[j].y, w, tot.y);
    tot.z = fmaf(a[j].z, w, tot.z);
    tot.w = fmaf(a[j].w, w, tot.w);
  }
  red_s[part][col] = tot;
  __syncthreads();
  if (part == 0) {
    float4 r = red_s[0][col];
#pragma unroll
    for (int p = 1; p < 16; ++p) {
      const float4 v = red_s[p][col];
      r.x += v.x;
      r.y += v.y;
      r.z += v.z;
      r.w += v.w;
    }
    const float lt = lt_s;
    float o[4] = {round_bf(r.x / lt), round_bf(r.y / lt), round_bf(r.z / lt), round_bf(r.w / lt)};
    if (packed_gate) {
      o[0] *= round_bf(sigmoid_f(bf_lo(graw.x)));
      o[1] *= round_bf(sigmoid_f(bf_hi(graw.x)));
      o[2] *= round_bf(sigmoid_f(bf_lo(graw.y)));
      o[3] *= round_bf(sigmoid_f(bf_hi(graw.y)));
    }
    *reinterpret_cast<uint2*>(out + (size_t)h * kAD + d0) = make_uint2(pack_bf2(o[0], o[1]), pack_bf2(o[2], o[3]));
  }
}

// Combine launch for a split count (partials per thread = ceil(splits / 16)).
void launch_combine(const float* acc, const float* ml, const uint16_t* gate, uint16_t* out, int QH,
                    int splits, long long* advance, hipStream_t stream) {
  const unsigned grid = (unsigned)(4 * QH);
  if (splits <= 32)
    gqa_decode_combine<2><<<grid, 256, 0, stream>>>(acc, ml, gate, out, splits, advance);
  else if (splits <= 64)
    gqa_decode_combine<4><<<grid, 256, 0, stream>>>(acc, ml, gate, out, splits, advance);
  else
    gqa_decode_combine<8><<<grid, 256, 0, stream>>>(acc, ml, gate, out, splits, advance);
}

// ------------------------------------------------- causal prefill (MFMA)
// Flash attention on the matrix cores, v_mfma_f32_16x16x32_bf16. Operand
// layouts (wave64): A[16 x 32]: lane l holds row l%16, 8 consecutive k at
// 8*(l/16); B[32 x 16]: lane l holds column l%16, the same 8 k; C[16 x 16]:
// lane l holds rows 4*(l/16) + i (i = 0..3) of column l%16.
// Grid (query tiles of 16 rows, KVH, B); the G waves of a workgroup are the G
// query heads of one KV head over the same 16 rows, so they share the K rows
// (L1) and the V tile (LDS). Per 32-key iteration and wave:
//   S = Q K^T: Q (A operand, rows x dims) stays in registers, K rows are the
//     B operand in their natural layout (16 contiguous bytes per lane);
//   online softmax on the C layout (row max / sum over the 16 lanes of a DPP
//     row), scale and causal mask applied to S in fp32;
//   O += P V: P is split into bf16 hi + lo parts (p - hi rounded again, so P
//     keeps ~16 mantissa bits: two MFMAs instead of the one of a plain bf16 P)
//     and moved through a wave-private LDS tile into the A layout; V is staged
//     transposed in LDS (double-buffered, one barrier per iteration) so the
//     B operand is again 16 contiguous bytes per lane.
// Keys past the valid end are masked to -inf and their V rows staged as
// zeros (the cache beyond the prompt may hold any bits).
Q35_DEV q35_f32x4 mfma_16x16x32(const uint4 a, const uint4 b, q35_f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(q35_bf16x8, a),
                                                 __builtin_bit_cast(q35_bf16x8, b), c, 0, 0, 0);
}

constexpr int kVtStride = 40;  // bf16 per transposed V row: 32 keys + pad
constexpr int kPStride = 40;   // bf16 per P row: 32 keys + pad

template <int G>
__global__ __launch_bounds__(G * 64) void gqa_prefill_mfma(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ Kc, const uint16_t* __restrict__ Vc,
    uint16_t* __restrict__ out, int B, int QH, int KVH, int L, int cache_len, int kv_start_host,
    const long long* __restrict__ valid_len, float scale) {
  const int lane = threadIdx.x & 63;
  const int wid = threadIdx.x >> 6;
  const int tile = gridDim.x - 1 - blockIdx.x;  // heavy (late) tiles first
  const int kvh = blockIdx.y;
  const int b = blockIdx.z;
  const int h = kvh * G + wid;
  const int q0 = tile * 16;
  long long ks = valid_len ? valid_len[0] - L + kv_start_host : (long long)kv_start_host;
  if (ks < 0) ks = 0;
  if (ks + L > cache_len) ks = cache_len - L;
  const int kv_start = (int)ks;
  const int col = lane & 15;  // A row / B column / C column
  const int kg = lane >> 4;   // k group of 8 / C row group of 4

  // Q operand: row q0 + col (clamped), dims 8*kg + 32t.
  const uint16_t* qp = q + (((size_t)b * QH + h) * L + min(q0 + col, L - 1)) * kAD + kg * 8;
  uint4 qa[8];
#pragma unroll
  for (int t = 0; t < 8; ++t) qa[t] = *reinterpret_cast<const uint4*>(qp + 32 * t);
  int row_abs[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) row_abs[i] = kv_start + min(q0 + 4 * kg + i, L - 1);
  const int n_keys = min(kv_start + min(q0 + 16, L), cache_len);
  const uint16_t* Kh = Kc + ((size_t)b * KVH + kvh) * cache_len * kAD;
  const uint16_t* Vh = Vc + ((size_t)b * KVH + kvh) * cache_len * kAD;

  __shared__ alignas(16) uint16_t vt_s[2][kAD * kVtStride];
  __shared__ alignas(16) uint16_t p_s[G][2][16 * kPStride];
  q35_f32x4 o[16];
#pragma unroll
  for (int d = 0; d < 16; ++d) o[d] = {0.f, 0.f, 0.f, 0.f};
  float m[4], l[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    m[i] = -INFINITY;
    l[i] = 0.f;
  }
  const int nblk = (n_keys + 31) / 32;
  // Global loads of one 32-key block: the K operand of its two 16-key halves
  // (key kb + 16*sb + col, dims 8*kg + 32t) and this thread's share of V rows
  // for the transposed staging. Block blk + 1 is requested before block blk
  // is computed, so the loop does not wait on memory.
  constexpr int VPER = (32 * (kAD / 8) + G * 64 - 1) / (G * 64);
  auto load_block = [&](int blk, uint4 (&kv)[2][8], uint4 (&vr)[VPER]) {
    const int kb = blk * 32;
#pragma unroll
    for (int sb = 0; sb < 2; ++sb) {
      const uint16_t* kr = Kh + (size_t)min(kb + 16 * sb + col, n_keys - 1) * kAD + kg * 8;
#pragma unroll
      for (int t = 0; t < 8; ++t) kv[sb][t] = *reinterpret_cast<const uint4*>(kr + 32 * t);
    }
#pragma unroll
    for (int j = 0; j < VPER; ++j) {
      const int pi = min((int)threadIdx.x + j * G * 64, 32 * (kAD / 8) - 1);
      const int k = pi & 31, dg = pi >> 5;
      vr[j] = *reinterpret_cast<const uint4*>(Vh + (size_t)min(kb + k, n_keys - 1) * kAD + dg * 8);
    }
  };
  uint4 kv[2][8], vr[VPER];
  load_block(0, kv, vr);
  for (int blk = 0; blk < nblk; ++blk) {
    const int kb = blk * 32;
    uint16_t* vt = vt_s[blk & 1];
    uint4 kn[2][8], vn[VPER];
    load_block(min(blk + 1, nblk - 1), kn, vn);
    // Stage V^T: (key, 8-dim group) pairs, vt[dim][key]; masked keys as zeros.
#pragma unroll
    for (int j = 0; j < VPER; ++j) {
      const int pi = (int)threadIdx.x + j * G * 64;
      if (pi < 32 * (kAD / 8)) {
        const int k = pi & 31, dg = pi >> 5;
        const uint4 v = kb + k < n_keys ? vr[j] : make_uint4(0, 0, 0, 0);
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          vt[(dg * 8 + 2 * e) * kVtStride + k] = (uint16_t)(w[e] & 0xffffu);
          vt[(dg * 8 + 2 * e + 1) * kVtStride + k] = (uint16_t)(w[e] >> 16);
        }
      }
    }
    // S = Q K^T, then scale, causal mask and online softmax per row.
    q35_f32x4 s[2];
#pragma unroll
    for (int sb = 0; sb < 2; ++sb) {
      s[sb] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int t = 0; t < 8; ++t) s[sb] = mfma_16x16x32(qa[t], kv[sb][t], s[sb]);
    }
    float corr[4];
    uint16_t* ps_hi = p_s[wid][0];
    uint16_t* ps_lo = p_s[wid][1];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float sv[2];
#pragma unroll
      for (int sb = 0; sb < 2; ++sb) {
        const int key = kb + 16 * sb + col;
        sv[sb] = (key <= row_abs[i] && key < n_keys) ? s[sb][i] * scale : -INFINITY;
      }
      const float m_new = fmaxf(m[i], row16_max(fmaxf(sv[0], sv[1])));
      // A row without any valid key so far keeps m = -inf: subtract 0 then.
      const float m_sub = m_new == -INFINITY ? 0.f : m_new;
      corr[i] = expf(m[i] - m_sub);
      const float p0 = expf(sv[0] - m_sub), p1 = expf(sv[1] - m_sub);
      l[i] = l[i] * corr[i] + row16_sum(p0 + p1);
      m[i] = m_new;
      const uint32_t h0 = f2bf(p0), h1 = f2bf(p1);
      ps_hi[(4 * kg + i) * kPStride + col] = (uint16_t)h0;
      ps_hi[(4 * kg + i) * kPStride + 16 + col] = (uint16_t)h1;
      ps_lo[(4 * kg + i) * kPStride + col] = (uint16_t)f2bf(p0 - bf2f(h0));
      ps_lo[(4 * kg + i) * kPStride + 16 + col] = (uint16_t)f2bf(p1 - bf2f(h1));
    }
    __syncthreads();  // V^T staged by every wave; this wave's P tile written
    // O += P V: A = P rows x keys (row col, keys 8*kg..), B = V^T (dims x keys).
    const uint4 pa_hi = *reinterpret_cast<const uint4*>(ps_hi + col * kPStride + kg * 8);
    const uint4 pa_lo = *reinterpret_cast<const uint4*>(ps_lo + col * kPStride + kg * 8);
#pragma unroll
    for (int d = 0; d < 16; ++d) {
#pragma unroll
      for (int i = 0; i < 4; ++i) o[d][i] *= corr[i];
      const uint4 vb = *reinterpret_cast<const uint4*>(vt + (d * 16 + col) * kVtStride + kg * 8);
      o[d] = mfma_16x16x32(pa_hi, vb, o[d]);
      o[d] = mfma_16x16x32(pa_lo, vb, o[d]);
    }
#pragma unroll
    for (int sb = 0; sb < 2; ++sb)
#pragma unroll
      for (int t = 0; t < 8; ++t) kv[sb][t] = kn[sb][t];
#pragma unroll
    for (int j = 0; j < VPER; ++j) vr[j] = vn[j];
  }
  // out[b, row, h*D + 16d + col] = bf16(O / l) for the valid rows.
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = q0 + 4 * kg + i;
    if (r < L) {
      const float inv = 1.0f / l[i];
      uint16_t* orow = out + ((size_t)b * L + r) * QH * kAD + h * kAD + col;
#pragma unroll
      for (int d = 0; d < 16; ++d) orow[16 * d] = (uint16_t)f2bf(o[d][i] * inv);
    }
  }
}

// ------------------------------------------ causal prefill, 64-key blocks
// Grid (query tiles of 16 rows, heavy first; KVH; B). A workgroup has 2G
// waves: wave w serves query head g = w % G of the KV head over key half
// kh = w / G (keys 32kh..32kh+31 of every 64-key block), with its own online
// softmax; the two halves of a head are merged in LDS at the end. Per block
// the K and V rows are staged once for all waves in their natural [key][dim]
// layout (16-byte stores, double-buffered, one barrier per block; the next
// block is loaded to registers before the current one is computed).
//   S = Q K^T: Q rows (A operand) stay in registers, K rows are read from LDS
//     as the B operand (16 contiguous bytes per lane);
//   O += P V: P is kept as bf16 hi + lo (~16 mantissa bits, two MFMAs); the
//     wave writes P^T [key][row] (4 rows = 8 bytes per lane) and reads the A
//     operand back with the gfx950 transpose read ds_read_b64_tr_b16, which
//     also turns row-major V into the B operand. Within each 16-lane group g
//     the read returns to lane 16g + i, element e, the 16-bit word at
//     address(lane 16g + 4e + i/4) + (i % 4); so lane 16g + 4e + q pointing at
//     row 8g + 4h + e, column 16t + 4q gives lane 16g + i the 4 rows
//     8g + 4h .. 8g + 4h + 3 of column 16t + i: read h = 0, 1 fill the 8
//     consecutive k of an MFMA operand.
// Keys past the valid end are clamped to the last valid row on load (finite
// values) and masked to -inf in S, so they add exact zeros.
typedef short q35_i16x4 __attribute__((ext_vector_type(4)));
Q35_DEV uint2 lds_read_tr16(const uint16_t* p) {
  const q35_i16x4 v =
      __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) q35_i16x4*)(p));
  return __builtin_bit_cast(uint2, v);
}

constexpr int kFaKeys = 64;         // keys per block
constexpr int kFaRow = kAD + 16;    // padded K/V row in LDS (elements)
constexpr int kFaPt = 16 + 4;       // padded P^T row (16 query rows)

template <int G>
__global__ __launch_bounds__(2 * G * 64) void gqa_prefill_fa(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ Kc, const uint16_t* __restrict__ Vc,
    uint16_t* __restrict__ out, int B, int QH, int KVH, int L, int cache_len, int kv_start_host,
    const long long* __restrict__ valid_len, float scale, int sb, int smax,
    float* __restrict__ part) {
  constexpr int NW = 2 * G;
  constexpr int NT = NW * 64;
  constexpr int PER = kFaKeys * (kAD / 8) / NT;  // 16-byte K (and V) groups per thread
  static_assert(PER * NT == kFaKeys * (kAD / 8), "block must split evenly");
  const int lane = threadIdx.x & 63;
  const int wid = threadIdx.x >> 6;
  const int g = wid % G, kh = wid / G;
  const int ntiles = gridDim.x / smax;
  const int tile = ntiles - 1 - (int)blockIdx.x / smax;  // heavy (late) tiles first
  const int split = (int)blockIdx.x % smax;
  const int kvh = blockIdx.y;
  const int b = blockIdx.z;
  const int h = kvh * G + g;
  const int q0 = tile * 16;
  long long ks = valid_len ? valid_len[0] - L + kv_start_host : (long long)kv_start_host;
  if (ks < 0) ks = 0;
  if (ks + L > cache_len) ks = cache_len - L;
  const int kv_start = (int)ks;
  const int col = lane & 15;  // A row / B column / C column
  const int kg = lane >> 4;   // k group of 8 / C row group of 4
  // transpose-read addressing: lane 16*kg + 4e + tq reads row 4e-offset, column 4tq
  const int te = (lane & 15) >> 2, tq = lane & 3;

  const uint16_t* qp = q + (((size_t)b * QH + h) * L + min(q0 + col, L - 1)) * kAD + kg * 8;
  uint4 qa[8];
#pragma unroll
  for (int t = 0; t < 8; ++t) qa[t] = *reinterpret_cast<const uint4*>(qp + 32 * t);
  int row_abs[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) row_abs[i] = kv_start + min(q0 + 4 * kg + i, L - 1);
  const int n_keys = min(kv_start + min(q0 + 16, L), cache_len);
  const int nblk = (n_keys + kFaKeys - 1) / kFaKeys;
  // This workgroup's key blocks [b0, b1) of the tile (sb blocks per split).
  const int nsplit = (nblk + sb - 1) / sb;
  if (split >= nsplit) return;  // whole workgroup: no barrier is skipped
  const int b0 = split * sb, b1 = min(b0 + sb, nblk);
  const uint16_t* Kh = Kc + ((size_t)b * KVH + kvh) * cache_len * kAD;
  const uint16_t* Vh = Vc + ((size_t)b * KVH + kvh) * cache_len * kAD;

  __shared__ alignas(16) uint16_t kv_s[2][2][kFaKeys * kFaRow];  // [buf][K, V][key][dim]
  __shared__ alignas(16) uint16_t pt_s[NW][2][32 * kFaPt];       // [wave][hi, lo][key][row]

  uint4 kr[PER], vr[PER];
#define Q35_FA_LOAD(blk)                                                                 \
  do {                                                                                   \
    _Pragma("unroll") for (int j = 0; j < PER; ++j) {                                     \
      const int gi = (int)threadIdx.x + j * NT;                                           \
      const int key = min((blk) * kFaKeys + (gi >> 5), n_keys - 1);                       \
      const size_t off = (size_t)key * kAD + (gi & 31) * 8;                               \
      kr[j] = *reinterpret_cast<const uint4*>(Kh + off);                                  \
      vr[j] = *reinterpret_cast<const uint4*>(Vh + off);                                  \
    }                                                                                     \
  } while (0)
#define Q35_FA_STORE(buf)                                                                \
  do {                                                                                   \
    _Pragma("unroll") for (int j = 0; j < PER; ++j) {                                     \
      const int gi = (int)threadIdx.x + j * NT;                                           \
      const int off = (gi >> 5) * kFaRow + (gi & 31) * 8;                                 \
      *reinterpret_cast<uint4*>(&kv_s[buf][0][off]) = kr[j];                              \
      *reinterpret_cast<uint4*>(&kv_s[buf][1][off]) = vr[j];                              \
    }                                                                                     \
  } while (0)

  q35_f32x4 o[16];
#pragma unroll
  for (int d = 0; d < 16; ++d) o[d] = {0.f, 0.f, 0.f, 0.f};
  float m[4], l[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    m[i] = -INFINITY;
    l[i] = 0.f;
  }
  uint16_t* pt_hi = pt_s[wid][0];
  uint16_t* pt_lo = pt_s[wid][1];

  Q35_FA_LOAD(b0);
  Q35_FA_STORE(0);
  __syncthreads();
  for (int blk = b0; blk < b1; ++blk) {
    const int buf = (blk - b0) & 1;
    Q35_FA_LOAD(min(blk + 1, b1 - 1));  // in flight while this block is computed
    const uint16_t* Ks = kv_s[buf][0] + 32 * kh * kFaRow;
    const uint16_t* Vs = kv_s[buf][1] + 32 * kh * kFaRow;
    const int kb = blk * kFaKeys + 32 * kh;  // first key of this wave's half
    // S = Q K^T over the wave's 32 keys (two 16-key column tiles).
    q35_f32x4 s[2];
#pragma unroll
    for (int st = 0; st < 2; ++st) {
      s[st] = {0.f, 0.f, 0.f, 0.f};
      const uint16_t* krow = Ks + (16 * st + col) * kFaRow + 8 * kg;
#pragma unroll
      for (int t = 0; t < 8; ++t)
        s[st] = mfma_16x16x32(qa[t], *reinterpret_cast<const uint4*>(krow + 32 * t), s[st]);
    }
    // Online softmax per row; P^T as bf16 hi + lo, 4 rows (8 bytes) per store.
    float corr[4], p[2][4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float sv[2];
#pragma unroll
      for (int st = 0; st < 2; ++st) {
        const int key = kb + 16 * st + col;
        sv[st] = (key <= row_abs[i] && key < n_keys) ? s[st][i] * scale : -INFINITY;
      }
      const float m_new = fmaxf(m[i], row16_max(fmaxf(sv[0], sv[1])));
      // A row without any valid key so far keeps m = -inf: subtract 0 then.
      const float m_sub = m_new == -INFINITY ? 0.f : m_new;
      corr[i] = expf(m[i] - m_sub);
      p[0][i] = expf(sv[0] - m_sub);
      p[1][i] = expf(sv[1] - m_sub);
      l[i] = l[i] * corr[i] + row16_sum(p[0][i] + p[1][i]);
      m[i] = m_new;
    }
#pragma unroll
    for (int st = 0; st < 2; ++st) {
      float hi[4], lo[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        hi[i] = round_bf(p[st][i]);
        lo[i] = p[st][i] - hi[i];
      }
      const int off = (16 * st + col) * kFaPt + 4 * kg;
      *reinterpret_cast<uint2*>(pt_hi + off) = make_uint2(pack_bf2(hi[0], hi[1]), pack_bf2(hi[2], hi[3]));
      *reinterpret_cast<uint2*>(pt_lo + off) = make_uint2(pack_bf2(lo[0], lo[1]), pack_bf2(lo[2], lo[3]));
    }
    // P operand (rows x 32 keys) back through the transpose read; the wave's
    // own LDS stores above complete before its later reads (in-order LDS).
    uint4 pa_hi, pa_lo;
    {
      const int off0 = (8 * kg + te) * kFaPt + 4 * tq;
      const int off1 = (8 * kg + 4 + te) * kFaPt + 4 * tq;
      const uint2 h0 = lds_read_tr16(pt_hi + off0), h1 = lds_read_tr16(pt_hi + off1);
      const uint2 l0 = lds_read_tr16(pt_lo + off0), l1 = lds_read_tr16(pt_lo + off1);
      pa_hi = make_uint4(h0.x, h0.y, h1.x, h1.y);
      pa_lo = make_uint4(l0.x, l0.y, l1.x, l1.y);
    }
    // O += P V; V rows 8kg + 4h + te of the wave's half, dims 16d + 4tq.
    const uint16_t* v0 = Vs + (8 * kg + te) * kFaRow + 4 * tq;
    const uint16_t* v1 = Vs + (8 * kg + 4 + te) * kFaRow + 4 * tq;
#pragma unroll
    for (int d = 0; d < 16; ++d) {
#pragma unroll
      for (int i = 0; i < 4; ++i) o[d][i] *= corr[i];
      const uint2 a = lds_read_tr16(v0 + 16 * d), c = lds_read_tr16(v1 + 16 * d);
      const uint4 vb = make_uint4(a.x, a.y, c.x, c.y);
      o[d] = mfma_16x16x32(pa_hi, vb, o[d]);
      o[d] = mfma_16x16x32(pa_lo, vb, o[d]);
    }
    Q35_FA_STORE(buf ^ 1);
    __syncthreads();
  }
#undef Q35_FA_LOAD
#undef Q35_FA_STORE

  // Merge the two key halves of each head: half 1 leaves (O, m, l) in LDS
  // (the K/V buffers are free after the last barrier), half 0 combines and
  // writes out[b, row, h*D + 16d + col] = bf16(O / l) for the valid rows.
  float* mo = reinterpret_cast<float*>(&kv_s[0][0][0]);  // [G][16 rows][kAD]
  float* ml = mo + G * 16 * kAD;                           // [G][16 rows][2]
  if (kh == 1) {
#pragma unroll
    for (int d = 0; d < 16; ++d)
#pragma unroll
      for (int i = 0; i < 4; ++i) mo[(g * 16 + 4 * kg + i) * kAD + 16 * d + col] = o[d][i];
    if (col == 0) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        ml[(g * 16 + 4 * kg + i) * 2] = m[i];
        ml[(g * 16 + 4 * kg + i) * 2 + 1] = l[i];
      }
    }
  }
  __syncthreads();
  if (kh == 0) {
    // One split: the final rows. Several: this split's (O, m, l) record, O
    // relative to m and not yet divided by l; gqa_prefill_merge combines them.
    float* rec = nsplit > 1 ? part + ((((size_t)b * KVH + kvh) * ntiles + tile) * smax + split) *
                                         (size_t)(G * 16 * (kAD + 2))
                            : nullptr;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = q0 + 4 * kg + i;
      const int rr = g * 16 + 4 * kg + i;
      const float m1 = ml[rr * 2], l1 = ml[rr * 2 + 1];
      const float mm = fmaxf(m[i], m1);
      const float f0 = m[i] == -INFINITY ? 0.f : expf(m[i] - mm);
      const float f1 = m1 == -INFINITY ? 0.f : expf(m1 - mm);
      const float lt = l[i] * f0 + l1 * f1;
      if (rec) {
#pragma unroll
        for (int d = 0; d < 16; ++d)
          rec[rr * kAD + 16 * d + col] = o[d][i] * f0 + mo[rr * kAD + 16 * d + col] * f1;
        if (col == 0) {
          rec[G * 16 * kAD + rr * 2] = mm;
          rec[G * 16 * kAD + rr * 2 + 1] = lt;
        }
      } else if (r < L) {
        const float inv = 1.0f / lt;
        uint16_t* orow = out + ((size_t)b * L + r) * QH * kAD + h * kAD + col;
#pragma unroll
        for (int d = 0; d < 16; ++d) {
          const float v = o[d][i] * f0 + mo[rr * kAD + 16 * d + col] * f1;
          orow[16 * d] = (uint16_t)f2bf(v * inv);
        }
      }
    }
  }
}

// Merge of the split records of the query tiles with more than one split:
// one thread per (query head g, row r, 16 dims), G*256 threads per (tile, KV
// head); O = sum_s O_s e^{m_s - M} / sum_s l_s e^{m_s - M}, M = max_s m_s.
template <int G>
__global__ __launch_bounds__(G * 256) void gqa_prefill_merge(
    const float* __restrict__ part, uint16_t* __restrict__ out, int B, int QH, int KVH, int L,
    int cache_len, int kv_start_host, const long long* __restrict__ valid_len, int sb, int smax) {
  const int t = threadIdx.x;
  const int g = t >> 8, r = (t >> 4) & 15, dq = t & 15;
  const int tile = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
  const int ntiles = gridDim.x;
  const int q0 = tile * 16;
  long long ks = valid_len ? valid_len[0] - L + kv_start_host : (long long)kv_start_host;
  if (ks < 0) ks = 0;
  if (ks + L > cache_len) ks = cache_len - L;
  const int n_keys = min((int)ks + min(q0 + 16, L), cache_len);
  const int nblk = (n_keys + kFaKeys - 1) / kFaKeys;
  const int nsplit = (nblk + sb - 1) / sb;
  if (nsplit <= 1 || q0 + r >= L) return;  // no barrier in this kernel
  const size_t rs = (size_t)G * 16 * (kAD + 2);
  const float* rec0 = part + (((size_t)b * KVH + kvh) * ntiles + tile) * smax * rs;
  const int rr = g * 16 + r;
  float mx = -INFINITY;
  for (int sp = 0; sp < nsplit; ++sp) mx = fmaxf(mx, rec0[sp * rs + G * 16 * kAD + rr * 2]);
  float acc[16];
#pragma unroll
  for (int e = 0; e < 16; ++e) acc[e] = 0.f;
  float lt = 0.f;
  for (int sp = 0; sp < nsplit; ++sp) {
    const float* rec = rec0 + sp * rs;
    const float ms = rec[G * 16 * kAD + rr * 2];
    const float f = ms == -INFINITY ? 0.f : expf(ms - mx);
    lt += rec[G * 16 * kAD + rr * 2 + 1] * f;
    const float4* v = reinterpret_cast<const float4*>(rec + rr * kAD + 16 * dq);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float4 x = v[j];
      acc[4 * j] = fmaf(x.x, f, acc[4 * j]);
      acc[4 * j + 1] = fmaf(x.y, f, acc[4 * j + 1]);
      acc[4 * j + 2] = fmaf(x.z, f, acc[4 * j + 2]);
      acc[4 * j + 3] = fmaf(x.w, f, acc[4 * j + 3]);
    }
  }
  const float inv = 1.0f / lt;
#pragma unroll
  for (int e = 0; e < 16; ++e) acc[e] *= inv;
  uint4* o = reinterpret_cast<uint4*>(out + ((size_t)b * L + q0 + r) * QH * kAD + (kvh * G + g) * kAD + 16 * dq);
  o[0] = pack8(acc);
  o[1] = pack8(acc + 8);
}

// ---------------------------------------------------------- causal prefill
// q [B, QH, L, D], K/V [B, KVH, cache_len, D] (the prompt at cache offset
// kv_start), out [B, L, QH*D]. Query row i of a head attends to keys
// [0, kv_start + i]. One wave per (batch, head, query row); 4 keys per
// iteration, lane = (key kk = lane/16, 16-dim slice); online softmax in fp32.
__global__ __launch_bounds__(256) void gqa_prefill_rows(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ Kc, const uint16_t* __restrict__ Vc,
    uint16_t* __restrict__ out, int B, int QH, int KVH, int L, int cache_len, int kv_start_host,
    const long long* __restrict__ valid_len, float scale) {
  const int lane = threadIdx.x & 63;
  const long long wv = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (wv >= (long long)B * QH * L) return;
  // With a device length the prompt starts at valid_len - L + kv_start
  // (kv_start = 0 when the length already counts these L tokens, L when it
  // holds the start); the bound keeps reads in the cache.
  long long ks = valid_len ? valid_len[0] - L + kv_start_host : (long long)kv_start_host;
  if (ks < 0) ks = 0;
  if (ks + L > cache_len) ks = cache_len - L;
  const int kv_start = (int)ks;
  // Heavy (late) rows first so that the tail of the grid is short.
  const int i = L - 1 - (int)(wv % L);
  const int h = (int)((wv / L) % QH);
  const int b = (int)(wv / ((long long)L * QH));
  const int kvh = h / (QH / KVH);
  const int ds = lane & 15;
  const uint16_t* qr = q + (((size_t)b * QH + h) * L + i) * kAD + ds * 16;
  float qf[16], t8[8];
  unpack8(*reinterpret_cast<const uint4*>(qr), t8);
  for (int j = 0; j < 8; ++j) qf[j] = t8[j] * scale;
  unpack8(*reinterpret_cast<const uint4*>(qr + 8), t8);
  for (int j = 0; j < 8; ++j) qf[8 + j] = t8[j] * scale;
  const uint16_t* Kh = Kc + ((size_t)b * KVH + kvh) * cache_len * kAD;
  const uint16_t* Vh = Vc + ((size_t)b * KVH + kvh) * cache_len * kAD;
  const int n = kv_start + i + 1;
  float m = -INFINITY, l = 0.f, acc[4] = {0.f, 0.f, 0.f, 0.f};
  for (int t0 = 0; t0 < n; t0 += 4) {
    const int tok = t0 + (lane >> 4);
    const bool live = tok < n;
    float s = 0.f;
    if (live) {
      const uint16_t* kr = Kh + (size_t)tok * kAD + ds * 16;
      unpack8(*reinterpret_cast<const uint4*>(kr), t8);
      for (int j = 0; j < 8; ++j) s = fmaf(qf[j], t8[j], s);
      unpack8(*reinterpret_cast<const uint4*>(kr + 8), t8);
      for (int j = 0; j < 8; ++j) s = fmaf(qf[8 + j], t8[j], s);
    }
    uint2 vv[4];
    for (int k = 0; k < 4; ++k)
      vv[k] = t0 + k < n ? *reinterpret_cast<const uint2*>(Vh + (size_t)(t0 + k) * kAD + 4 * lane)
                         : make_uint2(0, 0);
    s = row16_sum(s);
    s = live ? s : -INFINITY;
    float sc[4];
    for (int k = 0; k < 4; ++k) sc[k] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(s), 16 * k));
    const float m_new = fmaxf(m, fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3])));
    const float corr = expf(m - m_new);
    float p[4];
    for (int k = 0; k < 4; ++k) p[k] = expf(sc[k] - m_new);
    l = l * corr + ((p[0] + p[1]) + (p[2] + p[3]));
    for (int d = 0; d < 4; ++d) acc[d] *= corr;
    for (int k = 0; k < 4; ++k) {
      acc[0] = fmaf(p[k], bf_lo(vv[k].x), acc[0]);
      acc[1] = fmaf(p[k], bf_hi(vv[k].x), acc[1]);
      acc[2] = fmaf(p[k], bf_lo(vv[k].y), acc[2]);
      acc[3] = fmaf(p[k], bf_hi(vv[k].y), acc[3]);
    }
    m = m_new;
  }
  uint16_t* orow = out + ((size_t)b * L + i) * QH * kAD + h * kAD + 4 * lane;
  const float inv = 1.0f / l;
  *reinterpret_cast<uint2*>(orow) = make_uint2(pack_bf2(acc[0] * inv, acc[1] * inv),
                                               pack_bf2(acc[2] * inv, acc[3] * inv));
}

}  // namespace

extern "C" {

int q35_qgkv_norm_rope(const void* packed, const void* q_w, const void* k_w, int w_f32,
                       const void* cos, const void* sin, void* q_out, void* k_out, void* v_out,
                       const void* cache_start, int B, int L, int QH, int KVH, int D,
                       int rotary_dim, int cache_len, hipStream_t stream) {
  Q35_CHECK_ARG(B >= 0 && L >= 0 && QH > 0 && KVH > 0 && KVH <= QH);
  Q35_CHECK_ARG(D == 64 || D == 128 || D == 256);
  const int E = D / 64;
  Q35_CHECK_ARG(rotary_dim >= 0 && rotary_dim <= D && rotary_dim % (2 * E) == 0);
  Q35_CHECK_ARG(!cache_start || cache_len > 0);
  const long long waves = (long long)B * L * QH;
  if (waves == 0) return 0;
  Q35_CHECK_ARG(waves < (1ll << 31));
  const unsigned grid = (unsigned)((waves + 3) / 4);
  const long long* cs = (const long long*)cache_start;
  if (D == kAD && rotary_dim > 0 && rotary_dim % 8 == 0 && q35_aligned8(packed) && q35_aligned8(q_w) &&
      q35_aligned8(k_w) && q35_aligned8(cos) && q35_aligned8(sin) && q35_aligned8(q_out) &&
      q35_aligned8(k_out) && q35_aligned8(v_out)) {
    qgkv_norm_rope_256<<<grid, 256, 0, stream>>>(
        (const uint16_t*)packed, q_w, k_w, w_f32, (const uint16_t*)cos, (const uint16_t*)sin,
        (uint16_t*)q_out, (uint16_t*)k_out, (uint16_t*)v_out, cs, B, L, QH, KVH, rotary_dim, cache_len);
    return q35_last_error();
  }
#define Q35_QGKV(EE)                                                                          \
  qgkv_norm_rope_k<EE><<<grid, 256, 0, stream>>>(                                             \
      (const uint16_t*)packed, q_w, k_w, w_f32, (const uint16_t*)cos, (const uint16_t*)sin,   \
      (uint16_t*)q_out, (uint16_t*)k_out, (uint16_t*)v_out, cs, B, L, QH, KVH, D, rotary_dim, \
      cache_len)
  if (E == 1) Q35_QGKV(1);
  else if (E == 2) Q35_QGKV(2);
  else Q35_QGKV(4);
#undef Q35_QGKV
  return q35_last_error();
}

// Split count and chunk length for a cache of cache_len tokens: chosen from
// the capacity only (never the valid length), so a captured graph stays valid.
// A chunk is a whole number of 32-token workgroup iterations and there are at
// most 128 splits per KV head (the combine requests them all at once).
int q35_gqa_decode_splits(int cache_len, int kv_heads, int* chunk_out) {
  if (cache_len <= 0 || kv_heads <= 0) return 0;
  long long chunk = ((long long)cache_len + kMaxSplits - 1) / kMaxSplits;
  chunk = (chunk + kIterTok - 1) / kIterTok * kIterTok;
  const int splits = (int)((cache_len + chunk - 1) / chunk);
  if (chunk_out) *chunk_out = (int)chunk;
  return splits;
}

// Workspace floats: acc[QH*splits*D] then ml[QH*splits*2].
long long q35_gqa_decode_workspace(int cache_len, int q_heads, int kv_heads, int D) {
  const int splits = q35_gqa_decode_splits(cache_len, kv_heads, nullptr);
  return (long long)q_heads * splits * (D + 2);
}

int q35_gqa_decode(const void* q, const void* K, const void* V, const void* valid_len, float scale,
                   const void* packed_gate, void* out, void* workspace, long long workspace_floats,
                   int QH, int KVH, int D, int cache_len, hipStream_t stream) {
  Q35_CHECK_ARG(D == kAD && KVH > 0 && QH % KVH == 0 && cache_len > 0);
  const int G = QH / KVH;
  Q35_CHECK_ARG(G == 1 || G == 2 || G == 4 || G == 8);
  int chunk = 0;
  const int splits = q35_gqa_decode_splits(cache_len, KVH, &chunk);
  Q35_CHECK_ARG(splits <= kMaxSplits);
  Q35_CHECK_ARG(workspace_floats >= q35_gqa_decode_workspace(cache_len, QH, KVH, D));
  Q35_CHECK_ARG(q35_aligned16(q) && q35_aligned16(K) && q35_aligned16(V) && q35_aligned16(workspace));
  Q35_CHECK_ARG(q35_aligned8(out) && q35_aligned8(packed_gate));
  float* acc = (float*)workspace;
  float* ml = acc + (size_t)QH * splits * D;
  dim3 grid(KVH, splits);
  const FusedQ none{};
#define Q35_GQA(GG)                                                                                    \
  gqa_decode_split<GG, false><<<grid, kSplitWaves * 64, 0, stream>>>((const uint16_t*)q, (const uint16_t*)K,       \
                                                        (const uint16_t*)V,                           \
                                                        (const long long*)valid_len, acc, ml,         \
                                                        cache_len, chunk, splits, scale, none)
  if (G == 1) Q35_GQA(1);
  else if (G == 2) Q35_GQA(2);
  else if (G == 4) Q35_GQA(4);
  else Q35_GQA(8);
#undef Q35_GQA
  int e = q35_last_error();
  if (e) return e;
  launch_combine(acc, ml, (const uint16_t*)packed_gate, (uint16_t*)out, QH, splits, nullptr, stream);
  return q35_last_error();
}

// One decode token of a full-attention layer after its packed projection:
// Q/K RMSNorm + RoPE (cos/sin from the device positions and inv_freq), K/V
// written into the static cache at index *cache_len_dev, split-K attention
// over the cache plus the new token, LSE combine, sigmoid gate, and
// *cache_len_dev += 1. Two launches; nothing is read on the host.
int q35_gqa_decode_fused(const void* packed, const void* q_w, const void* k_w, int w_f32,
                         const void* inv_freq, const void* pos_t, const void* pos_h,
                         const void* pos_w, int sec_h, int sec_w, int rotary_dim, void* K, void* V,
                         void* cache_len_dev, float scale, void* out, void* workspace,
                         long long workspace_floats, int QH, int KVH, int D, int cache_len,
                         hipStream_t stream) {
  Q35_CHECK_ARG(D == kAD && KVH > 0 && QH % KVH == 0 && cache_len > 0);
  Q35_CHECK_ARG(packed && q_w && k_w && inv_freq && pos_t && K && V && cache_len_dev && out);
  // The in-kernel rotary table holds rot/2 <= 64 frequencies, one per lane.
  Q35_CHECK_ARG(rotary_dim > 0 && rotary_dim <= 128 && rotary_dim % 8 == 0);
  Q35_CHECK_ARG(sec_h >= 0 && sec_w >= 0 && 3 * sec_h <= rotary_dim && 3 * sec_w <= rotary_dim);
  const int G = QH / KVH;
  Q35_CHECK_ARG(G == 1 || G == 2 || G == 4 || G == 8);
  int chunk = 0;
  const int splits = q35_gqa_decode_splits(cache_len, KVH, &chunk);
  Q35_CHECK_ARG(splits <= kMaxSplits);
  Q35_CHECK_ARG(workspace_floats >= q35_gqa_decode_workspace(cache_len, QH, KVH, D));
  Q35_CHECK_ARG(q35_aligned16(K) && q35_aligned16(V) && q35_aligned16(workspace));
  Q35_CHECK_ARG(q35_aligned4(inv_freq) && q35_aligned8(packed) && q35_aligned8(q_w) && q35_aligned8(k_w));
  Q35_CHECK_ARG(q35_aligned8(out));
  float* acc = (float*)workspace;
  float* ml = acc + (size_t)QH * splits * D;
  FusedQ f;
  f.packed = (const uint16_t*)packed;
  f.q_w = q_w;
  f.k_w = k_w;
  f.w_f32 = w_f32;
  f.inv_freq = (const float*)inv_freq;
  f.pos_t = (const long long*)pos_t;
  f.pos_h = (const long long*)(pos_h ? pos_h : pos_t);
  f.pos_w = (const long long*)(pos_w ? pos_w : pos_t);
  f.sec_h = sec_h;
  f.sec_w = sec_w;
  f.rot = rotary_dim;
  f.k_cache = (uint16_t*)K;
  f.v_cache = (uint16_t*)V;
  dim3 grid(KVH, splits);
#define Q35_GQA(GG)                                                                                 \
  gqa_decode_split<GG, true><<<grid, kSplitWaves * 64, 0, stream>>>(nullptr, (const uint16_t*)K,                \
                                                       (const uint16_t*)V,                         \
                                                       (const long long*)cache_len_dev, acc, ml,   \
                                                       cache_len, chunk, splits, scale, f)
  if (G == 1) Q35_GQA(1);
  else if (G == 2) Q35_GQA(2);
  else if (G == 4) Q35_GQA(4);
  else Q35_GQA(8);
#undef Q35_GQA
  int e = q35_last_error();
  if (e) return e;
  launch_combine(acc, ml, (const uint16_t*)packed, (uint16_t*)out, QH, splits,
                 (long long*)cache_len_dev, stream);
  return q35_last_error();
}

// Split plan of the 64-key-block prefill kernel: query tile t (16 rows) has
// nblk(t) key blocks and splits them into ranges of sb blocks, one workgroup
// each. sb starts at 4 and grows until the workgroups of a prompt that starts
// at key 0 fit one round on the device's CUs (one workgroup per CU: the
// kernel takes 156 KB of LDS); smax = the splits of a tile covering the whole
// cache sizes the grid and the workspace. The plan depends only on
// (B, KVH, L, cache_len), so q35_gqa_prefill_workspace sees the same one.
constexpr int kFaSplitBlocks = 4;
static int fa_device_cus() {
  static int cus = 0;
  if (cus == 0) {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) == hipSuccess &&
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0)
      cus = n;
    else
      cus = 256;
  }
  return cus;
}
static void fa_plan(int B, int KVH, int L, int cache_len, int* sb_out, int* smax_out) {
  const int nblk_max = (cache_len + kFaKeys - 1) / kFaKeys;
  const int ntiles = (L + 15) / 16;
  const long long budget = fa_device_cus();
  int sb = kFaSplitBlocks;
  for (; sb < nblk_max; ++sb) {
    long long wgs = 0;
    for (int t = 0; t < ntiles; ++t) {
      const int nb = (min(16 * t + 16, L) + kFaKeys - 1) / kFaKeys;
      wgs += (nb + sb - 1) / sb;
    }
    if (wgs * B * KVH <= budget) break;
  }
  *sb_out = sb;
  *smax_out = (nblk_max + sb - 1) / sb;
}

long long q35_gqa_prefill_workspace(int B, int QH, int KVH, int L, int cache_len) {
  if (B <= 0 || KVH <= 0 || QH <= 0 || QH % KVH || L <= 0 || cache_len <= 0) return 0;
  const int G = QH / KVH;
  if (G != 2 && G != 4) return 0;
  int sb, smax;
  fa_plan(B, KVH, L, cache_len, &sb, &smax);
  if (smax <= 1) return 0;
  return (long long)B * KVH * ((L + 15) / 16) * smax * G * 16 * (kAD + 2);
}

int q35_gqa_prefill(const void* q, const void* K, const void* V, void* out, int B, int QH, int KVH,
                    int D, int L, int cache_len, int kv_start, const void* valid_len, float scale,
                    void* workspace, long long workspace_floats, hipStream_t stream) {
  Q35_CHECK_ARG(D == kAD && KVH > 0 && QH % KVH == 0 && B >= 0 && L >= 0);
  Q35_CHECK_ARG(L <= cache_len && (valid_len || (kv_start >= 0 && kv_start + L <= cache_len)));
  Q35_CHECK_ARG(q35_aligned16(q) && q35_aligned16(K) && q35_aligned16(V) && q35_aligned16(out));
  if ((long long)B * QH * L == 0) return 0;
  const int G = QH / KVH;
  if ((G == 1 || G == 2 || G == 4 || G == 8) && B < 65536 && KVH < 65536) {
    dim3 grid((unsigned)((L + 15) / 16), (unsigned)KVH, (unsigned)B);
#define Q35_PF(GG)                                                                                  \
  gqa_prefill_mfma<GG><<<grid, GG * 64, 0, stream>>>((const uint16_t*)q, (const uint16_t*)K,       \
                                                     (const uint16_t*)V, (uint16_t*)out, B, QH, KVH, \
                                                     L, cache_len, kv_start,                       \
                                                     (const long long*)valid_len, scale)
    if (G == 2 || G == 4) {
      // Long query tiles split their key range over workgroups of at most
      // kFaSplitBlocks blocks when the workspace holds the split records.
      const int ntiles = (L + 15) / 16;
      int sb, smax;
      fa_plan(B, KVH, L, cache_len, &sb, &smax);
      const long long need = q35_gqa_prefill_workspace(B, QH, KVH, L, cache_len);
      if (smax <= 1 || !workspace || workspace_floats < need) {
        smax = 1;
        sb = (cache_len + kFaKeys - 1) / kFaKeys;
      }
      Q35_CHECK_ARG((long long)ntiles * smax < (1ll << 31));
      dim3 fgrid((unsigned)(ntiles * smax), (unsigned)KVH, (unsigned)B);
#define Q35_FA(GG)                                                                               \
  do {                                                                                         \
    gqa_prefill_fa<GG><<<fgrid, 2 * GG * 64, 0, stream>>>(                                     \
        (const uint16_t*)q, (const uint16_t*)K, (const uint16_t*)V, (uint16_t*)out, B, QH, KVH,  \
        L, cache_len, kv_start, (const long long*)valid_len, scale, sb, smax,                    \
        (float*)workspace);                                                                      \
    if (smax > 1)                                                                              \
      gqa_prefill_merge<GG><<<grid, GG * 256, 0, stream>>>(                                    \
          (const float*)workspace, (uint16_t*)out, B, QH, KVH, L, cache_len, kv_start,           \
          (const long long*)valid_len, sb, smax);                                                \
  } while (0)
      if (G == 2) Q35_FA(2);
      else Q35_FA(4);
#undef Q35_FA
    } else if (G == 1) {
      Q35_PF(1);
    } else {
      Q35_PF(8);
    }
#undef Q35_PF
    return q35_last_error();
  }
  const long long waves = (long long)B * QH * L;
  Q35_CHECK_ARG(waves < (1ll << 31));
  gqa_prefill_rows<<<(unsigned)((waves + 3) / 4), 256, 0, stream>>>(
      (const uint16_t*)q, (const uint16_t*)K, (const uint16_t*)V, (uint16_t*)out, B, QH, KVH, L,
      cache_len, kv_start, (const long long*)valid_len, scale);
  return q35_last_error();
}

}  // extern "C"
