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
// read from HBM exactly once per step. D = 256.
//   QK: lane = (token tg = lane/16 of a 4-token group, 16-dim slice lane%16);
//       per-token scores are reduced over the 16-lane DPP row.
//   PV: lane owns dims 4*lane..4*lane+3; p values are broadcast by readlane.
// Each wave runs an online softmax over its tokens; the 4 waves are merged in
// LDS and the workgroup writes (acc[D], m, l) per query head and split.
constexpr int kAD = 256;
constexpr int kMaxG = 8;

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

// Q/K RMSNorm (1 + w) + partial RoPE of one 256-wide head held by a wave
// (lane: dims 4*lane..+3), with cos/sin computed from the positions exactly as
// Transformers' rotary table does: freq_i = pos * inv_freq[i] (fp32),
// cos/sin in fp32 rounded to bf16; dims c and c + rot/2 share freq c mod rot/2.
Q35_DEV void norm_rope_row(const uint16_t* __restrict__ src, const void* w, int w_f32,
                           const FusedQ& f, int lane, float (&o)[4]) {
  float x[4], n[4];
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    x[e] = bf2f(src[lane * 4 + e]);
    ss += x[e] * x[e];
  }
  const float inv = rsqrt_cr(wave_sum(ss) / (float)kAD + 1.0e-6f);
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int c = lane * 4 + e;
    const float wc = w_f32 ? reinterpret_cast<const float*>(w)[c] : bf2f(reinterpret_cast<const uint16_t*>(w)[c]);
    n[e] = round_bf(x[e] * inv * (1.0f + wc));
  }
  const int half = f.rot / 2;
  const int shift = half / 4;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int c = lane * 4 + e;
    const int partner_lane = c < half ? lane + shift : lane - shift;
    const float pn = __shfl(n[e], partner_lane & 63, 64);
    if (c < f.rot) {
      const int i = c < half ? c : c - half;
      const long long* pp = f.pos_t;
      if (i % 3 == 1 && i < 3 * f.sec_h) pp = f.pos_h;
      if (i % 3 == 2 && i < 3 * f.sec_w) pp = f.pos_w;
      const float ang = (float)pp[0] * f.inv_freq[i];
      const float cs = round_bf(cosf(ang)), sn = round_bf(sinf(ang));
      const float qc = round_bf(n[e] * cs);
      const float rh = c < half ? -pn : pn;
      o[e] = round_bf(qc + round_bf(rh * sn));
    } else {
      o[e] = n[e];
    }
  }
}

template <int G, bool FUSED>
__global__ __launch_bounds__(256) void gqa_decode_split(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ Kc, const uint16_t* __restrict__ Vc,
    const long long* __restrict__ valid_len, float* __restrict__ acc_out, float* __restrict__ ml_out,
    int cache_len, int chunk, int splits, float scale, const FusedQ fq) {
  const int lane = threadIdx.x & 63;
  const int wid = threadIdx.x >> 6;
  const int kvh = blockIdx.x;
  const int split = blockIdx.y;
  const int QH = G * gridDim.x;
  // FUSED: valid_len counts the tokens before this one; the new token sits at
  // index n_old and is attended from LDS by the workgroup that owns it.
  const long long n_old = FUSED ? valid_len[0] : 0;
  const int n_cached = FUSED ? (int)min((long long)cache_len, n_old)
                             : (int)min((long long)cache_len, valid_len[0]);
  const int start = split * chunk;
  const int end = min(start + chunk, n_cached);
  const bool owns_new = FUSED && n_old >= start && n_old < start + chunk;

  __shared__ float q_s[FUSED ? G : 1][kAD];
  __shared__ float kn_s[FUSED ? kAD : 1], vn_s[FUSED ? kAD : 1];
  if (FUSED) {
    for (int g = wid; g < G; g += 4) {
      float o[4];
      norm_rope_row(fq.packed + (size_t)(kvh * G + g) * 2 * kAD, fq.q_w, fq.w_f32, fq, lane, o);
      *reinterpret_cast<float4*>(&q_s[g][4 * lane]) =
          make_float4(o[0] * scale, o[1] * scale, o[2] * scale, o[3] * scale);
    }
    if (owns_new && wid == 0) {
      float o[4];
      const uint16_t* krow = fq.packed + (size_t)2 * QH * kAD + (size_t)kvh * kAD;
      const uint16_t* vrow = krow + (size_t)gridDim.x * kAD;
      norm_rope_row(krow, fq.k_w, fq.w_f32, fq, lane, o);
      const uint2 vraw = *reinterpret_cast<const uint2*>(vrow + 4 * lane);
      *reinterpret_cast<float4*>(&kn_s[4 * lane]) = make_float4(o[0], o[1], o[2], o[3]);
      *reinterpret_cast<float4*>(&vn_s[4 * lane]) =
          make_float4(bf_lo(vraw.x), bf_hi(vraw.x), bf_lo(vraw.y), bf_hi(vraw.y));
      if (n_old < cache_len) {
        const size_t off = ((size_t)kvh * cache_len + (size_t)n_old) * kAD + 4 * lane;
        *reinterpret_cast<uint2*>(fq.k_cache + off) = make_uint2(pack_bf2(o[0], o[1]), pack_bf2(o[2], o[3]));
        *reinterpret_cast<uint2*>(fq.v_cache + off) = vraw;
      }
    }
    __syncthreads();
  }

  // q slices for QK (16 dims of the lane's slice, per head), pre-scaled in fp32.
  const int ds = lane & 15;
  float qf[G][16];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    if (FUSED) {
#pragma unroll
      for (int j = 0; j < 16; ++j) qf[g][j] = q_s[g][ds * 16 + j];
    } else {
      const uint16_t* qh = q + (size_t)(kvh * G + g) * kAD + ds * 16;
      float t8[8];
      unpack8(*reinterpret_cast<const uint4*>(qh), t8);
#pragma unroll
      for (int j = 0; j < 8; ++j) qf[g][j] = t8[j] * scale;
      unpack8(*reinterpret_cast<const uint4*>(qh + 8), t8);
#pragma unroll
      for (int j = 0; j < 8; ++j) qf[g][8 + j] = t8[j] * scale;
    }
  }

  float m[G], l[G], acc[G][4];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = -INFINITY;
    l[g] = 0.f;
    acc[g][0] = acc[g][1] = acc[g][2] = acc[g][3] = 0.f;
  }
  const uint16_t* Kh = Kc + (size_t)kvh * cache_len * kAD;
  const uint16_t* Vh = Vc + (size_t)kvh * cache_len * kAD;
  // Tokens of this wave: groups of 4, interleaved across the 4 waves.
  for (int t0 = start + wid * 4; t0 < end; t0 += 16) {
    const int tok = t0 + (lane >> 4);
    const bool live = tok < end;
    float kf[16];
    if (live) {
      float t8[8];
      unpack8(*reinterpret_cast<const uint4*>(Kh + (size_t)tok * kAD + ds * 16), t8);
#pragma unroll
      for (int j = 0; j < 8; ++j) kf[j] = t8[j];
      unpack8(*reinterpret_cast<const uint4*>(Kh + (size_t)tok * kAD + ds * 16 + 8), t8);
#pragma unroll
      for (int j = 0; j < 8; ++j) kf[8 + j] = t8[j];
    } else {
#pragma unroll
      for (int j = 0; j < 16; ++j) kf[j] = 0.f;
    }
    // V rows of the 4 tokens, dims 4*lane..+3.
    uint2 vv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      vv[i] = t0 + i < end ? *reinterpret_cast<const uint2*>(Vh + (size_t)(t0 + i) * kAD + 4 * lane)
                           : make_uint2(0, 0);
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float s = 0.f;
#pragma unroll
      for (int j = 0; j < 16; ++j) s = fmaf(qf[g][j], kf[j], s);
      s = row16_sum(s);
      s = live ? s : -INFINITY;
      float sc[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) sc[i] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(s), 16 * i));
      const float mx = fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3]));
      const float m_new = fmaxf(m[g], mx);
      const float corr = expf(m[g] - m_new);
      float p[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) p[i] = expf(sc[i] - m_new);
      l[g] = l[g] * corr + ((p[0] + p[1]) + (p[2] + p[3]));
#pragma unroll
      for (int d = 0; d < 4; ++d) acc[g][d] *= corr;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        acc[g][0] = fmaf(p[i], bf_lo(vv[i].x), acc[g][0]);
        acc[g][1] = fmaf(p[i], bf_hi(vv[i].x), acc[g][1]);
        acc[g][2] = fmaf(p[i], bf_lo(vv[i].y), acc[g][2]);
        acc[g][3] = fmaf(p[i], bf_hi(vv[i].y), acc[g][3]);
      }
      m[g] = m_new;
    }
  }
  // The new token (FUSED): wave 0 of the owning workgroup folds it in.
  if (owns_new && wid == 0) {
    const float4 kn = *reinterpret_cast<const float4*>(&kn_s[4 * lane]);
    const float4 vn = *reinterpret_cast<const float4*>(&vn_s[4 * lane]);
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float4 qv = *reinterpret_cast<const float4*>(&q_s[g][4 * lane]);
      float sdot = qv.x * kn.x;
      sdot = fmaf(qv.y, kn.y, sdot);
      sdot = fmaf(qv.z, kn.z, sdot);
      sdot = fmaf(qv.w, kn.w, sdot);
      const float sc = wave_sum(sdot);
      const float m_new = fmaxf(m[g], sc);
      const float corr = expf(m[g] - m_new);
      const float p = expf(sc - m_new);
      l[g] = l[g] * corr + p;
      acc[g][0] = fmaf(p, vn.x, acc[g][0] * corr);
      acc[g][1] = fmaf(p, vn.y, acc[g][1] * corr);
      acc[g][2] = fmaf(p, vn.z, acc[g][2] * corr);
      acc[g][3] = fmaf(p, vn.w, acc[g][3] * corr);
      m[g] = m_new;
    }
  }
  // Merge the 4 waves.
  __shared__ float m_s[4][kMaxG], l_s[4][kMaxG];
  __shared__ float a_s[4][kMaxG][kAD];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    if (lane == 0) {
      m_s[wid][g] = m[g];
      l_s[wid][g] = l[g];
    }
    *reinterpret_cast<float4*>(&a_s[wid][g][4 * lane]) = make_float4(acc[g][0], acc[g][1], acc[g][2], acc[g][3]);
  }
  __syncthreads();
  for (int idx = threadIdx.x; idx < G * kAD; idx += 256) {
    const int g = idx / kAD, d = idx - g * kAD;
    float mm = -INFINITY;
    for (int w = 0; w < 4; ++w) mm = fmaxf(mm, m_s[w][g]);
    float a = 0.f, ll = 0.f;
    for (int w = 0; w < 4; ++w) {
      const float f = m_s[w][g] == -INFINITY ? 0.f : expf(m_s[w][g] - mm);
      a += a_s[w][g][d] * f;
      ll += l_s[w][g] * f;
    }
    const int slot = (kvh * G + g) * splits + split;
    acc_out[(size_t)slot * kAD + d] = a;
    if (d == 0) {
      ml_out[slot * 2] = mm;
      ml_out[slot * 2 + 1] = ll;
    }
  }
}

// Log-sum-exp merge of the splits -> bf16, optionally times bf16(sigmoid(gate))
// [reference kernels.py:1007-1028 and 285-333]. One workgroup per query head.
__global__ __launch_bounds__(256) void gqa_decode_combine(const float* __restrict__ acc,
                                                          const float* __restrict__ ml,
                                                          const uint16_t* __restrict__ packed_gate,
                                                          uint16_t* __restrict__ out, int splits,
                                                          long long* advance_len) {
  const int h = blockIdx.x;
  // The split kernel that read the length has completed (stream order).
  if (advance_len && h == 0 && threadIdx.x == 0) advance_len[0] += 1;
  __shared__ float w_s[1024];
  __shared__ float mx_s, l_s;
  if (threadIdx.x < 64) {
    float mx = -INFINITY;
    for (int s = threadIdx.x; s < splits; s += 64) mx = fmaxf(mx, ml[(h * splits + s) * 2]);
    mx = wave_max(mx);
    float lt = 0.f;
    for (int s = threadIdx.x; s < splits; s += 64) {
      const float ms = ml[(h * splits + s) * 2];
      const float f = ms == -INFINITY ? 0.f : expf(ms - mx);
      w_s[s] = f;
      lt += ml[(h * splits + s) * 2 + 1] * f;
    }
    lt = wave_sum(lt);
    if (threadIdx.x == 0) {
      mx_s = mx;
      l_s = lt;
    }
  }
  __syncthreads();
  const int d = threadIdx.x;
  float tot = 0.f;
  for (int s = 0; s < splits; ++s) tot = fmaf(acc[(size_t)(h * splits + s) * kAD + d], w_s[s], tot);
  float o = round_bf(tot / l_s);
  if (packed_gate) {
    const float g = bf2f(packed_gate[h * 2 * kAD + kAD + d]);
    o = o * round_bf(sigmoid_f(g));
  }
  out[(size_t)h * kAD + d] = (uint16_t)f2bf(o);
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
  // With a device length (static cache, already including these L tokens)
  // the prompt starts at valid_len - L; the bound keeps reads in the cache.
  long long ks = valid_len ? valid_len[0] - L : (long long)kv_start_host;
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
int q35_gqa_decode_splits(int cache_len, int kv_heads, int* chunk_out) {
  if (cache_len <= 0 || kv_heads <= 0) return 0;
  long long chunk = ((long long)cache_len * kv_heads + 255) / 256;
  chunk = (chunk + 15) / 16 * 16;
  if (chunk < 16) chunk = 16;
  if (chunk > 1024) chunk = 1024;
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
  Q35_CHECK_ARG(splits <= 1024);
  Q35_CHECK_ARG(workspace_floats >= q35_gqa_decode_workspace(cache_len, QH, KVH, D));
  Q35_CHECK_ARG(q35_aligned16(q) && q35_aligned16(K) && q35_aligned16(V) && q35_aligned16(workspace));
  float* acc = (float*)workspace;
  float* ml = acc + (size_t)QH * splits * D;
  dim3 grid(KVH, splits);
  const FusedQ none{};
#define Q35_GQA(GG)                                                                                    \
  gqa_decode_split<GG, false><<<grid, 256, 0, stream>>>((const uint16_t*)q, (const uint16_t*)K,       \
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
  gqa_decode_combine<<<QH, kAD, 0, stream>>>(acc, ml, (const uint16_t*)packed_gate, (uint16_t*)out,
                                             splits, nullptr);
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
  Q35_CHECK_ARG(rotary_dim > 0 && rotary_dim <= D && rotary_dim % 8 == 0);
  Q35_CHECK_ARG(sec_h >= 0 && sec_w >= 0 && 3 * sec_h <= rotary_dim && 3 * sec_w <= rotary_dim);
  const int G = QH / KVH;
  Q35_CHECK_ARG(G == 1 || G == 2 || G == 4 || G == 8);
  int chunk = 0;
  const int splits = q35_gqa_decode_splits(cache_len, KVH, &chunk);
  Q35_CHECK_ARG(splits <= 1024);
  Q35_CHECK_ARG(workspace_floats >= q35_gqa_decode_workspace(cache_len, QH, KVH, D));
  Q35_CHECK_ARG(q35_aligned16(K) && q35_aligned16(V) && q35_aligned16(workspace));
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
  gqa_decode_split<GG, true><<<grid, 256, 0, stream>>>(nullptr, (const uint16_t*)K,                \
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
  gqa_decode_combine<<<QH, kAD, 0, stream>>>(acc, ml, (const uint16_t*)packed, (uint16_t*)out,
                                             splits, (long long*)cache_len_dev);
  return q35_last_error();
}

int q35_gqa_prefill(const void* q, const void* K, const void* V, void* out, int B, int QH, int KVH,
                    int D, int L, int cache_len, int kv_start, const void* valid_len, float scale,
                    hipStream_t stream) {
  Q35_CHECK_ARG(D == kAD && KVH > 0 && QH % KVH == 0 && B >= 0 && L >= 0);
  Q35_CHECK_ARG(L <= cache_len && (valid_len || (kv_start >= 0 && kv_start + L <= cache_len)));
  Q35_CHECK_ARG(q35_aligned16(q) && q35_aligned16(K) && q35_aligned16(V) && q35_aligned16(out));
  const long long waves = (long long)B * QH * L;
  if (waves == 0) return 0;
  Q35_CHECK_ARG(waves < (1ll << 31));
  gqa_prefill_rows<<<(unsigned)((waves + 3) / 4), 256, 0, stream>>>(
      (const uint16_t*)q, (const uint16_t*)K, (const uint16_t*)V, (uint16_t*)out, B, QH, KVH, L,
      cache_len, kv_start, (const long long*)valid_len, scale);
  return q35_last_error();
}

}  // extern "C"
