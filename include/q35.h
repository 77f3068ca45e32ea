/* libq35 — MI355X (gfx950) decode hot path for the Qwen3.5-2B-class text
 * decoder, as a plain C ABI.
 *
 * Conventions for every entry point:
 *   - pointers are device pointers; bf16 tensors are raw 16-bit patterns;
 *   - sizes are element counts; tensors are dense row-major unless a stride
 *     argument says otherwise;
 *   - all work is enqueued on `stream` (a hipStream_t passed as void*); no
 *     entry point synchronises, allocates device memory or reads device data
 *     on the host, so every call can be captured in a hipGraph;
 *   - the return value is 0 or a hipError_t code; invalid sizes return
 *     hipErrorInvalidValue (1) before anything is launched.
 *   - `*_f32` flags say whether a small parameter vector is fp32 (1) or
 *     bf16 (0).
 *
 * Each declaration names the reference interface it replaces
 * (PingGuoLiZiJvZi/ppu, paths relative to the repository root).
 */
#ifndef Q35_H
#define Q35_H

#ifdef __cplusplus
extern "C" {
#endif

/* ABI version of this header; q35_abi_version() must return it. */
#define Q35_ABI_VERSION 5
int q35_abi_version(void);

/* Zero n device buffers in one launch per 128: ptrs[i] (16-byte aligned) holds
 * nbytes[i] bytes; ptrs and nbytes are host arrays. Replaces the per-tensor
 * zero_() calls of Transformers' Cache.reset() on a reused generation cache
 * (evaluation_wrapper.py:350-352). */
int q35_zero_buffers(void* const* ptrs, const long long* nbytes, int n, void* stream);

/* Measurement utility with no counterpart in the reference: read nbytes
 * (multiple of 16; p 16-byte aligned) once with the non-temporal 16-byte
 * loads of the GEMV weight stream, one workgroup per CU, and write one XOR
 * word per thread to out (out_words >= 256 * CUs; the workgroup count goes
 * to *workgroups_out when not null). Timing it gives the HBM read rate the
 * decode GEMVs can reach on this device. */
int q35_stream_read(const void* p, long long nbytes, void* out, long long out_words, int* workgroups_out,
                    void* stream);

/* Measurement utility with no counterpart in the reference: the same read as
 * one round of requests (workgroups = max(ceil(nbytes / 32 KiB),
 * min(CUs, ceil(nbytes / 4 KiB))), so no lane issues more than 8 loads and
 * every byte is requested at once); out_words >= 256 * that count, which
 * goes to *workgroups_out when not null. Timing it gives the read floor of a
 * small kernel that must fetch nbytes in one launch. */
int q35_stream_read_round(const void* p, long long nbytes, void* out, long long out_words,
                          int* workgroups_out, void* stream);

/* ---- norms and elementwise ------------------------------------------- */

/* rms_norm: y = bf16(x * rsqrt(mean(x^2) + eps) * (1 + w)), rows x width.
 * Replaces qwen35_fused/kernels.py:44 (rms_norm, kernel :24-53). */
int q35_rmsnorm(const void* x, const void* w, int w_f32, void* y, int rows, int width, float eps,
                void* stream);

/* The prefill's embedding lookup and the first layer's input RMSNorm in one
 * launch: r_out[r] = table[ids[r]] (ids int64, clamped to [0, table_rows) as
 * the decode step's gather), y[r] = rms_norm(r_out[r]) with q35_rmsnorm's
 * arithmetic. Replaces embed_tokens(input_ids) (qwen35_fused/integration.py:403)
 * followed by the first layer's rms_norm (kernels.py:44). r_out may be null;
 * widths 512, 1024, 2048, 4096. */
int q35_embed_rmsnorm(const void* table, int table_rows, const void* ids, const void* w, int w_f32,
                      void* r_out, void* y, int rows, int width, float eps, void* stream);

/* residual_add_rms_norm: r' = bf16(residual + update); y = rms_norm(r').
 * Replaces qwen35_fused/kernels.py:85 (kernel :56-112). */
int q35_residual_rmsnorm(const void* residual, const void* update, const void* w, int w_f32,
                         void* residual_out, void* y, int rows, int width, float eps,
                         void* stream);

/* gated_rms_norm: y = bf16(bf16(bf16(rms(x)) * bf16(w)) * silu(gate)).
 * Replaces qwen35_fused/kernels.py:139 (kernel :115-155). */
int q35_gated_rmsnorm(const void* x, const void* gate, const void* w, int w_f32, void* y,
                      int rows, int width, float eps, void* stream);

/* Gated RMSNorm over 128-wide rows whose gate sits inside a wider packed row:
 * gate row r at gate + (r / group_rows) * group_stride + (r % group_rows) * 128
 * (elements). The prefill form of the call at qwen35_fused/integration.py:264-271,
 * where z is a slice of the packed projection (no copy of z). */
int q35_gated_rmsnorm_grouped(const void* x, const void* gate, int group_rows,
                              long long group_stride, const void* w, int w_f32, void* y, int rows,
                              float eps, void* stream);

/* silu_and_mul: out[r, c] = bf16(bf16(silu(p[r, c])) * p[r, width + c]).
 * Replaces qwen35_fused/kernels.py:170 (kernel :158-180). */
int q35_silu_mul(const void* packed, void* out, long long rows, int width, void* stream);

/* q35_silu_mul on the transposed product of a packed [gate; up] projection:
 * packed_t [2 * width, rows] channel-major (what W @ X^T gives), out [rows,
 * width] token-major, same arithmetic. width % 64 == 0, rows % 8 == 0. The
 * prefill MLP computes its gate/up GEMM in that orientation (the library's
 * kernel for it is faster) and this entry transposes back while it applies
 * silu_and_mul (reference kernels.py:170, integration.py:183-185). */
int q35_silu_mul_t(const void* packed_t, void* out, int rows, int width, void* stream);

/* attention_gate_mul: out = bf16(x * bf16(sigmoid(gate))), gate read from the
 * packed QGKV row. Replaces qwen35_fused/kernels.py:312 (kernel :285-333).
 * advance (optional int64 device scalar): *advance += amount in the same
 * launch, the static cache's cumulative_length.add_ of a prefill
 * (integration.py:338) moved after the attention that reads the start. */
int q35_attn_gate_mul(const void* x, const void* packed, void* out, long long tokens, int hidden,
                      int packed_stride, int head_dim, void* advance, long long amount,
                      void* stream);

/* ---- bf16 GEMV (M = 1) ------------------------------------------------- */

/* y[N] = bf16(W[N,K] . xa) where xa depends on `prologue`:
 *   0: xa = x;  1: xa = rms_norm(x, norm_w);  2: r' = bf16(x + u), xa = rms_norm(r', norm_w);
 *   3: xa = gated_rms_norm(x, gate = u, norm_w) over heads of 128 (K % 512 == 0).
 * residual_out / x_norm_out (optional) receive r' and xa.
 * Replaces the decode F.linear call sites qwen35_fused/integration.py:185,245,272,298-302,359,
 * fused with the residual_add_rms_norm of integration.py:478-499 (prologues 1, 2) or the
 * gated_rms_norm of integration.py:266-271 (prologue 3). */
int q35_gemv_bf16(const void* W, const void* x, const void* u, const void* norm_w, int norm_w_f32,
                  float eps, void* residual_out, void* x_norm_out, void* y, int N, int K,
                  int prologue, void* stream);

/* x_row (optional int64 device scalar, prologue 1 only): x is row *x_row of an
 * [x_rows, K] table (the token embedding lookup of integration.py:402-403) and the raw
 * row is stored to residual_out.
 * q35_gemv_bf16 (prologues 0-2) whose epilogue also runs, for rows n < conv_channels,
 * the single-token causal conv update on y[n]: conv_out[n] = bf16(silu(bf16(sum_t
 * conv_w[n,t] * window[t]))), window = (conv_state[n,1:], y[n]), conv_state shifted in
 * place. Replaces integration.py:245 (packed DeltaNet projection) followed by
 * qwen35_fused/kernels.py:659 (causal_conv1d_fused at L == 1, kernel :622-656). */
int q35_gemv_conv(const void* W, const void* x, const void* u, const void* norm_w, int norm_w_f32,
                  float eps, void* residual_out, void* y, int N, int K, int prologue,
                  const void* conv_w, void* conv_state, void* conv_out, int conv_channels,
                  int conv_kw, const void* x_row, int x_rows, void* stream);

/* y[N] = bf16(bf16(silu(bf16(W[n].xa))) * bf16(W[N+n].xa)), W = [gate; up] of [2N, K];
 * prologue as q35_gemv_bf16. Replaces qwen35_fused/kernels.py:232 (ppu_swiglu_gemv,
 * kernel :183-263). */
int q35_swiglu_gemv(const void* W, const void* x, const void* u, const void* norm_w,
                    int norm_w_f32, float eps, void* residual_out, void* x_norm_out, void* y,
                    int N, int K, int prologue, void* stream);

/* int8-weight (A8W8) forms of the three GEMVs above, for one token: W is int8
 * [N, K] (SwiGLU: [2N, K]) with fp32 per-channel scales s_w; the activation
 * after the prologue (rounded to bf16) is quantised per token inside every
 * workgroup (s_x = absmax/127, q = sat(rint(x*127/absmax))), int32 dot4
 * accumulation, y = bf16(float(acc) * s_x * s_w[n]); SwiGLU dequantises gate
 * and up to bf16 first. K a multiple of 1024 (1, 2, 4 or 6 KiB rows).
 * Optional acc_out int32 (per output row; SwiGLU [2N]), xq_out int8 [K] and
 * sx_out fp32 [1] (written by block 0). Each replaces the reference's
 * norm kernel (kernels.py:44/85/139) followed by PPUA8W8Linear.forward
 * (explore_runtime_quantization.py:161-181) and, for SwiGLU, silu_and_mul
 * (kernels.py:158). */
int q35_gemv_i8(const void* Wq, const void* s_w, const void* x, const void* u, const void* norm_w,
                int norm_w_f32, float eps, void* residual_out, void* x_norm_out, void* y,
                void* acc_out, void* xq_out, void* sx_out, int N, int K, int prologue,
                void* stream);
int q35_gemv_i8_conv(const void* Wq, const void* s_w, const void* x, const void* u,
                     const void* norm_w, int norm_w_f32, float eps, void* residual_out, void* y,
                     int N, int K, int prologue, const void* conv_w, void* conv_state,
                     void* conv_out, int conv_channels, int conv_kw, const void* x_row, int x_rows,
                     void* stream);
int q35_swiglu_gemv_i8(const void* Wq, const void* s_w, const void* x, const void* u,
                       const void* norm_w, int norm_w_f32, float eps, void* residual_out,
                       void* x_norm_out, void* y, void* acc_out, int N, int K, int prologue,
                       void* stream);

/* ---- lm_head GEMV + top-1 -------------------------------------------- */

/* Workspace slots (8 bytes each) for q35_lm_head_top1. */
long long q35_lm_head_top1_workspace(int V, int K);
/* out[0] (int64) = argmax_v bf16(W[v] . x), lowest index on ties; no logits stored.
 * mirror (optional, 8-byte aligned, device-addressable: device memory or the
 * q35_host_device_ptr address of pinned host memory) receives the same index
 * from the same launch, so a host loop reads a captured step's token without a
 * copy after it. With advance (int64 device array of n_advance <= 64) every
 * element is incremented after the token is written (the token feedback and
 * position += 1 of graph.py:78-79).
 * Replaces qwen35_fused/kernels.py:1146 (lm_head_argmax, kernels :1093-1143). */
int q35_lm_head_top1(const void* W, const void* x, int V, int K, void* workspace,
                     long long workspace_slots, void* out, void* mirror, void* advance,
                     int n_advance, void* stream);
/* *dev = the address kernels use for the pinned, device-mapped host memory at
 * `host` (hipHostMalloc / torch pin_memory); hipErrorInvalidValue for any
 * other pointer. For the mirror argument of the top-1 entries; no
 * counterpart in the reference (its loop copies the token to the host). */
int q35_host_device_ptr(const void* host, void** dev);
/* No counterpart in the reference: q35_lm_head_top1 for callers that cannot
 * allocate device memory (code under hipGraph capture, tight serving loops,
 * harnesses that forbid hipMalloc). Same result and arguments minus the
 * workspace: the candidate keys go to a fixed array in the library's device
 * memory (65,536 8-byte slots, one copy per GPU, kept until the process
 * ends). Limit: the K = 2048 path (16-byte aligned W and x) takes any
 * V < 2^30; other shapes need (V + 3) / 4 slots, so V <= 262,141, and larger
 * V returns hipErrorInvalidValue before any launch. Allocates nothing. All
 * calls on one GPU share the array: calls that overlap on one GPU (two
 * streams at once) race. */
int q35_lm_head_top1_noalloc(const void* W, const void* x, int V, int K, void* out,
                             void* advance, int n_advance, void* stream);
/* Set-up of the current device for q35_lm_head_top1_noalloc: resolves this
 * GPU's address of its fixed array (a runtime query). Call once per device,
 * with that device current, before the first no-alloc call made under graph
 * capture (otherwise the first call on a device resolves it). No counterpart
 * in the reference. */
int q35_init(void);
/* The same index as q35_lm_head_top1 (replaces the same reference call,
 * qwen35_fused/kernels.py:1146), found with half the weight bytes: an int8
 * copy of W screens every row with a rigorous bound on the difference to the
 * row's bf16 logit, and only the rows the bound cannot exclude are recomputed
 * with q35_lm_head_top1's arithmetic (bit-identical result for any weights;
 * the number of recomputed rows sets the cost). K = 2048; W, Wq, x and the
 * workspace 16-byte aligned. q35_lm_head_screen_prep makes Wq [V, K] int8 and
 * s, c [V] fp32 from W once; workspace of
 * q35_lm_head_top1_screened_workspace(V, K) bytes; out, mirror and advance as
 * for q35_lm_head_top1. */
int q35_lm_head_screen_prep(const void* W, int V, int K, void* Wq, void* s, void* c, void* stream);
long long q35_lm_head_top1_screened_workspace(int V, int K);
int q35_lm_head_top1_screened(const void* W, const void* Wq, const void* s, const void* c,
                              const void* x, int V, int K, void* workspace,
                              long long workspace_bytes, void* out, void* mirror, void* advance,
                              int n_advance, void* stream);
/* Where a screened top-1 workspace for vocabulary V keeps the number of rows
 * each workgroup recomputed exactly (uint32 each, written by every call):
 * returns the byte offset, *n the count. Their sum is the call's bf16 row
 * reads beyond the int8 screen (for monitoring; no reference counterpart). */
long long q35_lm_head_screened_counts(int V, int* n);

/* ---- DeltaNet --------------------------------------------------------- */

/* causal_conv1d_fused for L == 1: state shift, 4-tap conv, bf16 round, SiLU.
 * x row stride in_stride >= C. Replaces qwen35_fused/kernels.py:659 (kernel :622-656). */
int q35_conv1d_update(const void* x, const void* w, void* state, void* out, int B, int C,
                      int in_stride, int kw, void* stream);
/* causal_conv1d_fused for L > 1 (zero history; last kw inputs saved to state).
 * Replaces qwen35_fused/kernels.py:659 (kernel :576-619). */
int q35_conv1d_prefill(const void* x, const void* w, void* state, void* out, int B, int L, int C,
                       int in_stride, int kw, void* stream);

/* One decode step of the gated delta rule for all heads (D = 128), state fp32
 * in place. fuse_conv: src is the raw packed projection and conv1d runs first;
 * fuse_gnorm: out is the gated RMSNorm of the core output (z from packed).
 * Replaces qwen35_fused/kernels.py:854 (delta_recurrent_fused, kernel :768-851),
 * fused with :659 and :139 as integration.py:254-271 chains them. */
int q35_delta_decode(const void* src, int src_stride, const void* packed, int packed_stride,
                     const void* conv_w, void* conv_state, int kw, const void* a_log,
                     const void* dt_bias, int params_f32, void* state, const void* norm_w,
                     int norm_w_f32, float norm_eps, void* out, int B, int H, int D,
                     int fuse_conv, int fuse_gnorm, void* stream);

/* Workspace floats for q35_delta_prefill: 4 per (batch, token, head), plus for
 * L >= 64 53377 per (batch, head, 64-token chunk) (28800 chunk operands, 1
 * decay, 24576 state / delta snapshots) and 3 of alignment. */
long long q35_delta_prefill_workspace(int B, int L, int H);
/* Gated delta rule over L tokens (per-token factors precomputed): a token scan
 * below 64 tokens, the closed form over 64-token chunks on the matrix cores
 * from 64 on. Replaces qwen35_fused/kernels.py:854 with precompute_factors
 * (kernels :713-851). */
int q35_delta_prefill(const void* qkv, int qkv_stride, const void* packed, int packed_stride,
                      const void* a_log, const void* dt_bias, int params_f32, void* state,
                      void* out, void* workspace, long long workspace_floats, int B, int L, int H,
                      int D, void* stream);

/* q35_delta_prefill followed by the gated RMSNorm of every (token, head) row:
 * y[b, t, h, :] = bf16(bf16(bf16(o * rsqrt(mean(o^2) + eps)) * bf16(norm_w)) *
 * silu(z)), o the core output and z = packed[token, 3*H*D + h*D ...]. For L >=
 * 64 the norm runs inside the chunked output kernel (out is not written);
 * below, out receives the core output and a norm launch follows. Replaces
 * the delta_recurrent_fused + gated_rms_norm pair at integration.py:255-271
 * (kernels.py:854 and :139) for prefill. */
int q35_delta_prefill_gated(const void* qkv, int qkv_stride, const void* packed, int packed_stride,
                            const void* a_log, const void* dt_bias, int params_f32, void* state,
                            void* out, void* workspace, long long workspace_floats, int B, int L,
                            int H, int D, const void* norm_w, int norm_w_f32, float eps, void* y,
                            void* stream);

/* q35_delta_prefill_gated with the prefill causal conv folded in: packed is
 * the raw projection [B, L, packed_stride] (conv channels [0, 3*H*D), then z,
 * a, b), conv_w the [3*H*D, 4] taps; the chunk prep computes the conv + SiLU
 * of its rows itself (the bf16 conv output is never stored) and conv_state
 * [B, 3*H*D, 4] receives the last four input rows, as q35_conv1d_prefill
 * leaves it. L >= 64 only (the chunked path). Replaces the
 * causal_conv1d_fused + delta_recurrent_fused + gated_rms_norm chain of
 * integration.py:244-271 (kernels.py:659, :854, :139) for prefill. */
int q35_delta_prefill_gated_conv(const void* packed, int packed_stride, const void* conv_w,
                                 void* conv_state, const void* a_log, const void* dt_bias,
                                 int params_f32, void* state, void* out, void* workspace,
                                 long long workspace_floats, int B, int L, int H, int D,
                                 const void* norm_w, int norm_w_f32, float eps, void* y,
                                 void* stream);

/* ---- full attention --------------------------------------------------- */

/* qgkv_norm_rope: per-head Q/K RMSNorm (1 + w), partial RoPE, Q to [B,QH,L,D];
 * K/V to [B,KVH,L,D], or into the static cache at *cache_start + t when
 * cache_start (int64 device scalar) is given. Positions outside the cache are
 * not written. Replaces qwen35_fused/kernels.py:507 (kernel :419-505). */
int q35_qgkv_norm_rope(const void* packed, const void* q_w, const void* k_w, int w_f32,
                       const void* cos, const void* sin, void* q_out, void* k_out, void* v_out,
                       const void* cache_start, int B, int L, int QH, int KVH, int D,
                       int rotary_dim, int cache_len, void* stream);

/* Split count for a cache capacity (chunk length in *chunk_out): at most 128
 * splits per KV head, chunks of whole 32-token workgroup iterations. */
int q35_gqa_decode_splits(int cache_len, int kv_heads, int* chunk_out);
/* Workspace floats for q35_gqa_decode. */
long long q35_gqa_decode_workspace(int cache_len, int q_heads, int kv_heads, int D);
/* gqa_decode_attention over a static cache; valid_len is an int64 device
 * scalar. With packed_gate (the packed QGKV row) the sigmoid gate of
 * attention_gate_mul is applied to the bf16 output. out [QH*D] bf16.
 * Replaces qwen35_fused/kernels.py:1031 (kernels :940-1028), optionally fused
 * with :312 as integration.py:343-358 chains them. */
int q35_gqa_decode(const void* q, const void* K, const void* V, const void* valid_len, float scale,
                   const void* packed_gate, void* out, void* workspace, long long workspace_floats,
                   int QH, int KVH, int D, int cache_len, void* stream);

/* One decode token of a full-attention layer after its packed projection: Q/K RMSNorm
 * (1 + w) and partial RoPE computed in the kernel (cos/sin from the int64 device
 * positions pos_t/pos_h/pos_w and fp32 inv_freq, interleaved multimodal sections sec_h,
 * sec_w as Transformers' rotary table), K/V stored into the static cache at index
 * *cache_len_dev, split-K attention over the cache and the new token, combine, sigmoid
 * gate, and *cache_len_dev += 1. out [QH*D] bf16. rotary_dim <= 128 (one
 * frequency per lane). Replaces the chain
 * integration.py:298-358 (qgkv_norm_rope :507, cumulative_length.add_, gqa_decode_attention
 * :1031, attention_gate_mul :312) after the packed projection. */
int q35_gqa_decode_fused(const void* packed, const void* q_w, const void* k_w, int w_f32,
                         const void* inv_freq, const void* pos_t, const void* pos_h,
                         const void* pos_w, int sec_h, int sec_w, int rotary_dim, void* K, void* V,
                         void* cache_len_dev, float scale, void* out, void* workspace,
                         long long workspace_floats, int QH, int KVH, int D, int cache_len,
                         void* stream);

/* Causal GQA prefill attention: q [B,QH,L,D], K/V [B,KVH,cache_len,D] holding
 * the L prompt tokens from position start; query row i attends to keys
 * [0, start + i]. start = *valid_len - L + kv_start when valid_len (int64
 * device scalar) is given (kv_start = 0 when it already counts the L tokens,
 * L when it still holds the start), else kv_start. out [B,L,QH*D].
 * Replaces the prefill ALL_ATTENTION_FUNCTIONS call of
 * qwen35_fused/integration.py:360-372. */
int q35_gqa_prefill(const void* q, const void* K, const void* V, void* out, int B, int QH, int KVH,
                    int D, int L, int cache_len, int kv_start, const void* valid_len, float scale,
                    void* workspace, long long workspace_floats, void* stream);

/* Floats of workspace q35_gqa_prefill uses to split the key range of long
 * query tiles across workgroups (0: no split applies). With a smaller or
 * null workspace the call still runs, without splitting. */
long long q35_gqa_prefill_workspace(int B, int QH, int KVH, int L, int cache_len);

/* ---- A8W8 -------------------------------------------------------------- */

/* Per-output-channel weight quantisation (int8 + fp32 scale).
 * Replaces explore_runtime_quantization.py:142-155 (PPUA8W8Linear.__init__). */
int q35_quant_weight_i8(const void* W, void* Wq, void* scale, int N, int K, void* stream);
/* Per-token dynamic symmetric int8 quantisation (vLLM scaled_int8_quant rule),
 * one workgroup per row: K a multiple of 8 and at most 8192, x 16-byte and xq
 * 8-byte aligned. Replaces the call at explore_runtime_quantization.py:167-172. */
int q35_quant_act_i8(const void* x, void* xq, void* scale, int M, int K, void* stream);
/* attention_gate_mul (qwen35_fused/kernels.py:312) followed by the per-token
 * int8 quantisation of the o_proj input that the A8W8 linear applies
 * (explore_runtime_quantization.py:167-172), in one launch: the same bits as
 * q35_attn_gate_mul -> q35_quant_act_i8; the gated bf16 rows are never
 * stored. hidden and head_dim multiples of 8, hidden <= 8192, packed_stride a
 * multiple of 8; advance / amount as for q35_attn_gate_mul. */
int q35_attn_gate_quant(const void* x, const void* packed, void* xq, void* scale, long long tokens,
                        int hidden, int packed_stride, int head_dim, void* advance, long long amount,
                        void* stream);
/* y[M,N] = bf16(int32(xq . Wq) * s_x[m] * s_w[n]). With x (bf16) the per-token
 * quantisation is done here and xq/s_x receive it (fused into the GEMV launch
 * for M == 1 and for small M*K at K = 2048/6144, where they are optional);
 * with x == NULL, xq/s_x are inputs. 2..16 tokens at K = 2048/6144 run on the
 * int8 matrix cores. acc_out (optional) gets the int32 sums.
 * Replaces explore_runtime_quantization.py:161-181 (PPUA8W8Linear.forward). */
int q35_gemv_a8w8(const void* x, void* xq, void* s_x, const void* Wq, const void* s_w, void* y,
                  void* acc_out, int M, int N, int K, void* stream);

/* Prefill SwiGLU of the packed [gate; up] A8W8 GEMM on its int32 accumulators
 * acc[M, 2N]: y[M,N] = bf16(bf16(silu(g)) * u), g and u dequantised as in
 * q35_dequant_i32 (N % 8 == 0, acc/s_w/y 16-byte aligned). Replaces the
 * dequant of explore_runtime_quantization.py:173-180 followed by silu_and_mul
 * (kernels.py:158-180) at integration.py:183-185. */
int q35_dequant_swiglu_i32(const void* acc, const void* s_x, const void* s_w, void* y, int M, int N,
                           void* stream);

/* Prefill GEMM on the matrix cores, C = A[M,K] . B[N,K]^T with both operands
 * K-contiguous, of one kind:
 *   0  bf16 A, B -> C bf16 = bf16(fp32 sum)                        F.linear at the prefill
 *      sites integration.py:183,245,272,298,359
 *   1  bf16, B = [gate; up] [2N, K] -> C[M,N] = bf16(bf16(silu(bf16 g)) * bf16 u)
 *      F.linear on the packed gate/up weight + silu_and_mul, integration.py:183-185
 *      and kernels.py:158-180
 *   2  int8 A, B -> C int32 = exact sum                            the int8 GEMM of
 *      explore_runtime_quantization.py:173-180 (accumulators for the fused
 *      dequant kernels below)
 *   3  int8 -> C bf16 = bf16(float(acc) * s_x[m] * s_w[n])         the same with its
 *      dequant (q35_dequant_i32's values)
 *   4  int8, B = [gate; up] -> SwiGLU of the dequantised bf16 gate and up
 *      (q35_dequant_swiglu_i32's values)
 * s_x [M] and s_w [N] (kind 4: [2N]) fp32 are used by kinds 3 and 4 only.
 * K * (element bytes) must be a multiple of 128 (the stage width); A and B
 * 16-byte aligned; each operand below 2^32 bytes (bf16: 2^31 elements).
 * tile < 0 picks the library's plan (tile and K splits by output shape);
 * otherwise tile 0-8 (outputs per workgroup: 0, 4, 5 256x192; 1, 6, 7
 * 128x128; 2 256x128; 3 128x192; 8 128x64; SwiGLU kinds: half as many
 * output columns; 5-8 store from registers and take kinds 0 and 2 only)
 * with `splits` workgroups per tile along K (1-8, dividing the stage count;
 * tiles 1, 2, 3, 6, 7, 8 and kinds 0, 2, 3 only). A plan that splits K needs a workspace of
 * q35_gemm_workspace bytes (arrival counters + partial tiles), zero-filled
 * before its first use; each launch leaves the counters at zero again (after
 * a launch that failed part way, zero it again). Two launches that overlap in
 * time must not share a workspace. No allocation, no host synchronisation. */
long long q35_gemm_workspace(int M, int N, int K, int kind, int tile, int splits);
int q35_gemm(const void* A, const void* B, void* C, int M, int N, int K, int kind, const void* s_x,
             const void* s_w, int tile, int splits, void* workspace, long long workspace_bytes,
             void* stream);

/* A8W8 prefill between the int8 GEMMs of a layer: residual add of the
 * dequantised accumulators of the previous GEMM (q35_dequant_i32's values) +
 * RMSNorm (width 2048, (1 + w) weight) with the normalised rows quantised per
 * token for the next GEMM (q35_quant_act_i8's rule): the same bits as
 * q35_dequant_i32 -> q35_residual_rmsnorm -> q35_quant_act_i8 in one launch.
 * y (bf16 normalised rows) and yq/s_y may each be null, not both. Replaces
 * the dequant of explore_runtime_quantization.py:173-180, the residual norm of
 * integration.py:456-499 and the activation quant of
 * explore_runtime_quantization.py:167-172 at the A8W8 prefill sites. */
int q35_residual_rmsnorm_dequant_quant(const void* x, const void* acc, const void* s_x,
                                       const void* s_w, const void* w, int w_f32, void* r_out,
                                       void* y, void* yq, void* s_y, int rows, int width, float eps,
                                       void* stream);
/* A8W8 prefill MLP: q35_dequant_swiglu_i32's SwiGLU of the packed [gate; up]
 * accumulators acc[M, 2N], quantised per token into yq[M, N] int8 and s_y[M]
 * (q35_quant_act_i8's rule) for the down projection; the bf16 activation is
 * never stored. N % 8 == 0, N <= 6144. Replaces silu_and_mul
 * (kernels.py:158-180) + the activation quant of the down projection's
 * PPUA8W8Linear at integration.py:183-187. */
int q35_dequant_swiglu_quant(const void* acc, const void* s_x, const void* s_w, void* yq, void* s_y,
                             int M, int N, void* stream);

/* y[M,N] = bf16(float(acc[m,n]) * s_x[m] * s_w[n]) for int32 accumulators of an
 * int8 GEMM (the prefill A8W8 path; N % 8 == 0). Same dequant epilogue as
 * q35_gemv_a8w8, replacing the output stage of explore_runtime_quantization.py:173-180. */
int q35_dequant_i32(const void* acc, const void* s_x, const void* s_w, void* y, int M, int N,
                    void* stream);

/* ---------------------------------------------------------- vision encoder */
/* Vision LayerNorm over rows of `width`: y = bf16((x - mean) * rsqrt(var +
 * eps) * w + b), mean and variance in fp32; w and b both bf16 or both fp32
 * (p_f32). Replaces layer_norm (kernels.py:1186-1218). */
int q35_layernorm(const void* x, const void* w, const void* b, int p_f32, void* y, int rows,
                  int width, float eps, void* stream);
/* residual_out = bf16(residual + update); y = q35_layernorm(residual_out).
 * Replaces residual_add_layer_norm (kernels.py:1221-1280). */
int q35_residual_layernorm(const void* residual, const void* update, const void* w, const void* b,
                           int p_f32, void* residual_out, void* y, int rows, int width, float eps,
                           void* stream);
/* out[r] = bf16(hidden[r] + bf16(sum_n table[indices[r, n]] * weights[r, n])),
 * the sum an fp32 FMA chain in neighbour order; indices int64 [rows,
 * neighbors] (clamped to [0, table_rows)), weights fp32 or bf16 (w_f32).
 * Replaces position_embed_add (kernels.py:1283-1336). */
int q35_position_embed_add(const void* hidden, const void* table, int table_rows,
                           const void* indices, const void* weights, int w_f32, void* out, int rows,
                           int width, int neighbors, void* stream);
/* packed [tokens, 3*heads*dim] = [q heads | k heads | v heads] per token ->
 * q, k, v [1, heads, tokens, dim]; q and k get rotate-half RoPE in fp32
 * (x*cos + (sign*x_partner)*sin, partner = c +- dim/2), cos/sin [tokens, dim]
 * fp32 or bf16 (cs_f32); dim even. Replaces vision_qkv_rope
 * (kernels.py:336-416). */
int q35_vision_qkv_rope(const void* packed, const void* cos, const void* sin, int cs_f32, void* q,
                        void* k, void* v, int tokens, int heads, int dim, void* stream);
/* Non-causal attention of the vision blocks: q, k, v [heads, tokens, dim]
 * (bf16, 16-byte aligned, dim % 8 == 0, dim <= 128), each query over the keys
 * of its own image (cu_seqlens: n_images + 1 int32 offsets, or null for one
 * image), fp32 softmax, P rounded to bf16 for the P.V product; out [tokens,
 * heads*dim] bf16. No counterpart among the reference's kernels: it replaces
 * the Transformers attention-interface call of the vision attention
 * (integration.py:671-731). */
int q35_vision_attention(const void* q, const void* k, const void* v, void* out,
                         const void* cu_seqlens, int n_images, int tokens, int heads, int dim,
                         float scale, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* Q35_H */
