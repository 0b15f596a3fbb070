/*
 * libqwen35_fp8_hip.so -- MI355X (gfx950) batch-1 FP8 decode path for
 * Qwen3.5-shaped hybrid models.
 *
 * Conventions (all entry points):
 *   - pointers are device pointers owned by the caller; activations are bf16
 *     (uint16 bit patterns), weights E4M3FN bytes, norm weights fp32 unless
 *     stated, GatedDeltaNet norm weight bf16;
 *   - `stream` is a hipStream_t (the reference passed cudaStream_t); launches
 *     are asynchronous on it;
 *   - scale-mode code `kb` (the reference's `K_blocks`): kb > 1 -> 128x128
 *     block scales [ceil(N/128), kb]; kb == 1 -> one scale per row [N];
 *     kb < 0 -> per-row-per-block [N, -kb].
 *
 * Section 1 re-exports the reference's ctypes ABI with identical names,
 * argument order and meaning (bf16 scale_inv, void return).  Section 2 holds
 * the native entry points (fp32 scale_inv, int status: 0 ok, -1 error with
 * qh_last_error()).
 */
#ifndef QWEN35_FP8_HIP_H
#define QWEN35_FP8_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* qh_stream_t; /* hipStream_t */

/* ========================= 1. reference ABI (bf16 scales) ================= */

/* replaces fp8_gemm_batch, qwen3_infer/csrc/fp8_kernels.cu:72-89 (bound at main.py:108) */
void fp8_gemm_batch(const void* x_bf16, const void* w_fp8, const void* w_scale_bf16, void* y_bf16,
                    int M, int N, int K, int K_blocks, qh_stream_t stream);

/* replaces launch_gemv_v4_extern, fused_kernels.cu:1328-1336 (main.py:119) */
void launch_gemv_v4_extern(const void* x, const void* w, const void* s, void* y, int N, int K,
                           int K_blk, qh_stream_t stream);

/* replaces launch_gemv_v3_extern, fused_kernels.cu:981-989 (same kernel as v4 here) */
void launch_gemv_v3_extern(const void* x, const void* w, const void* s, void* y, int N, int K,
                           int K_blk, qh_stream_t stream);

/* replaces launch_linear_in_proj4, fused_kernels.cu:1338-1354 (main.py:123-132) */
void launch_linear_in_proj4(const void* x, const void* w0, const void* s0, void* y0, int n0,
                            int kb0, const void* w1, const void* s1, void* y1, int n1, int kb1,
                            const void* w2, const void* s2, void* y2, int n2, int kb2,
                            const void* w3, const void* s3, void* y3, int n3, int kb3, int K,
                            qh_stream_t stream);

/* replaces launch_fused_qkv, fused_kernels.cu:991-1007 (main.py:133-140) */
void launch_fused_qkv(const void* x, const void* w_q, const void* w_k, const void* w_v,
                      const void* s_q, const void* s_k, const void* s_v, void* q_out, void* k_out,
                      void* v_out, int K, int N_q, int N_k, int N_v, int K_blk, int N_q_blk,
                      int N_k_blk, int N_v_blk, qh_stream_t stream);

/* replaces launch_fused_gate_up, fused_kernels.cu:1009-1025 (main.py:141-148) */
void launch_fused_gate_up(const void* x, const void* w_gate, const void* w_up, const void* s_gate,
                          const void* s_up, void* gate_out, void* up_out, int K, int N_gate,
                          int N_up, int K_blk, int N_gate_blk, int N_up_blk, qh_stream_t stream);

/* replaces launch_rmsnorm_ip, fused_kernels.cu:1055-1062 (main.py:149-153) */
void launch_rmsnorm_ip(void* x, const void* weight, int N, int D, float eps, qh_stream_t stream);

/* replaces launch_rmsnorm_out, fused_kernels.cu:1045-1053 (main.py:154-162) */
void launch_rmsnorm_out(const void* x, const void* weight, void* out, int N, int D, float eps,
                        qh_stream_t stream);

/* replaces launch_fused_attn, fused_kernels.cu:1027-1043 (main.py:168-172) */
void launch_fused_attn(const void* q, const void* k_cache, const void* v_cache, void* output,
                       int seq_len, int max_seq_len, int head_dim, int n_heads, int n_kv_heads,
                       qh_stream_t stream);

/* replaces launch_fused_attn_v2, fused_kernels.cu:1300-1326 (main.py:163-167) */
void launch_fused_attn_v2(const void* q, const void* k_cache, const void* v_cache, void* output,
                          int seq_len, int max_seq_len, int head_dim, int n_heads, int n_kv_heads,
                          qh_stream_t stream);

/* replaces layer_pre_attn, fused_kernels.cu:1066-1091 (main.py:184-193).
 * The checkpoint's q_proj rows are per-head [q_h | gate_h] (main.py:1001); the
 * reference's opt-in fused path splits q_out as [first half | second half]
 * (main.py:1292-1294).  With a q/gate head dim set (qh_set_qgate_head_dim, or
 * the environment variable QH_QGATE_HEAD_DIM when it is left at -1), q_out is
 * written de-interleaved, [q_0 .. q_{H-1} | gate_0 .. gate_{H-1}], which makes
 * that split correct; with 0 (the default) the rows keep the checkpoint order. */
void layer_pre_attn(const void* hidden, const float* norm_weight, const void* w_q, const void* s_q,
                    int N_q, int N_q_blk, const void* w_k, const void* s_k, int N_k, int N_k_blk,
                    const void* w_v, const void* s_v, int N_v, int N_v_blk, void* q_out,
                    void* k_out, void* v_out, void* norm_ws, int h_dim, int K_blk,
                    qh_stream_t stream);

/* Head dim of layer_pre_attn's q/gate de-interleave: d > 0 on, 0 off, -1 (the
 * initial value) follow QH_QGATE_HEAD_DIM.  No counterpart in the reference,
 * whose opt-in path carries the split bug.  Returns 0, or -1 for d < -1. */
int qh_set_qgate_head_dim(int d);

/* replaces layer_post_attn, fused_kernels.cu:1102-1150 (main.py:194-206) */
void layer_post_attn(const void* hidden, const void* attn_out, const void* w_o, const void* s_o,
                     int N_o, int N_o_blk, const float* norm_weight, const void* w_g,
                     const void* s_g, int N_g, int N_g_blk, const void* w_u, const void* s_u,
                     int N_u, int N_u_blk, const void* w_d, const void* s_d, int N_d, int N_d_blk,
                     void* output, void* ws, void* gate_buf, void* up_buf, void* silu_buf,
                     int h_dim, int attn_dim, int K_blk_o, int K_blk_gu, int K_blk_d,
                     qh_stream_t stream);

/* replaces layer_post_o_fp8_mlp, fused_kernels.cu:1156-1195 (main.py:207-217) */
void layer_post_o_fp8_mlp(const void* hidden, const void* o_out, const float* norm_weight,
                          const void* w_g, const void* s_g, int N_g, const void* w_u,
                          const void* s_u, int N_u, const void* w_d, const void* s_d, int N_d,
                          void* output, void* ws, void* gate_buf, void* up_buf, void* silu_buf,
                          int h_dim, int K_blk_gu, int K_blk_d, qh_stream_t stream);

/* replaces layer_mid_attn, fused_kernels.cu:1224-1297 (main.py:173-183) */
void layer_mid_attn(void* q_buf, void* k_buf, const void* v_buf, void* attn_out,
                    const float* q_norm_weight, const float* k_norm_weight,
                    const float* cos_table, const float* sin_table, void* k_cache, void* v_cache,
                    int pos, int past_len, int total_seq, int max_seq_len, int head_dim,
                    int rotary_dim, int n_heads, int n_kv_heads, qh_stream_t stream);

/* replaces launch_prepare_linear_gates, fused_kernels.cu:942-954 (main.py:218-225) */
void launch_prepare_linear_gates(const void* a, const void* beta_in, const float* A_log,
                                 const float* dt_bias, void* g_out, void* beta_out, int heads,
                                 qh_stream_t stream);

/* replaces launch_rmsnorm_gated_decode, fused_kernels.cu:956-965 (main.py:226-229) */
void launch_rmsnorm_gated_decode(const void* core, const void* z, const void* weight, void* out,
                                 int heads, int head_dim, float eps, qh_stream_t stream);

/* replaces launch_delta_rule_decode, fused_kernels.cu:967-979 (main.py:231-240) */
void launch_delta_rule_decode(const void* q, const void* k, const void* v, const void* g,
                              const void* beta, void* state, void* output, int n_heads,
                              int head_dim, qh_stream_t stream);

/* ========================= 2. native entry points (fp32 scales) ============ */

/* Last error message of the calling thread (no reference counterpart: the
 * reference kernels have no error channel). */
const char* qh_last_error(void);
void qh_clear_error(void);
int qh_abi_version(void);

/* Grouped block-scaled GEMV, up to 4 segments sharing x (generalises
 * launch_gemv_v4_extern / launch_linear_in_proj4 / launch_fused_qkv).
 * Prologue: x := bf16(x + x2) if x2; x := (1+w) RMSNorm(x) if norm_w.
 * Epilogue (nseg == 1): y := bf16(res + bf16(Wx)), res = res1 or bf16(res1+res2).
 * scales_bf16 selects bf16 scale_inv (reference format) instead of fp32. */
int qh_gemv_e4m3(const void* x, const void* x2, const float* norm_w, float eps, int K,
                 const void* res1, const void* res2, int nseg, const void* w0, const void* s0,
                 void* y0, int n0, int kb0, const void* w1, const void* s1, void* y1, int n1,
                 int kb1, const void* w2, const void* s2, void* y2, int n2, int kb2,
                 const void* w3, const void* s3, void* y3, int n3, int kb3, int scales_bf16,
                 qh_stream_t stream);

/* Paired gate/up GEMV, optional add + (1+w) RMSNorm prologue, SiLU(g)*u
 * epilogue on fp32 accumulators (fused_kernels.cu:398-479 semantics). */
int qh_mlp_gate_up(const void* x, const void* x2, const float* norm_w, float eps, int K,
                   const void* w_g, const void* s_g, const void* w_u, const void* s_u, int N,
                   int kb, void* m_out, void* g_out, void* u_out, int scales_bf16,
                   qh_stream_t stream);

/* Decode MLP block: h2 = bf16(h + o); out = bf16(h2 + down(silu(gate)*up of
 * RMSNorm(h2))) (layer_post_o_fp8_mlp semantics, fp32 scales). */
int qh_mlp_decode(const void* h, const void* o, const float* norm_w, float eps, int H,
                  const void* w_g, const void* s_g, const void* w_u, const void* s_u, int I,
                  int kb_gu, const void* w_d, const void* s_d, int kb_d, void* m_buf, void* out,
                  int scales_bf16, qh_stream_t stream);

/* (1+w) RMSNorm of `rows` rows of D (out may equal x). */
int qh_rmsnorm(const void* x, const float* w, void* out, int rows, int D, float eps,
               qh_stream_t stream);

/* Residual add + (1+w) RMSNorm of `rows` rows of D: h = bf16(h + o) in place,
 * out = bf16(h * rsqrt(mean(h^2) + eps) * (1 + w)); out must not alias h or o.
 * No reference counterpart: it fuses elem_add_kernel (fused_kernels.cu:553-559)
 * and the (1+w) RMSNorm (fused_kernels.cu:489-547) that main.py's prefill runs
 * back to back after every output projection (main.py:1550-1566). */
int qh_add_rmsnorm(void* h, const void* o, const float* w, void* out, int rows, int D, float eps,
                   qh_stream_t stream);

/* Scratch bytes for qh_attn_decode with nsplit > 1.  Layout (4-byte words):
 * group arrival counters [n_kv][8], then the split records
 * [n_kv][nsplit][8][head_dim + 2] and, above 8 splits, the level-2 records
 * [n_kv][8][8][head_dim + 2] of the two-level merge.  The counters must be
 * zero before the first call; the kernel returns them to zero itself. */
size_t qh_attn_scratch_bytes(int n_kv_heads, int nsplit, int head_dim);

/* Full-attention decode (layer_mid_attn + the sigmoid output gate of
 * main.py:1059): q/k head RMSNorm, partial RoPE, KV write, split-K GQA
 * attention.  Position t = *pos_dev (device) if pos_dev else pos. */
int qh_attn_decode(const void* q, int q_stride, const void* gate, int gate_stride,
                   const void* k_new, const void* v_new, const float* q_norm_w,
                   const float* k_norm_w, const float* cos_t, const float* sin_t, void* k_cache,
                   void* v_cache, int max_seq, int head_dim, int rot, int n_heads, int n_kv,
                   const int* pos_dev, int pos, int nsplit, void* scratch, unsigned* counters,
                   void* out, float eps, qh_stream_t stream);

/* Allocation-free variant of qh_attn_decode, same arguments without scratch
 * and counters.  No counterpart in the reference; it is for callers that
 * cannot allocate (code under HIP graph capture, serving loops that forbid
 * hipMalloc): the split partials and arrival counters live in a fixed
 * library array (8 MiB + 2304 bytes per GPU, held until the process ends).
 * Limits: n_kv <= 64, nsplit 1..64, n_heads / n_kv <= 8 and
 * qh_attn_scratch_bytes(n_kv, nsplit, head_dim) <= 8 MiB (records are laid
 * out for up to 8 query heads per KV head; at head_dim 256, 16 KV heads take
 * up to 55 splits and 8 KV heads all 64); larger shapes return -1.  The first call on a device looks up the
 * array's address (make it outside graph capture).  Every call on one GPU
 * shares the array: calls that overlap on one GPU race. */
int qh_attn_decode_noalloc(const void* q, int q_stride, const void* gate, int gate_stride,
                           const void* k_new, const void* v_new, const float* q_norm_w,
                           const float* k_norm_w, const float* cos_t, const float* sin_t,
                           void* k_cache, void* v_cache, int max_seq, int head_dim, int rot,
                           int n_heads, int n_kv, const int* pos_dev, int pos, int nsplit,
                           void* out, float eps, qh_stream_t stream);

/* GatedDeltaNet decode step: causal conv update (4-slot ring indexed by
 * position), gates, l2norm, delta rule (state in place), gated RMSNorm
 * (main.py:1064-1162 with launch_delta_rule_decode semantics).  `core` is an
 * fp32 scratch of Hv*dv floats; `counters` Hv zero-initialised uints. */
int qh_gdn_decode(const void* mixed, const void* a, const void* b, const void* z,
                  void* conv_ring, const void* conv_w, const float* A_log, const float* dt_bias,
                  const void* norm_w, float* state, void* core, void* out, unsigned* counters,
                  const int* pos_dev, int pos, int Hk, int Hv, int dk, int dv, float eps,
                  qh_stream_t stream);

/* Measurement helper with no counterpart in the reference: reads `bytes`
 * bytes at src (16-byte aligned, a non-zero multiple of 16, at most 2^31) in one launch of
 * min(out_len, 4 x CUs) workgroups with 16-byte loads, each wave streaming a
 * contiguous share as the GEMVs' waves stream their rows, and writes one XOR
 * checksum of 32-bit words per workgroup to out.  The XOR of those checksums
 * is the XOR of all words.  Its time is the plain-read floor that bench.py
 * sets the decode kernels' times against. */
int qh_read_stream(const void* src, size_t bytes, unsigned* out, int out_len, qh_stream_t stream);

/* Scratch bytes for qh_lm_head_argmax. */
size_t qh_lm_head_scratch_bytes(int N);

/* bf16 lm_head GEMV (F.linear, main.py:1600-1601) with the fused final RMSNorm
 * and greedy argmax (lowest index on ties); optional token history, position
 * increment and next-token embedding gather. */
int qh_lm_head_argmax(const void* x, const float* norm_w, float eps, int K, const void* w, int N,
                      void* logits, void* scratch, unsigned* counter, int64_t* tok_out,
                      int64_t* tok_hist, int hist_len, int* pos_dev, const void* embed,
                      void* embed_out, qh_stream_t stream);

/* Workspace bytes for qh_sample_top_p over a V-entry vocabulary. */
size_t qh_sample_workspace_size(int V);

/* replaces top_p_sample, main.py:49-87 (called at main.py:1726-1727): nucleus
 * sampling of one bf16 logits row entirely on the device.  temperature > 0
 * scales the logits; rep_penalty > 1 penalises the distinct ids of the window
 * hist[max(lo, p - window) .. p), p = *pos_dev + pos_offset (pos when pos_dev
 * is null), lo = *lo_dev (0 when null), window <= 64, slots clipped to
 * [0, hist_len) (hist_len > 0 when hist is given); top-min(2000, V)
 * candidates normalised against the full vocabulary, full-softmax fallback
 * when their mass is below top_p, top-p cut, one draw (SplitMix64 of seed and
 * *counter, which advances by one).  Writes *tok_out, hist[p] when hist is
 * given, and the token's row of embed [V, D] into h when embed is given.
 * info (optional, 16 int64): cut key, kept at that key, kept count, fallback
 * flag, kept mass (2^-40 units), draw bits, drawn key, rank, top-k mass, max,
 * Z, log-partition (fp32 bits), token, counter used, window size.
 * ws: qh_sample_workspace_size(V) bytes, 256-byte aligned, zeroed once (its
 * arrival counters reset themselves); calls sharing one workspace must not
 * overlap. */
int qh_sample_top_p(const void* logits, int V, float temperature, float top_p, float rep_penalty,
                    int64_t* hist, int hist_len, const int* pos_dev, int pos, int pos_offset,
                    const int* lo_dev,
                    int window, uint64_t seed, uint64_t* counter, void* ws, int64_t* tok_out,
                    const void* embed, void* h, int D, int64_t* info, qh_stream_t stream);

/* Embedding row gather (F.embedding, main.py:1587); ids outside [0, vocab)
 * give a zero row. */
int qh_embed(const void* table, const int64_t* ids, void* out, int n, int K, int vocab,
             qh_stream_t stream);

/* bf16 elementwise add (elem_add_kernel, fused_kernels.cu:553-559). */
int qh_add_bf16(const void* a, const void* b, void* out, int n, qh_stream_t stream);

/* GatedDeltaNet gates (launch_prepare_linear_gates semantics, torch softplus). */
int qh_linear_gates(const void* a, const void* b, const float* A_log, const float* dt_bias,
                    float* g_out, void* beta_out, int heads, qh_stream_t stream);

/* Gated RMSNorm per head; bf16_steps=1 follows main.py:1152-1158, 0 the
 * fused kernel fused_kernels.cu:592-618. */
int qh_gated_rmsnorm(const void* core, const void* z, const void* w, void* out, int heads,
                     int head_dim, float eps, int bf16_steps, qh_stream_t stream);

/* GatedDeltaNet decode step up to the bf16 core [Hv*dv] (no gated norm): one
 * wave per value head and 8 value columns, conv ring and state updated in
 * place.  No counterpart in the reference, whose delta_rule_decode_kernel
 * (fused_kernels.cu:623-684) is followed by the gated norm as its own step;
 * pair it with qh_gemv_e4m3_gated.  dk = dv = 128, Hv % 8 == 0. */
int qh_gdn_decode_core(const void* mixed, const void* a, const void* b, void* conv_ring,
                       const void* conv_w, const float* A_log, const float* dt_bias, float* state,
                       void* core, const int* pos_dev, int pos, int Hk, int Hv, int dk, int dv,
                       qh_stream_t stream);

/* Single-segment E4M3 GEMV whose activation is the per-head gated RMSNorm of
 * core with gate z (main.py:1152-1158, head dim d = 128), optional residual
 * res.  No counterpart in the reference, which normalises and then runs
 * launch_gemv_v4_extern.  K % 512 == 0, 128x128 block scales. */
int qh_gemv_e4m3_gated(const void* core, const void* z, const void* norm_w, int d, float eps, int K,
                       const void* res, const void* w, const void* s, void* y, int n, int kb,
                       int scales_bf16, qh_stream_t stream);

/* Workspace bytes for qh_gemm_e4m3 / qh_gemm_e4m3_grouped /
 * qh_gemm_e4m3_add_rmsnorm (a fixed 16 MiB of split-K partials, whatever M and
 * K).  The workspace is optional: with ws null the GEMM does not split K.  A
 * non-null ws must come with ws_bytes >= this size and be 256-byte aligned, or
 * the call fails before any launch; no plan puts more partials in it than
 * ws_bytes.  Calls sharing a workspace must not overlap. */
size_t qh_gemm_workspace_size(int M, int K);

/* Prefill GEMM on the fp8 matrix cores (fp8_gemm_batch semantics). */
int qh_gemm_e4m3(const void* x, const void* w, const void* s, void* y, int M, int N, int K,
                 int kb, int scales_bf16, void* ws, size_t ws_bytes, qh_stream_t stream);

/* Output projection + residual add + (1+w) RMSNorm, the batch prefill's step
 * after o_proj / out_proj / down: o = bf16(x . deq(W)^T) (M x N scratch, not
 * written when the split-K finish fuses all three), h = bf16(h + o) in place,
 * hn = bf16(h * rsqrt(mean(h^2) + eps) * (1 + norm_w)); norm_w null: the add
 * only.  x, o, h, hn distinct; ws as qh_gemm_e4m3 (null: no split).  No
 * reference counterpart: main.py:1550-1566 runs fp8_gemm_batch, the add and
 * the norm as separate steps. */
int qh_gemm_e4m3_add_rmsnorm(const void* x, const void* w, const void* s, void* o, int M, int N, int K,
                             int kb, int scales_bf16, void* h, const float* norm_w, void* hn, float eps,
                             void* ws, size_t ws_bytes, qh_stream_t stream);

/* Grouped prefill GEMM; no counterpart in the reference, which runs each
 * projection as its own fp8_gemm_batch (main.py:262-269).  Up to 4 projections
 * of one activation x [M, K] (segment t: y_t [M, n_t] = bf16(x . deq(w_t)^T),
 * scale mode kb_t) in one launch; ws as for qh_gemm_e4m3 (optional). */
int qh_gemm_e4m3_grouped(const void* x, int M, int K, int nseg, const void* w0, const void* s0,
                         void* y0, int n0, int kb0, const void* w1, const void* s1, void* y1,
                         int n1, int kb1, const void* w2, const void* s2, void* y2, int n2,
                         int kb2, const void* w3, const void* s3, void* y3, int n3, int kb3,
                         int scales_bf16, void* ws, size_t ws_bytes, qh_stream_t stream);

/* ---- batch prefill pieces (the reference runs these in torch) ---------- */

/* q/k head (1+w) RMSNorm + partial RoPE (q kept fp32, k cached bf16) and the
 * KV-cache write for M tokens at positions past.. (replaces main.py:1034-1043). */
int qh_attn_prep(const void* q_all, const void* k, const void* v, const float* q_norm_w,
                 const float* k_norm_w, const float* cos_t, const float* sin_t, float* q_out,
                 void* k_cache, void* v_cache, int M, int Hq, int Hkv, int D, int rot, int past,
                 int max_seq, float eps, qh_stream_t stream);

/* Causal GQA attention (fp32 softmax) with the bf16 sigmoid output gate for M
 * query tokens (replaces main.py:1043-1059). */
int qh_attn_prefill(const float* q, const void* gate, int gate_mstride, int gate_hstride,
                    const void* k_cache, const void* v_cache, void* out, int M, int Hq, int Hkv,
                    int D, int past, int max_seq, qh_stream_t stream);

/* GatedDeltaNet prefill front: causal conv + SiLU over the sequence (conv ring
 * updated), bf16-step l2norm of q/k, per-token gates (replaces
 * main.py:1097-1128). */
int qh_gdn_prep(const void* mixed, void* conv_ring, const void* conv_w, const void* a,
                const void* b, const float* A_log, const float* dt_bias, void* y, void* qn,
                void* kn, float* g, void* beta, int M, int Hk, int Hv, int dk, int dv, int past,
                qh_stream_t stream);

/* GatedDeltaNet prefill scan: recurrent gated delta rule from the stored
 * state (updated in place) and the gated RMSNorm per token and head (replaces
 * main.py:1139-1158, transformers torch_chunk_gated_delta_rule). */
int qh_gdn_scan(const void* qn, const void* kn, const void* y, const float* g, const void* beta,
                const void* z, const void* norm_w, float* state, void* out, int M, int Hk, int Hv,
                int dk, int dv, float eps, qh_stream_t stream);

/* Workspace bytes of qh_gdn_chunk for M tokens and Hv value heads
 * (Hv * ceil(M / 64) * 99328). */
size_t qh_gdn_chunk_workspace_size(int M, int Hv);

/* qh_gdn_scan in the chunked (WY) form the reference's prefill uses
 * (main.py:1139-1149, transformers torch_chunk_gated_delta_rule, chunk 64)
 * on the bf16 matrix cores: same operands and results (dk = dv = 128), plus a
 * device workspace of qh_gdn_chunk_workspace_size(M, Hv) bytes. */
int qh_gdn_chunk(const void* qn, const void* kn, const void* y, const float* g, const void* beta,
                 const void* z, const void* norm_w, float* state, void* out, int M, int Hk, int Hv,
                 int dk, int dv, float eps, void* ws, size_t ws_bytes, qh_stream_t stream);

/* m = bf16(bf16(silu(g)) * u), the M > 1 MLP glue (replaces main.py:1213-1215). */
int qh_silu_mul(const void* g, const void* u, void* m, size_t n, qh_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* QWEN35_FP8_HIP_H */
