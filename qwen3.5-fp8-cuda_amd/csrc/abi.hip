// C-ABI of libqwen35_fp8_hip.so.
//
// Two families of entry points, all declared in include/qwen35_fp8_hip.h:
//   1. The reference engine's ctypes ABI (same names, argument order and
//      meaning as qwen3_infer/csrc/fused_kernels.cu:940-1356 and
//      fp8_kernels.cu:68-91): bf16 scale_inv, `void` return, stream last.
//      Invalid arguments launch nothing and record a message for
//      qh_last_error() (the reference silently launches garbage or no-ops).
//   2. Native `qh_*` entry points used by this framework's host: fp32
//      scale_inv, device-resident positions for HIP-graph replay, fused
//      epilogues; they return 0 on success and -1 with qh_last_error() set.
// Every buffer is caller-owned device memory; the library allocates nothing.
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>

#include "qh_attn.h"
#include "qh_gdn.h"
#include "qh_gemm.h"
#include "qh_prefill.h"
#include "qh_sample.h"
#include "qh_kernels.h"
#include "qh_norm.h"

#define QH_EXPORT extern "C" __attribute__((visibility("default")))

namespace {
thread_local char g_err[512] = "";

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    qh_set_error("%s: launch failed: %s", what, hipGetErrorString(e));
    return -1;
  }
  return 0;
}

bool k_ok(int K, const char* what) {
  if (K <= 0 || (K % 8) != 0) {
    qh_set_error("%s: K=%d must be a positive multiple of 8", what, K);
    return false;
  }
  return true;
}

QhGemvSeg seg(const void* w, const void* s, void* y, int n, int kb) {
  QhGemvSeg g;
  g.w = (const uint8_t*)w;
  g.s = s;
  g.y = (uint16_t*)y;
  g.n = n;
  g.kb = kb;
  g.qgate_d = 0;
  return g;
}

QhGemvParams gemv_params(const void* x, int K) {
  QhGemvParams p;
  memset(&p, 0, sizeof(p));
  p.x = (const uint16_t*)x;
  p.K = K;
  p.eps = 1e-6f;
  return p;
}

int run_gemv(QhGemvParams& p, bool bf16_scales, const char* what, hipStream_t st) {
  if (!k_ok(p.K, what)) return -1;
  for (int i = 0; i < p.nseg; ++i) {
    if (p.seg[i].n < 0 || (p.seg[i].n > 0 && (!p.seg[i].w || !p.seg[i].s || !p.seg[i].y))) {
      qh_set_error("%s: segment %d has null pointers or negative rows", what, i);
      return -1;
    }
  }
  if (qh_launch_gemv(p, bf16_scales, st) != 0) return -1;
  return check_launch(what);
}

}  // namespace

void qh_set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

// ============================================================================
// Library info
// ============================================================================
QH_EXPORT const char* qh_last_error(void) { return g_err; }
QH_EXPORT void qh_clear_error(void) { g_err[0] = '\0'; }
QH_EXPORT int qh_abi_version(void) { return 1; }

// ============================================================================
// Reference ABI (bf16 scales)
// ============================================================================
QH_EXPORT void launch_gemv_v4_extern(const void* x, const void* w, const void* s, void* y, int N,
                                     int K, int K_blk, hipStream_t stream) {
  QhGemvParams p = gemv_params(x, K);
  p.nseg = 1;
  p.seg[0] = seg(w, s, y, N, K_blk);
  run_gemv(p, true, "launch_gemv_v4_extern", stream);
}

QH_EXPORT void launch_gemv_v3_extern(const void* x, const void* w, const void* s, void* y, int N,
                                     int K, int K_blk, hipStream_t stream) {
  launch_gemv_v4_extern(x, w, s, y, N, K, K_blk, stream);
}

QH_EXPORT void launch_linear_in_proj4(const void* x, const void* w0, const void* s0, void* y0,
                                      int n0, int kb0, const void* w1, const void* s1, void* y1,
                                      int n1, int kb1, const void* w2, const void* s2, void* y2,
                                      int n2, int kb2, const void* w3, const void* s3, void* y3,
                                      int n3, int kb3, int K, hipStream_t stream) {
  QhGemvParams p = gemv_params(x, K);
  p.nseg = 4;
  p.seg[0] = seg(w0, s0, y0, n0, kb0);
  p.seg[1] = seg(w1, s1, y1, n1, kb1);
  p.seg[2] = seg(w2, s2, y2, n2, kb2);
  p.seg[3] = seg(w3, s3, y3, n3, kb3);
  run_gemv(p, true, "launch_linear_in_proj4", stream);
}

QH_EXPORT void launch_fused_qkv(const void* x, const void* w_q, const void* w_k, const void* w_v,
                                const void* s_q, const void* s_k, const void* s_v, void* q_out,
                                void* k_out, void* v_out, int K, int N_q, int N_k, int N_v,
                                int K_blk, int N_q_blk, int N_k_blk, int N_v_blk,
                                hipStream_t stream) {
  (void)N_q_blk; (void)N_k_blk; (void)N_v_blk;  // unused by the reference kernel too
  QhGemvParams p = gemv_params(x, K);
  p.nseg = 3;
  p.seg[0] = seg(w_q, s_q, q_out, N_q, K_blk);
  p.seg[1] = seg(w_k, s_k, k_out, N_k, K_blk);
  p.seg[2] = seg(w_v, s_v, v_out, N_v, K_blk);
  run_gemv(p, true, "launch_fused_qkv", stream);
}

QH_EXPORT void launch_fused_gate_up(const void* x, const void* w_gate, const void* w_up,
                                    const void* s_gate, const void* s_up, void* gate_out,
                                    void* up_out, int K, int N_gate, int N_up, int K_blk,
                                    int N_gate_blk, int N_up_blk, hipStream_t stream) {
  (void)N_gate_blk; (void)N_up_blk;
  QhGemvParams p = gemv_params(x, K);
  p.nseg = 2;
  p.seg[0] = seg(w_gate, s_gate, gate_out, N_gate, K_blk);
  p.seg[1] = seg(w_up, s_up, up_out, N_up, K_blk);
  run_gemv(p, true, "launch_fused_gate_up", stream);
}

QH_EXPORT void launch_rmsnorm_ip(void* x, const void* weight, int N, int D, float eps,
                                 hipStream_t stream) {
  if (N < 0 || D <= 0) {
    qh_set_error("launch_rmsnorm_ip: bad shape N=%d D=%d", N, D);
    return;
  }
  qh_launch_rmsnorm_rows(x, (const float*)weight, x, N, D, eps, stream);
  check_launch("launch_rmsnorm_ip");
}

QH_EXPORT void launch_rmsnorm_out(const void* x, const void* weight, void* out, int N, int D,
                                  float eps, hipStream_t stream) {
  if (N < 0 || D <= 0) {
    qh_set_error("launch_rmsnorm_out: bad shape N=%d D=%d", N, D);
    return;
  }
  qh_launch_rmsnorm_rows(x, (const float*)weight, out, N, D, eps, stream);
  check_launch("launch_rmsnorm_out");
}

static void attn_only(const char* what, const void* q, const void* k_cache, const void* v_cache,
                      void* output, int seq_len, int max_seq_len, int head_dim, int n_heads,
                      int n_kv_heads, hipStream_t stream) {
  QhAttnParams a;
  memset(&a, 0, sizeof(a));
  a.q = (const uint16_t*)q;
  a.q_stride = head_dim;
  a.k_cache = (uint16_t*)k_cache;
  a.v_cache = (uint16_t*)v_cache;
  a.max_seq = max_seq_len;
  a.n_heads = n_heads;
  a.n_kv = n_kv_heads;
  a.rope_pos = 0;
  a.slot = 0;  // no new token (k_new is null): nothing is written
  a.total = seq_len;
  a.nsplit = 1;
  a.out = (uint16_t*)output;
  a.eps = 1e-6f;
  if (seq_len < 1 || seq_len > max_seq_len) {
    qh_set_error("%s: seq_len=%d out of range (max %d)", what, seq_len, max_seq_len);
    return;
  }
  if (qh_launch_attn(a, head_dim, stream) == 0) check_launch(what);
}

QH_EXPORT void launch_fused_attn(const void* q, const void* k_cache, const void* v_cache,
                                 void* output, int seq_len, int max_seq_len, int head_dim,
                                 int n_heads, int n_kv_heads, hipStream_t stream) {
  attn_only("launch_fused_attn", q, k_cache, v_cache, output, seq_len, max_seq_len, head_dim,
            n_heads, n_kv_heads, stream);
}

QH_EXPORT void launch_fused_attn_v2(const void* q, const void* k_cache, const void* v_cache,
                                    void* output, int seq_len, int max_seq_len, int head_dim,
                                    int n_heads, int n_kv_heads, hipStream_t stream) {
  attn_only("launch_fused_attn_v2", q, k_cache, v_cache, output, seq_len, max_seq_len, head_dim,
            n_heads, n_kv_heads, stream);
}

// Q/gate layout of layer_pre_attn's q output.  The checkpoint's q_proj rows
// are per-head [q_h | gate_h] (main.py:1001), but the reference's opt-in fused
// full-attention path reads q_buf as [all q heads | all gates]
// (main.py:1292-1294).  With a head dim d set here (or by the environment
// variable QH_QGATE_HEAD_DIM, for an unmodified main.py), layer_pre_attn
// stores q de-interleaved so that split is the right one; 0 keeps the
// checkpoint order, like the reference kernel.
static int g_qgate_d = -1;  // -1: take QH_QGATE_HEAD_DIM
static int qgate_head_dim() {
  if (g_qgate_d >= 0) return g_qgate_d;
  const char* e = getenv("QH_QGATE_HEAD_DIM");
  return e ? atoi(e) : 0;
}

QH_EXPORT int qh_set_qgate_head_dim(int d) {
  if (d < -1) {
    qh_set_error("qh_set_qgate_head_dim: d=%d (use -1, 0 or a head dim)", d);
    return -1;
  }
  g_qgate_d = d;
  return 0;
}

QH_EXPORT void layer_pre_attn(const void* hidden, const float* norm_weight, const void* w_q,
                              const void* s_q, int N_q, int N_q_blk, const void* w_k,
                              const void* s_k, int N_k, int N_k_blk, const void* w_v,
                              const void* s_v, int N_v, int N_v_blk, void* q_out, void* k_out,
                              void* v_out, void* norm_ws, int h_dim, int K_blk,
                              hipStream_t stream) {
  (void)N_q_blk; (void)N_k_blk; (void)N_v_blk;
  const int d = qgate_head_dim();
  if (d > 0 && (N_q % (2 * d)) != 0) {
    qh_set_error("layer_pre_attn: N_q=%d is not a whole number of [q | gate] heads of 2 x %d", N_q,
                 d);
    return;
  }
  qh_launch_rmsnorm_rows(hidden, norm_weight, norm_ws, 1, h_dim, 1e-6f, stream);
  QhGemvParams p = gemv_params(norm_ws, h_dim);
  p.nseg = 3;
  p.seg[0] = seg(w_q, s_q, q_out, N_q, K_blk);
  p.seg[0].qgate_d = d > 0 ? d : 0;
  p.seg[1] = seg(w_k, s_k, k_out, N_k, K_blk);
  p.seg[2] = seg(w_v, s_v, v_out, N_v, K_blk);
  run_gemv(p, true, "layer_pre_attn", stream);
}

QH_EXPORT void layer_post_o_fp8_mlp(const void* hidden, const void* o_out,
                                    const float* norm_weight, const void* w_g, const void* s_g,
                                    int N_g, const void* w_u, const void* s_u, int N_u,
                                    const void* w_d, const void* s_d, int N_d, void* output,
                                    void* ws, void* gate_buf, void* up_buf, void* silu_buf,
                                    int h_dim, int K_blk_gu, int K_blk_d, hipStream_t stream) {
  (void)ws;
  if (N_g != N_u || !k_ok(h_dim, "layer_post_o_fp8_mlp") || !k_ok(N_g, "layer_post_o_fp8_mlp"))
    return;
  QhMlpParams m;
  memset(&m, 0, sizeof(m));
  m.x = (const uint16_t*)hidden;
  m.x2 = (const uint16_t*)o_out;
  m.norm_w = norm_weight;
  m.eps = 1e-6f;
  m.K = h_dim;
  m.wg = (const uint8_t*)w_g;
  m.sg = s_g;
  m.wu = (const uint8_t*)w_u;
  m.su = s_u;
  m.N = N_g;
  m.kb = K_blk_gu;
  m.m_out = (uint16_t*)silu_buf;
  m.g_out = (uint16_t*)gate_buf;
  m.u_out = (uint16_t*)up_buf;
  if (qh_launch_mlp(m, true, stream) != 0 || check_launch("layer_post_o_fp8_mlp") != 0) return;
  QhGemvParams p = gemv_params(silu_buf, N_g);
  p.nseg = 1;
  p.seg[0] = seg(w_d, s_d, output, N_d, K_blk_d);
  p.res1 = (const uint16_t*)hidden;
  p.res2 = (const uint16_t*)o_out;
  run_gemv(p, true, "layer_post_o_fp8_mlp", stream);
}

QH_EXPORT void layer_post_attn(const void* hidden, const void* attn_out, const void* w_o,
                               const void* s_o, int N_o, int N_o_blk, const float* norm_weight,
                               const void* w_g, const void* s_g, int N_g, int N_g_blk,
                               const void* w_u, const void* s_u, int N_u, int N_u_blk,
                               const void* w_d, const void* s_d, int N_d, int N_d_blk,
                               void* output, void* ws, void* gate_buf, void* up_buf,
                               void* silu_buf, int h_dim, int attn_dim, int K_blk_o, int K_blk_gu,
                               int K_blk_d, hipStream_t stream) {
  (void)N_o_blk; (void)N_g_blk; (void)N_u_blk; (void)N_d_blk; (void)ws;
  if (N_o != h_dim) {
    qh_set_error("layer_post_attn: N_o=%d must equal h_dim=%d", N_o, h_dim);
    return;
  }
  // output = bf16(hidden + bf16(W_o attn_out))
  QhGemvParams p = gemv_params(attn_out, attn_dim);
  p.nseg = 1;
  p.seg[0] = seg(w_o, s_o, output, N_o, K_blk_o);
  p.res1 = (const uint16_t*)hidden;
  if (run_gemv(p, true, "layer_post_attn", stream) != 0) return;
  if (N_g != N_u || !k_ok(N_g, "layer_post_attn")) return;
  QhMlpParams m;
  memset(&m, 0, sizeof(m));
  m.x = (const uint16_t*)output;
  m.norm_w = norm_weight;
  m.eps = 1e-6f;
  m.K = h_dim;
  m.wg = (const uint8_t*)w_g;
  m.sg = s_g;
  m.wu = (const uint8_t*)w_u;
  m.su = s_u;
  m.N = N_g;
  m.kb = K_blk_gu;
  m.m_out = (uint16_t*)silu_buf;
  m.g_out = (uint16_t*)gate_buf;
  m.u_out = (uint16_t*)up_buf;
  if (qh_launch_mlp(m, true, stream) != 0 || check_launch("layer_post_attn") != 0) return;
  QhGemvParams d = gemv_params(silu_buf, N_g);
  d.nseg = 1;
  d.seg[0] = seg(w_d, s_d, output, N_d, K_blk_d);
  d.res1 = (const uint16_t*)output;
  run_gemv(d, true, "layer_post_attn", stream);
}

QH_EXPORT void layer_mid_attn(void* q_buf, void* k_buf, const void* v_buf, void* attn_out,
                              const float* q_norm_weight, const float* k_norm_weight,
                              const float* cos_table, const float* sin_table, void* k_cache,
                              void* v_cache, int pos, int past_len, int total_seq,
                              int max_seq_len, int head_dim, int rotary_dim, int n_heads,
                              int n_kv_heads, hipStream_t stream) {
  QhAttnParams a;
  memset(&a, 0, sizeof(a));
  a.q = (const uint16_t*)q_buf;
  a.q_stride = head_dim;
  a.k_new = (const uint16_t*)k_buf;
  a.v_new = (const uint16_t*)v_buf;
  a.q_wb = (uint16_t*)q_buf;
  a.k_wb = (uint16_t*)k_buf;
  a.q_norm_w = q_norm_weight;
  a.k_norm_w = k_norm_weight;
  a.cos_t = cos_table;
  a.sin_t = sin_table;
  a.k_cache = (uint16_t*)k_cache;
  a.v_cache = (uint16_t*)v_cache;
  a.max_seq = max_seq_len;
  a.rot = rotary_dim;
  a.n_heads = n_heads;
  a.n_kv = n_kv_heads;
  a.rope_pos = pos;
  a.slot = past_len;
  a.total = total_seq;
  a.nsplit = 1;
  a.out = (uint16_t*)attn_out;
  a.eps = 1e-6f;
  if (qh_launch_attn(a, head_dim, stream) == 0) check_launch("layer_mid_attn");
}

QH_EXPORT void launch_prepare_linear_gates(const void* a, const void* beta_in, const float* A_log,
                                           const float* dt_bias, void* g_out, void* beta_out,
                                           int heads, hipStream_t stream) {
  qh_launch_linear_gates(a, beta_in, A_log, dt_bias, (float*)g_out, beta_out, heads, stream);
  check_launch("launch_prepare_linear_gates");
}

QH_EXPORT void launch_rmsnorm_gated_decode(const void* core, const void* z, const void* weight,
                                           void* out, int heads, int head_dim, float eps,
                                           hipStream_t stream) {
  if (head_dim <= 0 || head_dim > 256) {
    qh_set_error("launch_rmsnorm_gated_decode: head_dim=%d unsupported (<= 256)", head_dim);
    return;
  }
  qh_launch_gated_rmsnorm(core, z, weight, out, heads, head_dim, eps, 0, stream);
  check_launch("launch_rmsnorm_gated_decode");
}

QH_EXPORT void launch_delta_rule_decode(const void* q, const void* k, const void* v, const void* g,
                                        const void* beta, void* state, void* output, int n_heads,
                                        int head_dim, hipStream_t stream) {
  if (qh_launch_delta_rule(q, k, v, (const float*)g, beta, (float*)state, output, n_heads,
                           head_dim, stream) == 0)
    check_launch("launch_delta_rule_decode");
}

QH_EXPORT void fp8_gemm_batch(const void* x_bf16, const void* w_fp8, const void* w_scale_bf16,
                              void* y_bf16, int M, int N, int K, int K_blocks,
                              hipStream_t stream) {
  if (M <= 0) return;
  if (!k_ok(K, "fp8_gemm_batch")) return;
  if (qh_launch_gemm_e4m3(x_bf16, w_fp8, w_scale_bf16, y_bf16, M, N, K, K_blocks, true, stream) == 0)
    check_launch("fp8_gemm_batch");
}

// ============================================================================
// Native entry points (fp32 scale_inv)
// ============================================================================
// Grouped block-scaled GEMV sharing one activation vector (up to 4 segments).
QH_EXPORT int qh_gemv_e4m3(const void* x, const void* x2, const float* norm_w, float eps, int K,
                           const void* res1, const void* res2, int nseg, const void* w0,
                           const void* s0, void* y0, int n0, int kb0, const void* w1,
                           const void* s1, void* y1, int n1, int kb1, const void* w2,
                           const void* s2, void* y2, int n2, int kb2, const void* w3,
                           const void* s3, void* y3, int n3, int kb3, int scales_bf16,
                           hipStream_t stream) {
  if (nseg < 1 || nseg > 4) {
    qh_set_error("qh_gemv_e4m3: nseg=%d must be 1..4", nseg);
    return -1;
  }
  QhGemvParams p = gemv_params(x, K);
  p.x2 = (const uint16_t*)x2;
  p.norm_w = norm_w;
  p.eps = eps;
  p.res1 = (const uint16_t*)res1;
  p.res2 = (const uint16_t*)res2;
  p.nseg = nseg;
  p.seg[0] = seg(w0, s0, y0, n0, kb0);
  p.seg[1] = seg(w1, s1, y1, n1, kb1);
  p.seg[2] = seg(w2, s2, y2, n2, kb2);
  p.seg[3] = seg(w3, s3, y3, n3, kb3);
  if ((res1 || res2) && nseg != 1) {
    qh_set_error("qh_gemv_e4m3: residual epilogue needs a single segment");
    return -1;
  }
  return run_gemv(p, scales_bf16 != 0, "qh_gemv_e4m3", stream);
}

// Paired gate/up GEMV with (1+w) RMSNorm prologue and SiLU(gate)*up epilogue.
QH_EXPORT int qh_mlp_gate_up(const void* x, const void* x2, const float* norm_w, float eps, int K,
                             const void* w_g, const void* s_g, const void* w_u, const void* s_u,
                             int N, int kb, void* m_out, void* g_out, void* u_out,
                             int scales_bf16, hipStream_t stream) {
  if (!k_ok(K, "qh_mlp_gate_up")) return -1;
  QhMlpParams m;
  memset(&m, 0, sizeof(m));
  m.x = (const uint16_t*)x;
  m.x2 = (const uint16_t*)x2;
  m.norm_w = norm_w;
  m.eps = eps;
  m.K = K;
  m.wg = (const uint8_t*)w_g;
  m.sg = s_g;
  m.wu = (const uint8_t*)w_u;
  m.su = s_u;
  m.N = N;
  m.kb = kb;
  m.m_out = (uint16_t*)m_out;
  m.g_out = (uint16_t*)g_out;
  m.u_out = (uint16_t*)u_out;
  if (qh_launch_mlp(m, scales_bf16 != 0, stream) != 0) return -1;
  return check_launch("qh_mlp_gate_up");
}

// Whole decode MLP: h2 = bf16(h + o) (o optional), m = silu(g)*u of
// RMSNorm(h2), out = bf16(h2 + bf16(W_d m)).
QH_EXPORT int qh_mlp_decode(const void* h, const void* o, const float* norm_w, float eps, int H,
                            const void* w_g, const void* s_g, const void* w_u, const void* s_u,
                            int I, int kb_gu, const void* w_d, const void* s_d, int kb_d,
                            void* m_buf, void* out, int scales_bf16, hipStream_t stream) {
  if (qh_mlp_gate_up(h, o, norm_w, eps, H, w_g, s_g, w_u, s_u, I, kb_gu, m_buf, nullptr, nullptr,
                     scales_bf16, stream) != 0)
    return -1;
  return qh_gemv_e4m3(m_buf, nullptr, nullptr, eps, I, h, o, 1, w_d, s_d, out, H, kb_d, nullptr,
                      nullptr, nullptr, 0, 0, nullptr, nullptr, nullptr, 0, 0, nullptr, nullptr,
                      nullptr, 0, 0, scales_bf16, stream);
}

QH_EXPORT int qh_rmsnorm(const void* x, const float* w, void* out, int rows, int D, float eps,
                         hipStream_t stream) {
  if (rows < 0 || D <= 0) {
    qh_set_error("qh_rmsnorm: bad shape rows=%d D=%d", rows, D);
    return -1;
  }
  qh_launch_rmsnorm_rows(x, w, out, rows, D, eps, stream);
  return check_launch("qh_rmsnorm");
}

QH_EXPORT int qh_add_rmsnorm(void* h, const void* o, const float* w, void* out, int rows, int D,
                             float eps, hipStream_t stream) {
  if (rows < 0 || D <= 0) {
    qh_set_error("qh_add_rmsnorm: bad shape rows=%d D=%d", rows, D);
    return -1;
  }
  if (rows > 0 && (!h || !o || !w || !out)) {
    qh_set_error("qh_add_rmsnorm: null pointer");
    return -1;
  }
  if (out == h || out == o) {
    qh_set_error("qh_add_rmsnorm: out must not alias h or o");
    return -1;
  }
  qh_launch_add_rmsnorm_rows(h, o, w, out, rows, D, eps, stream);
  return check_launch("qh_add_rmsnorm");
}

QH_EXPORT size_t qh_attn_scratch_bytes(int n_kv_heads, int nsplit, int head_dim) {
  return qh_attn_scratch_floats(n_kv_heads, nsplit, head_dim) * sizeof(float);
}

// Full-attention decode: q/k head norm, partial RoPE, KV-cache write, split-K
// GQA attention and the optional sigmoid output gate.  pos_dev (device int) or
// the host pos gives the token position t: RoPE at t, cache slot t, t+1 keys.
QH_EXPORT int qh_attn_decode(const void* q, int q_stride, const void* gate, int gate_stride,
                             const void* k_new, const void* v_new, const float* q_norm_w,
                             const float* k_norm_w, const float* cos_t, const float* sin_t,
                             void* k_cache, void* v_cache, int max_seq, int head_dim, int rot,
                             int n_heads, int n_kv, const int* pos_dev, int pos, int nsplit,
                             void* scratch, unsigned* counters, void* out, float eps,
                             hipStream_t stream) {
  QhAttnParams a;
  memset(&a, 0, sizeof(a));
  a.q = (const uint16_t*)q;
  a.q_stride = q_stride;
  a.gate = (const uint16_t*)gate;
  a.gate_stride = gate_stride;
  a.k_new = (const uint16_t*)k_new;
  a.v_new = (const uint16_t*)v_new;
  a.q_norm_w = q_norm_w;
  a.k_norm_w = k_norm_w;
  a.cos_t = cos_t;
  a.sin_t = sin_t;
  a.k_cache = (uint16_t*)k_cache;
  a.v_cache = (uint16_t*)v_cache;
  a.max_seq = max_seq;
  a.rot = rot;
  a.n_heads = n_heads;
  a.n_kv = n_kv;
  a.pos_dev = pos_dev;
  a.rope_pos = pos;
  a.slot = pos;
  a.total = pos + 1;
  a.nsplit = nsplit;
  // the scratch opens with the group counters [n_kv][8], then the records
  a.gcounters = (unsigned*)scratch;
  a.part = scratch ? (float*)scratch + (size_t)n_kv * 8 : nullptr;
  a.counters = counters;
  a.out = (uint16_t*)out;
  a.eps = eps;
  if (qh_launch_attn(a, head_dim, stream) != 0) return -1;
  return check_launch("qh_attn_decode");
}

QH_EXPORT int qh_gdn_decode(const void* mixed, const void* a, const void* b, const void* z,
                            void* conv_ring, const void* conv_w, const float* A_log,
                            const float* dt_bias, const void* norm_w, float* state, void* core,
                            void* out, unsigned* counters, const int* pos_dev, int pos, int Hk,
                            int Hv, int dk, int dv, float eps, hipStream_t stream) {
  QhGdnParams g;
  memset(&g, 0, sizeof(g));
  g.mixed = (const uint16_t*)mixed;
  g.a = (const uint16_t*)a;
  g.b = (const uint16_t*)b;
  g.z = (const uint16_t*)z;
  g.conv_ring = (uint16_t*)conv_ring;
  g.conv_w = (const uint16_t*)conv_w;
  g.A_log = A_log;
  g.dt_bias = dt_bias;
  g.norm_w = (const uint16_t*)norm_w;
  g.state = state;
  g.core = (float*)core;
  g.out = (uint16_t*)out;
  g.counters = counters;
  g.pos_dev = pos_dev;
  g.pos = pos;
  g.Hk = Hk;
  g.Hv = Hv;
  g.dk = dk;
  g.dv = dv;
  g.eps = eps;
  if (qh_launch_gdn_decode(g, stream) != 0) return -1;
  return check_launch("qh_gdn_decode");
}

// GatedDeltaNet decode step up to the bf16 core (no reference counterpart:
// the reference's delta_rule_decode_kernel, fused_kernels.cu:623-684, is
// followed by the gated norm as its own step).  One wave per value head and 8
// value columns; the gated RMSNorm is qh_gemv_e4m3_gated's prologue.
QH_EXPORT int qh_gdn_decode_core(const void* mixed, const void* a, const void* b, void* conv_ring,
                                 const void* conv_w, const float* A_log, const float* dt_bias,
                                 float* state, void* core, const int* pos_dev, int pos, int Hk,
                                 int Hv, int dk, int dv, hipStream_t stream) {
  if (!mixed || !a || !b || !conv_ring || !conv_w || !A_log || !dt_bias || !state || !core) {
    qh_set_error("qh_gdn_decode_core: null pointer argument");
    return -1;
  }
  QhGdnParams g;
  memset(&g, 0, sizeof(g));
  g.mixed = (const uint16_t*)mixed;
  g.a = (const uint16_t*)a;
  g.b = (const uint16_t*)b;
  g.conv_ring = (uint16_t*)conv_ring;
  g.conv_w = (const uint16_t*)conv_w;
  g.A_log = A_log;
  g.dt_bias = dt_bias;
  g.state = state;
  g.out = (uint16_t*)core;
  g.pos_dev = pos_dev;
  g.pos = pos;
  g.Hk = Hk;
  g.Hv = Hv;
  g.dk = dk;
  g.dv = dv;
  if (qh_launch_gdn_decode_core(g, stream) != 0) return -1;
  return check_launch("qh_gdn_decode_core");
}

// Single-segment E4M3 GEMV whose activation is the GatedDeltaNet gated
// RMSNorm of core with gate z (main.py:1152-1158: per head of d = 128,
// bf16(bf16(bf16(core * rs) * w) * bf16(silu(z)))), optional residual res.
// No reference counterpart (the reference normalises, then runs
// launch_gemv_v4_extern).  Fast-path shapes: K % 512 == 0, 128x128 scales.
QH_EXPORT int qh_gemv_e4m3_gated(const void* core, const void* z, const void* norm_w, int d,
                                 float eps, int K, const void* res, const void* w, const void* s,
                                 void* y, int n, int kb, int scales_bf16, hipStream_t stream) {
  if (!core || !z || !norm_w) {
    qh_set_error("qh_gemv_e4m3_gated: null core, gate or norm weight");
    return -1;
  }
  QhGemvParams p = gemv_params(core, K);
  p.x2 = (const uint16_t*)z;
  p.gnorm_w = (const uint16_t*)norm_w;
  p.gnorm_d = d;
  p.eps = eps;
  p.res1 = (const uint16_t*)res;
  p.nseg = 1;
  p.seg[0] = seg(w, s, y, n, kb);
  return run_gemv(p, scales_bf16 != 0, "qh_gemv_e4m3_gated", stream);
}

// Plain read of `bytes` bytes (one XOR checksum per workgroup into out, at
// most out_len workgroups): the measured read floor.
QH_EXPORT int qh_read_stream(const void* src, size_t bytes, unsigned* out, int out_len, hipStream_t stream) {
  if (qh_launch_read_stream(src, bytes, out, out_len, stream) != 0) return -1;
  return check_launch("qh_read_stream");
}

QH_EXPORT size_t qh_lm_head_scratch_bytes(int N) {
  return (size_t)qh_lm_head_grid(N) * (sizeof(float) + sizeof(int));
}

// bf16 lm_head GEMV with fused final (1+w) RMSNorm and greedy argmax.  The
// last block writes the token (int64) to tok_out; with pos_dev it also stores
// it at tok_hist[*pos_dev] (when in range) and increments *pos_dev; with embed
// it copies embed[token] into embed_out for the next step.
QH_EXPORT int qh_lm_head_argmax(const void* x, const float* norm_w, float eps, int K,
                                const void* w, int N, void* logits, void* scratch,
                                unsigned* counter, int64_t* tok_out, int64_t* tok_hist,
                                int hist_len, int* pos_dev, const void* embed, void* embed_out,
                                hipStream_t stream) {
  if (!k_ok(K, "qh_lm_head_argmax")) return -1;
  if (N <= 0 || !scratch || !counter || !tok_out) {
    qh_set_error("qh_lm_head_argmax: N=%d, scratch/counter/tok_out required", N);
    return -1;
  }
  QhLmHeadParams p;
  memset(&p, 0, sizeof(p));
  const int grid = qh_lm_head_grid(N);
  p.x = (const uint16_t*)x;
  p.norm_w = norm_w;
  p.eps = eps;
  p.K = K;
  p.w = (const uint16_t*)w;
  p.N = N;
  p.logits = (uint16_t*)logits;
  p.part_val = (float*)scratch;
  p.part_idx = (int*)((float*)scratch + grid);
  p.counter = counter;
  p.tok_out = tok_out;
  p.tok_hist = tok_hist;
  p.hist_len = hist_len;
  p.pos = pos_dev;
  p.embed = (const uint16_t*)embed;
  p.embed_out = (uint16_t*)embed_out;
  if (qh_launch_lm_head(p, grid, stream) != 0) return -1;
  return check_launch("qh_lm_head_argmax");
}

QH_EXPORT size_t qh_sample_workspace_size(int V) { return qh_sample_workspace_bytes(V); }

// Nucleus sampling of one bf16 logits row (main.py:49-87) on the device.
QH_EXPORT int qh_sample_top_p(const void* logits, int V, float temperature, float top_p,
                              float rep_penalty, int64_t* hist, int hist_len,
                              const int* pos_dev, int pos,
                              int pos_offset, const int* lo_dev, int window, uint64_t seed,
                              uint64_t* counter, void* ws, int64_t* tok_out, const void* embed,
                              void* h, int D, int64_t* info, hipStream_t stream) {
  QhSampleParams p;
  memset(&p, 0, sizeof(p));
  p.logits = (const uint16_t*)logits;
  p.V = V;
  p.temperature = temperature;
  p.top_p = top_p;
  p.rep_penalty = rep_penalty;
  p.hist = hist;
  p.hist_len = hist_len;
  p.pos_dev = pos_dev;
  p.pos = pos;
  p.pos_offset = pos_offset;
  p.lo_dev = lo_dev;
  p.window = window;
  p.seed = seed;
  p.counter = counter;
  p.ws = (uint8_t*)ws;
  p.tok_out = tok_out;
  p.embed = (const uint16_t*)embed;
  p.h = (uint16_t*)h;
  p.D = D;
  p.info = info;
  if (qh_launch_sample(p, stream) != 0) return -1;
  return check_launch("qh_sample_top_p");
}

QH_EXPORT int qh_embed(const void* table, const int64_t* ids, void* out, int n, int K, int vocab,
                       hipStream_t stream) {
  qh_launch_embed_gather(table, ids, out, n, K, vocab, stream);
  return check_launch("qh_embed");
}

QH_EXPORT int qh_add_bf16(const void* a, const void* b, void* out, int n, hipStream_t stream) {
  qh_launch_add_bf16(a, b, out, n, stream);
  return check_launch("qh_add_bf16");
}

QH_EXPORT int qh_linear_gates(const void* a, const void* b, const float* A_log,
                              const float* dt_bias, float* g_out, void* beta_out, int heads,
                              hipStream_t stream) {
  qh_launch_linear_gates(a, b, A_log, dt_bias, g_out, beta_out, heads, stream);
  return check_launch("qh_linear_gates");
}

QH_EXPORT int qh_gated_rmsnorm(const void* core, const void* z, const void* w, void* out,
                               int heads, int head_dim, float eps, int bf16_steps,
                               hipStream_t stream) {
  if (head_dim <= 0 || head_dim > 256) {
    qh_set_error("qh_gated_rmsnorm: head_dim=%d unsupported (<= 256)", head_dim);
    return -1;
  }
  qh_launch_gated_rmsnorm(core, z, w, out, heads, head_dim, eps, bf16_steps, stream);
  return check_launch("qh_gated_rmsnorm");
}

QH_EXPORT size_t qh_gemm_workspace_size(int M, int K) { return qh_gemm_workspace_bytes(M, K); }

// A caller workspace for split-K partials is either absent (ws null: K is not
// split) or ws_bytes >= qh_gemm_workspace_size bytes, 256-byte aligned.  The
// check runs before anything touches the device, and the plan never puts more
// partials in the workspace than ws_bytes.
static bool gemm_ws_ok(const void* ws, size_t ws_bytes, int M, int K, const char* what) {
  if (!ws) return true;
  const size_t need = qh_gemm_workspace_bytes(M, K);
  if (ws_bytes < need) {
    qh_set_error("%s: workspace of %zu bytes is smaller than qh_gemm_workspace_size (%zu)", what, ws_bytes,
                 need);
    return false;
  }
  if ((uintptr_t)ws % 256 != 0) {
    qh_set_error("%s: workspace must be 256-byte aligned", what);
    return false;
  }
  return true;
}

// Prefill block-scaled E4M3 GEMM: Y[M,N] = bf16(X[M,K] . deq(W)[N,K]^T) on the
// fp8 matrix cores.  `ws` (ws_bytes >= qh_gemm_workspace_size, optional) holds
// split-K partials; without it the GEMM does not split K.
QH_EXPORT int qh_gemm_e4m3(const void* x, const void* w, const void* s, void* y, int M, int N,
                           int K, int kb, int scales_bf16, void* ws, size_t ws_bytes, hipStream_t stream) {
  if (!k_ok(K, "qh_gemm_e4m3")) return -1;
  if (!gemm_ws_ok(ws, ws_bytes, M, K, "qh_gemm_e4m3")) return -1;
  if (M <= 0 || N <= 0) return 0;
  const int rc = ws ? qh_launch_gemm_e4m3_ws(x, w, s, y, M, N, K, kb, scales_bf16 != 0, ws, ws_bytes, stream)
                    : qh_launch_gemm_e4m3(x, w, s, y, M, N, K, kb, scales_bf16 != 0, stream);
  if (rc != 0) return -1;
  return check_launch("qh_gemm_e4m3");
}

// Output projection + residual add + (1+w) RMSNorm (no reference counterpart:
// main.py's prefill runs fp8_gemm_batch, the add and the norm as three steps,
// main.py:1550-1566).  o = bf16(x W^T) (scratch; not written when the split-K
// finish does all three), h = bf16(h + o) in place, hn = RMSNorm(h) with
// (1 + norm_w) (norm_w null: the add only).
QH_EXPORT int qh_gemm_e4m3_add_rmsnorm(const void* x, const void* w, const void* s, void* o, int M, int N, int K,
                                       int kb, int scales_bf16, void* h, const float* norm_w, void* hn, float eps,
                                       void* ws, size_t ws_bytes, hipStream_t stream) {
  if (K <= 0 || K % 128 != 0) {
    qh_set_error("qh_gemm_e4m3_add_rmsnorm: K=%d must be a positive multiple of 128", K);
    return -1;
  }
  if (!gemm_ws_ok(ws, ws_bytes, M, K, "qh_gemm_e4m3_add_rmsnorm")) return -1;
  if (M < 0 || N < 0) {
    qh_set_error("qh_gemm_e4m3_add_rmsnorm: bad shape M=%d N=%d", M, N);
    return -1;
  }
  if (M == 0 || N == 0) return 0;
  if (!x || !w || !s || !o || !h || (norm_w && !hn)) {
    qh_set_error("qh_gemm_e4m3_add_rmsnorm: null pointer");
    return -1;
  }
  if (o == h || o == x || h == x || (norm_w && (hn == h || hn == o || hn == x))) {
    qh_set_error("qh_gemm_e4m3_add_rmsnorm: x, o, h and hn must be distinct buffers");
    return -1;
  }
  if (qh_launch_gemm_e4m3_add_rmsnorm(x, w, s, o, M, N, K, kb, scales_bf16 != 0, h, norm_w, hn, eps, ws,
                                      ws_bytes, stream) != 0)
    return -1;
  return check_launch("qh_gemm_e4m3_add_rmsnorm");
}

// Grouped prefill GEMM (no reference counterpart: the reference runs each
// projection as its own fp8_gemm_batch, main.py:262-269).  Up to 4
// projections of the same activation X[M, K] -- segment t:
// Y_t[M, n_t] = bf16(X . deq(W_t)^T), scale mode kb_t -- with one activation
// split and one launch.  `ws` / `ws_bytes` as for qh_gemm_e4m3 (optional).
QH_EXPORT int qh_gemm_e4m3_grouped(const void* x, int M, int K, int nseg, const void* w0,
                                   const void* s0, void* y0, int n0, int kb0, const void* w1,
                                   const void* s1, void* y1, int n1, int kb1, const void* w2,
                                   const void* s2, void* y2, int n2, int kb2, const void* w3,
                                   const void* s3, void* y3, int n3, int kb3, int scales_bf16,
                                   void* ws, size_t ws_bytes, hipStream_t stream) {
  if (!k_ok(K, "qh_gemm_e4m3_grouped")) return -1;
  if (!gemm_ws_ok(ws, ws_bytes, M, K, "qh_gemm_e4m3_grouped")) return -1;
  if (!x) {
    qh_set_error("qh_gemm_e4m3_grouped: null activation");
    return -1;
  }
  if (M <= 0) return 0;
  const QhGemmSeg seg[4] = {{w0, s0, y0, n0, kb0}, {w1, s1, y1, n1, kb1},
                            {w2, s2, y2, n2, kb2}, {w3, s3, y3, n3, kb3}};
  if (qh_launch_gemm_e4m3_group_ws(x, M, K, seg, nseg, scales_bf16 != 0, ws, ws_bytes, stream) != 0) return -1;
  return check_launch("qh_gemm_e4m3_grouped");
}

// ---- batch prefill pieces (the reference runs these in torch) -------------------
// q/k head norm + partial RoPE (q kept fp32) + KV-cache write for M tokens at
// positions past.. (main.py:1034-1043).
QH_EXPORT int qh_attn_prep(const void* q_all, const void* k, const void* v, const float* q_norm_w,
                           const float* k_norm_w, const float* cos_t, const float* sin_t,
                           float* q_out, void* k_cache, void* v_cache, int M, int Hq, int Hkv,
                           int D, int rot, int past, int max_seq, float eps, hipStream_t stream) {
  QhAttnPrepParams p = {(const uint16_t*)q_all, (const uint16_t*)k, (const uint16_t*)v, q_norm_w,
                        k_norm_w, cos_t, sin_t, q_out, (uint16_t*)k_cache, (uint16_t*)v_cache,
                        M, Hq, Hkv, D, rot, past, max_seq, eps};
  if (qh_launch_attn_prep(p, stream) != 0) return -1;
  return check_launch("qh_attn_prep");
}

// Causal GQA attention with the sigmoid output gate for M query tokens
// (main.py:1043-1059).
QH_EXPORT int qh_attn_prefill(const float* q, const void* gate, int gate_mstride, int gate_hstride,
                              const void* k_cache, const void* v_cache, void* out, int M, int Hq,
                              int Hkv, int D, int past, int max_seq, hipStream_t stream) {
  QhAttnPrefillParams p = {q, (const uint16_t*)gate, gate_mstride, gate_hstride,
                           (const uint16_t*)k_cache, (const uint16_t*)v_cache, (uint16_t*)out,
                           M, Hq, Hkv, D, past, max_seq};
  if (qh_launch_attn_prefill(p, stream) != 0) return -1;
  return check_launch("qh_attn_prefill");
}

// GatedDeltaNet prefill front: causal conv + SiLU over the sequence (conv
// ring updated), bf16-step l2norm of q/k, per-token gates (main.py:1097-1128).
QH_EXPORT int qh_gdn_prep(const void* mixed, void* conv_ring, const void* conv_w, const void* a,
                          const void* b, const float* A_log, const float* dt_bias, void* y, void* qn,
                          void* kn, float* g, void* beta, int M, int Hk, int Hv, int dk, int dv,
                          int past, hipStream_t stream) {
  QhGdnPrepParams p = {(const uint16_t*)mixed, (uint16_t*)conv_ring, (const uint16_t*)conv_w,
                       (const uint16_t*)a, (const uint16_t*)b, A_log, dt_bias, (uint16_t*)y,
                       (uint16_t*)qn, (uint16_t*)kn, g, (uint16_t*)beta, M,
                       2 * Hk * dk + Hv * dv, Hk, Hv, dk, dv, past};
  if (qh_launch_gdn_prep(p, stream) != 0) return -1;
  return check_launch("qh_gdn_prep");
}

// GatedDeltaNet prefill scan: recurrent gated delta rule over the M tokens from
// the stored state (updated in place), gated RMSNorm per token and head
// (main.py:1139-1158).
QH_EXPORT int qh_gdn_scan(const void* qn, const void* kn, const void* y, const float* g,
                          const void* beta, const void* z, const void* norm_w, float* state,
                          void* out, int M, int Hk, int Hv, int dk, int dv, float eps,
                          hipStream_t stream) {
  QhGdnScanParams p = {(const uint16_t*)qn, (const uint16_t*)kn, (const uint16_t*)y, g,
                       (const uint16_t*)beta, (const uint16_t*)z, (const uint16_t*)norm_w, state,
                       (uint16_t*)out, M, 2 * Hk * dk + Hv * dv, Hk, Hv, dk, dv, eps};
  if (qh_launch_gdn_scan(p, stream) != 0) return -1;
  return check_launch("qh_gdn_scan");
}

// Workspace bytes of qh_gdn_chunk for M tokens and Hv value heads.
QH_EXPORT size_t qh_gdn_chunk_workspace_size(int M, int Hv) { return qh_gdn_chunk_ws_bytes(M, Hv); }

// qh_gdn_scan in the chunked (WY) form of torch_chunk_gated_delta_rule, the
// reference's prefill algorithm (main.py:1139-1149), on the matrix cores:
// same operands and results, plus a workspace of qh_gdn_chunk_workspace_size.
QH_EXPORT int qh_gdn_chunk(const void* qn, const void* kn, const void* y, const float* g,
                           const void* beta, const void* z, const void* norm_w, float* state,
                           void* out, int M, int Hk, int Hv, int dk, int dv, float eps, void* ws,
                           size_t ws_bytes, hipStream_t stream) {
  QhGdnScanParams p = {(const uint16_t*)qn, (const uint16_t*)kn, (const uint16_t*)y, g,
                       (const uint16_t*)beta, (const uint16_t*)z, (const uint16_t*)norm_w, state,
                       (uint16_t*)out, M, 2 * Hk * dk + Hv * dv, Hk, Hv, dk, dv, eps};
  if (qh_launch_gdn_chunk(p, (float*)ws, ws_bytes, stream) != 0) return -1;
  return check_launch("qh_gdn_chunk");
}

// m = bf16(bf16(silu(g)) * u), the M > 1 MLP glue (main.py:1213-1215).
QH_EXPORT int qh_silu_mul(const void* g, const void* u, void* m, size_t n, hipStream_t stream) {
  if (qh_launch_silu_mul((const uint16_t*)g, (const uint16_t*)u, (uint16_t*)m, n, stream) != 0)
    return -1;
  return check_launch("qh_silu_mul");
}
