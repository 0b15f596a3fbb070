// Launch descriptors for the batch prefill kernels (prefill.hip): the
// reference's s > 1 path (main.py:1550-1566) for a prompt of M tokens at
// positions past .. past + M - 1.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

// q/k head norm + partial RoPE + KV-cache write (main.py:1034-1043).
struct QhAttnPrepParams {
  const uint16_t* q_all;  // [M, Hq, 2D] bf16: per head [q | gate]
  const uint16_t* k;      // [M, Hkv, D] bf16
  const uint16_t* v;      // [M, Hkv, D] bf16
  const float* q_norm_w;  // [D] (1+w)
  const float* k_norm_w;
  const float* cos_t;     // [max_pos, rot] fp32
  const float* sin_t;
  float* q_out;           // [M, Hq, D] fp32: normed (bf16) then rotated, not rounded
  uint16_t* k_cache;      // [Hkv, max_seq, D]
  uint16_t* v_cache;
  int M, Hq, Hkv, D, rot, past, max_seq;
  float eps;
};

// Causal GQA attention over the cache with the sigmoid output gate
// (main.py:1043-1059): out[m, h] = bf16(bf16(softmax(q k^T / sqrt(D)) v) *
// bf16(sigmoid(gate))).
struct QhAttnPrefillParams {
  const float* q;          // [M, Hq, D] fp32
  const uint16_t* gate;    // head h of token m at gate + m * gate_mstride + h * gate_hstride
  int gate_mstride, gate_hstride;
  const uint16_t* k_cache; // [Hkv, max_seq, D]
  const uint16_t* v_cache;
  uint16_t* out;           // [M, Hq * D]
  int M, Hq, Hkv, D, past, max_seq;
};

// Causal depthwise conv (window 4) + SiLU over the sequence, conv ring
// update, bf16-step l2norm of q/k, per-token gates (main.py:1097-1128).
struct QhGdnPrepParams {
  const uint16_t* mixed;   // [M, C] bf16 (C = 2 Hk dk + Hv dv)
  uint16_t* conv_ring;     // [C, 4] bf16 ring, slot t % 4 holds x_t
  const uint16_t* conv_w;  // [C, 4] bf16
  const uint16_t* a;       // [M, Hv] bf16
  const uint16_t* b;       // [M, Hv] bf16
  const float* A_log;      // [Hv]
  const float* dt_bias;    // [Hv]
  uint16_t* y;             // [M, C] bf16 conv output (q | k | v)
  uint16_t* qn;            // [M, Hk, dk] bf16 l2-normalised q (bf16 steps)
  uint16_t* kn;            // [M, Hk, dk]
  float* g;                // [M, Hv] fp32
  uint16_t* beta;          // [M, Hv] bf16
  int M, C, Hk, Hv, dk, dv, past;
};

// Recurrent gated delta rule over the prompt from the stored state, then the
// gated RMSNorm per token and head (main.py:1139-1158).
struct QhGdnScanParams {
  const uint16_t* qn;      // [M, Hk, dk] bf16
  const uint16_t* kn;
  const uint16_t* y;       // [M, C] conv output; v at offset 2 Hk dk
  const float* g;          // [M, Hv]
  const uint16_t* beta;    // [M, Hv]
  const uint16_t* z;       // [M, Hv dv] bf16
  const uint16_t* norm_w;  // [dv] bf16
  float* state;            // [Hv, dk, dv] fp32, updated in place
  uint16_t* out;           // [M, Hv dv] bf16
  int M, C, Hk, Hv, dk, dv;
  float eps;
};

int qh_launch_attn_prep(const QhAttnPrepParams& p, hipStream_t st);
int qh_launch_attn_prefill(const QhAttnPrefillParams& p, hipStream_t st);
int qh_launch_gdn_prep(const QhGdnPrepParams& p, hipStream_t st);
int qh_launch_gdn_scan(const QhGdnScanParams& p, hipStream_t st);
// gated RMSNorm of the bf16 core in p.out, in place (gdn_gated_norm_kernel)
int qh_launch_gdn_gated_norm(const QhGdnScanParams& p, hipStream_t st);
// Chunked (WY) form of qh_launch_gdn_scan on the matrix cores (gdn_chunk.hip);
// ws: qh_gdn_chunk_ws_bytes(M, Hv) bytes, 16-byte aligned.
size_t qh_gdn_chunk_ws_bytes(int M, int Hv);
int qh_launch_gdn_chunk(const QhGdnScanParams& p, float* ws, size_t ws_bytes, hipStream_t st);
int qh_launch_silu_mul(const uint16_t* g, const uint16_t* u, uint16_t* m, size_t n, hipStream_t st);
void qh_set_error(const char* fmt, ...);
