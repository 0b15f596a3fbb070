// Launch descriptor for the GatedDeltaNet decode step (gdn.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

struct QhGdnParams {
  const uint16_t* mixed;    // [conv_dim] bf16: in_proj_qkv output before the conv
  const uint16_t* a;        // [Hv] bf16
  const uint16_t* b;        // [Hv] bf16
  const uint16_t* z;        // [Hv * dv] bf16
  uint16_t* conv_ring;      // [conv_dim, 4] bf16 ring, slot t % 4 holds x_t
  const uint16_t* conv_w;   // [conv_dim, 4] bf16
  const float* A_log;       // [Hv]
  const float* dt_bias;     // [Hv]
  const uint16_t* norm_w;   // [dv] bf16 (plain weight)
  float* state;             // [Hv, dk, dv] fp32, updated in place
  float* core;              // optional [Hv * dv] fp32: the bf16-rounded delta-rule output
  uint16_t* out;            // [Hv * dv] bf16 gated output
  unsigned* counters;       // unused (kept for the entry point's signature)
  const int* pos_dev;       // optional device position t
  int pos;                  // host position when pos_dev is null
  int Hk, Hv, dk, dv;
  float eps;
};

int qh_launch_gdn_decode(const QhGdnParams& p, hipStream_t st);
// bf16 core output to p.out, no gated norm (one wave per head and 8 columns)
int qh_launch_gdn_decode_core(const QhGdnParams& p, hipStream_t st);
int qh_launch_delta_rule(const void* q, const void* k, const void* v, const float* g,
                         const void* beta, float* state, void* out, int n_heads, int head_dim,
                         hipStream_t st);
void qh_set_error(const char* fmt, ...);
