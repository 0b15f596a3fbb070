// Launch descriptor for the decode attention kernel (attention.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

struct QhAttnParams {
  const uint16_t* q;        // head h at q + h * q_stride (bf16, pre-norm, pre-RoPE)
  int q_stride;
  const uint16_t* gate;     // optional output gate, head h at gate + h * gate_stride
  int gate_stride;
  const uint16_t* k_new;    // optional [n_kv, D] new key (pre-norm, pre-RoPE)
  const uint16_t* v_new;    // [n_kv, D] new value
  uint16_t* q_wb;           // optional write-back of the normalised + rotated q [n_heads, D]
  uint16_t* k_wb;           // optional write-back of the normalised + rotated k [n_kv, D]
  const float* q_norm_w;    // optional (1+w) head norm weights [D]
  const float* k_norm_w;
  const float* cos_t;       // [max_pos, rot] fp32
  const float* sin_t;
  uint16_t* k_cache;        // [n_kv, max_seq, D] bf16
  uint16_t* v_cache;
  int max_seq;
  int rot;
  int n_heads;
  int n_kv;
  const int* pos_dev;       // optional device position t: rope = slot = t, total = t + 1
  int rope_pos;             // host positions, used when pos_dev is null
  int slot;
  int total;
  int nsplit;               // position splits per KV head (1 = no scratch needed)
  float* part;              // split records, then the level-2 records (nsplit > 8)
  unsigned* counters;       // [n_kv] zero-initialised arrival counters
  unsigned* gcounters;      // [n_kv][8] zero-initialised group counters (nsplit > 8)
  uint16_t* out;            // [n_heads, D] bf16
  float eps;
};

size_t qh_attn_scratch_floats(int n_kv, int nsplit, int head_dim);
int qh_launch_attn(const QhAttnParams& p, int head_dim, hipStream_t st);
void qh_set_error(const char* fmt, ...);
