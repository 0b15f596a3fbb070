// Host-side launch descriptors shared by the kernel translation units and the
// C-ABI layer (abi.hip).  Plain structs of device pointers and sizes; no torch
// types anywhere in this library.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

// One output segment of a (grouped) block-scaled E4M3 GEMV: y = W x.
struct QhGemvSeg {
  const uint8_t* w;  // [n, K] E4M3FN bytes, row-major
  const void* s;     // scales (fp32 or bf16, see QhGemvParams::scale_bf16)
  uint16_t* y;       // bf16 [n]
  int n;             // rows
  int kb;            // scale-mode code (reference `K_blocks` encoding)
  int qgate_d;       // 0: y[row]; d > 0: rows are per-head [q_h | gate_h] blocks
                     // of 2d, stored de-interleaved as [q_0..q_{H-1} | gate_0..]
};

// Grouped GEMV sharing one activation vector.  Optional prologue: x := bf16(x +
// x2), then x := (1+w) RMSNorm(x).  Optional epilogue: y := bf16(res + bf16(Wx)),
// where res := res1 or bf16(res1 + res2).
struct QhGemvParams {
  const uint16_t* x;
  const uint16_t* x2;
  const float* norm_w;
  const uint16_t* res1;
  const uint16_t* res2;
  float eps;
  int K;
  int nseg;
  int gtotal;      // filled by the launcher
  int gstart[5];   // filled by the launcher
  QhGemvSeg seg[4];
  // Optional per-head gated RMSNorm prologue (fast path only): x is the
  // GatedDeltaNet core, x2 its gate z, gnorm_w the bf16 norm weights [gnorm_d].
  const uint16_t* gnorm_w;
  int gnorm_d;
};

// Paired gate/up GEMV with the SiLU(gate)*up epilogue (fp32 accumulators).
struct QhMlpParams {
  const uint16_t* x;
  const uint16_t* x2;
  const float* norm_w;
  float eps;
  int K;
  const uint8_t* wg;
  const void* sg;
  const uint8_t* wu;
  const void* su;
  int N;
  int kb;
  uint16_t* m_out;  // bf16(silu(g) * u)
  uint16_t* g_out;  // optional bf16(g)
  uint16_t* u_out;  // optional bf16(u)
};

// bf16 lm_head GEMV fused with the final (1+w) RMSNorm and greedy argmax.
struct QhLmHeadParams {
  const uint16_t* x;
  const float* norm_w;  // optional final norm
  float eps;
  int K;
  const uint16_t* w;    // bf16 [N, K]
  int N;
  uint16_t* logits;     // optional bf16 [N]
  float* part_val;      // [grid] scratch
  int* part_idx;        // [grid] scratch
  unsigned* counter;    // zero-initialised; reset by the last block
  int64_t* tok_out;     // argmax (int64, like torch.argmax)
  int64_t* tok_hist;    // optional: tok_hist[*pos] = token (before the increment)
  int hist_len;         // entries in tok_hist
  int* pos;             // optional: ++ by the last block
  const uint16_t* embed;  // optional: copy embed[tok] ...
  uint16_t* embed_out;    // ... into this [K] buffer for the next step
};

int qh_launch_gemv(QhGemvParams p, bool scale_bf16, hipStream_t st);
int qh_launch_mlp(QhMlpParams p, bool scale_bf16, hipStream_t st);
int qh_launch_lm_head(QhLmHeadParams p, int grid, hipStream_t st);
int qh_lm_head_grid(int N);
int qh_launch_read_stream(const void* src, uint64_t bytes, unsigned* out, int out_len, hipStream_t st);

void qh_set_error(const char* fmt, ...);
