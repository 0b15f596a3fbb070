// Launchers for the row-normalisation / elementwise kernels (norm.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

void qh_launch_rmsnorm_rows(const void* x, const float* w, void* out, int rows, int D, float eps,
                            hipStream_t st);
// h = bf16(h + o) in place, out = (1+w) RMSNorm of h; out must not alias h or o.
void qh_launch_add_rmsnorm_rows(void* h, const void* o, const float* w, void* out, int rows, int D,
                                float eps, hipStream_t st);
void qh_launch_linear_gates(const void* a, const void* b, const float* A_log, const float* dt_bias,
                            float* g_out, void* beta_out, int heads, hipStream_t st);
void qh_launch_gated_rmsnorm(const void* core, const void* z, const void* w, void* out, int heads,
                             int head_dim, float eps, int bf16_steps, hipStream_t st);
void qh_launch_add_bf16(const void* a, const void* b, void* out, int n, hipStream_t st);
void qh_launch_embed_gather(const void* table, const int64_t* ids, void* out, int n, int K,
                            int vocab, hipStream_t st);
