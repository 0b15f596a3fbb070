// Row-wise normalisation and small elementwise kernels.
//
//  * (1+w) RMSNorm, in place or out of place, one 256-thread block per row:
//    y = bf16((x * rsqrt(mean(x^2) + eps)) * (1 + w)), w fp32
//    (reference: qwen3_infer/csrc/fused_kernels.cu:489-547; main.py:898-933).
//  * GatedDeltaNet decode gates: g = -exp(A_log) * softplus(a + dt_bias) (fp32),
//    beta = bf16(sigmoid(b))  (fused_kernels.cu:575-590; main.py:1120-1122).
//  * Gated RMSNorm of the GatedDeltaNet output, per head, plain (not 1+w) weight
//    (fused_kernels.cu:592-618; main.py:1152-1158).  `bf16_steps` selects the
//    rounding points of main.py's torch path (bf16 after the norm, after the
//    weight product and after silu(z)); otherwise everything stays fp32 and
//    only the output is rounded, like the reference's fused kernel.
//  * bf16 residual add and embedding-row gather.
#include "qh_common.h"
#include "qh_norm.h"

namespace {

__global__ __launch_bounds__(256) void rmsnorm_rows_kernel(const uint16_t* x, const float* w,
                                                           uint16_t* out, int D, float eps) {
  __shared__ float red[4];
  const uint16_t* xr = x + (size_t)blockIdx.x * D;
  uint16_t* yr = out + (size_t)blockIdx.x * D;
  float ss = 0.0f;
  for (int i = threadIdx.x; i < D; i += 256) {
    const float v = bf2f(xr[i]);
    ss = fmaf(v, v, ss);
  }
  ss = block_sum_256(ss, red);
  const float rms = rsqrtf(ss / (float)D + eps);
  for (int i = threadIdx.x; i < D; i += 256) yr[i] = f2bf(bf2f(xr[i]) * rms * (1.0f + w[i]));
}

__global__ void linear_gates_kernel(const uint16_t* a, const uint16_t* b, const float* A_log,
                                    const float* dt_bias, float* g_out, uint16_t* beta_out,
                                    int heads) {
  const int h = blockIdx.x * blockDim.x + threadIdx.x;
  if (h >= heads) return;
  g_out[h] = -__expf(A_log[h]) * qh_softplus(bf2f(a[h]) + dt_bias[h]);
  beta_out[h] = f2bf(qh_sigmoid(bf2f(b[h])));
}

// One block of `head_dim` threads (<= 256, a multiple of 64) per head.
__global__ __launch_bounds__(256) void gated_rmsnorm_kernel(const uint16_t* core, const uint16_t* z,
                                                            const uint16_t* w, uint16_t* out,
                                                            int head_dim, float eps, int bf16_steps) {
  __shared__ float red[4];
  const int d = threadIdx.x;
  const size_t off = (size_t)blockIdx.x * head_dim + d;
  const bool ok = d < head_dim;
  const float x = ok ? bf2f(core[off]) : 0.0f;
  float ss = wave_sum(x * x);
  if ((d & 63) == 0) red[d >> 6] = ss;
  __syncthreads();
  ss = 0.0f;
  for (int i = 0; i < (int)(blockDim.x >> 6); ++i) ss += red[i];
  if (!ok) return;
  const float r = rsqrtf(ss / (float)head_dim + eps);
  const float zv = bf2f(z[off]);
  const float wv = bf2f(w[d]);
  float y;
  if (bf16_steps) {
    const float normed = rbf(rbf(x * r) * wv);
    y = normed * rbf(qh_silu(zv));
  } else {
    y = x * r * wv * qh_silu(zv);
  }
  out[off] = f2bf(y);
}

__global__ void add_bf16_kernel(const uint16_t* a, const uint16_t* b, uint16_t* out, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) out[i] = f2bf(bf2f(a[i]) + bf2f(b[i]));
}

// Ids outside [0, vocab) produce a zero row instead of an out-of-bounds read.
__global__ void embed_gather_kernel(const uint16_t* table, const int64_t* ids, uint16_t* out,
                                    int K, int vocab) {
  const int64_t id = ids[blockIdx.x];
  const bool ok = id >= 0 && id < vocab;
  const uint16_t* src = table + (ok ? (size_t)id * K : 0);
  uint16_t* dst = out + (size_t)blockIdx.x * K;
  for (int k = threadIdx.x; k < K; k += blockDim.x) dst[k] = ok ? src[k] : (uint16_t)0;
}

}  // namespace

void qh_launch_rmsnorm_rows(const void* x, const float* w, void* out, int rows, int D, float eps,
                            hipStream_t st) {
  if (rows <= 0) return;
  hipLaunchKernelGGL(rmsnorm_rows_kernel, dim3(rows), dim3(256), 0, st, (const uint16_t*)x, w,
                     (uint16_t*)out, D, eps);
}

void qh_launch_linear_gates(const void* a, const void* b, const float* A_log, const float* dt_bias,
                            float* g_out, void* beta_out, int heads, hipStream_t st) {
  if (heads <= 0) return;
  hipLaunchKernelGGL(linear_gates_kernel, dim3((heads + 63) / 64), dim3(64), 0, st,
                     (const uint16_t*)a, (const uint16_t*)b, A_log, dt_bias, g_out,
                     (uint16_t*)beta_out, heads);
}

void qh_launch_gated_rmsnorm(const void* core, const void* z, const void* w, void* out, int heads,
                             int head_dim, float eps, int bf16_steps, hipStream_t st) {
  if (heads <= 0) return;
  const int threads = ((head_dim + 63) / 64) * 64;
  hipLaunchKernelGGL(gated_rmsnorm_kernel, dim3(heads), dim3(threads), 0, st,
                     (const uint16_t*)core, (const uint16_t*)z, (const uint16_t*)w,
                     (uint16_t*)out, head_dim, eps, bf16_steps);
}

void qh_launch_add_bf16(const void* a, const void* b, void* out, int n, hipStream_t st) {
  if (n <= 0) return;
  hipLaunchKernelGGL(add_bf16_kernel, dim3((n + 255) / 256), dim3(256), 0, st, (const uint16_t*)a,
                     (const uint16_t*)b, (uint16_t*)out, n);
}

void qh_launch_embed_gather(const void* table, const int64_t* ids, void* out, int n, int K,
                            int vocab, hipStream_t st) {
  if (n <= 0) return;
  hipLaunchKernelGGL(embed_gather_kernel, dim3(n), dim3(256), 0, st, (const uint16_t*)table, ids,
                     (uint16_t*)out, K, vocab);
}
