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
//  * bf16 residual add, fused residual add + (1+w) RMSNorm of whole rows (the
//    batch prefill's pattern after every out_proj / o_proj / down), and
//    embedding-row gather.
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
  g_out[h] = -expf(A_log[h]) * qh_softplus(bf2f(a[h]) + dt_bias[h]);
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

// Residual add + (1+w) RMSNorm of whole rows, one 256-thread block per row:
//   h = bf16(h + o)  (stored back when o is given), out = bf16(h * rsqrt(mean(h^2) + eps) * (1 + w)),
// the rounding points of the reference's separate add and norm
// (fused_kernels.cu:553-559, 489-547).  Each thread holds up to V 8-element
// vectors of the row in registers, so the row is read once with 16-byte loads.
// Requires D % 8 == 0, D <= 2048 V and 16-byte aligned rows and weights.
template <int V>
__global__ __launch_bounds__(256) void add_rmsnorm_rows_kernel(uint16_t* h, const uint16_t* o, const float* w,
                                                               uint16_t* out, int D, float eps) {
  __shared__ float red[4];
  const int t = threadIdx.x, nv = D >> 3;
  uint16_t* hr = h + (size_t)blockIdx.x * D;
  const uint16_t* orow = o ? o + (size_t)blockIdx.x * D : nullptr;
  // Every load first, at a clamped vector index (a vector past nv is loaded
  // and not used), so h, o and the norm weights share one round trip; o
  // through a buffer resource (an empty range when o is null).
  const auto orr = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(orow), (short)0, orow ? D * 2 : 0,
                                                     0x00020000);
  u32x4 av[V], bv[V];
  float4 wv0[V], wv1[V];
#pragma unroll
  for (int v = 0; v < V; ++v) {
    const int ic = min(t + 256 * v, nv - 1);
    av[v] = *(const u32x4*)(hr + 8 * ic);
    bv[v] = __builtin_amdgcn_raw_buffer_load_b128(orr, (uint32_t)ic * 16u, 0, 0);
    wv0[v] = *(const float4*)(w + 8 * ic);
    wv1[v] = *(const float4*)(w + 8 * ic + 4);
  }
  float xv[V][8];
  float ss = 0.0f;
#pragma unroll
  for (int v = 0; v < V; ++v) {
    const int i = t + 256 * v;
    if (i < nv) {
      u32x4 a = av[v];
      if (orow) {
        const u32x4 b = bv[v];
        u32x4 sum;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float lo = rbf(bf_lo(a[q]) + bf_lo(b[q])), hi = rbf(bf_hi(a[q]) + bf_hi(b[q]));
          sum[q] = (__float_as_uint(lo) >> 16) | (__float_as_uint(hi) & 0xFFFF0000u);
        }
        a = sum;
        *(u32x4*)(hr + 8 * i) = a;
      }
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        xv[v][2 * q] = bf_lo(a[q]);
        xv[v][2 * q + 1] = bf_hi(a[q]);
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) ss = fmaf(xv[v][e], xv[v][e], ss);
    }
  }
  ss = block_sum_256(ss, red);
  const float rms = rsqrtf(ss / (float)D + eps);
  uint16_t* yr = out + (size_t)blockIdx.x * D;
#pragma unroll
  for (int v = 0; v < V; ++v) {
    const int i = t + 256 * v;
    if (i < nv) {
      const float4 w0 = wv0[v], w1 = wv1[v];
      const float wv[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
      u32x4 y;
#pragma unroll
      for (int q = 0; q < 4; ++q)
        y[q] = (uint32_t)f2bf(xv[v][2 * q] * rms * (1.0f + wv[2 * q])) |
               ((uint32_t)f2bf(xv[v][2 * q + 1] * rms * (1.0f + wv[2 * q + 1])) << 16);
      *(u32x4*)(yr + 8 * i) = y;
    }
  }
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

namespace {
bool rows_vectorizable(const void* a, const void* b, const void* w, const void* out, int D) {
  const auto al = [](const void* p) { return p == nullptr || (uintptr_t)p % 16 == 0; };
  return D > 0 && D % 8 == 0 && D <= 2048 * 4 && al(a) && al(b) && al(w) && al(out);
}

template <int V>
void launch_add_rmsnorm_v(void* h, const void* o, const float* w, void* out, int rows, int D, float eps,
                          hipStream_t st) {
  hipLaunchKernelGGL((add_rmsnorm_rows_kernel<V>), dim3(rows), dim3(256), 0, st, (uint16_t*)h,
                     (const uint16_t*)o, w, (uint16_t*)out, D, eps);
}

// The vector kernel for D <= 8192 (8 elements per thread per vector).
bool launch_add_rmsnorm_vec(void* h, const void* o, const float* w, void* out, int rows, int D, float eps,
                            hipStream_t st) {
  if (!rows_vectorizable(h, o, w, out, D)) return false;
  const int v = (D / 8 + 255) / 256;
  if (v <= 1) launch_add_rmsnorm_v<1>(h, o, w, out, rows, D, eps, st);
  else if (v == 2) launch_add_rmsnorm_v<2>(h, o, w, out, rows, D, eps, st);
  else launch_add_rmsnorm_v<4>(h, o, w, out, rows, D, eps, st);
  return true;
}
}  // namespace

void qh_launch_rmsnorm_rows(const void* x, const float* w, void* out, int rows, int D, float eps,
                            hipStream_t st) {
  if (rows <= 0 || D <= 0) return;
  if (launch_add_rmsnorm_vec(const_cast<void*>(x), nullptr, w, out, rows, D, eps, st)) return;
  hipLaunchKernelGGL(rmsnorm_rows_kernel, dim3(rows), dim3(256), 0, st, (const uint16_t*)x, w,
                     (uint16_t*)out, D, eps);
}

void qh_launch_add_rmsnorm_rows(void* h, const void* o, const float* w, void* out, int rows, int D,
                                float eps, hipStream_t st) {
  if (rows <= 0 || D <= 0) return;
  if (launch_add_rmsnorm_vec(h, o, w, out, rows, D, eps, st)) return;
  qh_launch_add_bf16(h, o, h, rows * D, st);
  hipLaunchKernelGGL(rmsnorm_rows_kernel, dim3(rows), dim3(256), 0, st, (const uint16_t*)h, w,
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
