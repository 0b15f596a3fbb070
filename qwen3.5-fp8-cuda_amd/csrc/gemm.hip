// Prefill block-scaled E4M3 GEMM on the gfx950 fp8 matrix cores.
//
// Semantics (reference: qwen3_infer/csrc/fp8_kernels.cu:23-64
// fp8_gemm_batch_kernel; caller main.py:262-269):
//   Y[m, n] = bf16( sum_kb s[n, kb] * sum_{k in kb} X[m, k] * e4m3(W[n, k]) )
//
// The activations are bf16, the matrix cores take E4M3 on both sides, so X is
// split into two E4M3 terms per row: with s_x = max|X[m,:]| / 448,
//   hi = e4m3(X / s_x),  lo = e4m3(X / s_x - hi),  X ~= s_x * (hi + lo)
// (about 8 significant bits, like bf16).  Both terms meet the same W tile in
// v_mfma_f32_32x32x16_fp8_fp8 and accumulate into one per-K-block partial,
// which is scaled by the W block scale and added to the fp32 accumulator; the
// row scale s_x is applied once in the epilogue.
//
// Tiling: 128x128 output tile per 256-thread workgroup, 64x64 per wave (2x2
// MFMA tiles of 32x32).  Within a 128-wide K block, lane half h owns bytes
// [64h, 64h+64) of its row for both operands (a K permutation shared by A and
// B, so the contraction is unchanged), which makes every operand fetch a
// contiguous 16-byte load.
#include <mutex>

#include "qh_common.h"
#include "qh_gemm.h"

namespace {

typedef float v16f __attribute__((ext_vector_type(16)));

__global__ __launch_bounds__(256) void quant_rows_kernel(const uint16_t* x, uint8_t* xhi,
                                                         uint8_t* xlo, float* sx, int K) {
  __shared__ float red[4];
  const int row = blockIdx.x;
  const uint16_t* xr = x + (size_t)row * K;
  float amax = 0.0f;
  for (int k = threadIdx.x * 8; k < K; k += 256 * 8) {
    const u32x4 v = *(const u32x4*)(xr + k);
    amax = fmaxf(amax, fmaxf(fmaxf(fabsf(bf_lo(v.x)), fabsf(bf_hi(v.x))),
                             fmaxf(fabsf(bf_lo(v.y)), fabsf(bf_hi(v.y)))));
    amax = fmaxf(amax, fmaxf(fmaxf(fabsf(bf_lo(v.z)), fabsf(bf_hi(v.z))),
                             fmaxf(fabsf(bf_lo(v.w)), fabsf(bf_hi(v.w)))));
  }
  amax = wave_max(amax);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = amax;
  __syncthreads();
  amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const float s = amax > 0.0f ? amax / 448.0f : 1.0f;
  const float inv = 1.0f / s;
  if (threadIdx.x == 0) sx[row] = s;
  for (int k = threadIdx.x * 8; k < K; k += 256 * 8) {
    const u32x4 v = *(const u32x4*)(xr + k);
    float f[8] = {bf_lo(v.x), bf_hi(v.x), bf_lo(v.y), bf_hi(v.y),
                  bf_lo(v.z), bf_hi(v.z), bf_lo(v.w), bf_hi(v.w)};
    uint32_t hi[2], lo[2];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      float a[4], r[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) a[e] = fminf(fmaxf(f[4 * q + e] * inv, -448.0f), 448.0f);
      uint32_t h = __builtin_amdgcn_cvt_pk_fp8_f32(a[0], a[1], 0u, false);
      h = __builtin_amdgcn_cvt_pk_fp8_f32(a[2], a[3], h, true);
      const qh_f32x2 h01 = e4m3x2_lo_f32(h), h23 = e4m3x2_hi_f32(h);
      r[0] = a[0] - h01.x; r[1] = a[1] - h01.y; r[2] = a[2] - h23.x; r[3] = a[3] - h23.y;
      uint32_t l = __builtin_amdgcn_cvt_pk_fp8_f32(r[0], r[1], 0u, false);
      l = __builtin_amdgcn_cvt_pk_fp8_f32(r[2], r[3], l, true);
      hi[q] = h;
      lo[q] = l;
    }
    *(u32x2*)(xhi + (size_t)row * K + k) = u32x2{hi[0], hi[1]};
    *(u32x2*)(xlo + (size_t)row * K + k) = u32x2{lo[0], lo[1]};
  }
}

__device__ __forceinline__ long as_long(uint32_t a, uint32_t b) {
  return (long)(((uint64_t)b << 32) | (uint64_t)a);
}

template <typename ScaleT>
__global__ __launch_bounds__(256) void gemm_e4m3_kernel(const uint8_t* xhi, const uint8_t* xlo,
                                                        const float* sx, const uint8_t* w,
                                                        const ScaleT* sw, uint16_t* y, int M,
                                                        int N, int K, int kb_code) {
  const int lane = threadIdx.x & 63;
  const int wid = threadIdx.x >> 6;
  const int m0 = blockIdx.y * 128 + (wid >> 1) * 64;
  const int n0 = blockIdx.x * 128 + (wid & 1) * 64;
  const int r = lane & 31, h = lane >> 5;

  const uint8_t* ah[2];
  const uint8_t* al[2];
  const uint8_t* bw[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int m = min(m0 + 32 * i + r, M - 1);
    ah[i] = xhi + (size_t)m * K + 64 * h;
    al[i] = xlo + (size_t)m * K + 64 * h;
    const int n = min(n0 + 32 * i + r, N - 1);
    bw[i] = w + (size_t)n * K + 64 * h;
  }
  v16f acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

  const int KB = K / 128;
  for (int kb = 0; kb < KB; ++kb) {
    const int ko = kb * 128;
    u32x4 A[2][4], L[2][4], B[2][4];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        A[i][q] = *(const u32x4*)(ah[i] + ko + 16 * q);
        L[i][q] = *(const u32x4*)(al[i] + ko + 16 * q);
        B[i][q] = __builtin_nontemporal_load((const u32x4*)(bw[i] + ko + 16 * q));
      }
    float swj[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int n = min(n0 + 32 * j + r, N - 1);
      swj[j] = load_scale<ScaleT>(sw, scale_index(kb_code, n, kb));
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        v16f t;
#pragma unroll
        for (int e = 0; e < 16; ++e) t[e] = 0.0f;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          t = __builtin_amdgcn_mfma_f32_32x32x16_fp8_fp8(as_long(A[i][q].x, A[i][q].y),
                                                         as_long(B[j][q].x, B[j][q].y), t, 0, 0, 0);
          t = __builtin_amdgcn_mfma_f32_32x32x16_fp8_fp8(as_long(A[i][q].z, A[i][q].w),
                                                         as_long(B[j][q].z, B[j][q].w), t, 0, 0, 0);
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          t = __builtin_amdgcn_mfma_f32_32x32x16_fp8_fp8(as_long(L[i][q].x, L[i][q].y),
                                                         as_long(B[j][q].x, B[j][q].y), t, 0, 0, 0);
          t = __builtin_amdgcn_mfma_f32_32x32x16_fp8_fp8(as_long(L[i][q].z, L[i][q].w),
                                                         as_long(B[j][q].z, B[j][q].w), t, 0, 0, 0);
        }
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[i][j][e] = fmaf(t[e], swj[j], acc[i][j][e]);
      }
    }
  }

  // C layout of a 32x32 tile: lane -> column lane%32, value e -> row
  // 8*(e/4) + 4*(lane/32) + e%4.
#pragma unroll
  for (int i = 0; i < 2; ++i) {
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int m = m0 + 32 * i + 8 * (e >> 2) + 4 * h + (e & 3);
      if (m >= M) continue;
      const float s = sx[m];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int n = n0 + 32 * j + r;
        if (n < N) y[(size_t)m * N + n] = f2bf(acc[i][j][e] * s);
      }
    }
  }
}

std::mutex g_ws_mu;
void* g_ws = nullptr;
size_t g_ws_bytes = 0;

}  // namespace

size_t qh_gemm_workspace_bytes(int M, int K) {
  return (size_t)M * K * 2 + (size_t)M * sizeof(float) + 256;
}

int qh_launch_gemm_e4m3_ws(const void* x, const void* w, const void* s, void* y, int M, int N,
                           int K, int kb, bool scale_bf16, void* ws, hipStream_t st) {
  if (K % 128 != 0) {
    qh_set_error("gemm: K=%d must be a multiple of 128", K);
    return -1;
  }
  uint8_t* xhi = (uint8_t*)ws;
  uint8_t* xlo = xhi + (size_t)M * K;
  float* sx = (float*)(((uintptr_t)(xlo + (size_t)M * K) + 255) & ~(uintptr_t)255);
  hipLaunchKernelGGL(quant_rows_kernel, dim3(M), dim3(256), 0, st, (const uint16_t*)x, xhi, xlo,
                     sx, K);
  dim3 grid((N + 127) / 128, (M + 127) / 128);
  if (scale_bf16)
    hipLaunchKernelGGL(gemm_e4m3_kernel<uint16_t>, grid, dim3(256), 0, st, xhi, xlo, sx,
                       (const uint8_t*)w, (const uint16_t*)s, (uint16_t*)y, M, N, K, kb);
  else
    hipLaunchKernelGGL(gemm_e4m3_kernel<float>, grid, dim3(256), 0, st, xhi, xlo, sx,
                       (const uint8_t*)w, (const float*)s, (uint16_t*)y, M, N, K, kb);
  return 0;
}

// Without a caller workspace, the library keeps one internal buffer that grows
// on demand (hipMalloc outside any captured region; the reference ABI passes
// no workspace).
int qh_launch_gemm_e4m3(const void* x, const void* w, const void* s, void* y, int M, int N, int K,
                        int kb, bool scale_bf16, hipStream_t st) {
  const size_t need = qh_gemm_workspace_bytes(M, K);
  void* ws = nullptr;
  {
    std::lock_guard<std::mutex> lk(g_ws_mu);
    if (g_ws_bytes < need) {
      if (g_ws) {
        (void)hipStreamSynchronize(st);
        (void)hipFree(g_ws);
        g_ws = nullptr;
        g_ws_bytes = 0;
      }
      if (hipMalloc(&g_ws, need) != hipSuccess) {
        g_ws = nullptr;
        qh_set_error("gemm: workspace allocation of %zu bytes failed", need);
        return -1;
      }
      g_ws_bytes = need;
    }
    ws = g_ws;
  }
  return qh_launch_gemm_e4m3_ws(x, w, s, y, M, N, K, kb, scale_bf16, ws, st);
}
