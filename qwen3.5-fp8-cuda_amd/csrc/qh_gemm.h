// Launchers for the prefill E4M3 GEMM (gemm.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>

// One projection of a grouped GEMM: Y[M, N] (row stride N) from W[N, K] with
// scales s in scale mode kb (as the GEMV's K_blocks).
struct QhGemmSeg {
  const void* w;
  const void* s;
  void* y;
  int N;
  int kb;
};

size_t qh_gemm_workspace_bytes(int M, int K);
int qh_launch_gemm_e4m3_group_ws(const void* x, int M, int K, const QhGemmSeg* seg, int nseg,
                                 bool scale_bf16, void* ws, size_t ws_bytes, hipStream_t st);
int qh_launch_gemm_e4m3_ws(const void* x, const void* w, const void* s, void* y, int M, int N,
                           int K, int kb, bool scale_bf16, void* ws, size_t ws_bytes, hipStream_t st);
int qh_launch_gemm_e4m3_add_rmsnorm(const void* x, const void* w, const void* s, void* o, int M, int N, int K,
                                    int kb, bool scale_bf16, void* h, const float* norm_w, void* hn, float eps,
                                    void* ws, size_t ws_bytes, hipStream_t st);
int qh_launch_gemm_e4m3(const void* x, const void* w, const void* s, void* y, int M, int N, int K,
                        int kb, bool scale_bf16, hipStream_t st);
void qh_set_error(const char* fmt, ...);
