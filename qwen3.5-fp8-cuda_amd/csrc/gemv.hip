// Block-scaled E4M3 GEMV family for batch-1 decode on gfx950.
//
// Semantics (reference: qwen3_infer/csrc/fused_kernels.cu:91-151 gemv_v4_kernel,
// 398-479 fused_gate_up_silu_v4_kernel; main.py:242-261 fp8_linear):
//   y[n] = bf16( sum_kb s[n,kb] * sum_{k in kb} x[k] * e4m3(W[n,k]) ), fp32 acc.
//
// Design (wave64, HBM streaming):
//   * a wave owns R consecutive rows at a time; its 64 lanes split K into
//     8-element chunks (lane l takes chunks l, l+64, ...), so one wave-wide
//     load of a row is 512 contiguous bytes and every lane keeps the same K
//     slice for all rows it ever touches;
//   * the activation slice (CPL = K/512 chunks of 8 bf16) is loaded once per
//     wave into registers, together with the optional (1+w) RMSNorm prologue;
//   * weights stream with non-temporal 8-byte loads, R*CPL of them in flight
//     per wave; E4M3 pairs become bf16 pairs with v_cvt_scalef32_pk_bf16_fp8
//     and meet the activations in v_dot2_f32_bf16;
//   * the fp32 scale of the 128-wide K block is applied once per 8-element
//     partial (an FMA), and partials meet in a 64-lane shuffle reduction.
#include "qh_common.h"
#include "qh_kernels.h"

#include <algorithm>

namespace {

__device__ __forceinline__ u32x2 ld_w8(const uint8_t* p) {
  return __builtin_nontemporal_load((const u32x2*)p);
}
__device__ __forceinline__ u32x4 ld_w16(const uint16_t* p) {
  return __builtin_nontemporal_load((const u32x4*)p);
}

__device__ __forceinline__ u32x4 add_bf16x8(u32x4 a, u32x4 b) {
  u32x4 r;
  r.x = pack_bf2(bf_lo(a.x) + bf_lo(b.x), bf_hi(a.x) + bf_hi(b.x));
  r.y = pack_bf2(bf_lo(a.y) + bf_lo(b.y), bf_hi(a.y) + bf_hi(b.y));
  r.z = pack_bf2(bf_lo(a.z) + bf_lo(b.z), bf_hi(a.z) + bf_hi(b.z));
  r.w = pack_bf2(bf_lo(a.w) + bf_lo(b.w), bf_hi(a.w) + bf_hi(b.w));
  return r;
}

__device__ __forceinline__ float sumsq_bf16x8(u32x4 a, float s) {
  s = fmaf(bf_lo(a.x), bf_lo(a.x), s); s = fmaf(bf_hi(a.x), bf_hi(a.x), s);
  s = fmaf(bf_lo(a.y), bf_lo(a.y), s); s = fmaf(bf_hi(a.y), bf_hi(a.y), s);
  s = fmaf(bf_lo(a.z), bf_lo(a.z), s); s = fmaf(bf_hi(a.z), bf_hi(a.z), s);
  s = fmaf(bf_lo(a.w), bf_lo(a.w), s); s = fmaf(bf_hi(a.w), bf_hi(a.w), s);
  return s;
}

// y = bf16((x * rms) * (1 + w)) for 8 elements (reference order, fused_kernels.cu:545).
__device__ __forceinline__ u32x4 norm_bf16x8(u32x4 a, float rms, const float* w) {
  const f32x4 w0 = *(const f32x4*)w;
  const f32x4 w1 = *(const f32x4*)(w + 4);
  u32x4 r;
  r.x = pack_bf2(bf_lo(a.x) * rms * (1.0f + w0.x), bf_hi(a.x) * rms * (1.0f + w0.y));
  r.y = pack_bf2(bf_lo(a.y) * rms * (1.0f + w0.z), bf_hi(a.y) * rms * (1.0f + w0.w));
  r.z = pack_bf2(bf_lo(a.z) * rms * (1.0f + w1.x), bf_hi(a.z) * rms * (1.0f + w1.y));
  r.w = pack_bf2(bf_lo(a.w) * rms * (1.0f + w1.z), bf_hi(a.w) * rms * (1.0f + w1.w));
  return r;
}

// Loads this lane's activation slice (chunks lane + 64*j) and applies the
// optional add / RMSNorm prologue.  Chunks past K read as zero.
template <int CPL>
__device__ __forceinline__ void load_x_slice(u32x4 (&xr)[CPL], const uint16_t* x,
                                             const uint16_t* x2, const float* norm_w,
                                             float eps, int K, int lane) {
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const int c = lane + 64 * j;
    u32x4 a = {0u, 0u, 0u, 0u};
    if (c * 8 < K) {
      a = *(const u32x4*)(x + c * 8);
      if (x2) a = add_bf16x8(a, *(const u32x4*)(x2 + c * 8));
    }
    xr[j] = a;
  }
  if (norm_w) {
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < CPL; ++j) ss = sumsq_bf16x8(xr[j], ss);
    ss = wave_sum(ss);
    const float rms = rsqrtf(ss / (float)K + eps);
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      const int c = lane + 64 * j;
      if (c * 8 < K) xr[j] = norm_bf16x8(xr[j], rms, norm_w + c * 8);
    }
  }
}

template <int R>
__device__ __forceinline__ float pick_lane(const float (&acc)[R], int lane) {
  float v = acc[0];
#pragma unroll
  for (int r = 1; r < R; ++r)
    if (lane == r) v = acc[r];
  return v;
}

template <int CPL, int R, typename ScaleT>
__global__ __launch_bounds__(256) void gemv_e4m3_kernel(QhGemvParams p) {
  const int lane = threadIdx.x & 63;
  const int wid = threadIdx.x >> 6;
  const int K = p.K;
  u32x4 xr[CPL];
  load_x_slice<CPL>(xr, p.x, p.x2, p.norm_w, p.eps, K, lane);

  for (int g = blockIdx.x * 4 + wid; g < p.gtotal; g += gridDim.x * 4) {
    int si = 0;
#pragma unroll
    for (int t = 1; t < 4; ++t)
      if (t < p.nseg && g >= p.gstart[t]) si = t;
    const QhGemvSeg sg = p.seg[si];
    const int row0 = (g - p.gstart[si]) * R;

    u32x2 wr[R][CPL];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int row = min(row0 + r, sg.n - 1);
      const uint8_t* wrow = sg.w + (size_t)row * K;
#pragma unroll
      for (int j = 0; j < CPL; ++j) {
        const int c = lane + 64 * j;
        wr[r][j] = (c * 8 < K) ? ld_w8(wrow + c * 8) : u32x2{0u, 0u};
      }
    }

    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.0f;
    const ScaleT* s = (const ScaleT*)sg.s;
    if (sg.kb > 1) {
      // 128x128 block scales: the R rows share one 128-row block.
      const ScaleT* srow = s + (row0 >> 7) * sg.kb;
#pragma unroll
      for (int j = 0; j < CPL; ++j) {
        const int c = lane + 64 * j;
        if (c * 8 < K) {
          const float sc = load_scale<ScaleT>(srow, c >> 4);
#pragma unroll
          for (int r = 0; r < R; ++r)
            acc[r] = fmaf(dot8_e4m3_bf16(wr[r][j].x, wr[r][j].y, xr[j], 0.0f), sc, acc[r]);
        }
      }
    } else {
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int row = min(row0 + r, sg.n - 1);
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
          const int c = lane + 64 * j;
          if (c * 8 < K) {
            const float sc = load_scale<ScaleT>(s, scale_index(sg.kb, row, c >> 4));
            acc[r] = fmaf(dot8_e4m3_bf16(wr[r][j].x, wr[r][j].y, xr[j], 0.0f), sc, acc[r]);
          }
        }
      }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = wave_sum(acc[r]);

    const float v = pick_lane<R>(acc, lane);
    const int row = row0 + lane;
    if (lane < R && row < sg.n) {
      float y = rbf(v);
      if (p.res1) {
        float res = bf2f(p.res1[row]);
        if (p.res2) res = rbf(res + bf2f(p.res2[row]));
        y = res + y;
      }
      sg.y[row] = f2bf(y);
    }
  }
}

template <int CPL, int R, typename ScaleT>
__global__ __launch_bounds__(256) void mlp_gate_up_kernel(QhMlpParams p) {
  const int lane = threadIdx.x & 63;
  const int wid = threadIdx.x >> 6;
  const int K = p.K;
  u32x4 xr[CPL];
  load_x_slice<CPL>(xr, p.x, p.x2, p.norm_w, p.eps, K, lane);
  const int ngroups = (p.N + R - 1) / R;
  const ScaleT* sg = (const ScaleT*)p.sg;
  const ScaleT* su = (const ScaleT*)p.su;

  for (int g = blockIdx.x * 4 + wid; g < ngroups; g += gridDim.x * 4) {
    const int row0 = g * R;
    u32x2 wg[R][CPL], wu[R][CPL];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int row = min(row0 + r, p.N - 1);
      const uint8_t* gr = p.wg + (size_t)row * K;
      const uint8_t* ur = p.wu + (size_t)row * K;
#pragma unroll
      for (int j = 0; j < CPL; ++j) {
        const int c = lane + 64 * j;
        const bool ok = c * 8 < K;
        wg[r][j] = ok ? ld_w8(gr + c * 8) : u32x2{0u, 0u};
        wu[r][j] = ok ? ld_w8(ur + c * 8) : u32x2{0u, 0u};
      }
    }
    float ag[R], au[R];
#pragma unroll
    for (int r = 0; r < R; ++r) { ag[r] = 0.0f; au[r] = 0.0f; }
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int row = min(row0 + r, p.N - 1);
#pragma unroll
      for (int j = 0; j < CPL; ++j) {
        const int c = lane + 64 * j;
        if (c * 8 < K) {
          const int si = scale_index(p.kb, row, c >> 4);
          const float scg = load_scale<ScaleT>(sg, si);
          const float scu = load_scale<ScaleT>(su, si);
          ag[r] = fmaf(dot8_e4m3_bf16(wg[r][j].x, wg[r][j].y, xr[j], 0.0f), scg, ag[r]);
          au[r] = fmaf(dot8_e4m3_bf16(wu[r][j].x, wu[r][j].y, xr[j], 0.0f), scu, au[r]);
        }
      }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) { ag[r] = wave_sum(ag[r]); au[r] = wave_sum(au[r]); }
    const float gv = pick_lane<R>(ag, lane);
    const float uv = pick_lane<R>(au, lane);
    const int row = row0 + lane;
    if (lane < R && row < p.N) {
      // SiLU on the fp32 accumulators (fused_kernels.cu:476).
      p.m_out[row] = f2bf(qh_silu(gv) * uv);
      if (p.g_out) p.g_out[row] = f2bf(gv);
      if (p.u_out) p.u_out[row] = f2bf(uv);
    }
  }
}

// ---- bf16 lm_head GEMV + greedy argmax -------------------------------------
// torch.argmax order on the bf16 logits: NaN ranks above every number, and
// the lowest index wins ties.  Candidates start at (-inf, INT_MAX); the final
// index is clamped into [0, N) before it is used as an address.
__device__ __forceinline__ void amax_merge(float& v, int& i, float v2, int i2) {
  const bool n1 = v != v, n2 = v2 != v2;
  bool take;
  if (n1 || n2) take = n2 && (!n1 || i2 < i);
  else take = v2 > v || (v2 == v && i2 < i);
  if (take) { v = v2; i = i2; }
}

template <int CPL, int R>
__global__ __launch_bounds__(256) void lm_head_argmax_kernel(QhLmHeadParams p) {
  const int lane = threadIdx.x & 63;
  const int wid = threadIdx.x >> 6;
  const int K = p.K;
  u32x4 xr[CPL];
  load_x_slice<CPL>(xr, p.x, nullptr, p.norm_w, p.eps, K, lane);
  const int ngroups = (p.N + R - 1) / R;
  float best_v = -INFINITY;
  int best_i = 0x7fffffff;

  for (int g = blockIdx.x * 4 + wid; g < ngroups; g += gridDim.x * 4) {
    const int row0 = g * R;
    u32x4 wr[R][CPL];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int row = min(row0 + r, p.N - 1);
      const uint16_t* wrow = p.w + (size_t)row * K;
#pragma unroll
      for (int j = 0; j < CPL; ++j) {
        const int c = lane + 64 * j;
        wr[r][j] = (c * 8 < K) ? ld_w16(wrow + c * 8) : u32x4{0u, 0u, 0u, 0u};
      }
    }
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      acc[r] = 0.0f;
#pragma unroll
      for (int j = 0; j < CPL; ++j) acc[r] = dot8_bf16(wr[r][j], xr[j], acc[r]);
    }
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = wave_sum(acc[r]);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int row = row0 + r;
      if (row < p.N) {
        const float lv = rbf(acc[r]);
        amax_merge(best_v, best_i, lv, row);
        if (p.logits && lane == r) p.logits[row] = f2bf(acc[r]);
      }
    }
  }

  __shared__ float s_v[4];
  __shared__ int s_i[4];
  __shared__ int s_last;
  if (lane == 0) { s_v[wid] = best_v; s_i[wid] = best_i; }
  __syncthreads();
  if (threadIdx.x == 0) {
    float v = s_v[0];
    int i = s_i[0];
    for (int w = 1; w < 4; ++w) amax_merge(v, i, s_v[w], s_i[w]);
    p.part_val[blockIdx.x] = v;
    p.part_idx[blockIdx.x] = i;
    __threadfence();
    const unsigned prev = atomicAdd(p.counter, 1u);
    s_last = (prev == gridDim.x - 1);
  }
  __syncthreads();
  if (!s_last) return;
  __threadfence();
  float v = -INFINITY;
  int i = 0x7fffffff;
  for (int b = threadIdx.x; b < (int)gridDim.x; b += 256) {
    const float bv = __hip_atomic_load(&p.part_val[b], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int bi = __hip_atomic_load(&p.part_idx[b], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    amax_merge(v, i, bv, bi);
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float v2 = __shfl_xor(v, o, 64);
    const int i2 = __shfl_xor(i, o, 64);
    amax_merge(v, i, v2, i2);
  }
  __syncthreads();
  if (lane == 0) { s_v[wid] = v; s_i[wid] = i; }
  __syncthreads();
  if (threadIdx.x == 0) {
    float fv = s_v[0];
    int fi = s_i[0];
    for (int w = 1; w < 4; ++w) amax_merge(fv, fi, s_v[w], s_i[w]);
    fi = min(max(fi, 0), p.N - 1);
    s_i[0] = fi;
    p.tok_out[0] = (int64_t)fi;
    if (p.pos) {
      const int t = p.pos[0];
      if (p.tok_hist && t >= 0 && t < p.hist_len) p.tok_hist[t] = (int64_t)fi;
      p.pos[0] = t + 1;
    }
    __hip_atomic_store(p.counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  if (p.embed) {
    const uint16_t* src = p.embed + (size_t)s_i[0] * K;
    for (int k = threadIdx.x; k < K; k += 256) p.embed_out[k] = src[k];
  }
}

// ---- launchers ----------------------------------------------------------------
constexpr int kMaxGrid = 4096;

template <int CPL, int R, typename ScaleT>
void launch_gemv_t(const QhGemvParams& p, hipStream_t st) {
  const int grid = std::min(kMaxGrid, (p.gtotal + 3) / 4);
  hipLaunchKernelGGL((gemv_e4m3_kernel<CPL, R, ScaleT>), dim3(grid), dim3(256), 0, st, p);
}

template <int CPL, int R, typename ScaleT>
void launch_mlp_t(const QhMlpParams& p, hipStream_t st) {
  const int ng = (p.N + R - 1) / R;
  const int grid = std::min(kMaxGrid, (ng + 3) / 4);
  hipLaunchKernelGGL((mlp_gate_up_kernel<CPL, R, ScaleT>), dim3(grid), dim3(256), 0, st, p);
}

// Smallest supported chunks-per-lane >= ceil(K / 512); 0 when K is too large.
int pick_cpl(int K) {
  static const int kCpl[] = {1, 2, 3, 4, 5, 6, 8, 10, 12, 16, 18, 20, 24, 32};
  const int need = (K + 511) / 512;
  for (int c : kCpl)
    if (c >= need) return c;
  return 0;
}

#define QH_CPL_DISPATCH(CPL_VAL, CALL4, CALL2) \
  switch (CPL_VAL) {                           \
    case 1: CALL4(1); break;                   \
    case 2: CALL4(2); break;                   \
    case 3: CALL4(3); break;                   \
    case 4: CALL4(4); break;                   \
    case 5: CALL4(5); break;                   \
    case 6: CALL4(6); break;                   \
    case 8: CALL4(8); break;                   \
    case 10: CALL2(10); break;                 \
    case 12: CALL2(12); break;                 \
    case 16: CALL2(16); break;                 \
    case 18: CALL2(18); break;                 \
    case 20: CALL2(20); break;                 \
    case 24: CALL2(24); break;                 \
    case 32: CALL2(32); break;                 \
    default: return -1;                        \
  }

}  // namespace

int qh_launch_gemv(QhGemvParams p, bool scale_bf16, hipStream_t st) {
  const int cpl = pick_cpl(p.K);
  if (cpl == 0) {
    qh_set_error("gemv: K=%d exceeds the supported maximum (16384)", p.K);
    return -1;
  }
  const int R = cpl <= 8 ? 4 : 2;
  p.gstart[0] = 0;
  for (int i = 0; i < p.nseg; ++i) p.gstart[i + 1] = p.gstart[i] + (p.seg[i].n + R - 1) / R;
  for (int i = p.nseg + 1; i < 5; ++i) p.gstart[i] = p.gstart[p.nseg];
  p.gtotal = p.gstart[p.nseg];
  if (p.gtotal == 0) return 0;
#define G4(C) (scale_bf16 ? launch_gemv_t<C, 4, uint16_t>(p, st) : launch_gemv_t<C, 4, float>(p, st))
#define G2(C) (scale_bf16 ? launch_gemv_t<C, 2, uint16_t>(p, st) : launch_gemv_t<C, 2, float>(p, st))
  QH_CPL_DISPATCH(cpl, G4, G2)
#undef G4
#undef G2
  return 0;
}

int qh_launch_mlp(QhMlpParams p, bool scale_bf16, hipStream_t st) {
  const int cpl = pick_cpl(p.K);
  if (cpl == 0) {
    qh_set_error("mlp: K=%d exceeds the supported maximum (16384)", p.K);
    return -1;
  }
  if (p.N <= 0) return 0;
#define M4(C) (scale_bf16 ? launch_mlp_t<C, 4, uint16_t>(p, st) : launch_mlp_t<C, 4, float>(p, st))
#define M2(C) (scale_bf16 ? launch_mlp_t<C, 2, uint16_t>(p, st) : launch_mlp_t<C, 2, float>(p, st))
  QH_CPL_DISPATCH(cpl, M4, M2)
#undef M4
#undef M2
  return 0;
}

int qh_lm_head_grid(int N) {
  const int ng = (N + 3) / 4;
  return std::max(1, std::min(1024, (ng + 3) / 4));
}

int qh_launch_lm_head(QhLmHeadParams p, int grid, hipStream_t st) {
  const int cpl = pick_cpl(p.K);
  if (cpl == 0 || cpl > 8) {
    qh_set_error("lm_head: K=%d unsupported (need K <= 4096)", p.K);
    return -1;
  }
#define L4(C) hipLaunchKernelGGL((lm_head_argmax_kernel<C, 4>), dim3(grid), dim3(256), 0, st, p)
#define L2(C) (void)0
  QH_CPL_DISPATCH(cpl, L4, L2)
#undef L4
#undef L2
  return 0;
}
