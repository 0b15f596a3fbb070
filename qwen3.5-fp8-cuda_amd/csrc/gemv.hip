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
__device__ __forceinline__ u32x4 norm_bf16x8(u32x4 a, float rms, f32x4 w0, f32x4 w1) {
  u32x4 r;
  r.x = pack_bf2(bf_lo(a.x) * rms * (1.0f + w0.x), bf_hi(a.x) * rms * (1.0f + w0.y));
  r.y = pack_bf2(bf_lo(a.y) * rms * (1.0f + w0.z), bf_hi(a.y) * rms * (1.0f + w0.w));
  r.z = pack_bf2(bf_lo(a.z) * rms * (1.0f + w1.x), bf_hi(a.z) * rms * (1.0f + w1.y));
  r.w = pack_bf2(bf_lo(a.w) * rms * (1.0f + w1.z), bf_hi(a.w) * rms * (1.0f + w1.w));
  return r;
}

// Activation prologue, once per workgroup: x (optionally + x2, rounded to
// bf16) and the optional (1+w) RMSNorm are built cooperatively into LDS
// (sx, K bf16), then every wave copies its slice (chunks lane + 64*j, zero
// past K) into registers.  Callers issue their first row group's weight loads
// before calling this, so the weight stream overlaps the prologue.
template <int CPL>
__device__ __forceinline__ void block_x_prologue(u32x4 (&xr)[CPL], uint16_t* sx, float* red,
                                                 const uint16_t* x, const uint16_t* x2,
                                                 const float* norm_w, float eps, int K) {
  constexpr int MAXC = (CPL * 64 + 255) / 256;  // 8-element chunks per thread
  const int tid = threadIdx.x;
  const int nch = K / 8;
  const u32x4 zero = {0u, 0u, 0u, 0u};
  u32x4 v[MAXC];
  f32x4 w0[MAXC], w1[MAXC];
#pragma unroll
  for (int i = 0; i < MAXC; ++i) {
    const int c = tid + 256 * i;
    const int cc = c < nch ? c : 0;
    v[i] = *(const u32x4*)(x + cc * 8);
    if (norm_w) {
      w0[i] = *(const f32x4*)(norm_w + cc * 8);
      w1[i] = *(const f32x4*)(norm_w + cc * 8 + 4);
    }
  }
  if (x2) {
#pragma unroll
    for (int i = 0; i < MAXC; ++i) {
      const int c = tid + 256 * i;
      v[i] = add_bf16x8(v[i], *(const u32x4*)(x2 + (c < nch ? c : 0) * 8));
    }
  }
#pragma unroll
  for (int i = 0; i < MAXC; ++i) v[i] = tid + 256 * i < nch ? v[i] : zero;
  if (norm_w) {
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < MAXC; ++i) ss = sumsq_bf16x8(v[i], ss);
    ss = block_sum_256(ss, red);
    const float rms = rsqrtf(ss / (float)K + eps);
#pragma unroll
    for (int i = 0; i < MAXC; ++i) v[i] = norm_bf16x8(v[i], rms, w0[i], w1[i]);
  }
#pragma unroll
  for (int i = 0; i < MAXC; ++i) {
    const int c = tid + 256 * i;
    if (c < nch) *(u32x4*)(sx + c * 8) = v[i];
  }
  __syncthreads();
  const int lane = tid & 63;
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const int c = lane + 64 * j;
    xr[j] = c < nch ? *(const u32x4*)(sx + c * 8) : zero;
  }
}

// Loads R rows of this lane's weight chunks (non-temporal) and the matching
// fp32 scales; chunks past K get zero weights and a zero scale.
template <int CPL, int R, typename ScaleT>
__device__ __forceinline__ void load_rows(u32x2 (&wr)[R][CPL], float (&sc)[R][CPL],
                                          const uint8_t* w, const ScaleT* s, int kb, int n,
                                          int row0, int K, int lane) {
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int row = min(row0 + r, n - 1);
    const uint8_t* wrow = w + (size_t)row * K;
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      const int c = lane + 64 * j;
      wr[r][j] = ld_w8(wrow + (c * 8 < K ? c : 0) * 8);
    }
  }
  if (kb > 1) {
    // 128x128 block scales: the R rows (R divides 128) share one row block.
    const ScaleT* srow = s + (row0 >> 7) * kb;
    float b[CPL];
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      const int c = lane + 64 * j;
      b[j] = load_scale<ScaleT>(srow, c * 8 < K ? (c >> 4) : 0);
    }
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int j = 0; j < CPL; ++j) sc[r][j] = b[j];
  } else {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int row = min(row0 + r, n - 1);
#pragma unroll
      for (int j = 0; j < CPL; ++j) {
        const int c = lane + 64 * j;
        sc[r][j] = load_scale<ScaleT>(s, scale_index(kb, row, c * 8 < K ? (c >> 4) : 0));
      }
    }
  }
  const u32x2 z = {0u, 0u};
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const bool ok = (lane + 64 * j) * 8 < K;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      wr[r][j] = ok ? wr[r][j] : z;
      sc[r][j] = ok ? sc[r][j] : 0.0f;
    }
  }
}

template <int CPL, int R>
__device__ __forceinline__ void dot_rows(float (&acc)[R], const u32x2 (&wr)[R][CPL],
                                         const float (&sc)[R][CPL], const u32x4 (&xr)[CPL]) {
#pragma unroll
  for (int r = 0; r < R; ++r) {
    acc[r] = 0.0f;
#pragma unroll
    for (int j = 0; j < CPL; ++j)
      acc[r] = fmaf(dot8_e4m3_bf16(wr[r][j].x, wr[r][j].y, xr[j], 0.0f), sc[r][j], acc[r]);
  }
}

template <int CPL, int R, typename ScaleT>
__global__ __launch_bounds__(256) void gemv_e4m3_kernel(QhGemvParams p) {
  __shared__ __align__(16) uint16_t sx[CPL * 512];
  __shared__ float red[4];
  const int lane = threadIdx.x & 63;
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int K = p.K;
  const int stride = gridDim.x * 4;
  int g = blockIdx.x * 4 + wid;

  auto seg_of = [&](int gg, QhGemvSeg& sg) {
    int si = 0;
#pragma unroll
    for (int t = 1; t < 4; ++t)
      if (t < p.nseg && gg >= p.gstart[t]) si = t;
    sg = p.seg[si];
    return (gg - p.gstart[si]) * R;
  };
  u32x2 wr[R][CPL];
  float sc[R][CPL];
  QhGemvSeg sg;
  int row0 = 0;
  if (g < p.gtotal) {
    row0 = seg_of(g, sg);
    load_rows<CPL, R, ScaleT>(wr, sc, sg.w, (const ScaleT*)sg.s, sg.kb, sg.n, row0, K, lane);
  }
  u32x4 xr[CPL];
  block_x_prologue<CPL>(xr, sx, red, p.x, p.x2, p.norm_w, p.eps, K);

  while (g < p.gtotal) {
    float acc[R];
    dot_rows<CPL, R>(acc, wr, sc, xr);
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = wave_sum(acc[r]);
    // Every lane holds every row total after the butterfly; lane 0 stores
    // them with static indices (a lane-indexed pick would be lowered to a
    // dynamically indexed array spilled through LDS).
    if (lane == 0) {
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int row = row0 + r;
        if (row < sg.n) {
          float y = rbf(acc[r]);
          if (p.res1) {
            float res = bf2f(p.res1[row]);
            if (p.res2) res = rbf(res + bf2f(p.res2[row]));
            y = res + y;
          }
          sg.y[row] = f2bf(y);
        }
      }
    }
    g += stride;
    if (g < p.gtotal) {
      row0 = seg_of(g, sg);
      load_rows<CPL, R, ScaleT>(wr, sc, sg.w, (const ScaleT*)sg.s, sg.kb, sg.n, row0, K, lane);
    }
  }
}

template <int CPL, int R, typename ScaleT>
__global__ __launch_bounds__(256) void mlp_gate_up_kernel(QhMlpParams p) {
  __shared__ __align__(16) uint16_t sx[CPL * 512];
  __shared__ float red[4];
  const int lane = threadIdx.x & 63;
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int K = p.K;
  const int ngroups = (p.N + R - 1) / R;
  const int stride = gridDim.x * 4;
  int g = blockIdx.x * 4 + wid;
  u32x2 wg[R][CPL], wu[R][CPL];
  float sg[R][CPL], su[R][CPL];
  if (g < ngroups) {
    load_rows<CPL, R, ScaleT>(wg, sg, p.wg, (const ScaleT*)p.sg, p.kb, p.N, g * R, K, lane);
    load_rows<CPL, R, ScaleT>(wu, su, p.wu, (const ScaleT*)p.su, p.kb, p.N, g * R, K, lane);
  }
  u32x4 xr[CPL];
  block_x_prologue<CPL>(xr, sx, red, p.x, p.x2, p.norm_w, p.eps, K);

  while (g < ngroups) {
    const int row0 = g * R;
    float ag[R], au[R];
    dot_rows<CPL, R>(ag, wg, sg, xr);
    dot_rows<CPL, R>(au, wu, su, xr);
#pragma unroll
    for (int r = 0; r < R; ++r) { ag[r] = wave_sum(ag[r]); au[r] = wave_sum(au[r]); }
    if (lane == 0) {
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int row = row0 + r;
        if (row < p.N) {
          // SiLU on the fp32 accumulators (fused_kernels.cu:476).
          p.m_out[row] = f2bf(qh_silu(ag[r]) * au[r]);
          if (p.g_out) p.g_out[row] = f2bf(ag[r]);
          if (p.u_out) p.u_out[row] = f2bf(au[r]);
        }
      }
    }
    g += stride;
    if (g < ngroups) {
      load_rows<CPL, R, ScaleT>(wg, sg, p.wg, (const ScaleT*)p.sg, p.kb, p.N, g * R, K, lane);
      load_rows<CPL, R, ScaleT>(wu, su, p.wu, (const ScaleT*)p.su, p.kb, p.N, g * R, K, lane);
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
__device__ __forceinline__ void load_bf16_rows(u32x4 (&wr)[R][CPL], const uint16_t* w, int N,
                                               int row0, int K, int lane) {
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int row = min(row0 + r, N - 1);
    const uint16_t* wrow = w + (size_t)row * K;
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      const int c = lane + 64 * j;
      wr[r][j] = ld_w16(wrow + (c * 8 < K ? c : 0) * 8);
    }
  }
}

// Grid-stride over row groups with the next group's weights in flight while
// the current one is reduced (two register buffers).
template <int CPL, int R>
__global__ __launch_bounds__(256) void lm_head_argmax_kernel(QhLmHeadParams p) {
  const int lane = threadIdx.x & 63;
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int K = p.K;
  const int ngroups = (p.N + R - 1) / R;
  const int stride = gridDim.x * 4;
  float best_v = -INFINITY;
  int best_i = 0x7fffffff;

  __shared__ __align__(16) uint16_t sx[CPL * 512];
  __shared__ float red[4];
  int g = blockIdx.x * 4 + wid;
  u32x4 wa[R][CPL];
  if (g < ngroups) load_bf16_rows<CPL, R>(wa, p.w, p.N, g * R, K, lane);
  u32x4 xr[CPL];
  block_x_prologue<CPL>(xr, sx, red, p.x, nullptr, p.norm_w, p.eps, K);

  while (g < ngroups) {
    const int gn = g + stride;
    u32x4 wb[R][CPL];
    if (gn < ngroups) load_bf16_rows<CPL, R>(wb, p.w, p.N, gn * R, K, lane);
    const int row0 = g * R;
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      acc[r] = 0.0f;
#pragma unroll
      for (int j = 0; j < CPL; ++j) acc[r] = dot8_bf16(wa[r][j], xr[j], acc[r]);
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
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int j = 0; j < CPL; ++j) wa[r][j] = wb[r][j];
    g = gn;
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
    pub_store(&p.part_val[blockIdx.x], v);
    pub_store(&p.part_idx[blockIdx.x], i);
  }
  if (!arrive_last(p.counter, gridDim.x, &s_last)) return;
  float v = -INFINITY;
  int i = 0x7fffffff;
  for (int b = threadIdx.x; b < (int)gridDim.x; b += 256) amax_merge(v, i, pub_load(&p.part_val[b]), pub_load(&p.part_idx[b]));
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
    reset_counter(p.counter);
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
  return std::max(1, std::min(512, (ng + 3) / 4));
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
