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
//     partial (an FMA), and partials meet in a 64-lane shuffle reduction;
//   * the decode path runs the 128-bit paced kernels instead
//     (gemv_b128_kernel, mlp_b128_kernel): one workgroup per CU over a
//     contiguous row range, 16-byte loads, one or two rows per wave in flight.
#include "qh_common.h"
#include "qh_kernels.h"

#include <algorithm>
#include <map>
#include <mutex>

namespace {

// ---- buffer-resource loads ----------------------------------------------------
// Weights and scales are read through buffer resources sized to their tensor:
// a load at an offset past the range returns zero without touching memory.
// Rows past n, chunks past K and pipeline slots past the last group all use
// kOob, so every wave issues the same instruction stream (the compiler's
// in-order vmcnt bookkeeping then stays exact across the software pipeline)
// while only real bytes are fetched.  Tensors must be smaller than 2^31 bytes
// (checked by the launchers) so that kOob plus any folded immediate offset stays
// out of range.
constexpr uint32_t kOob = 0x80000000u;
typedef __amdgpu_buffer_rsrc_t qh_rsrc;

__device__ __forceinline__ qh_rsrc make_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ u32x2 bload_w8(qh_rsrc r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 2 /* nt: streaming */);
}
__device__ __forceinline__ uint16_t bload_u16(qh_rsrc r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0);
}
template <typename ScaleT> __device__ __forceinline__ float bload_scale(qh_rsrc r, uint32_t i);
template <> __device__ __forceinline__ float bload_scale<float>(qh_rsrc r, uint32_t i) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, i == kOob ? kOob : i * 4u, 0, 0));
}
template <> __device__ __forceinline__ float bload_scale<uint16_t>(qh_rsrc r, uint32_t i) {
  return bf2f(bload_u16(r, i == kOob ? kOob : i * 2u));
}

// Number of scale entries of an [n, K] matrix in scale mode kb (see scale_index).
__host__ __device__ __forceinline__ uint32_t scale_count(int kb, int n) {
  if (kb > 1) return (uint32_t)((n + 127) >> 7) * (uint32_t)kb;
  if (kb == 1) return (uint32_t)n;
  return (uint32_t)n * (uint32_t)(-kb);
}


// Output index of segment row `row`: the identity, or for a gated q
// projection (qgate_d = d, rows = H per-head blocks [q_h | gate_h] of 2d) the
// de-interleaved position in [q_0 .. q_{H-1} | gate_0 .. gate_{H-1}].
__device__ __forceinline__ int out_index(const QhGemvSeg& sg, int row) {
  const int d = sg.qgate_d;
  if (d <= 0) return row;
  const int h = row / (2 * d), w = row - h * 2 * d;
  return w < d ? h * d + w : (sg.n >> 1) + h * d + (w - d);
}

// ---- activation I/O -------------------------------------------------------------
__device__ __forceinline__ u32x4 ld_act8(const uint16_t* base, int elem) {
  return *(const u32x4*)(base + elem);
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
// past K) into registers.  Split in two: XIn's loads are issued first, then
// the caller issues its weight pipeline, then block_x_finish consumes XIn.
// Vector-memory counters complete in order, so loads issued after the weight
// stream would make the prologue wait for every weight load ahead of them.
template <int CPL, int NT = 256>
struct XIn {
  static constexpr int MAXC = (CPL * 64 + NT - 1) / NT;  // 8-element chunks per thread
  u32x4 v[MAXC], v2[MAXC];
  f32x4 w0[MAXC], w1[MAXC];
};

// Large K (CPL > 8, one row group in flight per wave): the activation loads are
// issued after the weights instead, so they hold no registers while the weight
// stream is issued; the first group's weights are needed before any compute
// anyway.
template <int CPL>
constexpr bool early_x() { return CPL <= 8; }

// gw: optional bf16 weights [gd] of a per-head gated RMSNorm (x = the
// GatedDeltaNet core, x2 = its gate z); a chunk's 8 weights are kept in w0 as
// raw bits.
template <int CPL, int NT = 256>
__device__ __forceinline__ void block_x_load(XIn<CPL, NT>& in, const uint16_t* x, const uint16_t* x2,
                                             const float* norm_w, int K, const uint16_t* gw = nullptr,
                                             int gd = 0) {
  const int tid = threadIdx.x;
  const int nch = K / 8;
#pragma unroll
  for (int i = 0; i < XIn<CPL, NT>::MAXC; ++i) {
    const int c = tid + NT * i;
    const int cc = c < nch ? c : 0;
    in.v[i] = ld_act8(x, cc * 8);
    if (x2) in.v2[i] = ld_act8(x2, cc * 8);
    if (gw) {
      in.w0[i] = __builtin_bit_cast(f32x4, *(const u32x4*)(gw + (cc * 8) % gd));
    } else if (norm_w) {
      in.w0[i] = *(const f32x4*)(norm_w + cc * 8);
      in.w1[i] = *(const f32x4*)(norm_w + cc * 8 + 4);
    }
  }
}

// Gated RMSNorm of one element with the reference's bf16 intermediates
// (main.py:1152-1158): bf16(bf16(c * rs) * w) * bf16(silu(z)), then bf16.
__device__ __forceinline__ float gated1(float c, float z, float rs, float w) {
  return rbf(rbf(c * rs) * w) * rbf(qh_silu_fast(z));
}
__device__ __forceinline__ u32x4 gated_bf16x8(u32x4 c, u32x4 z, float rs, u32x4 w) {
  u32x4 r;
  r.x = pack_bf2(gated1(bf_lo(c.x), bf_lo(z.x), rs, bf_lo(w.x)), gated1(bf_hi(c.x), bf_hi(z.x), rs, bf_hi(w.x)));
  r.y = pack_bf2(gated1(bf_lo(c.y), bf_lo(z.y), rs, bf_lo(w.y)), gated1(bf_hi(c.y), bf_hi(z.y), rs, bf_hi(w.y)));
  r.z = pack_bf2(gated1(bf_lo(c.z), bf_lo(z.z), rs, bf_lo(w.z)), gated1(bf_hi(c.z), bf_hi(z.z), rs, bf_hi(w.z)));
  r.w = pack_bf2(gated1(bf_lo(c.w), bf_lo(z.w), rs, bf_lo(w.w)), gated1(bf_hi(c.w), bf_hi(z.w), rs, bf_hi(w.w)));
  return r;
}

// Builds the (normalised) activation in LDS; returns after the barrier.
// gd > 0: the per-head gated RMSNorm (heads of gd = 128 elements: a head's 16
// chunks sit in 16 consecutive threads, an aligned lane group) instead of the
// x2 sum and the (1+w) RMSNorm.
// Bare barrier: waits for this wave's LDS writes, not for its vector-memory
// loads (__syncthreads' workgroup fence would also wait for every weight
// load in flight).
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

template <int NT>
__device__ __forceinline__ float block_sum_bare(float v, float* red) {
  v = wave_sum(v);
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  if (lane == 0) red[wid] = v;
  lds_barrier();
  float s = 0.0f;
#pragma unroll
  for (int w = 0; w < NT / 64; ++w) s += red[w];
  return s;
}

// BARE: the barriers wait for LDS only (the caller's loads stay in flight).
template <int CPL, int NT = 256, bool BARE = false>
__device__ __forceinline__ void block_x_finish(XIn<CPL, NT>& in, uint16_t* sx, float* red, bool has_x2,
                                               bool has_norm, float eps, int K, int gd = 0) {
  constexpr int MAXC = XIn<CPL, NT>::MAXC;
  const int tid = threadIdx.x;
  const int nch = K / 8;
  const u32x4 zero = {0u, 0u, 0u, 0u};
  u32x4 v[MAXC];
  if (gd > 0) {
#pragma unroll
    for (int i = 0; i < MAXC; ++i) {
      const bool in_k = tid + NT * i < nch;
      const float ss = column_sum<16>(sumsq_bf16x8(in_k ? in.v[i] : zero, 0.0f));
      const float rs = rsqrtf(ss / (float)gd + eps);
      v[i] = in_k ? gated_bf16x8(in.v[i], in.v2[i], rs, __builtin_bit_cast(u32x4, in.w0[i])) : zero;
    }
  } else {
#pragma unroll
    for (int i = 0; i < MAXC; ++i) {
      v[i] = has_x2 ? add_bf16x8(in.v[i], in.v2[i]) : in.v[i];
      v[i] = tid + NT * i < nch ? v[i] : zero;
    }
  }
  if (gd == 0 && has_norm) {
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < MAXC; ++i) ss = sumsq_bf16x8(v[i], ss);
    ss = BARE ? block_sum_bare<NT>(ss, red) : block_sum<NT>(ss, red);
    const float rms = rsqrtf(ss / (float)K + eps);
#pragma unroll
    for (int i = 0; i < MAXC; ++i) v[i] = norm_bf16x8(v[i], rms, in.w0[i], in.w1[i]);
  }
#pragma unroll
  for (int i = 0; i < MAXC; ++i) {
    const int c = tid + NT * i;
    if (c < nch) *(u32x4*)(sx + c * 8) = v[i];
  }
  if (BARE) lds_barrier();
  else __syncthreads();
}

// Prologue variant for large K: loads and combines x / x2 in one pass and
// fetches the norm weights only after the sum of squares, so at most MAXC
// chunks are live while a wave's weight loads are in flight.
template <int CPL, int NT = 256>
__device__ __forceinline__ void block_x_direct(uint16_t* sx, float* red, const uint16_t* x,
                                               const uint16_t* x2, const float* norm_w, float eps,
                                               int K) {
  constexpr int MAXC = XIn<CPL, NT>::MAXC;
  const int tid = threadIdx.x;
  const int nch = K / 8;
  const u32x4 zero = {0u, 0u, 0u, 0u};
  u32x4 v[MAXC];
#pragma unroll
  for (int i = 0; i < MAXC; ++i) {
    const int c = tid + NT * i;
    const int cc = c < nch ? c : 0;
    u32x4 a = ld_act8(x, cc * 8);
    if (x2) a = add_bf16x8(a, ld_act8(x2, cc * 8));
    v[i] = c < nch ? a : zero;
  }
  if (norm_w) {
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < MAXC; ++i) ss = sumsq_bf16x8(v[i], ss);
    ss = block_sum<NT>(ss, red);
    const float rms = rsqrtf(ss / (float)K + eps);
#pragma unroll
    for (int i = 0; i < MAXC; ++i) {
      const int cc = tid + NT * i < nch ? tid + NT * i : 0;
      v[i] = norm_bf16x8(v[i], rms, *(const f32x4*)(norm_w + cc * 8),
                         *(const f32x4*)(norm_w + cc * 8 + 4));
    }
  }
#pragma unroll
  for (int i = 0; i < MAXC; ++i) {
    const int c = tid + NT * i;
    if (c < nch) *(u32x4*)(sx + c * 8) = v[i];
  }
  __syncthreads();
}

// The lane's activation slice: chunk j holds x[8c .. 8c+8), c = lane + 64 j,
// zero past K.  XLDS (large K): chunks are read from LDS at every use instead
// of occupying 4*CPL registers for the kernel's lifetime.
template <int CPL, bool XLDS>
struct XSlice {
  u32x4 r[XLDS ? 1 : CPL];
  const uint16_t* sx;
  int nch, lane;
  __device__ __forceinline__ void init(const uint16_t* sx_, int K) {
    sx = sx_;
    nch = K / 8;
    lane = threadIdx.x & 63;
    if (!XLDS) {
#pragma unroll
      for (int j = 0; j < CPL; ++j) r[XLDS ? 0 : j] = get_lds(j);
    }
  }
  __device__ __forceinline__ u32x4 get_lds(int j) const {
    const int c = lane + 64 * j;
    const u32x4 zero = {0u, 0u, 0u, 0u};
    return c < nch ? *(const u32x4*)(sx + c * 8) : zero;
  }
  __device__ __forceinline__ u32x4 operator[](int j) const { return XLDS ? get_lds(j) : r[XLDS ? 0 : j]; }
};

// The fast path's register slice (K == 512 * CPL): chunk j of lane l is
// x[8c, 8c + 8) with c = l + 64 j, read once from the staged activation.
template <int CPL>
__device__ __forceinline__ void x_slice(u32x4 (&xr)[CPL], const uint16_t* sx) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int j = 0; j < CPL; ++j) xr[j] = *(const u32x4*)(sx + (lane + 64 * j) * 8);
}

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

// Issues the loads of R rows (row0 ..) of this lane's weight chunks and their
// fp32 scales.  BLK: 128x128 block scales, which the R rows (R divides 128,
// row0 a multiple of R) share, so one scale per chunk is loaded.  Rows past n,
// chunks past K and !valid groups load zeros.
template <int CPL, int R, bool BLK, typename ScaleT>
__device__ __forceinline__ void issue_rows(u32x2 (&wr)[R][CPL], float (&sc)[R][CPL], qh_rsrc wrs,
                                           qh_rsrc srs, int kb, int n, int row0, bool valid, int K,
                                           int lane) {
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int row = row0 + r;
    const bool okr = valid && row < n;
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      const int c = lane + 64 * j;
      const bool ok = okr && c * 8 < K;
      wr[r][j] = bload_w8(wrs, ok ? (uint32_t)row * (uint32_t)K + (uint32_t)c * 8u : kOob);
    }
  }
  if (BLK) {
    float b[CPL];
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      const int c = lane + 64 * j;
      const bool ok = valid && row0 < n && c * 8 < K;
      b[j] = bload_scale<ScaleT>(srs, ok ? (uint32_t)((row0 >> 7) * kb + (c >> 4)) : kOob);
    }
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int j = 0; j < CPL; ++j) sc[r][j] = b[j];
  } else {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int row = row0 + r;
#pragma unroll
      for (int j = 0; j < CPL; ++j) {
        const int c = lane + 64 * j;
        const bool ok = valid && row < n && c * 8 < K;
        sc[r][j] = bload_scale<ScaleT>(srs, ok ? (uint32_t)scale_index(kb, row, c >> 4) : kOob);
      }
    }
  }
}

template <int CPL, int R, bool XLDS>
__device__ __forceinline__ void dot_rows(float (&acc)[R], const u32x2 (&wr)[R][CPL],
                                         const float (&sc)[R][CPL], const XSlice<CPL, XLDS>& xs) {
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = 0.0f;
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const u32x4 xj = xs[j];
#pragma unroll
    for (int r = 0; r < R; ++r)
      acc[r] = fmaf(dot8_e4m3_bf16(wr[r][j].x, wr[r][j].y, xj, 0.0f), sc[r][j], acc[r]);
  }
}

// Software pipeline shared by the E4M3 GEMV kernels: a wave walks the row
// groups g0, g0 + stride, ... (stride = all waves of the grid) and keeps P
// groups' loads in flight (slot i % P holds group i), so the weight stream of
// a wave never waits a full memory round trip between groups.  The loop body
// is unrolled over the P slots so every register array is indexed statically.
// Minimum resident waves per SIMD asked of the compiler: decode GEMVs want every
// row group of the grid in flight at once (2560 rows of a K=9216 projection need
// three waves per SIMD on 256 CUs).
constexpr int gemv_min_waves(int cpl) { return cpl <= 8 ? 4 : 3; }

template <int CPL, int R, int P, bool BLK, typename ScaleT>
__global__ __launch_bounds__(256)
__attribute__((amdgpu_waves_per_eu(gemv_min_waves(CPL)))) void gemv_e4m3_kernel(QhGemvParams p) {
  __shared__ __align__(16) uint16_t sx[CPL * 512];
  __shared__ float red[4];
  const int lane = threadIdx.x & 63;
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int K = p.K;
  const int stride = gridDim.x * 4;
  int g = blockIdx.x * 4 + wid;

  u32x2 wr[P][R][CPL];
  float sc[P][R][CPL];
  float res[P][R];   // residual for lane r's row r (epilogue), prefetched with the slot
  int srow0[P], sseg[P];

  // Issues slot s = group gg's loads (zeros when gg is past the last group).
  auto issue = [&](auto& w_, auto& s_, float (&res_)[R], int& row0_, int& seg_, int gg) {
    int si = 0;
#pragma unroll
    for (int t = 1; t < 4; ++t)
      if (t < p.nseg && gg >= p.gstart[t]) si = t;
    const QhGemvSeg& sg = p.seg[si];
    const bool valid = gg < p.gtotal;
    row0_ = (gg - p.gstart[si]) * R;
    seg_ = si;
    const qh_rsrc wrs = make_rsrc(sg.w, (uint32_t)sg.n * (uint32_t)K);
    const qh_rsrc srs = make_rsrc(sg.s, scale_count(sg.kb, sg.n) * (uint32_t)sizeof(ScaleT));
    issue_rows<CPL, R, BLK, ScaleT>(w_, s_, wrs, srs, sg.kb, sg.n, row0_, valid, K, lane);
    if (p.res1) {
      const qh_rsrc r1 = make_rsrc(p.res1, (uint32_t)sg.n * 2u);
      const qh_rsrc r2 = make_rsrc(p.res2, p.res2 ? (uint32_t)sg.n * 2u : 0u);
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int row = row0_ + r;
        const uint32_t off = valid && row < sg.n ? (uint32_t)row * 2u : kOob;
        float v = bf2f(bload_u16(r1, off));
        if (p.res2) v = rbf(v + bf2f(bload_u16(r2, off)));
        res_[r] = v;
      }
    }
  };
  (void)res;

  XIn<CPL> xin;
  if (early_x<CPL>()) block_x_load<CPL>(xin, p.x, p.x2, p.norm_w, K);
#pragma unroll
  for (int s = 0; s < P; ++s) issue(wr[s], sc[s], res[s], srow0[s], sseg[s], g + s * stride);
  if (early_x<CPL>())
    block_x_finish<CPL>(xin, sx, red, p.x2 != nullptr, p.norm_w != nullptr, p.eps, K);
  else
    block_x_direct<CPL>(sx, red, p.x, p.x2, p.norm_w, p.eps, K);
  XSlice<CPL, (CPL > 8)> xs;
  xs.init(sx, K);

  for (;;) {
#pragma unroll
    for (int s = 0; s < P; ++s) {
      if (g >= p.gtotal) return;
      float acc[R];
      dot_rows<CPL, R>(acc, wr[s], sc[s], xs);
#pragma unroll
      for (int r = 0; r < R; ++r) acc[r] = wave_sum(acc[r]);
      // Every lane holds every row total after the butterfly; lane 0 stores
      // them with static indices (a lane-indexed pick would be lowered to a
      // dynamically indexed array spilled through LDS).
      if (lane == 0) {
        const QhGemvSeg& sg = p.seg[sseg[s]];
#pragma unroll
        for (int r = 0; r < R; ++r) {
          const int row = srow0[s] + r;
          if (row < sg.n) {
            float y = rbf(acc[r]);
            if (p.res1) y = res[s][r] + y;
            sg.y[out_index(sg, row)] = f2bf(y);
          }
        }
      }
      issue(wr[s], sc[s], res[s], srow0[s], sseg[s], g + P * stride);
      g += stride;
    }
  }
}

template <int CPL, int R, int P, bool BLK, typename ScaleT>
__global__ __launch_bounds__(256)
__attribute__((amdgpu_waves_per_eu(gemv_min_waves(CPL)))) void mlp_gate_up_kernel(QhMlpParams p) {
  __shared__ __align__(16) uint16_t sx[CPL * 512];
  __shared__ float red[4];
  const int lane = threadIdx.x & 63;
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int K = p.K;
  const int ngroups = (p.N + R - 1) / R;
  const int stride = gridDim.x * 4;
  int g = blockIdx.x * 4 + wid;
  const qh_rsrc wgr = make_rsrc(p.wg, (uint32_t)p.N * (uint32_t)K);
  const qh_rsrc wur = make_rsrc(p.wu, (uint32_t)p.N * (uint32_t)K);
  const uint32_t sbytes = scale_count(p.kb, p.N) * (uint32_t)sizeof(ScaleT);
  const qh_rsrc sgr = make_rsrc(p.sg, sbytes);
  const qh_rsrc sur = make_rsrc(p.su, sbytes);

  XIn<CPL> xin;
  if (early_x<CPL>()) block_x_load<CPL>(xin, p.x, p.x2, p.norm_w, K);
  u32x2 wg[P][R][CPL], wu[P][R][CPL];
  float sg[P][R][CPL], su[P][R][CPL];
#pragma unroll
  for (int s = 0; s < P; ++s) {
    const int gg = g + s * stride;
    issue_rows<CPL, R, BLK, ScaleT>(wg[s], sg[s], wgr, sgr, p.kb, p.N, gg * R, gg < ngroups, K, lane);
    issue_rows<CPL, R, BLK, ScaleT>(wu[s], su[s], wur, sur, p.kb, p.N, gg * R, gg < ngroups, K, lane);
  }
  if (early_x<CPL>())
    block_x_finish<CPL>(xin, sx, red, p.x2 != nullptr, p.norm_w != nullptr, p.eps, K);
  else
    block_x_direct<CPL>(sx, red, p.x, p.x2, p.norm_w, p.eps, K);
  XSlice<CPL, (CPL > 8)> xs;
  xs.init(sx, K);

  for (;;) {
#pragma unroll
    for (int s = 0; s < P; ++s) {
      if (g >= ngroups) return;
      const int row0 = g * R;
      float ag[R], au[R];
      dot_rows<CPL, R>(ag, wg[s], sg[s], xs);
      dot_rows<CPL, R>(au, wu[s], su[s], xs);
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
      const int gn = g + P * stride;
      issue_rows<CPL, R, BLK, ScaleT>(wg[s], sg[s], wgr, sgr, p.kb, p.N, gn * R, gn < ngroups, K, lane);
      issue_rows<CPL, R, BLK, ScaleT>(wu[s], su[s], wur, sur, p.kb, p.N, gn * R, gn < ngroups, K, lane);
      g += stride;
    }
  }
}

// ---- fast path: 128x128 block scales, K a multiple of 512 ---------------------
// One row per wave and iteration.  Every row gets its own buffer resource
// (base = the row, range = K bytes, or 0 when the slot has no row), so the
// lane offsets are the constants lane*8 + 512*j and the per-row address math
// is a few scalar instructions; the scales of the row's 128-row block come
// the same way (lane l, chunk j reads k-block 4j + l/16).  Row totals are
// reduced with DPP moves into a wave-uniform value.
// Scale registers per row: lane l holds the fp32 scale of k-block l (and
// 64 + l when K > 8192) of the row's 128-row block; a chunk's scale (k-block
// 4j + l/16) is fetched with ds_bpermute, which runs on the LDS crossbar and
// so takes no slot of the vector-memory counter the weight pipeline lives on.
template <int CPL>
constexpr int scale_regs() { return (CPL * 4 + 63) / 64; }

template <int CPL, typename ScaleT>
__device__ __forceinline__ void issue_fast(u32x2 (&w)[CPL], float (&sr_)[scale_regs<CPL>()],
                                           const uint8_t* W, const void* S, int row, bool valid,
                                           uint32_t lw, uint32_t lane) {
  constexpr int K = CPL * 512, KB = K / 128;
  const qh_rsrc wr = make_rsrc(W + (size_t)row * K, valid ? (uint32_t)K : 0u);
  const qh_rsrc sr = make_rsrc((const ScaleT*)S + (size_t)(row >> 7) * KB,
                               valid ? (uint32_t)(KB * sizeof(ScaleT)) : 0u);
#pragma unroll
  for (int j = 0; j < CPL; ++j) w[j] = bload_w8(wr, lw + 512u * j);
#pragma unroll
  for (int r = 0; r < scale_regs<CPL>(); ++r) {
    const uint32_t off = (lane + 64u * r) * (uint32_t)sizeof(ScaleT);
    if (sizeof(ScaleT) == 4)
      sr_[r] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(sr, off, 0, 0));
    else
      sr_[r] = bf2f(bload_u16(sr, off));
  }
}

template <int CPL>
__device__ __forceinline__ float dot_row(const u32x2 (&w)[CPL], const float (&sr_)[scale_regs<CPL>()],
                                         const u32x4 (&xs)[CPL], uint32_t q4) {
  float acc = 0.0f;
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    // k-block 4j + lane/16 lives in lane (4j + lane/16) % 64 of register j/16
    const float sc = __builtin_bit_cast(
        float, __builtin_amdgcn_ds_bpermute((int)(((4u * j) & 63u) * 4u + q4),
                                            __builtin_bit_cast(int, sr_[j >> 4])));
    acc = fmaf(dot8_e4m3_bf16(w[j].x, w[j].y, xs[j], 0.0f), sc, acc);
  }
  return acc;
}

// Fast-path pipeline shape per K (measured on MI355X at the decode shapes):
//   fast_depth: row groups a wave keeps in flight;
//   fast_lead: row groups issued before the wave waits for its activation.
// A launch puts ~20 MB of weight requests in flight at once, and at that queue
// depth every request -- the activation's included, although it is issued
// first -- takes ~3.5 us to return.  Waiting for the activation before most of
// the weight stream is issued lets the first dot products start as soon as
// the first rows land.
constexpr int fast_depth(int cpl) { return cpl <= 6 ? 4 : 1; }
constexpr int fast_lead(int cpl) { return cpl <= 6 ? 1 : 0; }
constexpr int mlp_fast_depth(int) { return 1; }
constexpr int mlp_fast_lead(int) { return 0; }

// Holds the wave until its first activation chunk (and every load issued
// before it) has arrived.
template <int CPL, int NT>
__device__ __forceinline__ void x_arrived(const XIn<CPL, NT>& in) {
  asm volatile("; activation %0" ::"v"(in.v[0].x) : "memory");
}

// Grouped E4M3 GEMV, workgroup `wg` of `nwg`: the activation loads go out
// first, then the weight pipeline.
template <int CPL, int P, typename ScaleT, int NT = 256>
__device__ __forceinline__ void gemv_fast_body(const QhGemvParams& p, int wg, int nwg, uint16_t* sx,
                                               float* red) {
  constexpr int K = CPL * 512;
  const int lane = threadIdx.x & 63;
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t lw = lane * 8u, q4 = (uint32_t)(lane >> 4) * 4u;
  constexpr int NW = NT / 64;
  const int stride = nwg * NW;
  int g = wg * NW + wid;

  u32x2 w[P][CPL];
  float sc[P][scale_regs<CPL>()];
  float res[P];
  int srow[P], sseg[P];
  auto issue_w = [&](u32x2 (&w_)[CPL], float (&sc_)[scale_regs<CPL>()], int& row_, int& seg_, int gg) {
    int si = 0;
#pragma unroll
    for (int t = 1; t < 4; ++t)
      if (t < p.nseg && gg >= p.gstart[t]) si = t;
    row_ = gg - p.gstart[si];
    seg_ = si;
    issue_fast<CPL, ScaleT>(w_, sc_, p.seg[si].w, p.seg[si].s, row_, gg < p.gtotal, lw, lane);
  };
  auto issue_res = [&](float& res_, int row_, int gg) {
    if (p.res1) {
      const bool valid = gg < p.gtotal;
      float v = bf2f(__builtin_amdgcn_raw_buffer_load_b16(make_rsrc(p.res1 + row_, valid ? 2u : 0u), 0,
                                                          0, 0));
      if (p.res2)
        v = rbf(v + bf2f(__builtin_amdgcn_raw_buffer_load_b16(
                        make_rsrc(p.res2 + row_, valid ? 2u : 0u), 0, 0, 0)));
      res_ = v;
    }
  };
  (void)res;

  XIn<CPL, NT> xin;
  block_x_load<CPL, NT>(xin, p.x, p.x2, p.norm_w, K, p.gnorm_w, p.gnorm_d);
#pragma unroll
  for (int s = 0; s < P; ++s) {
    if (s == fast_lead(CPL)) x_arrived(xin);
    issue_w(w[s], sc[s], srow[s], sseg[s], g + s * stride);
    issue_res(res[s], srow[s], g + s * stride);
  }
  u32x4 xr[CPL];
  block_x_finish<CPL, NT>(xin, sx, red, p.x2 != nullptr, p.norm_w != nullptr, p.eps, K,
                          p.gnorm_w ? p.gnorm_d : 0);
  x_slice<CPL>(xr, sx);

  for (;;) {
#pragma unroll
    for (int s = 0; s < P; ++s) {
      if (g >= p.gtotal) return;
      const float acc = wave_total(dot_row<CPL>(w[s], sc[s], xr, q4));
      if (lane == 0) {
        float y = rbf(acc);
        if (p.res1) y = res[s] + y;
        p.seg[sseg[s]].y[out_index(p.seg[sseg[s]], srow[s])] = f2bf(y);
      }
      issue_w(w[s], sc[s], srow[s], sseg[s], g + P * stride);
      issue_res(res[s], srow[s], g + P * stride);
      g += stride;
    }
  }
}

// Paired gate/up GEMV with the SiLU(g)*u epilogue, workgroup `wg` of `nwg`.
template <int CPL, int P, typename ScaleT, int NT = 256>
__device__ __forceinline__ void mlp_fast_body(const QhMlpParams& p, int wg, int nwg, uint16_t* sx,
                                              float* red) {
  constexpr int K = CPL * 512;
  const int lane = threadIdx.x & 63;
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t lw = lane * 8u, q4 = (uint32_t)(lane >> 4) * 4u;
  constexpr int NW = NT / 64;
  const int stride = nwg * NW;
  int g = wg * NW + wid;

  XIn<CPL, NT> xin;
  block_x_load<CPL, NT>(xin, p.x, p.x2, p.norm_w, K);
  u32x2 wg_[P][CPL], wu[P][CPL];
  float sg[P][scale_regs<CPL>()], su[P][scale_regs<CPL>()];
#pragma unroll
  for (int s = 0; s < P; ++s) {
    if (s == mlp_fast_lead(CPL)) x_arrived(xin);
    const int gg = g + s * stride;
    issue_fast<CPL, ScaleT>(wg_[s], sg[s], p.wg, p.sg, gg, gg < p.N, lw, lane);
    issue_fast<CPL, ScaleT>(wu[s], su[s], p.wu, p.su, gg, gg < p.N, lw, lane);
  }
  u32x4 xr[CPL];
  block_x_finish<CPL, NT>(xin, sx, red, p.x2 != nullptr, p.norm_w != nullptr, p.eps, K);
  x_slice<CPL>(xr, sx);

  for (;;) {
#pragma unroll
    for (int s = 0; s < P; ++s) {
      if (g >= p.N) return;
      const float ag = wave_total(dot_row<CPL>(wg_[s], sg[s], xr, q4));
      const float au = wave_total(dot_row<CPL>(wu[s], su[s], xr, q4));
      if (lane == 0) {
        // SiLU on the fp32 accumulators (fused_kernels.cu:476).
        p.m_out[g] = f2bf(qh_silu(ag) * au);
        if (p.g_out) p.g_out[g] = f2bf(ag);
        if (p.u_out) p.u_out[g] = f2bf(au);
      }
      const int gn = g + P * stride;
      issue_fast<CPL, ScaleT>(wg_[s], sg[s], p.wg, p.sg, gn, gn < p.N, lw, lane);
      issue_fast<CPL, ScaleT>(wu[s], su[s], p.wu, p.su, gn, gn < p.N, lw, lane);
      g += stride;
    }
  }
}

// Standalone fast kernels.
// The launchers run two workgroups per CU, i.e. two waves per SIMD, so that is
// the occupancy asked of the compiler (the register budget then holds the
// activation slice, the norm weights and the P-deep weight pipeline unspilled).
template <int CPL, int P, typename ScaleT, int NT = 256>
__global__ __launch_bounds__(NT)
__attribute__((amdgpu_waves_per_eu(2))) void gemv_fast_kernel(QhGemvParams p) {
  __shared__ __align__(16) uint16_t sx[CPL * 512];
  __shared__ float red[NT / 64];
  gemv_fast_body<CPL, P, ScaleT, NT>(p, blockIdx.x, gridDim.x, sx, red);
}

template <int CPL, int P, typename ScaleT, int NT = 256>
__global__ __launch_bounds__(NT)
__attribute__((amdgpu_waves_per_eu(2))) void mlp_fast_kernel(QhMlpParams p) {
  __shared__ __align__(16) uint16_t sx[CPL * 512];
  __shared__ float red[NT / 64];
  mlp_fast_body<CPL, P, ScaleT, NT>(p, blockIdx.x, gridDim.x, sx, red);
}

// ---- 128-bit paced GEMV (a CU's contiguous row range) ------------------------
// One 512-thread workgroup per CU owns a contiguous range of rows (row slots
// s = 0 .. nrows - 1; slot s belongs to wave s % 8).  Each wave issues its
// activation and residual loads, then keeps D row slots in flight: a slot is
// the row's bytes as 16-byte loads (chunk c of lane l covers bytes
// [16 (l + 64 c), +16), so one wave instruction reads 1 KB contiguous) and
// its k-block scales, in registers.  After a slot's dot product the wave
// issues the slot D further on into the same registers.  Every CU's share
// streams from its first cycle at about 5 KB in flight per wave (D = 2 for
// 2.5 KB rows, D = 1 from 4 KB): deeper pacing, the whole share at once, and
// direct-to-LDS loads all measured slower.
constexpr int kB128Threads = 512;
constexpr int kB128Waves = kB128Threads / 64;

// Row slots in flight per wave for KC 1 KB chunks per row.
constexpr int b128_depth(int kc) { return kc >= 4 ? 1 : 2; }

// Segment of grouped row g and its row index, chosen by scalar selects over
// the four segments' fields (an indexed p.seg[si] is a kernel-argument load
// and a wait per row).
__device__ __forceinline__ QhGemvSeg seg_of(const QhGemvParams& p, int g, int& row) {
  QhGemvSeg sg = p.seg[0];
  int g0 = 0;
#pragma unroll
  for (int t = 1; t < 4; ++t) {
    if (t < p.nseg && g >= p.gstart[t]) {
      sg = p.seg[t];
      g0 = p.gstart[t];
    }
  }
  row = g - g0;
  return sg;
}

// Scale registers of a row with KC 1 KB chunks: lane l holds k-block
// 64 r + l of the row's 128-row block.
template <int KC>
constexpr int b128_sregs() { return (KC * 8 + 63) / 64; }

// Lane partial of one row: chunk c holds k-block (l + 64 c) / 8 = 8 c + l / 8,
// i.e. lane (8 c + l / 8) % 64 of scale register c / 8 (fetched with
// ds_bpermute); chunks past K count zero.
template <int KC>
__device__ __forceinline__ float b128_dot(const u32x4 (&w)[KC], const float (&sc)[b128_sregs<KC>()],
                                          const u32x4 (&xa)[KC], const u32x4 (&xb)[KC], int K, int lane) {
  float acc = 0.0f;
#pragma unroll
  for (int c = 0; c < KC; ++c) {
    u32x4 ww = w[c];
    if (16 * (lane + 64 * c) >= K) ww = u32x4{0u, 0u, 0u, 0u};
    float d = dot8_e4m3_bf16(ww.x, ww.y, xa[c], 0.0f);
    d = dot8_e4m3_bf16(ww.z, ww.w, xb[c], d);
    const float scl = __builtin_bit_cast(
        float, __builtin_amdgcn_ds_bpermute((((lane >> 3) + 8 * c) & 63) * 4, __builtin_bit_cast(int, sc[c >> 3])));
    acc = fmaf(d, scl, acc);
  }
  return acc;
}

// This workgroup's contiguous range of n items (sizes differing by at most one).
__device__ __forceinline__ void b128_range(int n, int& r0, int& nrows) {
  const int G = gridDim.x, b = blockIdx.x;
  const int base = n / G, rem = n % G;
  nrows = base + (b < rem ? 1 : 0);
  r0 = b * base + min(b, rem);
}

// The activation slice of the 16-byte chunk layout, from the staged LDS copy.
template <int KC>
__device__ __forceinline__ void b128_x(u32x4 (&xa)[KC], u32x4 (&xb)[KC], const uint16_t* sx, int K, int lane) {
#pragma unroll
  for (int c = 0; c < KC; ++c) {
    const int e = 16 * (lane + 64 * c);
    const u32x4 zero = {0u, 0u, 0u, 0u};
    xa[c] = e < K ? *(const u32x4*)(sx + e) : zero;
    xb[c] = e < K ? *(const u32x4*)(sx + e + 8) : zero;
  }
}

// Scales of a row (no weights): lane l loads k-block 64 r + l of the row's
// 128-row block.
template <int KC, typename ScaleT>
__device__ __forceinline__ void b128_scales(float (&sc)[b128_sregs<KC>()], const void* S, int row, bool valid,
                                            int K, int lane) {
  const int KB = K / 128;
  const qh_rsrc sr = make_rsrc((const ScaleT*)S + (size_t)(row >> 7) * KB, valid ? (uint32_t)(KB * sizeof(ScaleT)) : 0u);
#pragma unroll
  for (int r = 0; r < b128_sregs<KC>(); ++r) {
    const uint32_t off = (lane + 64u * r) * (uint32_t)sizeof(ScaleT);
    if (sizeof(ScaleT) == 4)
      sc[r] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(sr, off, 0, 0));
    else
      sc[r] = bf2f(bload_u16(sr, off));
  }
}

// One row's bytes as 16-byte loads (rows past the range load nothing).
template <int KC>
__device__ __forceinline__ void b128_row(u32x4 (&w)[KC], const uint8_t* W, int row, bool valid, int K, int lane) {
  const qh_rsrc wr = make_rsrc(W + (size_t)row * K, valid ? (uint32_t)K : 0u);
#pragma unroll
  for (int c = 0; c < KC; ++c)
    w[c] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(wr, (uint32_t)(lane * 16 + c * 1024), 0,
                                                                          2 /* nt: streaming */));
}

// Slot I of this wave (row r0 + wid + 8 I): dot product from register set
// I % D, then slot I + D into the same set.  Unrolled at compile time, so
// every register index is static and the compiler's in-order vmcnt count
// waits for slot I's loads only.
template <int I, int KC, int RPW, int D>
__device__ __forceinline__ void b128_rows(const QhGemvParams& p, u32x4 (&w)[D][KC],
                                          const float (&sc)[RPW][b128_sregs<KC>()], const u32x4 (&xa)[KC],
                                          const u32x4 (&xb)[KC], float res, int r0, int mine, int lane, int wid) {
  if constexpr (I < RPW) {
    if (I >= mine) return;
    const int K = p.K;
    const float part = b128_dot<KC>(w[I % D], sc[I], xa, xb, K, lane);
    if constexpr (I + D < RPW) {
      const bool valid = I + D < mine;
      int row;
      const QhGemvSeg sn = seg_of(p, r0 + (valid ? wid + kB128Waves * (I + D) : 0), row);
      b128_row<KC>(w[I % D], sn.w, row, valid, K, lane);
    }
    const float tot = wave_total(part);
    int row;
    const QhGemvSeg sg = seg_of(p, r0 + wid + kB128Waves * I, row);
    const float rv = __shfl(res, I, 64);
    if (lane == 0) {
      float y = rbf(tot);
      if (p.res1) y = rv + y;
      sg.y[out_index(sg, row)] = f2bf(y);
    }
    b128_rows<I + 1, KC, RPW, D>(p, w, sc, xa, xb, res, r0, mine, lane, wid);
  }
}

// KC: 1 KB chunks per row; RPW: row slots per wave (at least the launch's).
template <int KC, int RPW, typename ScaleT>
__global__ __launch_bounds__(kB128Threads) void gemv_b128_kernel(QhGemvParams p) {
  constexpr int D = b128_depth(KC) < RPW ? b128_depth(KC) : RPW;
  constexpr int SR = b128_sregs<KC>();
  constexpr int W8 = kB128Waves;
  __shared__ __align__(16) uint16_t sx[KC * 1024];
  __shared__ float red[W8];
  const int K = p.K;
  const int lane = threadIdx.x & 63;
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  int r0, nrows;
  b128_range(p.gtotal, r0, nrows);
  if (nrows == 0) return;
  const int mine = (nrows - wid + W8 - 1) / W8;  // this wave's slots (<= RPW, checked on the host)

  // in this order (loads complete in order): activation, residuals, every
  // slot's scales, the first D slots' rows
  XIn<2 * KC, kB128Threads> xin;
  block_x_load<2 * KC, kB128Threads>(xin, p.x, p.x2, p.norm_w, K, p.gnorm_w, p.gnorm_d);
  // residuals of this wave's slots (lane i: slot wid + 8 i) as raw bf16 bits,
  // branch-free: one resource over the range, kOob past it or without res
  uint32_t r1, r2;
  {
    const uint32_t off = lane < mine ? (uint32_t)(r0 + wid + W8 * lane) * 2u : kOob;
    const uint32_t rb = (uint32_t)p.gtotal * 2u;
    r1 = bload_u16(make_rsrc(p.res1 ? p.res1 : p.x, p.res1 ? rb : 0u), off);
    r2 = bload_u16(make_rsrc(p.res2 ? p.res2 : p.x, p.res2 ? rb : 0u), off);
  }
  float sc[RPW][SR];
#pragma unroll
  for (int i = 0; i < RPW; ++i) {
    const bool valid = i < mine;
    int row;
    const QhGemvSeg sg = seg_of(p, r0 + (valid ? wid + W8 * i : 0), row);
    b128_scales<KC, ScaleT>(sc[i], sg.s, row, valid, K, lane);
  }
  u32x4 w[D][KC];
#pragma unroll
  for (int i = 0; i < D; ++i) {
    const bool valid = i < mine;
    int row;
    const QhGemvSeg sg = seg_of(p, r0 + (valid ? wid + W8 * i : 0), row);
    b128_row<KC>(w[i], sg.w, row, valid, K, lane);
  }
  block_x_finish<2 * KC, kB128Threads, true>(xin, sx, red, p.x2 != nullptr, p.norm_w != nullptr, p.eps, K,
                                             p.gnorm_w ? p.gnorm_d : 0);
  u32x4 xa[KC], xb[KC];
  b128_x<KC>(xa, xb, sx, K, lane);
  float res = 0.0f;
  if (p.res1) res = p.res2 ? rbf(bf2f((uint16_t)r1) + bf2f((uint16_t)r2)) : bf2f((uint16_t)r1);
  b128_rows<0, KC, RPW, D>(p, w, sc, xa, xb, res, r0, mine, lane, wid);
}

// Paired gate/up with the SiLU(g) * u epilogue: a slot is gate row r and up
// row r (5 KB at K = 2560; one slot in flight per wave).
template <int I, int KC, int RPW>
__device__ __forceinline__ void b128_pairs(const QhMlpParams& p, u32x4 (&wg)[KC], u32x4 (&wu)[KC],
                                           const float (&sg)[RPW][b128_sregs<KC>()],
                                           const float (&su)[RPW][b128_sregs<KC>()], const u32x4 (&xa)[KC],
                                           const u32x4 (&xb)[KC], int r0, int mine, int lane, int wid) {
  if constexpr (I < RPW) {
    if (I >= mine) return;
    const int K = p.K;
    const float pg = b128_dot<KC>(wg, sg[I], xa, xb, K, lane);
    const float pu = b128_dot<KC>(wu, su[I], xa, xb, K, lane);
    if constexpr (I + 1 < RPW) {
      const bool valid = I + 1 < mine;
      const int row = r0 + (valid ? wid + kB128Waves * (I + 1) : 0);
      b128_row<KC>(wg, p.wg, row, valid, K, lane);
      b128_row<KC>(wu, p.wu, row, valid, K, lane);
    }
    const float ag = wave_total(pg);
    const float au = wave_total(pu);
    if (lane == 0) {
      const int g = r0 + wid + kB128Waves * I;
      // SiLU on the fp32 accumulators (fused_kernels.cu:476).
      p.m_out[g] = f2bf(qh_silu(ag) * au);
      if (p.g_out) p.g_out[g] = f2bf(ag);
      if (p.u_out) p.u_out[g] = f2bf(au);
    }
    b128_pairs<I + 1, KC, RPW>(p, wg, wu, sg, su, xa, xb, r0, mine, lane, wid);
  }
}

template <int KC, int RPW, typename ScaleT>
__global__ __launch_bounds__(kB128Threads) void mlp_b128_kernel(QhMlpParams p) {
  constexpr int SR = b128_sregs<KC>();
  constexpr int W8 = kB128Waves;
  __shared__ __align__(16) uint16_t sx[KC * 1024];
  __shared__ float red[W8];
  const int K = p.K;
  const int lane = threadIdx.x & 63;
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  int r0, nrows;
  b128_range(p.N, r0, nrows);
  if (nrows == 0) return;
  const int mine = (nrows - wid + W8 - 1) / W8;

  XIn<2 * KC, kB128Threads> xin;
  block_x_load<2 * KC, kB128Threads>(xin, p.x, p.x2, p.norm_w, K);
  float sg[RPW][SR], su[RPW][SR];
#pragma unroll
  for (int i = 0; i < RPW; ++i) {
    const bool valid = i < mine;
    const int row = r0 + (valid ? wid + W8 * i : 0);
    b128_scales<KC, ScaleT>(sg[i], p.sg, row, valid, K, lane);
    b128_scales<KC, ScaleT>(su[i], p.su, row, valid, K, lane);
  }
  u32x4 wg[KC], wu[KC];
  {
    const bool valid = 0 < mine;
    const int row = r0 + wid;
    b128_row<KC>(wg, p.wg, row, valid, K, lane);
    b128_row<KC>(wu, p.wu, row, valid, K, lane);
  }
  block_x_finish<2 * KC, kB128Threads, true>(xin, sx, red, p.x2 != nullptr, p.norm_w != nullptr, p.eps, K);
  u32x4 xa[KC], xb[KC];
  b128_x<KC>(xa, xb, sx, K, lane);
  b128_pairs<0, KC, RPW>(p, wg, wu, sg, su, xa, xb, r0, mine, lane, wid);
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
  float best_v = -INFINITY;
  int best_i = 0x7fffffff;

  __shared__ __align__(16) uint16_t sx[CPL * 512];
  __shared__ float red[4];
  // Each wave streams a contiguous range of row groups (194.1 us for
  // 248320 x 2560 on MI355X, against 196.4 us with groups dealt round-robin
  // over the grid's waves).
  const int nwaves = gridDim.x * 4;
  const int per = (ngroups + nwaves - 1) / nwaves;
  int g = (blockIdx.x * 4 + wid) * per;
  const int gend = min(ngroups, g + per);
  const int stride = 1;
  u32x4 wa[R][CPL];
  if (g < gend) load_bf16_rows<CPL, R>(wa, p.w, p.N, g * R, K, lane);
  u32x4 xr[CPL];
  block_x_prologue<CPL>(xr, sx, red, p.x, nullptr, p.norm_w, p.eps, K);

  while (g < gend) {
    const int gn = g + stride;
    u32x4 wb[R][CPL];
    if (gn < gend) load_bf16_rows<CPL, R>(wb, p.w, p.N, gn * R, K, lane);
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
// Generic kernels (any scale mode, any K % 8 == 0): row-group size R and
// pipeline depth P per chunks-per-lane class: one row, one group in flight.
constexpr int gemv_rows(int cpl) { return cpl > 0 ? 1 : 1; }
constexpr int gemv_depth(int cpl) { return cpl > 0 ? 1 : 1; }
constexpr uint32_t kMaxBufferBytes = 0x7fffffffu;

int cu_count() {
  static int cus[16] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 16) return 256;
  if (cus[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n < 1) n = 256;
    cus[dev] = n;
  }
  return cus[dev];
}

// Workgroups of `fn` (256 threads) that fit on the current device at once.
int resident_blocks(const void* fn) {
  static std::mutex mu;
  static std::map<std::pair<const void*, int>, int> cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 256;
  std::lock_guard<std::mutex> lk(mu);
  auto it = cache.find({fn, dev});
  if (it != cache.end()) return it->second;
  int per_cu = 0, cus = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, 256, 0) != hipSuccess || per_cu < 1)
    per_cu = 1;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 1)
    cus = 1;
  const int n = per_cu * cus;
  cache[{fn, dev}] = n;
  return n;
}

template <int CPL, bool BLK, typename ScaleT>
void launch_gemv_t(const QhGemvParams& p, hipStream_t st) {
  constexpr int R = gemv_rows(CPL), P = gemv_depth(CPL);
  auto fn = gemv_e4m3_kernel<CPL, R, P, BLK, ScaleT>;
  const int grid = std::max(1, std::min(resident_blocks((const void*)fn), (p.gtotal + 3) / 4));
  hipLaunchKernelGGL(fn, dim3(grid), dim3(256), 0, st, p);
}

template <int CPL, bool BLK, typename ScaleT>
void launch_mlp_t(const QhMlpParams& p, hipStream_t st) {
  constexpr int R = gemv_rows(CPL), P = gemv_depth(CPL);
  auto fn = mlp_gate_up_kernel<CPL, R, P, BLK, ScaleT>;
  const int ng = (p.N + R - 1) / R;
  const int grid = std::max(1, std::min(resident_blocks((const void*)fn), (ng + 3) / 4));
  hipLaunchKernelGGL(fn, dim3(grid), dim3(256), 0, st, p);
}

template <int CPL, typename ScaleT>
void launch_gemv_fast_t(const QhGemvParams& p, hipStream_t st) {
  // Two workgroups per CU, each wave walking several rows, measured faster than
  // filling every slot.
  auto fn = gemv_fast_kernel<CPL, fast_depth(CPL), ScaleT>;
  const int grid = std::max(1, std::min({resident_blocks((const void*)fn), 2 * cu_count(), (p.gtotal + 3) / 4}));
  hipLaunchKernelGGL(fn, dim3(grid), dim3(256), 0, st, p);
}

// 128-bit paced kernels: every shape whose rows split over the CUs leave at
// most 64 slots per wave (K = 1024 KC for the instantiated KC, K % 512 == 0).
// Measured on MI355X against the register pipeline (gemv_fast_kernel /
// mlp_fast_kernel), graphs over more weight copies than the MALL holds:
//   12352 x 2560  8.43 -> 7.92 us    10240 x 2560  7.85 -> 6.81 us
//    9216 x 2560  7.08 -> 6.43 us     2560 x 9216  7.35 -> 6.47 us
//    2560 x 4096  5.01 -> 4.06 us     gate/up 2 x 9216 x 2560  9.48 -> 9.32 us
// Row slots per wave instantiated: 2, 5 or 7 (the launch's count rounded up).
inline int b128_rpw(int n) {
  const int need = (n + cu_count() - 1) / cu_count();
  const int per_wave = (need + kB128Waves - 1) / kB128Waves;
  return per_wave <= 2 ? 2 : per_wave <= 5 ? 5 : per_wave <= 7 ? 7 : 0;
}

template <typename ScaleT>
bool try_gemv_b128(const QhGemvParams& p, hipStream_t st) {
  if (p.K % 512 != 0) return false;
  const int rpw = b128_rpw(p.gtotal);
  const dim3 grid(cu_count()), block(kB128Threads);
#define B(KCV)                                                                                     \
  do {                                                                                             \
    if (rpw == 2) hipLaunchKernelGGL((gemv_b128_kernel<KCV, 2, ScaleT>), grid, block, 0, st, p);   \
    else if (rpw == 5) hipLaunchKernelGGL((gemv_b128_kernel<KCV, 5, ScaleT>), grid, block, 0, st, p); \
    else hipLaunchKernelGGL((gemv_b128_kernel<KCV, 7, ScaleT>), grid, block, 0, st, p);             \
    return true;                                                                                   \
  } while (0)
  if (rpw == 0) return false;
  switch ((p.K + 1023) / 1024) {
    case 1: B(1);
    case 2: B(2);
    case 3: B(3);
    case 4: B(4);
    case 5: B(5);
    case 6: B(6);
    case 8: B(8);
    case 9: B(9);
    default: return false;
  }
#undef B
}

template <typename ScaleT>
bool try_mlp_b128(const QhMlpParams& p, hipStream_t st) {
  if (p.K % 512 != 0) return false;
  const int rpw = b128_rpw(p.N);
  const dim3 grid(cu_count()), block(kB128Threads);
#define B(KCV)                                                                                    \
  do {                                                                                            \
    if (rpw == 2) hipLaunchKernelGGL((mlp_b128_kernel<KCV, 2, ScaleT>), grid, block, 0, st, p);   \
    else if (rpw == 5) hipLaunchKernelGGL((mlp_b128_kernel<KCV, 5, ScaleT>), grid, block, 0, st, p); \
    else hipLaunchKernelGGL((mlp_b128_kernel<KCV, 7, ScaleT>), grid, block, 0, st, p);             \
    return true;                                                                                  \
  } while (0)
  if (rpw == 0) return false;
  switch ((p.K + 1023) / 1024) {
    case 1: B(1);
    case 2: B(2);
    case 3: B(3);
    case 4: B(4);
    case 5: B(5);
    case 6: B(6);
    case 8: B(8);
    case 9: B(9);
    default: return false;
  }
#undef B
}

template <int CPL, typename ScaleT>
void launch_mlp_fast_t(const QhMlpParams& p, hipStream_t st) {
  auto fn = mlp_fast_kernel<CPL, mlp_fast_depth(CPL), ScaleT>;
  const int grid = std::max(1, std::min({resident_blocks((const void*)fn), 2 * cu_count(), (p.N + 3) / 4}));
  hipLaunchKernelGGL(fn, dim3(grid), dim3(256), 0, st, p);
}

// Fast-path K values (K = 512 * CPL); other K use the generic kernels.
#define QH_FAST_DISPATCH(CPL_VAL, CALL) \
  switch (CPL_VAL) {                    \
    case 2: CALL(2); return 0;          \
    case 4: CALL(4); return 0;          \
    case 5: CALL(5); return 0;          \
    case 6: CALL(6); return 0;          \
    case 8: CALL(8); return 0;          \
    case 10: CALL(10); return 0;        \
    case 12: CALL(12); return 0;        \
    case 16: CALL(16); return 0;        \
    case 18: CALL(18); return 0;        \
    default: break;                     \
  }

// Smallest supported chunks-per-lane >= ceil(K / 512); 0 when K is too large.
int pick_cpl(int K) {
  static const int kCpl[] = {1, 2, 3, 4, 5, 6, 8, 10, 12, 16, 18, 20, 24, 32};
  const int need = (K + 511) / 512;
  for (int c : kCpl)
    if (c >= need) return c;
  return 0;
}

#define QH_CPL_DISPATCH(CPL_VAL, CALL) \
  switch (CPL_VAL) {                     \
    case 1: CALL(1); break;              \
    case 2: CALL(2); break;              \
    case 3: CALL(3); break;              \
    case 4: CALL(4); break;              \
    case 5: CALL(5); break;              \
    case 6: CALL(6); break;              \
    case 8: CALL(8); break;              \
    case 10: CALL(10); break;            \
    case 12: CALL(12); break;            \
    case 16: CALL(16); break;            \
    case 18: CALL(18); break;            \
    case 20: CALL(20); break;            \
    case 24: CALL(24); break;            \
    case 32: CALL(32); break;            \
    default: return -1;                  \
  }

// ---- plain read stream (the measured read floor) ---------------------------
// Reads `bytes` bytes (< 2^31) with the lm_head's weight load (non-temporal,
// 16 bytes per lane, so one wave instruction reads 1 KB contiguous).  Wave w of
// the grid reads its own contiguous `wave_bytes` from byte w * wave_bytes, as
// the GEMVs' waves stream their rows, in batches of 8 loads with the next batch
// in flight while one is consumed, and writes one XOR checksum per workgroup so
// that no load is dead.  Each wave's loads go through a buffer resource over
// exactly its share: past the end they return zeros without memory traffic,
// so the loop has no branch and every wave runs the same trip count.  What one
// launch can read of the same bytes: the floor the decode kernels are measured
// against beside the 8 TB/s peak.
__global__ __launch_bounds__(256) void read_stream_kernel(const uint8_t* __restrict__ src, uint32_t bytes,
                                                          uint32_t wave_bytes, unsigned* __restrict__ out) {
  constexpr int U = 8;
  constexpr uint32_t kLoad = 64 * 16;  // bytes per wave load
  __shared__ unsigned red[4];
  const int lane = threadIdx.x & 63;
  const uint32_t w0 = (blockIdx.x * 4u + (threadIdx.x >> 6)) * wave_bytes;
  const uint32_t len = w0 < bytes ? min(wave_bytes, bytes - w0) : 0u;
  const qh_rsrc r = make_rsrc(src + (w0 < bytes ? w0 : 0u), len);
  const uint32_t batch = U * kLoad;
  const uint32_t nb = (wave_bytes + batch - 1) / batch;  // batches, the same in every wave
  uint32_t off = (uint32_t)lane * 16u;
  unsigned acc = 0;
  u32x4 va[U], vb[U];
  auto issue = [&](u32x4 (&v)[U], uint32_t o) {
#pragma unroll
    for (int u = 0; u < U; ++u) v[u] = __builtin_amdgcn_raw_buffer_load_b128(r, o + u * kLoad, 0, 2 /* nt */);
  };
  auto consume = [&](const u32x4 (&v)[U]) {
#pragma unroll
    for (int u = 0; u < U; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  };
  issue(va, off);
  for (uint32_t b = 0; b < nb; b += 2) {
    issue(vb, off + batch);
    consume(va);
    issue(va, off + 2 * batch);
    consume(vb);
    off += 2 * batch;
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) acc ^= (unsigned)__shfl_xor((int)acc, m, 64);
  if (lane == 0) red[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) out[blockIdx.x] = red[0] ^ red[1] ^ red[2] ^ red[3];
}

}  // namespace

int qh_launch_gemv(QhGemvParams p, bool scale_bf16, hipStream_t st) {
  const int cpl = pick_cpl(p.K);
  if (cpl == 0) {
    qh_set_error("gemv: K=%d exceeds the supported maximum (16384)", p.K);
    return -1;
  }
  constexpr int R = 1;
  static_assert(gemv_rows(1) == R && gemv_rows(32) == R, "group size must not depend on CPL");
  bool blk = true;
  p.gstart[0] = 0;
  for (int i = 0; i < p.nseg; ++i) {
    const QhGemvSeg& sg = p.seg[i];
    const uint32_t sbytes = scale_count(sg.kb, sg.n) * (scale_bf16 ? 2u : 4u);
    if ((uint64_t)sg.n * (uint64_t)p.K > kMaxBufferBytes || sbytes > kMaxBufferBytes) {
      qh_set_error("gemv: segment %d (%d x %d) exceeds 2^31 bytes", i, sg.n, p.K);
      return -1;
    }
    blk = blk && sg.kb > 1;
    p.gstart[i + 1] = p.gstart[i] + (sg.n + R - 1) / R;
  }
  for (int i = p.nseg + 1; i < 5; ++i) p.gstart[i] = p.gstart[p.nseg];
  p.gtotal = p.gstart[p.nseg];
  if (p.gtotal == 0) return 0;
  bool fast = p.K % 512 == 0;
  for (int i = 0; i < p.nseg; ++i) fast = fast && p.seg[i].kb == p.K / 128;
  if (p.gnorm_w && (!fast || p.gnorm_d != 128 || !p.x2 || p.norm_w)) {
    qh_set_error("gemv: the gated-norm prologue needs K %% 512 == 0, 128x128 block scales, head "
                 "dim 128 (got %d) and a gate vector, and excludes the (1+w) norm",
                 p.gnorm_d);
    return -1;
  }
  if (fast && (scale_bf16 ? try_gemv_b128<uint16_t>(p, st) : try_gemv_b128<float>(p, st))) return 0;
  if (fast) {
#define F(C) (scale_bf16 ? launch_gemv_fast_t<C, uint16_t>(p, st) : launch_gemv_fast_t<C, float>(p, st))
    QH_FAST_DISPATCH(p.K / 512, F)
#undef F
  }
#define G(C)                                                              \
  (blk ? (scale_bf16 ? launch_gemv_t<C, true, uint16_t>(p, st)             \
                     : launch_gemv_t<C, true, float>(p, st))               \
       : (scale_bf16 ? launch_gemv_t<C, false, uint16_t>(p, st)            \
                     : launch_gemv_t<C, false, float>(p, st)))
  QH_CPL_DISPATCH(cpl, G)
#undef G
  return 0;
}

int qh_launch_mlp(QhMlpParams p, bool scale_bf16, hipStream_t st) {
  const int cpl = pick_cpl(p.K);
  if (cpl == 0) {
    qh_set_error("mlp: K=%d exceeds the supported maximum (16384)", p.K);
    return -1;
  }
  if (p.N <= 0) return 0;
  if ((uint64_t)p.N * (uint64_t)p.K > kMaxBufferBytes) {
    qh_set_error("mlp: %d x %d exceeds 2^31 bytes", p.N, p.K);
    return -1;
  }
  if (p.K % 512 == 0 && p.kb == p.K / 128 &&
      (scale_bf16 ? try_mlp_b128<uint16_t>(p, st) : try_mlp_b128<float>(p, st)))
    return 0;
  if (p.K % 512 == 0 && p.kb == p.K / 128) {
#define F(C) (scale_bf16 ? launch_mlp_fast_t<C, uint16_t>(p, st) : launch_mlp_fast_t<C, float>(p, st))
    QH_FAST_DISPATCH(p.K / 512, F)
#undef F
  }
  const bool blk = p.kb > 1;
#define M(C)                                                              \
  (blk ? (scale_bf16 ? launch_mlp_t<C, true, uint16_t>(p, st)              \
                     : launch_mlp_t<C, true, float>(p, st))                \
       : (scale_bf16 ? launch_mlp_t<C, false, uint16_t>(p, st)             \
                     : launch_mlp_t<C, false, float>(p, st)))
  QH_CPL_DISPATCH(cpl, M)
#undef M
  return 0;
}

int qh_launch_read_stream(const void* src, uint64_t bytes, unsigned* out, int out_len, hipStream_t st) {
  if (!src || !out || out_len < 1 || bytes == 0 || bytes % 16 != 0 || bytes > (1ull << 31) ||
      ((uintptr_t)src & 15) != 0) {
    qh_set_error("read_stream: needs a 16-byte aligned source, a non-zero multiple of 16 bytes up to "
                 "2^31 (got %llu) and an output of at least one word", (unsigned long long)bytes);
    return -1;
  }
  const int grid = std::min(out_len, 4 * cu_count());
  // each wave's share, whole 1 KB wave loads
  const uint64_t waves = 4ull * (uint64_t)grid;
  const uint32_t wave_bytes = (uint32_t)((bytes + waves * 1024 - 1) / (waves * 1024) * 1024);
  hipLaunchKernelGGL(read_stream_kernel, dim3(grid), dim3(256), 0, st, (const uint8_t*)src, (uint32_t)bytes,
                     wave_bytes, out);
  return 0;
}

int qh_lm_head_grid(int N) {
  // 512 workgroups (two per CU): 768 and 1024 measured 200.3 and 208.6 us
  // against 194.1 us.
  const int ng = (N + 3) / 4;
  return std::max(1, std::min(512, (ng + 3) / 4));
}

int qh_launch_lm_head(QhLmHeadParams p, int grid, hipStream_t st) {
  const int cpl = pick_cpl(p.K);
  if (cpl == 0 || cpl > 8) {
    qh_set_error("lm_head: K=%d unsupported (need K <= 4096)", p.K);
    return -1;
  }
  // Two-row groups, two in flight per wave: 186.5 us for 248320 x 2560 on
  // MI355X (6.8 TB/s), against 194 us with four-row groups.
#define L(C) hipLaunchKernelGGL((lm_head_argmax_kernel<(C <= 8 ? C : 8), 2>), dim3(grid), dim3(256), 0, st, p)
  QH_CPL_DISPATCH(cpl, L)
#undef L
  return 0;
}
