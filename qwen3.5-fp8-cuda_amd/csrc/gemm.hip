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
// v_mfma_scale_f32_32x32x64_f8f6f4 (E4M3 operands, its MX block-scale operands
// fixed at 2^0) and accumulate into one per-K-block partial, which is scaled by
// the W block scale and added to the fp32 accumulator; the row scale s_x is
// applied once in the epilogue.
//
// Tiling: BM x BN output tile per 256-thread workgroup (64x64, or 128x128 when
// there are enough tiles), a 2 x 2 grid of waves each holding (BM/2) x (BN/2)
// of 32x32 matrix-core tiles.  Each 128-wide K block of A hi, A lo and B is
// staged once per workgroup in LDS (rows padded to 144 bytes against bank
// conflicts, one or two stages), the next one or two blocks in registers
// while the current one is multiplied.  Within a K block, lane half h of a 32x32x64 instruction
// takes bytes [64q + 32h, +32) of its row in both operands: the same K
// permutation on A and B leaves the contraction unchanged.
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

// gfx950 variant: operands staged through LDS once per workgroup (the four
// waves of a tile share its A and B rows), the next K blocks loaded into
// registers while the current one is multiplied, and the 32x32x64 fp8
// matrix-core instruction (its block-scale operands fixed at 2^0: the
// checkpoint's fp32 block scale is applied per 128-wide K block in fp32).
// A, A_lo and B rows of a K block are 128 bytes; LDS rows are padded to 144
// bytes so the 32 rows a lane group reads at one column land in distinct banks.
typedef int v8i __attribute__((ext_vector_type(8)));
constexpr int kGRow = 144;                      // padded LDS row (bytes)

__device__ __forceinline__ v8i lds_v8(const uint8_t* p) {
  const u32x4 a = *(const u32x4*)p, b = *(const u32x4*)(p + 16);
  return v8i{(int)a.x, (int)a.y, (int)a.z, (int)a.w, (int)b.x, (int)b.y, (int)b.z, (int)b.w};
}

// LDS bytes of one K-block stage of a BM x BN tile: A hi, A lo (BM rows), B
// (BN rows), then the BN fp32 weight scales of the block.
constexpr int gemm_stage_bytes(int bm, int bn) { return (2 * bm + bn) * kGRow + bn * 4; }

// NST LDS stages (1 or 2) and D K blocks in flight in registers.  The K loop
// is unrolled by D so the register sets rotate statically; loads past the
// last block re-read it (no branch, so the in-order load counter waits only
// for the block about to be stored).  Requires (K / 128) % D == 0.
// Up to four projections of the same activation in one launch: segment t
// owns N tiles [tstart[t], tstart[t + 1]) of the grid's x dimension.
struct GemmGroup {
  const uint8_t* w[4];
  const void* s[4];
  uint16_t* y[4];
  int N[4];
  int kb[4];
  int tstart[4];
  int nseg;
};

template <typename ScaleT, int BM, int BN, int NST, int D>
// Split-K (part != null): blockIdx.z takes K blocks [z KB/S, (z+1) KB/S) of
// S = gridDim.z and stores its fp32 partial tile, unscaled, at
// part[(z M + m) ldp + global column]; gemm_splitk_reduce_kernel finishes.
__global__ __launch_bounds__(256) void gemm_e4m3_lds_kernel(const uint8_t* xhi, const uint8_t* xlo,
                                                            const float* sx, GemmGroup g, int M,
                                                            int K, float* part, int ldp) {
  constexpr int WM = BM / 2, WN = BN / 2;        // this wave's sub-tile (2 x 2 waves)
  constexpr int TI = WM / 32, TJ = WN / 32;      // 32x32 matrix-core tiles per wave
  constexpr int STAGE = gemm_stage_bytes(BM, BN);
  constexpr int PIECES = (2 * BM + BN) * 8;      // 16-byte pieces per K block
  constexpr int PPT = PIECES / 256;              // per thread
  static_assert(PIECES % 256 == 0 && TI >= 1 && TJ >= 1 && (NST == 1 || NST == 2), "tile shape");
  extern __shared__ __align__(16) uint8_t smem[];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wid = tid >> 6;
  // this workgroup's segment (uniform across the workgroup)
  int si = 0;
#pragma unroll
  for (int t = 1; t < 4; ++t)
    if (t < g.nseg && (int)blockIdx.x >= g.tstart[t]) si = t;
  const uint8_t* w = g.w[si];
  const ScaleT* sw = (const ScaleT*)g.s[si];
  uint16_t* y = g.y[si];
  const int N = g.N[si], kb_code = g.kb[si];
  const int mb = blockIdx.y * BM, nb = ((int)blockIdx.x - g.tstart[si]) * BN;
  const int wm = (wid >> 1) * WM, wn = (wid & 1) * WN;
  const int r = lane & 31, h = lane >> 5;
  const int KB = K / 128 / (int)gridDim.z;        // K blocks of this workgroup
  const int kb0 = (int)blockIdx.z * KB;

  // Global -> register staging: piece p is (operand row, 16-byte column) of
  // the stage's rows [A hi (BM) | A lo (BM) | B (BN)].
  // The block's weight scales travel with its operands and are staged in LDS
  // beside them: a scale loaded at use time would sit behind every prefetched
  // block in the in-order load counter and drain the pipeline at each K step.
  // Thread t loads the scale of tile column t % BN (every thread loads, so no
  // load sits under a branch).
  constexpr int SC_OFF = (2 * BM + BN) * kGRow;
  u32x4 st[D][PPT];
  float scv[D];
  auto gload = [&](u32x4 (&dst)[PPT], float& sdst, int kb) {
    kb = kb0 + min(kb, KB - 1);
    const int ko = kb * 128;
    sdst = load_scale<ScaleT>(sw, scale_index(kb_code, min(nb + tid % BN, N - 1), kb));
#pragma unroll
    for (int e = 0; e < PPT; ++e) {
      const int piece = tid + 256 * e;
      const int row = piece >> 3, c16 = (piece & 7) * 16;
      if (row < 2 * BM) {
        const int m = min(mb + (row % BM), M - 1);
        dst[e] = *(const u32x4*)((row < BM ? xhi : xlo) + (size_t)m * K + ko + c16);
      } else {
        const int n = min(nb + row - 2 * BM, N - 1);
        dst[e] = __builtin_nontemporal_load((const u32x4*)(w + (size_t)n * K + ko + c16));
      }
    }
  };
  auto sstore = [&](uint8_t* stage, const u32x4 (&src)[PPT], float sc) {
#pragma unroll
    for (int e = 0; e < PPT; ++e) {
      const int piece = tid + 256 * e;
      *(u32x4*)(stage + (piece >> 3) * kGRow + (piece & 7) * 16) = src[e];
    }
    if (tid < BN) *(float*)(stage + SC_OFF + tid * 4) = sc;
  };

  v16f acc[TI][TJ];
#pragma unroll
  for (int i = 0; i < TI; ++i)
#pragma unroll
    for (int j = 0; j < TJ; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

  auto mma_block = [&](const uint8_t* cur) {
    float swj[TJ];
#pragma unroll
    for (int j = 0; j < TJ; ++j) swj[j] = *(const float*)(cur + SC_OFF + (wn + 32 * j + r) * 4);
    v16f t[TI][TJ];
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
      for (int j = 0; j < TJ; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) t[i][j][e] = 0.0f;
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      // lane half h takes K bytes [64q + 32h, +32) of its row in both operands
      const int co = 64 * q + 32 * h;
      v8i ah[TI], al[TI], bw[TJ];
#pragma unroll
      for (int i = 0; i < TI; ++i) {
        ah[i] = lds_v8(cur + (wm + 32 * i + r) * kGRow + co);
        al[i] = lds_v8(cur + (BM + wm + 32 * i + r) * kGRow + co);
      }
#pragma unroll
      for (int j = 0; j < TJ; ++j) bw[j] = lds_v8(cur + (2 * BM + wn + 32 * j + r) * kGRow + co);
#pragma unroll
      for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j) {
          t[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(ah[i], bw[j], t[i][j], 0, 0, 0, 127, 0, 127);
          t[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(al[i], bw[j], t[i][j], 0, 0, 0, 127, 0, 127);
        }
    }
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
      for (int j = 0; j < TJ; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[i][j][e] = fmaf(t[i][j][e], swj[j], acc[i][j][e]);
  };

  // Prologue: blocks 0..D-1 in registers, block 0 in LDS stage 0, block D
  // loaded into the freed register set.
#pragma unroll
  for (int d = 0; d < D; ++d) gload(st[d], scv[d], d);
  sstore(smem, st[0], scv[0]);
  gload(st[0], scv[0], D);
  __syncthreads();
  // Invariant at step k: LDS stage (k % NST) holds block k, register set
  // (k + 1) % D holds block k + 1.
  for (int k0 = 0; k0 < KB; k0 += D) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      const int k = k0 + d;
      mma_block(smem + (NST == 2 ? (k & 1) * STAGE : 0));
      if constexpr (NST == 1) __syncthreads();   // one stage: every wave is done reading it
      const int nx = (d + 1) % D;   // static once the loop is unrolled
      sstore(smem + (NST == 2 ? ((k + 1) & 1) * STAGE : 0), st[nx], scv[nx]);
      gload(st[nx], scv[nx], k + 1 + D);
      __syncthreads();
    }
  }

  // C layout of a 32x32 tile: lane -> column lane%32, value e -> row
  // 8*(e/4) + 4*(lane/32) + e%4.
  if (part) {
    float* pz = part + (size_t)blockIdx.z * M * ldp;
    const int ng0 = (int)blockIdx.x * BN;
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int m = mb + wm + 32 * i + 8 * (e >> 2) + 4 * h + (e & 3);
        if (m >= M) continue;
#pragma unroll
        for (int j = 0; j < TJ; ++j) pz[(size_t)m * ldp + ng0 + wn + 32 * j + r] = acc[i][j][e];
      }
    return;
  }
#pragma unroll
  for (int i = 0; i < TI; ++i) {
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int m = mb + wm + 32 * i + 8 * (e >> 2) + 4 * h + (e & 3);
      if (m >= M) continue;
      const float s = sx[m];
#pragma unroll
      for (int j = 0; j < TJ; ++j) {
        const int n = nb + wn + 32 * j + r;
        if (n < N) y[(size_t)m * N + n] = f2bf(acc[i][j][e] * s);
      }
    }
  }
}

// Split-K finish: y = bf16(sx[m] * sum_z part[z][m][column]), summed in z
// order; columns past a segment's N (tile padding) are skipped.  Four
// columns per thread (segments start at multiples of 64 columns).
__global__ __launch_bounds__(256) void gemm_splitk_reduce_kernel(const float* part, int S, int M,
                                                                 int ldp, const float* sx,
                                                                 GemmGroup g, int bn) {
  const size_t q = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (q >= (size_t)M * ldp / 4) return;
  const int m = (int)(q / (ldp / 4)), ng = (int)(q % (ldp / 4)) * 4;
  const int tile = ng / bn;
  int si = 0;
#pragma unroll
  for (int t = 1; t < 4; ++t)
    if (t < g.nseg && tile >= g.tstart[t]) si = t;
  const int n = ng - g.tstart[si] * bn, N = g.N[si];
  if (n >= N) return;
  f32x4 acc = *(const f32x4*)(part + (size_t)m * ldp + ng);
  for (int z = 1; z < S; ++z) acc += *(const f32x4*)(part + ((size_t)z * M + m) * ldp + ng);
  const float s = sx[m];
  uint16_t* y = g.y[si] + (size_t)m * N + n;
#pragma unroll
  for (int c = 0; c < 4; ++c)
    if (n + c < N) y[c] = f2bf(acc[c] * s);
}

template <int BN>
GemmGroup make_group(const QhGemmSeg* seg, int nseg, int& tiles_n) {
  GemmGroup g = {};
  g.nseg = nseg;
  tiles_n = 0;
  for (int t = 0; t < nseg; ++t) {
    g.w[t] = (const uint8_t*)seg[t].w;
    g.s[t] = seg[t].s;
    g.y[t] = (uint16_t*)seg[t].y;
    g.N[t] = seg[t].N;
    g.kb[t] = seg[t].kb;
    g.tstart[t] = tiles_n;
    tiles_n += (seg[t].N + BN - 1) / BN;
  }
  return g;
}

template <typename ScaleT, int BM, int BN, int NST, int D>
void launch_gemm_lds(const uint8_t* xhi, const uint8_t* xlo, const float* sx, const QhGemmSeg* seg,
                     int nseg, int M, int K, hipStream_t st, int S = 1, float* part = nullptr) {
  int tiles_n = 0;
  const GemmGroup g = make_group<BN>(seg, nseg, tiles_n);
  dim3 grid(tiles_n, (M + BM - 1) / BM, S);
  const int ldp = tiles_n * BN;
  hipLaunchKernelGGL((gemm_e4m3_lds_kernel<ScaleT, BM, BN, NST, D>), grid, dim3(256),
                     NST * (size_t)gemm_stage_bytes(BM, BN), st, xhi, xlo, sx, g, M, K,
                     S > 1 ? part : nullptr, ldp);
  if (S > 1) {
    const size_t quads = (size_t)M * ldp / 4;
    hipLaunchKernelGGL(gemm_splitk_reduce_kernel, dim3((unsigned)((quads + 255) / 256)), dim3(256),
                       0, st, (const float*)part, S, M, ldp, sx, g, BN);
  }
}

// 64x64 tiles.  With at least three tiles per CU, one LDS stage (27.6 KB)
// lets four workgroups share a CU; with fewer tiles, two stages and two K
// blocks in flight per workgroup.  M = 512: 9216 x 2560 50 us (1 stage) vs
// 55 us (2 stages); 2560 x 9216 67 us (2 stages, 2 in flight) vs 70 us.
// S > 1: split-K over S slices of K (partials in `part`); the variant is
// chosen by the workgroup count tiles * S and the per-slice K block count.
template <typename ScaleT>
void launch_gemm_small(const uint8_t* xhi, const uint8_t* xlo, const float* sx, const QhGemmSeg* seg,
                       int nseg, int M, int K, long tiles, hipStream_t st, int cus, int S,
                       float* part) {
  const int kbl = K / 128 / S;
  if (tiles * S >= 3L * cus)
    launch_gemm_lds<ScaleT, 64, 64, 1, 1>(xhi, xlo, sx, seg, nseg, M, K, st, S, part);
  else if (kbl % 2 == 0)
    launch_gemm_lds<ScaleT, 64, 64, 2, 2>(xhi, xlo, sx, seg, nseg, M, K, st, S, part);
  else
    launch_gemm_lds<ScaleT, 64, 64, 2, 1>(xhi, xlo, sx, seg, nseg, M, K, st, S, part);
}

std::mutex g_ws_mu;
void* g_ws = nullptr;
size_t g_ws_bytes = 0;

}  // namespace

// Workspace: the activation's hi and lo E4M3 terms (M x K bytes each), the
// row scales, then the split-K partials.  A split GEMM runs S * tiles <= 3 per
// CU workgroups of 64x64 fp32 partials, so kSplitPartBytes covers up to 1024
// of them (341 CUs).
constexpr size_t kSplitPartBytes = (size_t)1024 * 64 * 64 * sizeof(float);

size_t qh_gemm_workspace_bytes(int M, int K) {
  return (size_t)M * K * 2 + (size_t)M * sizeof(float) + 512 + kSplitPartBytes;
}

int qh_launch_gemm_e4m3_group_ws(const void* x, int M, int K, const QhGemmSeg* seg, int nseg,
                                 bool scale_bf16, void* ws, hipStream_t st) {
  if (K % 128 != 0) {
    qh_set_error("gemm: K=%d must be a multiple of 128", K);
    return -1;
  }
  if (nseg < 1 || nseg > 4) {
    qh_set_error("gemm: nseg=%d outside [1, 4]", nseg);
    return -1;
  }
  long tiles64 = 0, tiles128 = 0;
  for (int t = 0; t < nseg; ++t) {
    if (!seg[t].w || !seg[t].s || !seg[t].y || seg[t].N <= 0) {
      qh_set_error("gemm: segment %d: null pointer or N=%d", t, seg[t].N);
      return -1;
    }
    tiles64 += (seg[t].N + 63) / 64;
    tiles128 += (seg[t].N + 127) / 128;
  }
  uint8_t* xhi = (uint8_t*)ws;
  uint8_t* xlo = xhi + (size_t)M * K;
  float* sx = (float*)(((uintptr_t)(xlo + (size_t)M * K) + 255) & ~(uintptr_t)255);
  hipLaunchKernelGGL(quant_rows_kernel, dim3(M), dim3(256), 0, st, (const uint16_t*)x, xhi, xlo,
                     sx, K);
  // 64x64 tiles unless 128x128 tiles give at least two per CU: at prefill
  // sizes (M of a few hundred rows) the smaller tiles keep every CU busy and
  // measured faster (M = 512: 63 vs 89 us for 9216 x 2560).
  int cus = 256, dev = 0;
  if (hipGetDevice(&dev) == hipSuccess) hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  const bool small = tiles128 * ((M + 127) / 128) < 2L * cus;
  if (small) {
    const long tiles = tiles64 * ((M + 63) / 64);
    // Split-K when there are no more tiles than CUs: the largest S <= 8
    // dividing the K blocks with >= 4 blocks per slice and S * tiles <= 3 per
    // CU, so each workgroup walks fewer serial K steps.  The extra reduce
    // launch costs more than it saves above that (M = 128: 9216 x 2560, 288
    // tiles, 24.7 us unsplit vs 28.8 us in 2; 2560 x 9216, 80 tiles, 46.5 vs
    // 28.7 us in 8).
    const int KB = K / 128;
    int S = 1;
    for (int c = 8; c >= 2 && tiles <= cus; --c)
      if (KB % c == 0 && KB / c >= 4 && tiles * c <= 3L * cus &&
          (size_t)tiles * c * 64 * 64 * sizeof(float) <= kSplitPartBytes) {
        S = c;
        break;
      }
    float* part = (float*)(((uintptr_t)(sx + M) + 255) & ~(uintptr_t)255);
    if (scale_bf16) launch_gemm_small<uint16_t>(xhi, xlo, sx, seg, nseg, M, K, tiles, st, cus, S, part);
    else launch_gemm_small<float>(xhi, xlo, sx, seg, nseg, M, K, tiles, st, cus, S, part);
  } else {
    if (scale_bf16) launch_gemm_lds<uint16_t, 128, 128, 2, 1>(xhi, xlo, sx, seg, nseg, M, K, st);
    else launch_gemm_lds<float, 128, 128, 2, 1>(xhi, xlo, sx, seg, nseg, M, K, st);
  }
  return 0;
}

int qh_launch_gemm_e4m3_ws(const void* x, const void* w, const void* s, void* y, int M, int N,
                           int K, int kb, bool scale_bf16, void* ws, hipStream_t st) {
  const QhGemmSeg seg = {w, s, y, N, kb};
  return qh_launch_gemm_e4m3_group_ws(x, M, K, &seg, 1, scale_bf16, ws, st);
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
