// Prefill block-scaled E4M3 GEMM on the gfx950 matrix cores.
//
// Semantics (reference: qwen3_infer/csrc/fp8_kernels.cu:23-64
// fp8_gemm_batch_kernel; caller main.py:262-269):
//   Y[m, n] = bf16( sum_kb s[n, kb] * sum_{k in kb} X[m, k] * e4m3(W[n, k]) )
//
// Every E4M3 value is a bf16 value (3 mantissa bits, exponent -9 .. 8), so
// the weights are widened to bf16 exactly as they leave LDS for the matrix
// cores, and the bf16 activations go in unchanged: v_mfma_f32_32x32x16_bf16
// forms each product exactly in fp32, as the reference's dequantize-then-
// multiply does, for any activation range.  Each 128-wide K block's fp32
// partial is multiplied by the weight block scale and added to the fp32
// accumulator.  The weights stream from HBM as one byte each; the widening
// (two conversions per two weights) is repeated only by the M / 64 row tiles
// that share a weight tile, and costs half the matrix-core time of its block.
//
// Nothing is precomputed and no workspace is needed; a caller workspace only
// enables split-K (qh_gemm_e4m3 / qh_gemm_e4m3_grouped).  The reference entry
// point fp8_gemm_batch passes none and never splits.
//
// Tiling: 64 x BN output tile per 256-thread workgroup (the launchers use
// BN = 64), a 2 x 2 grid of waves each holding 32 x (BN/2) as BN/64 32x32
// matrix-core tiles; tiles are ordered so that the row tiles of one weight
// tile run on one XCD (see the kernel).  Each 128-wide K block of X (bf16, rows padded to 272 bytes) and W
// (E4M3, rows padded to 144 bytes) is staged once per workgroup in LDS (two
// stages), the next block in registers while the current one is multiplied.
// Operand layout of the 32x32x16 bf16 instruction (measured on gfx950):
// lane l holds A[l % 32][8 (l / 32) + r] and B[8 (l / 32) + r][l % 32],
// r = 0..7, and accumulator value e is C[8 (e / 4) + 4 (l / 32) + e % 4][l % 32].
#include "qh_common.h"
#include "qh_gemm.h"

namespace {

typedef float v16f __attribute__((ext_vector_type(16)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
constexpr int kARow = 272;                      // padded LDS row of the X tile (bytes)
constexpr int kBRow = 144;                      // padded LDS row of the W tile (bytes)
constexpr int kBM = 64;                         // output rows per tile

// Eight E4M3 weights (two words) widened to bf16, exactly.
__device__ __forceinline__ v8bf e4m3x8_bf16(u32x2 w) {
  const auto a = __builtin_amdgcn_cvt_pk_f32_fp8(w.x, false), b = __builtin_amdgcn_cvt_pk_f32_fp8(w.x, true);
  const auto c = __builtin_amdgcn_cvt_pk_f32_fp8(w.y, false), d = __builtin_amdgcn_cvt_pk_f32_fp8(w.y, true);
  return v8bf{(__bf16)a[0], (__bf16)a[1], (__bf16)b[0], (__bf16)b[1],
              (__bf16)c[0], (__bf16)c[1], (__bf16)d[0], (__bf16)d[1]};
}

// LDS of one K-block stage of a 64 x BN tile: X (64 rows), W (BN rows), the
// BN fp32 weight scales of the block.
constexpr int gemm_b_off() { return kBM * kARow; }
constexpr int gemm_scw_off(int bn) { return gemm_b_off() + bn * kBRow; }
constexpr int gemm_stage_bytes(int bn) { return gemm_scw_off(bn) + bn * 4; }

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

// NST LDS stages (1 or 2) and D K blocks in flight in registers.  The K loop
// is unrolled by D so the register sets rotate statically; loads past the
// last block re-read it (no branch, so the in-order load counter waits only
// for the block about to be stored).  Requires (K / 128 / gridDim.z) % D == 0.
// Split-K (part != null): blockIdx.z takes K blocks [z KB, (z+1) KB) and
// stores its fp32 partial tile at part[(z M + m) ldp + global column];
// gemm_splitk_reduce_kernel finishes.
template <typename ScaleT, int BN, int NST, int D>
__global__ __launch_bounds__(256) void gemm_e4m3_lds_kernel(const uint16_t* x, GemmGroup g, int M,
                                                            int K, float* part, int ldp, int tiles_n,
                                                            int tiles_m) {
  constexpr int BM = kBM;
  constexpr int WM = BM / 2, WN = BN / 2;        // this wave's sub-tile (2 x 2 waves)
  constexpr int TJ = WN / 32;                    // 32x32 matrix-core tiles per wave
  constexpr int STAGE = gemm_stage_bytes(BN);
  constexpr int BOFF = gemm_b_off(), SCW = gemm_scw_off(BN);
  constexpr int BPT = BN * 8 / 256;              // 16-byte W pieces per thread
  static_assert(WM == 32 && TJ >= 1 && BPT >= 1 && (NST == 1 || NST == 2), "tile shape");
  extern __shared__ __align__(16) uint8_t smem[];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wid = tid >> 6;
  // XCD-aware tile order: workgroups are dealt to the 8 XCDs round-robin by
  // index, so index q runs on XCD q % 8.  N tile tn goes to XCD tn % 8 with
  // all of its row tiles, which then share the W tile in that XCD's L2 (each
  // XCD reads the whole, small, activation once).  Indices past the last N
  // tile of their XCD have no tile.
  const int q = (int)blockIdx.x;
  const int tn = (q & 7) + 8 * ((q >> 3) / tiles_m), tm = (q >> 3) % tiles_m;
  if (tn >= tiles_n) return;
  // this workgroup's segment (uniform across the workgroup)
  int si = 0;
#pragma unroll
  for (int t = 1; t < 4; ++t)
    if (t < g.nseg && tn >= g.tstart[t]) si = t;
  const uint8_t* w = g.w[si];
  const ScaleT* sw = (const ScaleT*)g.s[si];
  uint16_t* y = g.y[si];
  const int N = g.N[si], kb_code = g.kb[si];
  const int mb = tm * BM, nb = (tn - g.tstart[si]) * BN;
  const int wm = (wid >> 1) * WM, wn = (wid & 1) * WN;
  const int r = lane & 31, h = lane >> 5;
  const int KB = K / 128 / (int)gridDim.z;        // K blocks of this workgroup
  const int kb0 = (int)blockIdx.z * KB;

  // X pieces t + 256 e (tile row p >> 4, 16-byte column p & 15) and W pieces
  // t + 256 e (row p >> 3, 16-byte column p & 7).  Rows past M or N re-read
  // the last one (their results are never stored).  The block's weight scales
  // travel with its operands and are staged in LDS beside them (a scale loaded
  // at use time would sit behind every prefetched block in the in-order load
  // counter): thread t loads the scale of tile column t % BN.
  u32x4 sa[D][4], sb[D][BPT];
  float scv[D];
  auto gload = [&](u32x4 (&da)[4], u32x4 (&db)[BPT], float& sdst, int kb) {
    kb = kb0 + min(kb, KB - 1);
    const int ko = kb * 128;
    sdst = load_scale<ScaleT>(sw, scale_index(kb_code, min(nb + tid % BN, N - 1), kb));
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int piece = tid + 256 * e;
      const int m = min(mb + (piece >> 4), M - 1);
      da[e] = *(const u32x4*)(x + (size_t)m * K + ko + (piece & 15) * 8);
    }
#pragma unroll
    for (int e = 0; e < BPT; ++e) {
      const int piece = tid + 256 * e;
      const int n = min(nb + (piece >> 3), N - 1);
      db[e] = *(const u32x4*)(w + (size_t)n * K + ko + (piece & 7) * 16);
    }
  };
  auto sstore = [&](uint8_t* stage, const u32x4 (&da)[4], const u32x4 (&db)[BPT], float sc) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int piece = tid + 256 * e;
      *(u32x4*)(stage + (piece >> 4) * kARow + (piece & 15) * 16) = da[e];
    }
#pragma unroll
    for (int e = 0; e < BPT; ++e) {
      const int piece = tid + 256 * e;
      *(u32x4*)(stage + BOFF + (piece >> 3) * kBRow + (piece & 7) * 16) = db[e];
    }
    if (tid < BN) *(float*)(stage + SCW + tid * 4) = sc;
  };

  v16f acc[TJ];
#pragma unroll
  for (int j = 0; j < TJ; ++j)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[j][e] = 0.0f;

  auto mma_block = [&](const uint8_t* cur) {
    float swj[TJ];
#pragma unroll
    for (int j = 0; j < TJ; ++j) swj[j] = *(const float*)(cur + SCW + (wn + 32 * j + r) * 4);
    v16f t[TJ];
#pragma unroll
    for (int j = 0; j < TJ; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) t[j][e] = 0.0f;
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) {  // 16-wide K steps of the block
      const v8bf a = *(const v8bf*)(cur + (wm + r) * kARow + 32 * kk + 16 * h);
#pragma unroll
      for (int j = 0; j < TJ; ++j) {
        const v8bf b = e4m3x8_bf16(*(const u32x2*)(cur + BOFF + (wn + 32 * j + r) * kBRow + 16 * kk + 8 * h));
        t[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, t[j], 0, 0, 0);
      }
    }
#pragma unroll
    for (int j = 0; j < TJ; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[j][e] = fmaf(t[j][e], swj[j], acc[j][e]);
  };

  // Prologue: blocks 0..D-1 in registers, block 0 in LDS stage 0, block D
  // loaded into the freed register set.
#pragma unroll
  for (int d = 0; d < D; ++d) gload(sa[d], sb[d], scv[d], d);
  sstore(smem, sa[0], sb[0], scv[0]);
  gload(sa[0], sb[0], scv[0], D);
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
      sstore(smem + (NST == 2 ? ((k + 1) & 1) * STAGE : 0), sa[nx], sb[nx], scv[nx]);
      gload(sa[nx], sb[nx], scv[nx], k + 1 + D);
      __syncthreads();
    }
  }

  // accumulator value e of tile j: row wm + 8 (e / 4) + 4 h + e % 4, column
  // wn + 32 j + r
  if (part) {
    float* pz = part + (size_t)blockIdx.z * M * ldp;
    const int ng0 = tn * BN;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int m = mb + wm + 8 * (e >> 2) + 4 * h + (e & 3);
      if (m >= M) continue;
#pragma unroll
      for (int j = 0; j < TJ; ++j) pz[(size_t)m * ldp + ng0 + wn + 32 * j + r] = acc[j][e];
    }
    return;
  }
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    const int m = mb + wm + 8 * (e >> 2) + 4 * h + (e & 3);
    if (m >= M) continue;
#pragma unroll
    for (int j = 0; j < TJ; ++j) {
      const int n = nb + wn + 32 * j + r;
      if (n < N) y[(size_t)m * N + n] = f2bf(acc[j][e]);
    }
  }
}

// Split-K finish: y = bf16(sum_z part[z][m][column]), summed in z order;
// columns past a segment's N (tile padding) are skipped.  Four columns per
// thread (segments start at multiples of 64 columns).
__global__ __launch_bounds__(256) void gemm_splitk_reduce_kernel(const float* part, int S, int M,
                                                                 int ldp, GemmGroup g, int bn) {
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
  uint16_t* y = g.y[si] + (size_t)m * N + n;
#pragma unroll
  for (int c = 0; c < 4; ++c)
    if (n + c < N) y[c] = f2bf(acc[c]);
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

template <typename ScaleT, int BN, int NST, int D>
void launch_gemm_lds(const uint16_t* x, const QhGemmSeg* seg, int nseg, int M, int K,
                     hipStream_t st, int S = 1, float* part = nullptr) {
  int tiles_n = 0;
  const GemmGroup g = make_group<BN>(seg, nseg, tiles_n);
  const int tiles_m = (M + kBM - 1) / kBM;
  dim3 grid(8 * ((tiles_n + 7) / 8) * tiles_m, 1, S);
  const int ldp = tiles_n * BN;
  hipLaunchKernelGGL((gemm_e4m3_lds_kernel<ScaleT, BN, NST, D>), grid, dim3(256),
                     NST * (size_t)gemm_stage_bytes(BN), st, x, g, M, K, S > 1 ? part : nullptr,
                     ldp, tiles_n, tiles_m);
  if (S > 1) {
    const size_t quads = (size_t)M * ldp / 4;
    hipLaunchKernelGGL(gemm_splitk_reduce_kernel, dim3((unsigned)((quads + 255) / 256)), dim3(256),
                       0, st, (const float*)part, S, M, ldp, g, BN);
  }
}

// 64x64 tiles.  With at least three tiles per CU, one LDS stage lets several
// workgroups share a CU; with fewer tiles, two stages and two K blocks in
// flight per workgroup.  S > 1: split-K over S slices of K (partials in
// `part`); the variant is chosen by the workgroup count tiles * S and the
// per-slice K block count.
template <typename ScaleT>
void launch_gemm_small(const uint16_t* x, const QhGemmSeg* seg, int nseg, int M, int K, long tiles,
                       hipStream_t st, int cus, int S, float* part) {
  const int kbl = K / 128 / S;
  if (tiles * S >= 3L * cus)
    launch_gemm_lds<ScaleT, 64, 1, 1>(x, seg, nseg, M, K, st, S, part);
  else if (kbl % 2 == 0)
    launch_gemm_lds<ScaleT, 64, 2, 2>(x, seg, nseg, M, K, st, S, part);
  else
    launch_gemm_lds<ScaleT, 64, 2, 1>(x, seg, nseg, M, K, st, S, part);
}

}  // namespace

// Split-K partials: a split GEMM runs S * tiles <= 3 per CU workgroups of
// 64x64 fp32 partials, so this covers up to 1024 of them (341 CUs).
constexpr size_t kSplitPartBytes = (size_t)1024 * 64 * 64 * sizeof(float);

size_t qh_gemm_workspace_bytes(int M, int K) {
  (void)M;
  (void)K;
  return kSplitPartBytes;
}

int qh_launch_gemm_e4m3_group_ws(const void* x, int M, int K, const QhGemmSeg* seg, int nseg,
                                 bool scale_bf16, void* ws, hipStream_t st) {
  if (K <= 0 || K % 128 != 0 || M <= 0) {
    qh_set_error("gemm: M=%d, K=%d: need M > 0 and K a positive multiple of 128", M, K);
    return -1;
  }
  if (!x || (uintptr_t)x % 16 != 0) {
    qh_set_error("gemm: the activation must be a 16-byte aligned device pointer");
    return -1;
  }
  if (nseg < 1 || nseg > 4) {
    qh_set_error("gemm: nseg=%d outside [1, 4]", nseg);
    return -1;
  }
  long tiles64 = 0;
  for (int t = 0; t < nseg; ++t) {
    if (!seg[t].w || !seg[t].s || !seg[t].y || seg[t].N <= 0) {
      qh_set_error("gemm: segment %d: null pointer or N=%d", t, seg[t].N);
      return -1;
    }
    tiles64 += (seg[t].N + 63) / 64;
  }
  const uint16_t* xa = (const uint16_t*)x;
  const long mt = (M + kBM - 1) / kBM;
  int cus = 256, dev = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    cus = 256;
  // 64x64 tiles: with the activation used as is, wider tiles only cut
  // occupancy (64 x 128 measured 59.7 us against 48.8 us for config 3a's
  // 512 x 9216 x 2560).
  const long tiles = tiles64 * mt;
  // Split-K (caller workspace only) when there are no more tiles than CUs:
  // the largest S <= 8 dividing the K blocks with >= 4 blocks per slice and
  // S * tiles <= 3 per CU, so each workgroup walks fewer serial K steps.
  const int KB = K / 128;
  int S = 1;
  for (int c = 8; ws && c >= 2 && tiles <= cus; --c)
    if (KB % c == 0 && KB / c >= 4 && tiles * c <= 3L * cus &&
        (size_t)tiles * c * 64 * 64 * sizeof(float) <= kSplitPartBytes) {
      S = c;
      break;
    }
  float* part = (float*)ws;
  if (scale_bf16) launch_gemm_small<uint16_t>(xa, seg, nseg, M, K, tiles, st, cus, S, part);
  else launch_gemm_small<float>(xa, seg, nseg, M, K, tiles, st, cus, S, part);
  return 0;
}

int qh_launch_gemm_e4m3_ws(const void* x, const void* w, const void* s, void* y, int M, int N,
                           int K, int kb, bool scale_bf16, void* ws, hipStream_t st) {
  const QhGemmSeg seg = {w, s, y, N, kb};
  return qh_launch_gemm_e4m3_group_ws(x, M, K, &seg, 1, scale_bf16, ws, st);
}

// Without a caller workspace (the reference ABI passes none): no split-K and
// nothing allocated.
int qh_launch_gemm_e4m3(const void* x, const void* w, const void* s, void* y, int M, int N, int K,
                        int kb, bool scale_bf16, hipStream_t st) {
  return qh_launch_gemm_e4m3_ws(x, w, s, y, M, N, K, kb, scale_bf16, nullptr, st);
}
