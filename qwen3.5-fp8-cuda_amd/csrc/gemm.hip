// Prefill block-scaled E4M3 GEMM on the gfx950 fp8 matrix cores.
//
// Semantics (reference: qwen3_infer/csrc/fp8_kernels.cu:23-64
// fp8_gemm_batch_kernel; caller main.py:262-269):
//   Y[m, n] = bf16( sum_kb s[n, kb] * sum_{k in kb} X[m, k] * e4m3(W[n, k]) )
//
// The activations are bf16 and the matrix cores take E4M3 on both sides, so
// each 32-element run of a row of X (one MX block of the matrix-core
// instruction) is split into two E4M3 terms while the A tile is staged:
//   E = floor(log2 max|x|) - 7 over the run (a power of two, E8M0),
//   hi = e4m3(x / 2^E),  lo = e4m3((x / 2^E - hi) * 16),
//   x = 2^E hi + 2^(E - 4) lo.
// A bf16 value has 8 significant bits; hi keeps the top 4 (rounded) and the
// remainder has at most 4, so the split is exact for every element within
// 2^13 of its run's maximum (smaller ones keep an absolute error below
// 2^-21 of that maximum).  A channel 1000x larger than its neighbours
// therefore costs the neighbours nothing.  Both terms meet the same W tile in
// v_mfma_scale_f32_32x32x64_f8f6f4 with their run exponents as the per-lane
// E8M0 A scales (W's scale operand fixed at 2^0), products are exact in fp32,
// and each 128-wide K block's partial is multiplied by the weight block scale
// and added to the fp32 accumulator.
//
// Nothing is precomputed: no activation pass, no workspace.  A caller
// workspace only enables split-K (qh_gemm_e4m3 / qh_gemm_e4m3_grouped); the
// reference entry point fp8_gemm_batch passes none and never splits.
//
// Tiling: 64 x BN output tile per 256-thread workgroup (BN = 64, or 128 when
// that still gives two tiles per CU), a 2 x 2 grid of waves each holding
// 32 x (BN/2) of 32x32 matrix-core tiles.  Each 128-wide K block of A hi, A lo
// and B is staged once per workgroup in LDS (rows padded to 144 bytes against
// bank conflicts, one or two stages), the next one or two blocks in registers
// while the current one is multiplied.  Operand layout of the 32x32x64
// instruction (measured on gfx950 with one-hot operands and distinct
// per-lane scales): lane (r, h) holds 32 bytes of row r, and its bytes 0-15
// belong to MX block 0 (scaled by lane r's scale byte), bytes 16-31 to block
// 1 (lane r + 32's).  So for the q-th 64-byte chunk of a K block, lane half h
// takes bytes [64q + 16h, +16) and [64q + 32 + 16h, +16) of its row in both
// operands: block 0 is run 2q, block 1 run 2q + 1, and lane half h supplies
// run 2q + h's exponent.
#include "qh_common.h"
#include "qh_gemm.h"

namespace {

typedef float v16f __attribute__((ext_vector_type(16)));
typedef int v8i __attribute__((ext_vector_type(8)));
constexpr int kGRow = 144;                      // padded LDS row (bytes)
constexpr int kBM = 64;                         // output rows per tile

// The two 16-byte K chunks a lane feeds the 32x32x64 instruction: bytes
// [0, 16) at p, [16, 32) at p + 32.
__device__ __forceinline__ v8i lds_operand(const uint8_t* p) {
  const u32x4 a = *(const u32x4*)p, b = *(const u32x4*)(p + 32);
  return v8i{(int)a.x, (int)a.y, (int)a.z, (int)a.w, (int)b.x, (int)b.y, (int)b.z, (int)b.w};
}

// Split of one 32-element bf16 run (16 packed words) into E4M3 hi and lo
// terms (32 bytes each) and the run's E8M0 exponent byte s of the hi term
// (the lo term's is s - 4).  s = biased exponent of max|x| - 7, kept in
// [4, 247]: then 2^(127 - s) is a normal fp32 and x * 2^(127 - s) < 256 (no
// saturation); an all-zero run gives zero terms.
__device__ __forceinline__ void split_run(const u32x4 (&v)[4], u32x4 (&hi)[2], u32x4 (&lo)[2],
                                          uint32_t& s) {
  float f[32];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    f[8 * c + 0] = bf_lo(v[c].x); f[8 * c + 1] = bf_hi(v[c].x);
    f[8 * c + 2] = bf_lo(v[c].y); f[8 * c + 3] = bf_hi(v[c].y);
    f[8 * c + 4] = bf_lo(v[c].z); f[8 * c + 5] = bf_hi(v[c].z);
    f[8 * c + 6] = bf_lo(v[c].w); f[8 * c + 7] = bf_hi(v[c].w);
  }
  float amax = 0.0f;
#pragma unroll
  for (int e = 0; e < 32; ++e) amax = fmaxf(amax, fabsf(f[e]));
  const int ex = (int)((__float_as_uint(amax) >> 23) & 0xFFu);
  s = (uint32_t)min(max(ex - 7, 4), 247);
  const float inv = __uint_as_float((254u - s) << 23);    // 2^(127 - s)
  uint32_t h[8], l[8];
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    float a[4], r[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) a[e] = f[4 * q + e] * inv;
    uint32_t hp = __builtin_amdgcn_cvt_pk_fp8_f32(a[0], a[1], 0u, false);
    hp = __builtin_amdgcn_cvt_pk_fp8_f32(a[2], a[3], hp, true);
    const qh_f32x2 h01 = e4m3x2_lo_f32(hp), h23 = e4m3x2_hi_f32(hp);
    r[0] = (a[0] - h01.x) * 16.0f; r[1] = (a[1] - h01.y) * 16.0f;
    r[2] = (a[2] - h23.x) * 16.0f; r[3] = (a[3] - h23.y) * 16.0f;
    uint32_t lp = __builtin_amdgcn_cvt_pk_fp8_f32(r[0], r[1], 0u, false);
    lp = __builtin_amdgcn_cvt_pk_fp8_f32(r[2], r[3], lp, true);
    h[q] = hp;
    l[q] = lp;
  }
  hi[0] = u32x4{h[0], h[1], h[2], h[3]};
  hi[1] = u32x4{h[4], h[5], h[6], h[7]};
  lo[0] = u32x4{l[0], l[1], l[2], l[3]};
  lo[1] = u32x4{l[4], l[5], l[6], l[7]};
}

// LDS of one K-block stage of a 64 x BN tile: A hi, A lo (64 rows), B (BN
// rows), the BN fp32 weight scales of the block, then the 64 rows' four run
// exponent bytes.
constexpr int gemm_scw_off(int bn) { return (2 * kBM + bn) * kGRow; }
constexpr int gemm_sca_off(int bn) { return gemm_scw_off(bn) + bn * 4; }
constexpr int gemm_stage_bytes(int bn) { return gemm_sca_off(bn) + kBM * 4; }

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
                                                            int K, float* part, int ldp) {
  constexpr int BM = kBM;
  constexpr int WM = BM / 2, WN = BN / 2;        // this wave's sub-tile (2 x 2 waves)
  constexpr int TJ = WN / 32;                    // 32x32 matrix-core tiles per wave
  constexpr int STAGE = gemm_stage_bytes(BN);
  constexpr int SCW = gemm_scw_off(BN), SCA = gemm_sca_off(BN);
  constexpr int BPT = BN * 8 / 256;              // 16-byte W pieces per thread
  static_assert(WM == 32 && TJ >= 1 && BPT >= 1 && (NST == 1 || NST == 2), "tile shape");
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
  // Thread t stages MX run (t & 3) of tile row t >> 2 (64 bf16 bytes) and W
  // pieces t + 256 e (row p >> 3, 16-byte column p & 7).  Rows past M or N
  // re-read the last one (their results are never stored).
  const int arow = tid >> 2, arun = tid & 3;
  const uint16_t* xa = x + (size_t)min(mb + arow, M - 1) * K + 32 * arun;

  // The block's weight scales travel with its operands and are staged in LDS
  // beside them: a scale loaded at use time would sit behind every prefetched
  // block in the in-order load counter.  Thread t loads the scale of tile
  // column t % BN (every thread loads, so no load sits under a branch).
  u32x4 sa[D][4], sb[D][BPT];
  float scv[D];
  auto gload = [&](u32x4 (&da)[4], u32x4 (&db)[BPT], float& sdst, int kb) {
    kb = kb0 + min(kb, KB - 1);
    const int ko = kb * 128;
    sdst = load_scale<ScaleT>(sw, scale_index(kb_code, min(nb + tid % BN, N - 1), kb));
#pragma unroll
    for (int c = 0; c < 4; ++c) da[c] = *(const u32x4*)(xa + ko + 8 * c);
#pragma unroll
    for (int e = 0; e < BPT; ++e) {
      const int piece = tid + 256 * e;
      const int n = min(nb + (piece >> 3), N - 1);
      db[e] = __builtin_nontemporal_load((const u32x4*)(w + (size_t)n * K + ko + (piece & 7) * 16));
    }
  };
  auto sstore = [&](uint8_t* stage, const u32x4 (&da)[4], const u32x4 (&db)[BPT], float sc) {
    u32x4 hi[2], lo[2];
    uint32_t s;
    split_run(da, hi, lo, s);
    uint8_t* ah = stage + arow * kGRow + 32 * arun;
    uint8_t* al = stage + (BM + arow) * kGRow + 32 * arun;
    *(u32x4*)ah = hi[0];
    *(u32x4*)(ah + 16) = hi[1];
    *(u32x4*)al = lo[0];
    *(u32x4*)(al + 16) = lo[1];
    stage[SCA + arow * 4 + arun] = (uint8_t)s;
#pragma unroll
    for (int e = 0; e < BPT; ++e) {
      const int piece = tid + 256 * e;
      *(u32x4*)(stage + (2 * BM + (piece >> 3)) * kGRow + (piece & 7) * 16) = db[e];
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
    // this lane's run exponents: byte 0 -> run h (q = 0), byte 2 -> run 2 + h
    // (q = 1); the lo term's are 4 lower (every byte >= 4: no borrow).  The
    // instruction reads byte 0 of its scale operand whatever OPSEL says, so
    // run 2 + h is shifted down for q = 1.
    const uint32_t ws_hi = *(const uint32_t*)(cur + SCA + (wm + r) * 4) >> (8 * h);
    const uint32_t ws_lo = ws_hi - 0x04040404u;
    v16f t[TJ];
#pragma unroll
    for (int j = 0; j < TJ; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) t[j][e] = 0.0f;
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int co = 64 * q + 16 * h;
      const v8i ah = lds_operand(cur + (wm + r) * kGRow + co);
      const v8i al = lds_operand(cur + (BM + wm + r) * kGRow + co);
      v8i bw[TJ];
#pragma unroll
      for (int j = 0; j < TJ; ++j) bw[j] = lds_operand(cur + (2 * BM + wn + 32 * j + r) * kGRow + co);
#pragma unroll
      for (int j = 0; j < TJ; ++j) {
        t[j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(ah, bw[j], t[j], 0, 0, 0,
                                                               (int)(ws_hi >> (16 * q)), 0, 127);
        t[j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(al, bw[j], t[j], 0, 0, 0,
                                                               (int)(ws_lo >> (16 * q)), 0, 127);
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

  // C layout of a 32x32 tile: lane -> column lane%32, value e -> row
  // 8*(e/4) + 4*(lane/32) + e%4.
  if (part) {
    float* pz = part + (size_t)blockIdx.z * M * ldp;
    const int ng0 = (int)blockIdx.x * BN;
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
  dim3 grid(tiles_n, (M + kBM - 1) / kBM, S);
  const int ldp = tiles_n * BN;
  hipLaunchKernelGGL((gemm_e4m3_lds_kernel<ScaleT, BN, NST, D>), grid, dim3(256),
                     NST * (size_t)gemm_stage_bytes(BN), st, x, g, M, K, S > 1 ? part : nullptr,
                     ldp);
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
  long tiles64 = 0, tiles128 = 0;
  for (int t = 0; t < nseg; ++t) {
    if (!seg[t].w || !seg[t].s || !seg[t].y || seg[t].N <= 0) {
      qh_set_error("gemm: segment %d: null pointer or N=%d", t, seg[t].N);
      return -1;
    }
    tiles64 += (seg[t].N + 63) / 64;
    tiles128 += (seg[t].N + 127) / 128;
  }
  const uint16_t* xa = (const uint16_t*)x;
  const long mt = (M + kBM - 1) / kBM;
  int cus = 256, dev = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    cus = 256;
  // 64x128 tiles while they give at least two per CU (the A split is shared by
  // twice the W rows); 64x64 below that, so every CU stays busy.
  if (tiles128 * mt >= 2L * cus) {
    if (scale_bf16) launch_gemm_lds<uint16_t, 128, 2, 1>(xa, seg, nseg, M, K, st);
    else launch_gemm_lds<float, 128, 2, 1>(xa, seg, nseg, M, K, st);
    return 0;
  }
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
