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
// (one conversion instruction per two weights) is repeated only by the M / 64
// row tiles that share a weight tile.
//
// Nothing is precomputed and no workspace is needed; a caller workspace only
// enables split-K (qh_gemm_e4m3 / qh_gemm_e4m3_grouped).  The reference entry
// point fp8_gemm_batch passes none and never splits.
//
// Two kernels, both with a 2 x 2 grid of waves per output tile in an
// XCD-aware tile order (the row tiles of one weight tile run on one XCD and
// share it in that XCD's L2):
//  - gemm_dma_kernel (every launch whose operands it can take): persistent
//    workgroups stream (tile or tile K slice, K block) units through a
//    two-stage LDS ring filled by direct-to-LDS loads, on 64 x 64 tiles
//    (three workgroups per CU), 64 x 128 (two) or 128 x 192 (one), the plan
//    (tile shape, K split) picked by a cost model with measured per-unit
//    cycles (gemm_plan); split-K partials are finished by
//    gemm_splitk_reduce_kernel or splitk_add_rmsnorm_kernel;
//  - gemm_e4m3_lds_kernel (fallback for unaligned weights or scales): one
//    workgroup per (64 x 64 tile, K slice), the next K blocks in registers
//    while the current one is multiplied.
// Operand layout of the 32x32x16 bf16 instruction (measured on gfx950):
// lane l holds A[l % 32][8 (l / 32) + r] and B[8 (l / 32) + r][l % 32],
// r = 0..7, and accumulator value e is C[8 (e / 4) + 4 (l / 32) + e % 4][l % 32].
#include "qh_common.h"
#include "qh_gemm.h"
#include "qh_norm.h"

namespace {

typedef float v16f __attribute__((ext_vector_type(16)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
constexpr int kARow = 272;                      // padded LDS row of the X tile (bytes)
constexpr int kBRow = 144;                      // padded LDS row of the W tile (bytes)
constexpr int kBM = 64;                         // output rows per tile

// Eight E4M3 weights (two words) widened to bf16, exactly: the scaled
// conversion with scale 1 turns two codes into two bf16 in one instruction
// (every finite E4M3 value, subnormals included, is a bf16 value; checked
// bit for bit against the fp32 route for all 256 codes).
__device__ __forceinline__ v8bf e4m3x8_bf16(u32x2 w) {
  const qh_bf16x2 a = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w.x, 1.0f, false);
  const qh_bf16x2 b = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w.x, 1.0f, true);
  const qh_bf16x2 c = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w.y, 1.0f, false);
  const qh_bf16x2 d = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w.y, 1.0f, true);
  return v8bf{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
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
  int sbytes[4];    // scale array bytes, rounded up to whole words (persistent kernel)
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

// ---- persistent LDS-ring variant ----------------------------------------------
// Persistent 256-thread workgroups (WPC per CU) walk their 64 x 64 output tiles
// (XCD-aware order, as above) as one stream of (tile, 128-wide K block) units.
// Each unit's X rows, W rows and per-column weight scales go straight from
// memory to an LDS stage (buffer_load ... lds through range-checked buffer
// resources based at the tile: rows past M or N read zeros), DS - 1 units
// ahead, so the loads in flight cost no registers and the stream does not
// drain between tiles.  16-byte slots are XOR-swizzled by row instead of padded
// (the loads fill whole 1 KB runs): X row r (256 B) keeps chunk c in slot
// c ^ (r % 16), so the 16-byte reads of 16 consecutive rows cover all 64
// banks; W row r (128 B) keeps it in slot c ^ ((r / 2) % 8), which spreads
// the 8-byte reads of 32 rows over the banks two to one.  Operands are read with
// inline-asm LDS reads, which the compiler does not track (it would otherwise
// wait for every outstanding ring load before each LDS read): each wave waits
// for its own loads of the unit (vmcnt), all waves meet at a barrier, and each
// matrix-core step waits only for its own two operand reads.
// LDS of one ring stage for 64 x BN tiles: X (64 rows), W (BN rows), and one
// 64-word copy of the column scales per wave.
// One ring stage of a BM x BN tile: X (BM rows x 128 bf16), W (BN rows x 128
// E4M3), the fp32 scales (or scale words) of the block: one 64-word slot per
// wave holding its own BN / 2 columns (BN <= 128), or three 64-column slots
// of the tile (BN = 192).
template <int BM, int BN>
struct Ring {
  static_assert((BM == 64 && (BN == 64 || BN == 128)) || (BM == 128 && BN == 192), "tile shape");
  static constexpr int A = BM * 256;
  static constexpr int B = BN * 128;
  static constexpr bool WSLOT = BN <= 128;        // per-wave scale slots
  static constexpr int NSC = WSLOT ? 4 : BN / 64;   // 256-byte scale slots
  static constexpr int STAGE = A + B + NSC * 256;  // 25,600 B (64 x 64) .. 58,112 B (128 x 192)
  static constexpr int XL = BM / 16;             // X loads (1 KB) per wave and unit
  static constexpr int WL = BN / 32;             // W loads (1 KB) per wave and unit
  static constexpr int LOADS = XL + WL + 1;      // per wave and unit: X, W, scales
};

typedef __amdgpu_buffer_rsrc_t rsrc_t;
typedef __attribute__((address_space(3))) void* lds_ptr;

__device__ __forceinline__ u32x4 ds_read16(uint32_t a) {
  u32x4 v;
  asm volatile("ds_read_b128 %0, %1" : "=v"(v) : "v"(a) : "memory");
  return v;
}
__device__ __forceinline__ u32x2 ds_read8(uint32_t a) {
  u32x2 v;
  asm volatile("ds_read_b64 %0, %1" : "=v"(v) : "v"(a) : "memory");
  return v;
}
__device__ __forceinline__ uint32_t ds_read4(uint32_t a) {
  uint32_t v;
  asm volatile("ds_read_b32 %0, %1" : "=v"(v) : "v"(a) : "memory");
  return v;
}
// Wait until at most N LDS reads are outstanding; a and b (the reads this
// wait completes) are tied to it so that no use moves above it.
template <int N>
__device__ __forceinline__ void lds_wait(u32x4& a, u32x2& b) {
  asm volatile("s_waitcnt lgkmcnt(%2)" : "+v"(a), "+v"(b) : "n"(N) : "memory");
}
template <int N>
__device__ __forceinline__ void lds_wait(u32x4& a, u32x4& b, u32x4& c) {
  asm volatile("s_waitcnt lgkmcnt(%3)" : "+v"(a), "+v"(b), "+v"(c) : "n"(N) : "memory");
}
template <int N>
__device__ __forceinline__ void lds_wait(u32x4& a, u32x4& b, u32x4& c, u32x4& d) {
  asm volatile("s_waitcnt lgkmcnt(%4)" : "+v"(a), "+v"(b), "+v"(c), "+v"(d) : "n"(N) : "memory");
}
template <int N>
__device__ __forceinline__ void lds_wait(u32x4& a, u32x4& b, u32x4& c, u32x4& d, u32x4& e) {
  asm volatile("s_waitcnt lgkmcnt(%5)" : "+v"(a), "+v"(b), "+v"(c), "+v"(d), "+v"(e) : "n"(N) : "memory");
}

// One work item of the walk (a tile, or with split-K one K slice of a tile)
// and its segment, all workgroup-uniform.
struct DmaTile {
  int tn, tm, nb, N, kb_code, sbytes, kb0;
  const uint8_t* w;
  const void* s;
  uint16_t* y;
};

// The group is indexed in place (a kernel argument: scalar loads), never
// copied to a local array.
// Item i of XCD xc: K slice i % S (K blocks kb0 .. kb0 + KBs - 1) of tile
// i / S.  The XCD's tiles (its ntx N tiles, all row tiles) go in groups of gm
// row tiles; within a group the row tile is fastest, so the items in flight
// at once share gm row tiles of X and a few N tiles of W in the XCD's L2.
template <int BN>
__device__ __forceinline__ DmaTile dma_tile(const GemmGroup& g, int xc, int i, int tiles_m, int S, int KBs,
                                            int ntx, int gm) {
  DmaTile d;
  d.kb0 = (i % S) * KBs;
  i /= S;
  const int grp = i / (gm * ntx), rr = i - grp * gm * ntx;
  const int gme = min(gm, tiles_m - grp * gm);
  d.tn = xc + 8 * (rr / gme);
  d.tm = grp * gm + rr % gme;
  int si = 0;
#pragma unroll
  for (int t = 1; t < 4; ++t)
    if (t < g.nseg && d.tn >= g.tstart[t]) si = t;
  d.w = g.w[si];
  d.s = g.s[si];
  d.y = g.y[si];
  d.N = g.N[si];
  d.kb_code = g.kb[si];
  d.sbytes = g.sbytes[si];
  d.nb = (d.tn - g.tstart[si]) * BN;
  return d;
}

// S > 1: each item is one K slice of a tile and its fp32 partial tile goes to
// part[(slice M + m) ldp + global column] (ldp = tiles_n BN) for a finishing
// kernel.  The four waves form a 2 x 2 grid of (BM / 2) x (BN / 2) sub-tiles:
// MI x NJ 32x32 matrix-core tiles per wave, where the MI activation reads
// and NJ weight reads of a K step are shared across them.
template <typename ScaleT, int DS, bool SPLIT, int BN, int BM, bool EARLY>
__global__ __launch_bounds__(256) void gemm_dma_kernel(const uint16_t* x, GemmGroup g, int M, int K,
                                                       int tiles_n, int tiles_m, int S_arg, float* part,
                                                       int ldp, int gm) {
  using R = Ring<BM, BN>;
  constexpr int NJ = BN / 64;       // 32-column matrix-core tiles per wave
  constexpr int MI = BM / 64;       // 32-row matrix-core tiles per wave
  const int S = SPLIT ? S_arg : 1;  // unsplit launches compile without the slice arithmetic
  extern __shared__ __align__(16) uint8_t smem[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane & 31, h = lane >> 5;
  const int wm = (wid >> 1) * (BM / 2), wn = (wid & 1) * (BN / 2);
  const int KB = K / 128 / S;  // K blocks per item
  // this workgroup's items: XCD xc, its j-th of P workgroups there; XCD xc
  // owns N tiles xc, xc + 8, ... with all their row tiles (row tile fastest)
  // and K slices, dealt round-robin to its workgroups
  const int xc = (int)blockIdx.x & 7, j = (int)blockIdx.x >> 3, P = (int)gridDim.x >> 3;
  const int nt_x = tiles_n > xc ? (tiles_n - xc + 7) / 8 : 0;  // N tiles of this XCD
  const int ntx = tiles_m * nt_x * S;
  const int my_tiles = j < ntx ? (ntx - j + P - 1) / P : 0;
  const int U = my_tiles * KB;
  if (U == 0) return;
  const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_ptr)smem;

  // lane-constant parts of the load offsets (the unit's K block is added);
  // fixed-size arrays: a lambda capturing an array whose bound depends on a
  // template parameter makes the host pass drop the kernel's launch stub
  uint32_t xo[8], wo[8];
#pragma unroll
  for (int i = 0; i < R::XL; ++i) {  // X: rows (BM / 4) wid + 4 i + lane / 16
    const int row = (BM / 4) * wid + 4 * i + (lane >> 4);
    xo[i] = ((uint32_t)row * (uint32_t)K + (uint32_t)(((lane & 15) ^ (row & 15)) * 8)) * 2u;
  }
#pragma unroll
  for (int i = 0; i < R::WL; ++i) {  // W: rows (BN / 4) wid + 8 i + lane / 8
    const int row = (BN / 4) * wid + 8 * i + (lane >> 3);
    wo[i] = (uint32_t)row * (uint32_t)K + (uint32_t)(((lane & 7) ^ ((row >> 1) & 7)) * 16);
  }
  // scales: per-wave slot w with the wave's BN / 2 columns (with BN 64,
  // lanes 32-63 repeat them), or slot w % 3 of the tile's columns (two waves
  // write slot 0 with the same words)
  const int sslot = R::WSLOT ? wid : wid % R::NSC;
  const int scol = R::WSLOT ? wn + (lane & (BN / 2 - 1)) : 64 * sslot + lane;
  const int soff = R::WSLOT ? wid * 256 - wn * 4 : 0;  // LDS byte offset of column c: soff + 4 c

  // issue cursor: the unit whose loads go out next (it stays on the last unit
  // once reached, so the ring keeps DS - 1 units of loads outstanding)
  int it = 0, ikb = 0;
  DmaTile itile = dma_tile<BN>(g, xc, j, tiles_m, S, KB, nt_x, gm);
  rsrc_t rx, rw, rs;
  auto bind = [&]() {
    const int rows_m = min(M - itile.tm * BM, BM), rows_n = min(itile.N - itile.nb, BN);
    rx = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(x + (size_t)itile.tm * BM * K), (short)0,
                                           rows_m * K * 2, 0x00020000);
    rw = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(itile.w + (size_t)itile.nb * K), (short)0,
                                           rows_n * K, 0x00020000);
    rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(itile.s), (short)0, itile.sbytes, 0x00020000);
  };
  bind();
  // load li of the issue cursor's unit into stage st: X loads, W loads,
  // then the scale words of the slot's 64 columns (aligned words)
  auto issue_one = [&](int st, int li) {
    uint8_t* stage = smem + st * R::STAGE;
    const int kb = itile.kb0 + ikb;
    const uint32_t ko = (uint32_t)kb * 256u;
    if (li < R::XL) {
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (lds_ptr)(stage + ((BM / 4) * wid + 4 * li) * 256), 16,
                                               xo[li] + ko, 0, 0, 0);
    } else if (li < R::XL + R::WL) {
      const int i = li - R::XL;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rw, (lds_ptr)(stage + R::A + ((BN / 4) * wid + 8 * i) * 128),
                                               16, wo[i] + (ko >> 1), 0, 0, 0);
    } else {
      const int si = scale_index(itile.kb_code, min(itile.nb + scol, itile.N - 1), kb);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_ptr)(stage + R::A + R::B + sslot * 256), 4,
                                               ((uint32_t)si * (uint32_t)sizeof(ScaleT)) & ~3u, 0, 0, 0);
    }
  };
  auto issue = [&](int st) {
#pragma unroll
    for (int li = 0; li < R::LOADS; ++li) issue_one(st, li);
  };
  // the loads of step q of 8: spread over the unit's matrix-core steps so
  // their issue overlaps the products in flight
  auto issue_step = [&](int st, int q) {
#pragma unroll
    for (int li = 0; li < R::LOADS; ++li)
      if (li * 8 / R::LOADS == q) issue_one(st, li);
  };
  auto advance = [&]() {
    if (ikb + 1 < KB) {
      ++ikb;
    } else if (it + 1 < my_tiles) {
      ++it;
      ikb = 0;
      itile = dma_tile<BN>(g, xc, j + it * P, tiles_m, S, KB, nt_x, gm);
      bind();
    }
  };

#pragma unroll
  for (int s = 0; s < DS - 1; ++s) {
    issue(s);
    advance();
  }

  // compute cursor
  int ckb = 0, ct = 0;
  DmaTile ctile = dma_tile<BN>(g, xc, j, tiles_m, S, KB, nt_x, gm);
  v16f acc[MI][NJ];
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int b = 0; b < NJ; ++b)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][b][e] = 0.0f;
  const int arow = wm + r;
  int st = 0;
  for (int u = 0; u < U; ++u) {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(R::LOADS * (DS - 2)) : "memory");
    __builtin_amdgcn_s_barrier();
    const int ist = st == 0 ? DS - 1 : st - 1;  // the stage the next unit's loads fill
    // EARLY (64 x 64 tiles): all of the next unit's loads before this unit's
    // LDS reads, so their latency is hidden behind the whole unit; wider
    // tiles spread them over the matrix-core steps, whose products in flight
    // then cover the issue (3700 x 18432 x 2560: 488 -> 426 us at 128 x 192)
    if constexpr (EARLY) {
      issue(ist);
      advance();
    }
    const uint32_t sa = lds0 + st * R::STAGE, sbb = sa + R::A, ssc = sbb + R::B;
    v16f t[MI][NJ];
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
      for (int b = 0; b < NJ; ++b)
#pragma unroll
        for (int e = 0; e < 16; ++e) t[i][b][e] = 0.0f;
    uint32_t sw[NJ];
    if constexpr (NJ == 1) {
      const int brow = wn + r;
      u32x4 av[8];
      u32x2 bv[8];
#pragma unroll
      for (int kk = 0; kk < 8; ++kk) {
        av[kk] = ds_read16(sa + arow * 256 + (((2 * kk + h) ^ (arow & 15)) << 4));
        bv[kk] = ds_read8(sbb + brow * 128 + ((kk ^ ((brow >> 1) & 7)) << 4) + 8 * h);
      }
      sw[0] = ds_read4(ssc + soff + (wn + r) * 4);
      // each step waits only for its own two operand reads
#define QH_DMA_STEP(kk)                                                                   \
  lds_wait<15 - 2 * (kk)>(av[kk], bv[kk]);                                                \
  t[0][0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8bf, av[kk]),    \
                                                    e4m3x8_bf16(bv[kk]), t[0][0], 0, 0, 0); \
  if constexpr (!EARLY) issue_step(ist, kk);                                              \
  __builtin_amdgcn_sched_barrier(0);
      QH_DMA_STEP(0) QH_DMA_STEP(1) QH_DMA_STEP(2) QH_DMA_STEP(3)
      QH_DMA_STEP(4) QH_DMA_STEP(5) QH_DMA_STEP(6) QH_DMA_STEP(7)
#undef QH_DMA_STEP
      asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(sw[0]) : : "memory");
    } else {
      // NJ 32-column tiles share each activation read and MI row tiles each
      // weight read.  Weights as 16-byte reads: lane half h holds chunk
      // 2 jj + h of its row and feeds half p to step 2 jj + p; the activation
      // operand is read in the same K order (bf16 chunk 4 jj + 2 h + p), so
      // both sides of a step see equal K.  Reads go out in step order, per
      // chunk pair jj: the NJ weight reads, then for p = 0, 1 the MI
      // activation reads; LDS reads complete in order, so step kk waits until
      // at most (total - reads through its own) are outstanding (capped at
      // 15, the counter's limit: issue stalls while it is full).
      constexpr int GR = NJ + 2 * MI;          // reads per chunk pair
      constexpr int TOT = 4 * GR + NJ;         // and the scale words
      u32x4 av[MI][8], bq[NJ][4];
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
#pragma unroll
        for (int b = 0; b < NJ; ++b) {
          const int brow = wn + 32 * b + r;
          bq[b][jj] = ds_read16(sbb + brow * 128 + (((2 * jj + h) ^ ((brow >> 1) & 7)) << 4));
        }
#pragma unroll
        for (int p = 0; p < 2; ++p)
#pragma unroll
          for (int i = 0; i < MI; ++i) {
            const int ar = arow + 32 * i;
            av[i][2 * jj + p] = ds_read16(sa + ar * 256 + (((4 * jj + 2 * h + p) ^ (ar & 15)) << 4));
          }
      }
#pragma unroll
      for (int b = 0; b < NJ; ++b) sw[b] = ds_read4(ssc + soff + (wn + 32 * b + r) * 4);
#define QH_WAITN(kk) (TOT - ((kk) >> 1) * GR - NJ - MI * (((kk) & 1) + 1) > 15 ? 15 \
                      : TOT - ((kk) >> 1) * GR - NJ - MI * (((kk) & 1) + 1))
#define QH_DMA_STEPG(kk)                                                                               \
  {                                                                                                    \
    if constexpr (MI == 1 && NJ == 2)                                                                  \
      lds_wait<QH_WAITN(kk)>(av[0][kk], bq[0][(kk) >> 1], bq[1][(kk) >> 1]);                          \
    else if constexpr (MI == 2 && NJ == 2)                                                             \
      lds_wait<QH_WAITN(kk)>(av[0][kk], av[1][kk], bq[0][(kk) >> 1], bq[1][(kk) >> 1]);               \
    else                                                                                               \
      lds_wait<QH_WAITN(kk)>(av[0][kk], av[MI - 1][kk], bq[0][(kk) >> 1], bq[1][(kk) >> 1],          \
                             bq[NJ - 1][(kk) >> 1]);                                                   \
    v8bf bb[NJ];                                                                                       \
    _Pragma("unroll") for (int b = 0; b < NJ; ++b) {                                                   \
      const u32x4 wq = bq[b][(kk) >> 1];                                                               \
      bb[b] = e4m3x8_bf16((kk) & 1 ? u32x2{wq.z, wq.w} : u32x2{wq.x, wq.y});                           \
    }                                                                                                  \
    _Pragma("unroll") for (int i = 0; i < MI; ++i) {                                                   \
      const v8bf a = __builtin_bit_cast(v8bf, av[i][kk]);                                              \
      _Pragma("unroll") for (int b = 0; b < NJ; ++b)                                                   \
        t[i][b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, bb[b], t[i][b], 0, 0, 0);                 \
    }                                                                                                  \
    if constexpr (!EARLY) issue_step(ist, kk);                                                         \
    __builtin_amdgcn_sched_barrier(0);                                                                 \
  }
      QH_DMA_STEPG(0) QH_DMA_STEPG(1) QH_DMA_STEPG(2) QH_DMA_STEPG(3)
      QH_DMA_STEPG(4) QH_DMA_STEPG(5) QH_DMA_STEPG(6) QH_DMA_STEPG(7)
#undef QH_DMA_STEPG
#undef QH_WAITN
      if constexpr (NJ == 2)
        asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(sw[0]), "+v"(sw[1]) : : "memory");
      else
        asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(sw[0]), "+v"(sw[1]), "+v"(sw[2]) : : "memory");
    }
    if constexpr (!EARLY) advance();
#pragma unroll
    for (int b = 0; b < NJ; ++b) {
      float scale;
      if constexpr (sizeof(ScaleT) == 4) {
        scale = __uint_as_float(sw[b]);
      } else {
        const int idx =
            scale_index(ctile.kb_code, min(ctile.nb + wn + 32 * b + r, ctile.N - 1), ctile.kb0 + ckb);
        scale = (idx & 1) ? bf_hi(sw[b]) : bf_lo(sw[b]);
      }
#pragma unroll
      for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[i][b][e] = fmaf(t[i][b][e], scale, acc[i][b][e]);
    }
    if (++ckb == KB) {  // the item is complete: store it, start the next one
#pragma unroll
      for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int b = 0; b < NJ; ++b) {
          const int n = ctile.nb + wn + 32 * b + r;
          if constexpr (SPLIT) {
            float* pz = part + (size_t)(ctile.kb0 / KB) * M * ldp + ctile.tn * BN + wn + 32 * b + r;
#pragma unroll
            for (int e = 0; e < 16; ++e) {
              const int m = ctile.tm * BM + wm + 32 * i + 8 * (e >> 2) + 4 * h + (e & 3);
              if (m < M) pz[(size_t)m * ldp] = acc[i][b][e];
              acc[i][b][e] = 0.0f;
            }
          } else {
#pragma unroll
            for (int e = 0; e < 16; ++e) {
              const int m = ctile.tm * BM + wm + 32 * i + 8 * (e >> 2) + 4 * h + (e & 3);
              if (m < M && n < ctile.N) ctile.y[(size_t)m * ctile.N + n] = f2bf(acc[i][b][e]);
              acc[i][b][e] = 0.0f;
            }
          }
        }
      ckb = 0;
      if (++ct < my_tiles) ctile = dma_tile<BN>(g, xc, j + ct * P, tiles_m, S, KB, nt_x, gm);
    }
    st = st == DS - 1 ? 0 : st + 1;
  }
  // no load may still be writing this workgroup's LDS when it exits
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

// Shape limit of the persistent kernel: its per-tile buffer ranges (up to
// 128 rows of K bf16, 192 rows of K E4M3) stay below 2^31 bytes.
inline bool gemm_dma_fits(int K) { return (long)128 * K * 2 < 0x7fffffffL; }

__global__ __launch_bounds__(256) void gemm_splitk_reduce_kernel(const float* part, int S, int M,
                                                                 int ldp, GemmGroup g, int bn);

// reduce = false leaves split-K partials for the caller's own finishing kernel
// (partial row stride: gemm_part_ldp).
template <typename ScaleT, int DS, int BN, int BM>
void launch_gemm_dma(const uint16_t* x, const QhGemmSeg* seg, int nseg, int M, int K, hipStream_t st,
                     int cus, int wpc, int S = 1, float* part = nullptr, bool reduce = true) {
  GemmGroup g = {};
  g.nseg = nseg;
  int tiles_n = 0;
  for (int t = 0; t < nseg; ++t) {
    g.w[t] = (const uint8_t*)seg[t].w;
    g.s[t] = seg[t].s;
    g.y[t] = (uint16_t*)seg[t].y;
    g.N[t] = seg[t].N;
    g.kb[t] = seg[t].kb;
    g.tstart[t] = tiles_n;
    tiles_n += (seg[t].N + BN - 1) / BN;
    const long n_scales = seg[t].kb > 1 ? (long)((seg[t].N + 127) / 128) * seg[t].kb
                          : seg[t].kb == 1 ? seg[t].N : (long)seg[t].N * (-seg[t].kb);
    // whole words: a 2-byte scale is read as the aligned word holding it
    g.sbytes[t] = (int)min((n_scales * (long)sizeof(ScaleT) + 3) & ~3L, 0x7fffffffL);
  }
  const int tiles_m = (M + BM - 1) / BM;
  // P workgroups per XCD: as many as the busiest XCD has items (XCD 0 owns
  // ceil(tiles_n / 8) N tiles), at most wpc per CU, so no workgroup there
  // takes a second item while others are idle
  const long busiest = (long)tiles_m * ((tiles_n + 7) / 8) * S;
  const int P = (int)max(1L, min((long)cus * wpc / 8, busiest));
  const int G = 8 * P;
  const int ldp = tiles_n * BN;
  // row tiles per group: all of them (row tile fastest) when X fits in 3 MB
  // of the XCD's 4 MB L2 or a workgroup takes at most two items (then the
  // workgroups sharing a CU share X rows in its L1), else about 1.5 MB of X
  // rows
  const long xbytes = (long)BM * K * 2;
  const int gm = tiles_m * xbytes <= 3L * 1024 * 1024 || busiest <= 2L * P
                     ? tiles_m
                     : (int)max(1L, min((long)tiles_m, (long)(1536 * 1024) / xbytes));
  constexpr size_t lds = (size_t)DS * Ring<BM, BN>::STAGE;
  constexpr bool early = BM == 64 && BN == 64;
  if (S > 1)
    hipLaunchKernelGGL((gemm_dma_kernel<ScaleT, DS, true, BN, BM, early>), dim3(G), dim3(256), lds, st, x, g, M,
                       K, tiles_n, tiles_m, S, part, ldp, gm);
  else
    hipLaunchKernelGGL((gemm_dma_kernel<ScaleT, DS, false, BN, BM, early>), dim3(G), dim3(256), lds, st, x, g, M,
                       K, tiles_n, tiles_m, 1, nullptr, ldp, gm);
  if (S > 1 && reduce) {
    const size_t quads = (size_t)M * ldp / 4;
    hipLaunchKernelGGL(gemm_splitk_reduce_kernel, dim3((unsigned)((quads + 255) / 256)), dim3(256), 0, st,
                       (const float*)part, S, M, ldp, g, BN);
  }
}

// sum_z p[z zs] (four floats), z in order, every load issued first
template <int S>
__device__ __forceinline__ f32x4 sum_slices(const float* p, size_t zs) {
  f32x4 a[S];
#pragma unroll
  for (int z = 0; z < S; ++z) a[z] = *(const f32x4*)(p + z * zs);
  f32x4 acc = a[0];
#pragma unroll
  for (int z = 1; z < S; ++z) acc += a[z];
  return acc;
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
  // the slices' loads all in flight (a runtime-count loop issued them one
  // round trip apart), summed in slice order
  const float* p = part + (size_t)m * ldp + ng;
  const size_t zs = (size_t)M * ldp;
  f32x4 acc;
  switch (S) {
    case 2: acc = sum_slices<2>(p, zs); break;
    case 3: acc = sum_slices<3>(p, zs); break;
    case 4: acc = sum_slices<4>(p, zs); break;
    case 5: acc = sum_slices<5>(p, zs); break;
    case 6: acc = sum_slices<6>(p, zs); break;
    case 7: acc = sum_slices<7>(p, zs); break;
    case 8: acc = sum_slices<8>(p, zs); break;
    default:
      acc = *(const f32x4*)p;
      for (int z = 1; z < S; ++z) acc += *(const f32x4*)(p + z * zs);
  }
  uint16_t* y = g.y[si] + (size_t)m * N + n;
#pragma unroll
  for (int c = 0; c < 4; ++c)
    if (n + c < N) y[c] = f2bf(acc[c]);
}

// Split-K finish fused with the residual add and the (1+w) RMSNorm that follow
// an output projection, one 256-thread block per row m of one N-wide segment:
//   o = bf16(sum_z part[z][m][:N])  (z in order, as gemm_splitk_reduce_kernel),
//   h = bf16(h + o) in place, hn = bf16(h * rsqrt(mean(h^2) + eps) * (1 + w))
// (no hn when w is null).  V 8-column vectors per thread stay in registers;
// requires N % 8 == 0, N <= 2048 V and 16-byte aligned rows.  SC > 0: the
// slice count as a constant, so all of a vector's partial loads are in flight
// at once (with a runtime count the loop issued them one round trip apart).
template <int V, int SC>
__global__ __launch_bounds__(256) void splitk_add_rmsnorm_kernel(const float* part, int S_arg, int M, int ldp, int N,
                                                                 uint16_t* h, const float* w, uint16_t* hn,
                                                                 float eps) {
  __shared__ float red[4];
  const int S = SC > 0 ? SC : S_arg;
  const int m = blockIdx.x, t = threadIdx.x, nv = N >> 3;
  uint16_t* hr = h + (size_t)m * N;
  // Every load first, at a clamped vector index (a vector past nv is loaded
  // and not used), so the partial slices, the residual row and the norm
  // weights share one round trip; the weights through a buffer resource
  // (none when w is null: an empty range, the loads read 0).
  const auto wr = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(w), (short)0, w ? N * 4 : 0, 0x00020000);
  f32x4 a0[V], a1[V];
  u32x4 hv[V], wq[V][2];
#pragma unroll
  for (int v = 0; v < V; ++v) {
    const int ic = min(t + 256 * v, nv - 1);
    const float* p0 = part + (size_t)m * ldp + 8 * ic;
    a0[v] = *(const f32x4*)p0;
    a1[v] = *(const f32x4*)(p0 + 4);
#pragma unroll
    for (int z = 1; z < S; ++z) {
      const float* pz = p0 + (size_t)z * M * ldp;
      a0[v] += *(const f32x4*)pz;
      a1[v] += *(const f32x4*)(pz + 4);
    }
    hv[v] = *(const u32x4*)(hr + 8 * ic);
    wq[v][0] = __builtin_amdgcn_raw_buffer_load_b128(wr, (uint32_t)ic * 32u, 0, 0);
    wq[v][1] = __builtin_amdgcn_raw_buffer_load_b128(wr, (uint32_t)ic * 32u + 16u, 0, 0);
  }
  float xv[V][8];
  float ss = 0.0f;
#pragma unroll
  for (int v = 0; v < V; ++v) {
    const int i = t + 256 * v;
    if (i < nv) {
      u32x4 sum;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float o_lo = rbf(q < 2 ? a0[v][2 * q] : a1[v][2 * q - 4]);
        const float o_hi = rbf(q < 2 ? a0[v][2 * q + 1] : a1[v][2 * q - 3]);
        xv[v][2 * q] = rbf(bf_lo(hv[v][q]) + o_lo);
        xv[v][2 * q + 1] = rbf(bf_hi(hv[v][q]) + o_hi);
        sum[q] = (__float_as_uint(xv[v][2 * q]) >> 16) | (__float_as_uint(xv[v][2 * q + 1]) & 0xFFFF0000u);
      }
      *(u32x4*)(hr + 8 * i) = sum;
#pragma unroll
      for (int e = 0; e < 8; ++e) ss = fmaf(xv[v][e], xv[v][e], ss);
    }
  }
  if (!w) return;
  ss = block_sum_256(ss, red);
  const float rms = rsqrtf(ss / (float)N + eps);
  uint16_t* yr = hn + (size_t)m * N;
#pragma unroll
  for (int v = 0; v < V; ++v) {
    const int i = t + 256 * v;
    if (i < nv) {
      float wv[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) wv[e] = __uint_as_float(wq[v][e >> 2][e & 3]);
      u32x4 y;
#pragma unroll
      for (int q = 0; q < 4; ++q)
        y[q] = (uint32_t)f2bf(xv[v][2 * q] * rms * (1.0f + wv[2 * q])) |
               ((uint32_t)f2bf(xv[v][2 * q + 1] * rms * (1.0f + wv[2 * q + 1])) << 16);
      *(u32x4*)(yr + 8 * i) = y;
    }
  }
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

namespace {
// Launch plan of the ring kernel: tile shape, workgroups per CU, K slices.
struct GemmPlan {
  int bm, bn, wpc, S;
};

// Cycles one workgroup spends per (tile, 128-wide K block) unit at its
// occupancy (64 x 64: three workgroups per CU, 64 x 128: two, 128 x 192:
// one), measured on MI355X at M = 512 (X fits the XCD's L2) and at M = 3700
// (grouped row tiles; X streams): 2.0 / 2.2 / 4.3 and 2.5 / 2.6 / 3.8
// thousand.  (128 x 128 tiles, 3.0 / 2.8 thousand, were never the fastest
// plan for a prefill shape.)
struct GemmShape {
  int bm, bn, wpc;
  double cycles_small, cycles_large;
};
constexpr GemmShape kGemmShapes[] = {{64, 64, 3, 2030.0, 2460.0}, {64, 128, 2, 2200.0, 2600.0},
                                     {128, 192, 1, 4280.0, 3760.0}};

// The plan with the shortest modelled time: units on the busiest XCD's
// busiest workgroup times the unit cost, plus, when K is split (caller
// workspace only, 2 .. 8 slices of >= 4 K blocks each), the partials'
// round trip through memory and the finishing launch (≈ 6 us: 128 x 10240 x
// 2560 took 17.7 us unsplit and 21.9 us in two slices).  Deeper rings for
// 64 x 64 tiles (three or four stages, fewer workgroups per CU) measured no
// faster at M = 128 and 512.
GemmPlan gemm_plan(int M, int K, const QhGemmSeg* seg, int nseg, int cus, const void* ws, size_t ws_bytes) {
  const int KB = K / 128;
  GemmPlan best = {64, 64, 3, 1};
  double best_t = 1e300;
  for (const GemmShape& c : kGemmShapes) {
    long tiles_n = 0;
    for (int t = 0; t < nseg; ++t) tiles_n += (seg[t].N + c.bn - 1) / c.bn;
    const long tiles_m = (M + c.bm - 1) / c.bm;
    const long slots = (long)cus * c.wpc / 8;  // workgroups per XCD
    for (int S = 1; S <= 8; ++S) {
      if (S > 1 && (!ws || KB % S != 0 || KB / S < 4 ||
                    (size_t)S * M * tiles_n * c.bn * sizeof(float) > ws_bytes))
        continue;
      const long items = tiles_m * ((tiles_n + 7) / 8) * S;
      const long per_wg = (items + slots - 1) / slots;
      double t = (double)per_wg * (KB / S) * (M > 1024 ? c.cycles_large : c.cycles_small);
      if (S > 1) t += (double)S * M * tiles_n * c.bn * 4.0 * 2.0 / 2048.0 + 13000.0;
      if (t < best_t * 0.98) {
        best_t = t;
        best = {c.bm, c.bn, c.wpc, S};
      }
    }
  }
  return best;
}

template <typename ScaleT>
void launch_gemm_plan(const GemmPlan& pl, const uint16_t* x, const QhGemmSeg* seg, int nseg, int M, int K,
                      hipStream_t st, int cus, float* part, bool reduce) {
  if (pl.bm == 128)
    launch_gemm_dma<ScaleT, 2, 192, 128>(x, seg, nseg, M, K, st, cus, pl.wpc, pl.S, part, reduce);
  else if (pl.bn == 128)
    launch_gemm_dma<ScaleT, 2, 128, 64>(x, seg, nseg, M, K, st, cus, pl.wpc, pl.S, part, reduce);
  else
    launch_gemm_dma<ScaleT, 2, 64, 64>(x, seg, nseg, M, K, st, cus, pl.wpc, pl.S, part, reduce);
}

// Split-K for the per-workgroup fallback kernel (caller workspace only) when
// there are no more tiles than CUs: the largest S <= 8 dividing the K blocks
// with >= 4 blocks per slice and S * tiles <= 3 per CU.
int gemm_split_count(int K, long tiles, int cus, const void* ws, size_t ws_bytes) {
  const int KB = K / 128;
  for (int c = 8; ws && c >= 2 && tiles <= cus; --c)
    if (KB % c == 0 && KB / c >= 4 && tiles * c <= 3L * cus &&
        (size_t)tiles * c * 64 * 64 * sizeof(float) <= ws_bytes)
      return c;
  return 1;
}
}  // namespace

size_t qh_gemm_workspace_bytes(int M, int K) {
  (void)M;
  (void)K;
  return kSplitPartBytes;
}

int qh_launch_gemm_e4m3_group_ws(const void* x, int M, int K, const QhGemmSeg* seg, int nseg,
                                 bool scale_bf16, void* ws, size_t ws_bytes, hipStream_t st) {
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
  // occupancy or (weights loaded straight into operand registers) the load
  // path's coalescing.
  const long tiles = tiles64 * mt;
  float* part = (float*)ws;
  // The persistent ring kernel when its direct-to-LDS loads can take the
  // operands as they are (16-byte aligned weights, word-aligned scales, tile
  // ranges < 2 GiB), with the modelled-fastest plan; the per-workgroup kernel
  // otherwise.
  bool ring = gemm_dma_fits(K);
  for (int t = 0; t < nseg; ++t)
    ring = ring && (uintptr_t)seg[t].w % 16 == 0 && (uintptr_t)seg[t].s % 4 == 0;
  if (ring) {
    const GemmPlan pl = gemm_plan(M, K, seg, nseg, cus, ws, ws_bytes);
    if (scale_bf16) launch_gemm_plan<uint16_t>(pl, xa, seg, nseg, M, K, st, cus, part, true);
    else launch_gemm_plan<float>(pl, xa, seg, nseg, M, K, st, cus, part, true);
    return 0;
  }
  const int S = gemm_split_count(K, tiles, cus, ws, ws_bytes);
  if (scale_bf16) launch_gemm_small<uint16_t>(xa, seg, nseg, M, K, tiles, st, cus, S, part);
  else launch_gemm_small<float>(xa, seg, nseg, M, K, tiles, st, cus, S, part);
  return 0;
}

// Output projection + residual + norm (the batch prefill's o_proj / out_proj /
// down): o = bf16(x W^T), h = bf16(h + o), hn = (1+w) RMSNorm(h) (none when
// norm_w is null).  When the GEMM splits K through the ring kernel and the
// rows fit its vector kernel, one row-wise kernel finishes the split, the add
// and the norm (o is not written); otherwise o is written and the fused
// add + norm kernel follows.
int qh_launch_gemm_e4m3_add_rmsnorm(const void* x, const void* w, const void* s, void* o, int M, int N, int K,
                                    int kb, bool scale_bf16, void* h, const float* norm_w, void* hn, float eps,
                                    void* ws, size_t ws_bytes, hipStream_t st) {
  const auto al16 = [](const void* p) { return p == nullptr || (uintptr_t)p % 16 == 0; };
  if (M > 0 && N > 0 && K > 0 && K % 128 == 0 && ws && x && (uintptr_t)x % 16 == 0 && w && s &&
      (uintptr_t)w % 16 == 0 && (uintptr_t)s % 4 == 0 && gemm_dma_fits(K) && N % 8 == 0 && N <= 8192 &&
      al16(h) && al16(hn) && al16(norm_w)) {
    int cus = 256, dev = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
      cus = 256;
    const QhGemmSeg seg = {w, s, o, N, kb};
    const GemmPlan pl = gemm_plan(M, K, &seg, 1, cus, ws, ws_bytes);
    if (pl.S > 1) {
      float* part = (float*)ws;
      if (scale_bf16) launch_gemm_plan<uint16_t>(pl, (const uint16_t*)x, &seg, 1, M, K, st, cus, part, false);
      else launch_gemm_plan<float>(pl, (const uint16_t*)x, &seg, 1, M, K, st, cus, part, false);
      const int S = pl.S, ldp = ((N + pl.bn - 1) / pl.bn) * pl.bn;
      const int v = (N / 8 + 255) / 256;
#define QH_SAN(V, SC)                                                                                          \
  hipLaunchKernelGGL((splitk_add_rmsnorm_kernel<V, SC>), dim3(M), dim3(256), 0, st, (const float*)part, S, M, ldp, N, \
                     (uint16_t*)h, norm_w, (uint16_t*)hn, eps)
#define QH_SAN_S(V)             \
  switch (S) {                  \
    case 2: QH_SAN(V, 2); break; \
    case 4: QH_SAN(V, 4); break; \
    case 8: QH_SAN(V, 8); break; \
    default: QH_SAN(V, 0); break; \
  }
      if (v <= 1) QH_SAN_S(1)
      else if (v == 2) QH_SAN_S(2)
      else QH_SAN_S(4)
#undef QH_SAN_S
#undef QH_SAN
      return 0;
    }
  }
  if (qh_launch_gemm_e4m3_ws(x, w, s, o, M, N, K, kb, scale_bf16, ws, ws_bytes, st) != 0) return -1;
  if (norm_w) qh_launch_add_rmsnorm_rows(h, o, norm_w, hn, M, N, eps, st);
  else qh_launch_add_bf16(h, o, h, M * N, st);
  return 0;
}

int qh_launch_gemm_e4m3_ws(const void* x, const void* w, const void* s, void* y, int M, int N,
                           int K, int kb, bool scale_bf16, void* ws, size_t ws_bytes, hipStream_t st) {
  const QhGemmSeg seg = {w, s, y, N, kb};
  return qh_launch_gemm_e4m3_group_ws(x, M, K, &seg, 1, scale_bf16, ws, ws_bytes, st);
}

// Without a caller workspace (the reference ABI passes none): no split-K and
// nothing allocated.
int qh_launch_gemm_e4m3(const void* x, const void* w, const void* s, void* y, int M, int N, int K,
                        int kb, bool scale_bf16, hipStream_t st) {
  return qh_launch_gemm_e4m3_ws(x, w, s, y, M, N, K, kb, scale_bf16, nullptr, 0, st);
}
