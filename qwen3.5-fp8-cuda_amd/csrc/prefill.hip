// Batch prefill kernels (s > 1) for gfx950: the attention and GatedDeltaNet
// pieces of the reference's prefill path that are not GEMMs (the projections
// run on the FP8 MFMA GEMM, gemm.hip).
//
// Semantics (reference main.py:1550-1566 _prefill_step, 1034-1059 attention,
// 1097-1158 GatedDeltaNet, 1203-1217 MLP with M > 1):
//   attention : q, k = bf16 (1+w) head RMSNorm; RoPE on dims [0, rot) in fp32
//               (q stays fp32, k is cached as bf16); causal softmax(q k^T /
//               sqrt(D)) v in fp32 -> bf16, times bf16(sigmoid(gate)) -> bf16
//   GDN       : y = bf16(silu(bf16(causal conv, window 4))); q, k l2-normalised
//               in bf16 steps (transformers l2norm on bf16 tensors); g, beta
//               as in decode; recurrent gated delta rule from the stored state;
//               gated RMSNorm with bf16 intermediates
//   MLP       : m = bf16(bf16(silu(bf16 gate)) * bf16 up)
#include "qh_common.h"
#include "qh_prefill.h"

#include <algorithm>

namespace {

constexpr int TP = 32;    // key positions per LDS tile
constexpr int MAXG = 8;   // query heads per KV head

// ---- q/k norm + RoPE + cache write: one wave per (token, head row) ---------
// Four (token, head) waves per 256-thread block; the cos / sin values of a
// lane's dims are loaded with its inputs (clamped to the table row), ahead of
// the norm, so RoPE waits for no further round trip.
template <int D>
__global__ __launch_bounds__(256) void attn_prep_kernel(QhAttnPrepParams p) {
  constexpr int NPL = D / 64;
  const int rows = p.Hq + p.Hkv;
  const int idx = (int)blockIdx.x * 4 + (int)(threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (idx >= p.M * rows) return;
  const int m = idx / rows, row = idx - m * rows;
  const int pos = p.past + m;
  const bool is_q = row < p.Hq;
  const int head = is_q ? row : row - p.Hq;
  const uint16_t* src = is_q ? p.q_all + ((size_t)m * p.Hq + head) * 2 * D
                             : p.k + ((size_t)m * p.Hkv + head) * D;
  const float* nw = is_q ? p.q_norm_w : p.k_norm_w;
  float v[NPL], cs[NPL], sn[NPL];
#pragma unroll
  for (int i = 0; i < NPL; ++i) v[i] = bf2f(src[lane * NPL + i]);
  if (p.rot > 0) {
    const float* cr = p.cos_t + (size_t)pos * p.rot;
    const float* sr = p.sin_t + (size_t)pos * p.rot;
#pragma unroll
    for (int i = 0; i < NPL; ++i) {
      const int c = min(lane * NPL + i, p.rot - 1);
      cs[i] = cr[c];
      sn[i] = sr[c];
    }
  }
  if (nw) {
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < NPL; ++i) ss = fmaf(v[i], v[i], ss);
    ss = wave_sum(ss);
    const float r = rsqrtf(ss / (float)D + p.eps);
#pragma unroll
    for (int i = 0; i < NPL; ++i) v[i] = rbf(v[i] * r * (1.0f + nw[lane * NPL + i]));
  }
  if (p.rot > 0) {
    const int half = p.rot >> 1;
    const int pm = half / NPL;  // partner lane distance (power of two, checked on the host)
#pragma unroll
    for (int i = 0; i < NPL; ++i) {
      const float partner = __shfl_xor(v[i], pm, 64);
      const int c = lane * NPL + i;
      if (c < half) v[i] = v[i] * cs[i] - partner * sn[i];
      else if (c < p.rot) v[i] = v[i] * cs[i] + partner * sn[i];
    }
  }
  if (is_q) {
    float* dst = p.q_out + ((size_t)m * p.Hq + head) * D + lane * NPL;
#pragma unroll
    for (int i = 0; i < NPL; ++i) dst[i] = v[i];
  } else {
    const size_t off = ((size_t)head * p.max_seq + pos) * D + lane * NPL;
    const uint16_t* vs = p.v + ((size_t)m * p.Hkv + head) * D + lane * NPL;
#pragma unroll
    for (int i = 0; i < NPL; ++i) {
      p.k_cache[off + i] = f2bf(v[i]);
      p.v_cache[off + i] = vs[i];
    }
  }
}

// ---- causal attention: one workgroup per (KV head, query token) -------------
// The 4 waves serve the query heads of the GQA group (heads wid, wid + 4, ...:
// HPW = ceil(G / 4) per wave); K/V tiles of 32 positions are staged in LDS and
// shared by those heads.  The tile loads are branch-free (rows past the
// query's last key read row t0 and are zeroed when staged) and the next tile
// is requested before the current one is used; the per-position dot product
// and the P V sum have constant trip counts and are unrolled, so their LDS
// reads go out together.  The arithmetic order is fixed: lane half h sums the
// q k products of dims h D/2 .. h D/2 + D/2 - 1 in order, the halves are
// added, and P V adds positions in order.
template <int D, int HPW>
__global__ __launch_bounds__(256) void attn_prefill_kernel(QhAttnPrefillParams p) {
  constexpr int NPL = D / 64;
  constexpr int KS = D + 8;
  __shared__ __align__(16) float sQ[4 * HPW][D];
  __shared__ __align__(16) uint16_t sK[TP * KS];
  __shared__ __align__(16) uint16_t sV[TP * D];
  __shared__ __align__(16) float sP[4 * HPW][TP];
  const int kvh = blockIdx.x, m = blockIdx.y;
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int G = p.Hq / p.Hkv;
  const int total = p.past + m + 1;
  const uint16_t* kbase = p.k_cache + (size_t)kvh * p.max_seq * D;
  const uint16_t* vbase = p.v_cache + (size_t)kvh * p.max_seq * D;

  // K/V tile staging: each thread moves PER 16-byte pieces of K and of V
  constexpr int PER = TP * (D / 8) / 256;
  u32x4 kreg[PER], vreg[PER];
  auto fetch = [&](int t0) {
#pragma unroll
    for (int e = 0; e < PER; ++e) {
      const int idx = threadIdx.x + 256 * e;
      const int pos = t0 + idx / (D / 8);
      const int c8 = (idx % (D / 8)) * 8;
      const int src = pos < total ? pos : t0;
      kreg[e] = *(const u32x4*)(kbase + (size_t)src * D + c8);
      vreg[e] = *(const u32x4*)(vbase + (size_t)src * D + c8);
    }
  };
  auto stage = [&](int t0) {
    const u32x4 zero = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int e = 0; e < PER; ++e) {
      const int idx = threadIdx.x + 256 * e;
      const int row = idx / (D / 8);
      const int c8 = (idx % (D / 8)) * 8;
      const bool in = t0 + row < total;
      *(u32x4*)(sK + row * KS + c8) = in ? kreg[e] : zero;
      *(u32x4*)(sV + row * D + c8) = in ? vreg[e] : zero;
    }
  };
  // the query heads and gates first (unconditional loads: a slot past the
  // group reads head 0 and is not used), then the first tile
  float qv[HPW][NPL], gate_v[HPW][NPL];
#pragma unroll
  for (int hi = 0; hi < HPW; ++hi) {
    const int gi = wid + 4 * hi < G ? wid + 4 * hi : 0;
    const int h = kvh * G + gi;
    const float* q = p.q + ((size_t)m * p.Hq + h) * D;
    const uint16_t* gp = p.gate + (size_t)m * p.gate_mstride + (size_t)h * p.gate_hstride;
#pragma unroll
    for (int i = 0; i < NPL; ++i) {
      qv[hi][i] = q[lane * NPL + i];
      gate_v[hi][i] = bf2f(gp[lane * NPL + i]);
    }
  }
  fetch(0);
#pragma unroll
  for (int hi = 0; hi < HPW; ++hi) {
    const int gi = wid + 4 * hi;
    if (gi < G) {
#pragma unroll
      for (int i = 0; i < NPL; ++i) sQ[gi][lane * NPL + i] = qv[hi][i];
    }
  }
  float mx[HPW], l[HPW], o[HPW][NPL];
#pragma unroll
  for (int hi = 0; hi < HPW; ++hi) {
    mx[hi] = -INFINITY;
    l[hi] = 0.0f;
#pragma unroll
    for (int i = 0; i < NPL; ++i) o[hi][i] = 0.0f;
  }
  const float scale = rsqrtf((float)D);
  const int prow = lane >> 1, half = lane & 1;
  for (int t0 = 0; t0 < total; t0 += TP) {
    stage(t0);
    __syncthreads();
    if (t0 + TP < total) fetch(t0 + TP);
    const bool valid = t0 + prow < total;
#pragma unroll
    for (int hi = 0; hi < HPW; ++hi) {
      const int gi = wid + 4 * hi;
      if (gi < G) {
        const uint16_t* kr = sK + prow * KS + half * (D / 2);
        const float* qr = &sQ[gi][half * (D / 2)];
        u32x4 k8[D / 16];
#pragma unroll
        for (int cc = 0; cc < D / 16; ++cc) k8[cc] = *(const u32x4*)(kr + 8 * cc);
        float dot = 0.0f;
#pragma unroll
        for (int cc = 0; cc < D / 16; ++cc) {
          const float4 qa = *(const float4*)(qr + 8 * cc);
          const float4 qb = *(const float4*)(qr + 8 * cc + 4);
          dot = fmaf(qa.x, bf_lo(k8[cc].x), dot);
          dot = fmaf(qa.y, bf_hi(k8[cc].x), dot);
          dot = fmaf(qa.z, bf_lo(k8[cc].y), dot);
          dot = fmaf(qa.w, bf_hi(k8[cc].y), dot);
          dot = fmaf(qb.x, bf_lo(k8[cc].z), dot);
          dot = fmaf(qb.y, bf_hi(k8[cc].z), dot);
          dot = fmaf(qb.z, bf_lo(k8[cc].w), dot);
          dot = fmaf(qb.w, bf_hi(k8[cc].w), dot);
        }
        dot += __shfl_xor(dot, 1, 64);
        const float sc = valid ? dot * scale : -INFINITY;
        const float nm = fmaxf(mx[hi], wave_max(sc));
        const float corr = __expf(mx[hi] - nm);
        const float pv = valid ? __expf(sc - nm) : 0.0f;
        l[hi] = l[hi] * corr + wave_sum(half == 0 ? pv : 0.0f);
        mx[hi] = nm;
        if (half == 0) sP[gi][prow] = pv;
#pragma unroll
        for (int i = 0; i < NPL; ++i) o[hi][i] *= corr;
      }
    }
    __syncthreads();
#pragma unroll
    for (int hi = 0; hi < HPW; ++hi) {
      const int gi = wid + 4 * hi;
      if (gi < G) {
#pragma unroll
        for (int j4 = 0; j4 < TP / 4; ++j4) {
          const float4 p4 = *(const float4*)&sP[gi][4 * j4];
          const float pj[4] = {p4.x, p4.y, p4.z, p4.w};
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            const uint16_t* vr = sV + (4 * j4 + u) * D + lane * NPL;
#pragma unroll
            for (int i = 0; i < NPL; ++i) o[hi][i] = fmaf(pj[u], bf2f(vr[i]), o[hi][i]);
          }
        }
      }
    }
    __syncthreads();
  }
#pragma unroll
  for (int hi = 0; hi < HPW; ++hi) {
    const int gi = wid + 4 * hi;
    if (gi < G) {
      const int h = kvh * G + gi;
      const float inv = 1.0f / l[hi];
      uint16_t* dst = p.out + (size_t)m * p.Hq * D + (size_t)h * D + lane * NPL;
#pragma unroll
      for (int i = 0; i < NPL; ++i)
        dst[i] = f2bf(rbf(o[hi][i] * inv) * rbf(qh_sigmoid(gate_v[hi][i])));
    }
  }
}

// ---- batch attention on the matrix cores (D = 256, 4 query heads per KV head) --
// One workgroup per (KV head, 32 query tokens); wave w is query head
// 4 kvh + w of the GQA group, so the 4 waves share every K / V tile in LDS.
// Tiles of 64 key positions; rows at or past the workgroup's last key (and
// past the prompt) read as zeros through the range-checked buffer resources.
// The next tile's K / V rows are loaded into registers while the current tile
// is computed.
//
// Scores are computed transposed, S^T = K Q^T on v_mfma_f32_32x32x16_bf16 (A = K
// rows, B = Q^T), so each lane owns one query row (lane % 32) and 16 of a
// 32-position block's scores: the row max and sum need one exchange with the
// partner lane (lane ^ 32, v_permlane32_swap).  The output is also transposed,
// O^T = V^T P^T (A = the V tile stored transposed in LDS, B = P^T), so a
// lane's 128 accumulators are its own query row and the online-softmax
// rescale stays in the lane.
//
// The rescale is lazy: the exponentials use a per-row reference max that is
// raised only when some row's running max passes it by more than kFaSlack, so
// p <= e^kFaSlack and O / l is unchanged up to fp32 rounding; most tiles skip
// the 128-accumulator rescale.  Only tiles that reach past the workgroup's
// first query position apply the causal mask.
//
// Precision as the reference's fp32 q . k, softmax and P . v: q (fp32) and P
// (fp32) enter as hi + lo bf16 pairs (hi = bf16(x), lo = bf16(x - hi), about
// 16 mantissa bits), each pair two matrix-core products that are exact in
// fp32; k and v are bf16 already.  q is scaled by 1/16 = 256^-1/2 first
// (exact).  The q hi parts stay in registers, the lo parts in a per-wave LDS
// area; a 16-dimension block's lo term is computed only when it is nonzero for
// some lane of the wave (the head-norm output is a bf16 value in every
// dimension RoPE does not rotate).
constexpr int kFaTile = 64;                    // key positions per tile
constexpr int kFaKRow = 256 * 2 + 16;          // padded K row in LDS (bytes)
constexpr int kFaVRow = kFaTile * 2 + 16;      // padded V^T row in LDS (bytes)
constexpr int kFaQRow = 256 * 2 + 16;          // padded q lo row in LDS (bytes)
constexpr int kFaV0 = kFaTile * kFaKRow;                       // 33,792
constexpr int kFaQ0 = kFaV0 + 256 * kFaVRow;                   // 70,656
constexpr int kFaLds = kFaQ0 + 4 * 32 * kFaQRow;               // 138,240 B
constexpr float kFaSlack = 8.0f;

typedef float v16f_fa __attribute__((ext_vector_type(16)));
typedef __bf16 v8bf_fa __attribute__((ext_vector_type(8)));

__device__ __forceinline__ uint32_t pack_bf2(float a, float b) {
  return (uint32_t)f2bf(a) | ((uint32_t)f2bf(b) << 16);
}
// 8 fp32 -> hi (bf16 of each) and lo (bf16 of each residual), packed
__device__ __forceinline__ void split8(const float (&v)[8], u32x4& hi, u32x4& lo) {
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const float a = v[2 * q], b = v[2 * q + 1];
    const float ah = rbf(a), bh = rbf(b);
    hi[q] = (__float_as_uint(ah) >> 16) | (__float_as_uint(bh) & 0xFFFF0000u);
    lo[q] = pack_bf2(a - ah, b - bh);
  }
}
// both lanes of a (lane, lane ^ 32) pair get max / sum of their two values
__device__ __forceinline__ float pair_max(float x) {
  const auto s = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(s[0]), __uint_as_float(s[1]));
}
__device__ __forceinline__ float pair_sum(float x) {
  const auto s = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(s[0]) + __uint_as_float(s[1]);
}

__global__ __launch_bounds__(256) void attn_prefill_mfma_kernel(QhAttnPrefillParams p) {
  extern __shared__ __align__(16) uint8_t smem[];
  uint8_t* sK = smem;
  uint8_t* sV = smem + kFaV0;
  // the last query blocks (the most tiles) are dispatched first
  const int kvh = blockIdx.x, m0 = (gridDim.y - 1 - blockIdx.y) * 32;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane & 31, h = lane >> 5;
  const int head = kvh * 4 + wid;
  const int qpos = p.past + m0 + r;      // its position
  const int kv_end = p.past + min(m0 + 32, p.M);
  const int q0pos = p.past + m0;         // the workgroup's first query position
  const uint16_t* kbase = p.k_cache + (size_t)kvh * p.max_seq * 256;
  const uint16_t* vbase = p.v_cache + (size_t)kvh * p.max_seq * 256;

  // K / V rows of this KV head through range-checked buffer resources: rows
  // at or past kv_end read as zeros, so the tile loads carry no branch
  const auto rk = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(kbase), (short)0, kv_end * 512,
                                                    0x00020000);
  const auto rv = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(vbase), (short)0, kv_end * 512,
                                                    0x00020000);
  // K: 64 rows x 32 chunks of 16 bytes, chunk tid + 256 i (coalesced).
  // V: thread (pg, dc) = (tid % 8, tid / 8) takes positions 8 pg .. + 7 of
  // dimensions 8 dc .. + 7 and stores them transposed.
  const int pg = tid & 7, dc = tid >> 3;
  u32x4 kv[8], vv[8];
  auto load_k = [&](int t0) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int c = tid + 256 * i;
      kv[i] = __builtin_amdgcn_raw_buffer_load_b128(rk, (uint32_t)((t0 + (c >> 5)) * 512 + (c & 31) * 16), 0, 0);
    }
  };
  auto load_v = [&](int t0) {
#pragma unroll
    for (int i = 0; i < 8; ++i)
      vv[i] = __builtin_amdgcn_raw_buffer_load_b128(rv, (uint32_t)((t0 + 8 * pg + i) * 512 + dc * 16), 0, 0);
  };
  load_k(0);
  load_v(0);

  // Q^T operand: dims 16 kk + 8 h .. + 7 of the lane's query, hi in
  // registers, lo in this wave's LDS rows.  The wave loads its 32 query rows
  // coalesced (row i by all 64 lanes, 4 dimensions each), splits them, and
  // hands the hi parts to the lanes that own them through the K / V area,
  // which is free until the first tile is stored.
  u32x4 qhi[16];
  uint32_t lo_mask = 0;  // 16-dimension blocks whose lo part is nonzero in this wave
  uint8_t* sQw = smem + kFaQ0 + wid * 32 * kFaQRow;
  uint8_t* sHw = smem + wid * 32 * kFaQRow;  // 4 x 16,896 B, below kFaQ0
  uint8_t* sQ = sQw + r * kFaQRow + 16 * h;
  {
    float4 qa[32];
#pragma unroll
    for (int i = 0; i < 32; ++i)
      qa[i] = *(const float4*)(p.q + ((size_t)min(m0 + i, p.M - 1) * p.Hq + head) * 256 + 4 * lane);
    __builtin_amdgcn_sched_barrier(0);
    uint64_t nzl = 0;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      const float v[4] = {qa[i].x * 0.0625f, qa[i].y * 0.0625f, qa[i].z * 0.0625f, qa[i].w * 0.0625f};
      u32x2 hi, lo;
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const float ah = rbf(v[2 * q]), bh = rbf(v[2 * q + 1]);
        hi[q] = (__float_as_uint(ah) >> 16) | (__float_as_uint(bh) & 0xFFFF0000u);
        lo[q] = pack_bf2(v[2 * q] - ah, v[2 * q + 1] - bh);
      }
      *(u32x2*)(sHw + i * kFaQRow + 8 * lane) = hi;
      *(u32x2*)(sQw + i * kFaQRow + 8 * lane) = lo;
      nzl |= __builtin_amdgcn_ballot_w64((lo.x | lo.y) != 0u);
    }
#pragma unroll
    for (int kk = 0; kk < 16; ++kk)
      if ((nzl >> (4 * kk)) & 0xFu) lo_mask |= 1u << kk;
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < 16; ++kk) qhi[kk] = *(const u32x4*)(sHw + r * kFaQRow + 32 * kk + 16 * h);
  }
  // lo terms for blocks 0 .. nlo - 1, four at a time (a block whose lo is
  // zero adds zero)
  const int nlo = lo_mask ? 32 - __builtin_clz(lo_mask) : 0;
  v16f_fa o[8];
#pragma unroll
  for (int d = 0; d < 8; ++d)
#pragma unroll
    for (int e = 0; e < 16; ++e) o[d][e] = 0.0f;
  float mref = -INFINITY, lrow = 0.0f;

  const uint8_t* ka_row = sK + r * kFaKRow + 16 * h;
  for (int t0 = 0; t0 < kv_end; t0 += kFaTile) {
    __syncthreads();  // every wave is done with the previous tile
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int c = tid + 256 * i;
      *(u32x4*)(sK + (c >> 5) * kFaKRow + (c & 31) * 16) = kv[i];
    }
    // V^T row 8 dc + j, positions 8 pg .. + 7: pairs of 16-bit halves
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint32_t sel = (j & 1) ? 0x07060302u : 0x05040100u;
      u32x4 col;
#pragma unroll
      for (int q = 0; q < 4; ++q) col[q] = __builtin_amdgcn_perm(vv[2 * q + 1][j >> 1], vv[2 * q][j >> 1], sel);
      *(u32x4*)(sV + (8 * dc + j) * kFaVRow + 16 * pg) = col;
    }
    __syncthreads();
    load_k(t0 + kFaTile);  // past kv_end: zeros, no memory traffic

    // S^T for the two 32-position blocks (two independent chains; four, with
    // the even and odd blocks summed afterwards, measured slower: 3.7 k ->
    // 4.0 k cycles per tile)
    v16f_fa s0, s1;
#pragma unroll
    for (int e = 0; e < 16; ++e) s0[e] = s1[e] = 0.0f;
#pragma unroll
    for (int kk = 0; kk < 16; ++kk) {
      const v8bf_fa ka0 = __builtin_bit_cast(v8bf_fa, *(const u32x4*)(ka_row + 32 * kk));
      const v8bf_fa ka1 = __builtin_bit_cast(v8bf_fa, *(const u32x4*)(ka_row + 32 * kFaKRow + 32 * kk));
      const v8bf_fa qb = __builtin_bit_cast(v8bf_fa, qhi[kk]);
      s0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ka0, qb, s0, 0, 0, 0);
      s1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ka1, qb, s1, 0, 0, 0);
    }
    for (int g = 0; g < nlo; g += 4) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int kk = g + i;
        const v8bf_fa ka0 = __builtin_bit_cast(v8bf_fa, *(const u32x4*)(ka_row + 32 * kk));
        const v8bf_fa ka1 = __builtin_bit_cast(v8bf_fa, *(const u32x4*)(ka_row + 32 * kFaKRow + 32 * kk));
        const v8bf_fa ql = __builtin_bit_cast(v8bf_fa, *(const u32x4*)(sQ + 32 * kk));
        s0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ka0, ql, s0, 0, 0, 0);
        s1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ka1, ql, s1, 0, 0, 0);
      }
    }
    // causal mask on tiles that reach past the first query position: score
    // e of block nt is position t0 + 32 nt + 8 (e / 4) + 4 h + e % 4
    if (t0 + kFaTile - 1 > q0pos) {
      const int lim = qpos - t0 - 4 * h;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int idx = 8 * (e >> 2) + (e & 3);
        s0[e] = idx <= lim ? s0[e] : -INFINITY;
        s1[e] = idx + 32 <= lim ? s1[e] : -INFINITY;
      }
    }
    float tmax = fmaxf(s0[0], s1[0]);
#pragma unroll
    for (int e = 1; e < 16; ++e) tmax = fmaxf(tmax, fmaxf(s0[e], s1[e]));
    tmax = pair_max(tmax);
    if (__builtin_amdgcn_ballot_w64(tmax > mref + kFaSlack) != 0) {
      // every row's first tile has position 0 unmasked, so mnew is finite
      const float mnew = fmaxf(mref, tmax);
      const float corr = mnew == mref ? 1.0f : __expf(mref - mnew);
      lrow *= corr;
#pragma unroll
      for (int d = 0; d < 8; ++d)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          float x = o[d][e], t;
          asm volatile("v_accvgpr_read_b32 %1, %0\n\tv_mul_f32_e32 %1, %2, %1\n\tv_accvgpr_write_b32 %0, %1"
                       : "+a"(x), "=&v"(t)
                       : "v"(corr));
          o[d][e] = x;
        }
      mref = mnew;
    }
    float psum = 0.0f;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      s0[e] = __expf(s0[e] - mref);
      s1[e] = __expf(s1[e] - mref);
      psum += s0[e] + s1[e];
    }
    lrow += pair_sum(psum);
    // P^T operand of block kk: positions 16 kk + 8 h .. + 7 of the lane's
    // row.  Lane h = 0 holds positions 0-3 and 8-11 of each 16, lane h = 1
    // positions 4-7 and 12-15; one swap of the middle pair gives both lanes
    // their 8 in order.
    u32x4 phi[4], plo[4];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const v16f_fa& sv = kk < 2 ? s0 : s1;
      const int b = 8 * (kk & 1);
      float v[8];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(sv[b + i]), __float_as_uint(sv[b + 4 + i]),
                                                         false, false);
        v[i] = __uint_as_float(sw[0]);
        v[4 + i] = __uint_as_float(sw[1]);
      }
      split8(v, phi[kk], plo[kk]);
    }
    load_v(t0 + kFaTile);
    // O^T += V^T P^T over 8 blocks of 32 dimensions; consecutive products
    // go to different accumulators
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      v8bf_fa va[8];
#pragma unroll
      for (int d = 0; d < 8; ++d)
        va[d] = __builtin_bit_cast(v8bf_fa, *(const u32x4*)(sV + (32 * d + r) * kFaVRow + 16 * h + 32 * kk));
#pragma unroll
      for (int d = 0; d < 8; ++d)
        o[d] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va[d], __builtin_bit_cast(v8bf_fa, phi[kk]), o[d], 0, 0, 0);
#pragma unroll
      for (int d = 0; d < 8; ++d)
        o[d] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va[d], __builtin_bit_cast(v8bf_fa, plo[kk]), o[d], 0, 0, 0);
    }
  }
  // out = bf16(bf16(O / l) * bf16(sigmoid(gate))) for the lane's query
  if (m0 + r >= p.M) return;
  const float inv = 1.0f / lrow;
  const uint16_t* gp = p.gate + (size_t)(m0 + r) * p.gate_mstride + (size_t)head * p.gate_hstride;
  uint16_t* dst = p.out + (size_t)(m0 + r) * p.Hq * 256 + (size_t)head * 256;
#pragma unroll
  for (int d = 0; d < 8; ++d)
#pragma unroll
    for (int b4 = 0; b4 < 4; ++b4) {
      const int dim = 32 * d + 8 * b4 + 4 * h;
      const u32x2 gw = *(const u32x2*)(gp + dim);
      const float g[4] = {bf_lo(gw.x), bf_hi(gw.x), bf_lo(gw.y), bf_hi(gw.y)};
      float y[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) y[i] = rbf(o[d][4 * b4 + i] * inv) * rbf(qh_sigmoid(g[i]));
      *(u32x2*)(dst + dim) = u32x2{pack_bf2(y[0], y[1]), pack_bf2(y[2], y[3])};
    }
}

// ---- GDN conv over the sequence: one thread per (token, channel) -------------
// x_t for t < 0 comes from the ring (positions past-3 .. past-1).  The ring is
// not written here (other threads still read it): gdn_norm_gates_kernel, the
// next launch, stores the last four positions.
__global__ __launch_bounds__(256) void gdn_conv_kernel(QhGdnPrepParams p) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (size_t)p.M * p.C) return;
  const int m = (int)(i / (size_t)p.C), c = (int)(i - (size_t)m * p.C);
  const uint16_t* ring = p.conv_ring + (size_t)c * 4;
  const uint16_t* w = p.conv_w + (size_t)c * 4;
  auto x_at = [&](int t) {  // x of prompt token t (t >= -3)
    return t >= 0 ? bf2f(p.mixed[(size_t)t * p.C + c]) : bf2f(ring[(p.past + t) & 3]);
  };
  const float x0 = x_at(m), x1 = x_at(m - 1), x2 = x_at(m - 2), x3 = x_at(m - 3);
  float acc = bf2f(w[3]) * x0;
  acc = fmaf(bf2f(w[2]), x1, acc);
  acc = fmaf(bf2f(w[1]), x2, acc);
  acc = fmaf(bf2f(w[0]), x3, acc);
  p.y[i] = f2bf(qh_silu(rbf(acc)));
}

// ---- q/k l2norm (bf16 steps) and gates: grid (M, 2 Hk + 1), one wave each ----
// blockIdx.y < 2 Hk: l2norm of q (y < Hk) or k of key head y % Hk; the last
// row computes the Hv gates of token m.
// The blocks of token 0 also store the ring's last four positions (slot
// (past + m) % 4 holds x of token m), once the conv has read it.
// Four (token, row) waves per 256-thread block (row < 2 Hk: the l2norm of a
// q or k head; row 2 Hk: the gates), each wave as the one-wave blocks it
// replaced.  Every thread of the grid also stores its share of the conv
// ring's last four positions (one (channel, position) copy per thread from
// 16 tokens; token 0's waves alone made one memory round trip per copy).
__global__ __launch_bounds__(256) void gdn_norm_gates_kernel(QhGdnPrepParams p) {
  const int rows = 2 * p.Hk + 1;
  const int idx = (int)blockIdx.x * 4 + (int)(threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (idx >= p.M * rows) return;
  const int m = idx / rows, row = idx - m * rows;
  {
    const int nt = min(4, p.M);
    const long total = (long)p.C * nt, nthr = (long)p.M * rows * 64;
    for (long it = (long)idx * 64 + lane; it < total; it += nthr) {
      const int c = (int)(it / nt), t = p.M - nt + (int)(it - (long)c * nt);
      p.conv_ring[(size_t)c * 4 + ((p.past + t) & 3)] = p.mixed[(size_t)t * p.C + c];
    }
  }
  if (row < 2 * p.Hk) {
    const bool is_k = row >= p.Hk;
    const int kh = row % p.Hk;
    const uint16_t* src = p.y + (size_t)m * p.C + (is_k ? p.Hk * p.dk : 0) + kh * p.dk;
    uint16_t* dst = (is_k ? p.kn : p.qn) + ((size_t)m * p.Hk + kh) * p.dk;
    float ss = 0.0f;
    for (int i = lane; i < p.dk; i += 64) {
      const float x = bf2f(src[i]);
      ss += rbf(x * x);
    }
    ss = wave_sum(ss);
    const float inv = rbf(rsqrtf(rbf(rbf(ss) + 1e-6f)));
    for (int i = lane; i < p.dk; i += 64) dst[i] = f2bf(bf2f(src[i]) * inv);
  } else if (lane < p.Hv) {
    const int h = lane;
    const float a = bf2f(p.a[(size_t)m * p.Hv + h]), b = bf2f(p.b[(size_t)m * p.Hv + h]);
    p.g[(size_t)m * p.Hv + h] = -expf(p.A_log[h]) * qh_softplus(a + p.dt_bias[h]);
    p.beta[(size_t)m * p.Hv + h] = f2bf(qh_sigmoid(b));
  }
}

// ---- recurrent scan: one wave per (head, COLS value columns) ---------------
// Lane l owns value column j = 8 cg + (l >> 3) of head h and state rows
// 16 (l & 7) .. +16 of it, so the two sums over the key dimension (S^T k and
// S^T q) are 8-lane butterflies inside the wave: a token needs no workgroup
// barrier, and the 16 waves of a head spread over the device.  q and k pass
// through a small per-wave LDS buffer (alternating halves by token parity).
// The operands of the next SCAN_AHEAD tokens are in flight in registers (a
// rotating set, the token loop unrolled by SCAN_AHEAD; loads past the prompt
// re-read its last token).  Every lane stores its column's output (the 8 lanes
// of a column hold the same value), so no vector-memory access sits under a
// branch and the load counter's waits stay exact.  The bf16 core output goes
// to `out`; gdn_gated_norm_kernel then applies the gated RMSNorm in place.
constexpr int SCAN_AHEAD = 8;

template <int COLS>
__global__ __launch_bounds__(64) void gdn_scan_kernel(QhGdnScanParams p) {
  constexpr int DK = 128, DV = 128, A = SCAN_AHEAD;
  constexpr int L = 64 / COLS;            // lanes per column
  constexpr int RPT = DK / L;             // state rows per lane
  constexpr int GROUPS = DV / COLS;       // waves per head
  static_assert(L == 8 || L == 16, "column width");
  __shared__ __align__(16) float sq[2][DK];
  __shared__ __align__(16) float sk[2][DK];
  const int h = blockIdx.x / GROUPS, cg = blockIdx.x % GROUPS;
  const int kh = h / (p.Hv / p.Hk);
  const int lane = threadIdx.x;
  const int r = lane & (L - 1);             // row group: rows RPT r .. +RPT
  const int j = cg * COLS + lane / L;
  float* col = p.state + (size_t)h * DK * DV + j;
  float S[RPT];
#pragma unroll
  for (int i = 0; i < RPT; ++i) S[i] = col[(size_t)(r * RPT + i) * DV];
  const float qscale = rsqrtf((float)DK);
  const size_t qk_off = (size_t)kh * DK + 2 * lane;  // a bf16 pair per lane
  const size_t v_off = (size_t)2 * p.Hk * DK + (size_t)h * DV + j;

  // raw bits: converting at load time would wait for the load
  uint32_t qq[A], kk[A];
  uint16_t vv[A], bb[A];
  float gg[A];
  auto fetch = [&](int m, int d) {
    m = min(m, p.M - 1);
    qq[d] = *(const uint32_t*)(p.qn + (size_t)m * p.Hk * DK + qk_off);
    kk[d] = *(const uint32_t*)(p.kn + (size_t)m * p.Hk * DK + qk_off);
    vv[d] = p.y[(size_t)m * p.C + v_off];
    gg[d] = p.g[(size_t)m * p.Hv + h];
    bb[d] = p.beta[(size_t)m * p.Hv + h];
  };
  auto step = [&](int m, int d) {
    // keep this token's conversions here: hoisted to the loop top they would
    // wait for every token's loads at once
    __builtin_amdgcn_sched_barrier(0);
    float* qs = sq[d & 1];
    float* ks = sk[d & 1];
    *(qh_f32x2*)(qs + 2 * lane) = qh_f32x2{bf_lo(qq[d]) * qscale, bf_hi(qq[d]) * qscale};
    *(qh_f32x2*)(ks + 2 * lane) = qh_f32x2{bf_lo(kk[d]), bf_hi(kk[d])};
    const float v = bf2f(vv[d]), decay = expf(gg[d]), beta = bf2f(bb[d]);
    fetch(m + A, d);
    __syncthreads();  // one wave: orders the LDS writes before the reads
    float kr[RPT], qr[RPT];
#pragma unroll
    for (int i = 0; i < RPT; i += 4) {
      *(f32x4*)(kr + i) = *(const f32x4*)(ks + r * RPT + i);
      *(f32x4*)(qr + i) = *(const f32x4*)(qs + r * RPT + i);
    }
    // four independent partial sums per lane (short dependency chains)
    float pp[4] = {0.0f, 0.0f, 0.0f, 0.0f}, op[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
      S[i] *= decay;
      pp[i & 3] = fmaf(S[i], kr[i], pp[i & 3]);
    }
    const float pred = column_sum<L>((pp[0] + pp[1]) + (pp[2] + pp[3]));
    const float delta = (v - pred) * beta;
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
      S[i] = fmaf(kr[i], delta, S[i]);
      op[i & 3] = fmaf(S[i], qr[i], op[i & 3]);
    }
    const float o = column_sum<L>((op[0] + op[1]) + (op[2] + op[3]));
    p.out[(size_t)m * p.Hv * DV + (size_t)h * DV + j] = f2bf(o);
  };
  // token by token, in order, as the loop re-issues them (the loop-entry
  // waits are derived from this order)
#pragma unroll
  for (int d = 0; d < A; ++d) {
    fetch(d, d);
    __builtin_amdgcn_sched_barrier(0);
  }
  int m0 = 0;
  for (; m0 + A <= p.M; m0 += A) {
#pragma unroll
    for (int d = 0; d < A; ++d) step(m0 + d, d);
  }
#pragma unroll
  for (int d = 0; d < A; ++d)
    if (m0 + d < p.M) step(m0 + d, d);
#pragma unroll
  for (int i = 0; i < RPT; ++i) col[(size_t)(r * RPT + i) * DV] = S[i];
}

// ---- gated RMSNorm of the scan output, in place: one 128-thread block per
// (token, head) (main.py:1152-1158) --------------------------------------------
// One wave per (token, head), four per block, no LDS or barrier: lane j
// holds elements j and j + 64 and the two 64-element sums are added as the
// two-wave kernel below does, so the results are the same bit for bit.
__global__ __launch_bounds__(256) void gdn_gated_norm_wave_kernel(QhGdnScanParams p) {
  const int idx = (int)blockIdx.x * 4 + (threadIdx.x >> 6), j = threadIdx.x & 63;
  if (idx >= p.M * p.Hv) return;
  const size_t o = (size_t)idx * 128 + j;  // token idx / Hv, head idx % Hv: rows of Hv * 128
  const float c0 = bf2f(p.out[o]), c1 = bf2f(p.out[o + 64]);
  const float z0 = bf2f(p.z[o]), z1 = bf2f(p.z[o + 64]);
  const float w0 = bf2f(p.norm_w[j]), w1 = bf2f(p.norm_w[j + 64]);
  const float rs = rsqrtf((wave_sum(c0 * c0) + wave_sum(c1 * c1)) / 128.0f + p.eps);
  p.out[o] = f2bf(rbf(rbf(c0 * rs) * w0) * rbf(qh_silu(z0)));
  p.out[o + 64] = f2bf(rbf(rbf(c1 * rs) * w1) * rbf(qh_silu(z1)));
}
__global__ __launch_bounds__(128) void gdn_gated_norm_kernel(QhGdnScanParams p) {
  __shared__ float red2[2];
  const int m = blockIdx.x, h = blockIdx.y, j = threadIdx.x;
  const size_t o = (size_t)m * p.Hv * 128 + (size_t)h * 128 + j;
  const float core = bf2f(p.out[o]);
  const float zv = bf2f(p.z[o]), nw = bf2f(p.norm_w[j]);
  const float s2 = wave_sum(core * core);
  if ((j & 63) == 0) red2[j >> 6] = s2;
  __syncthreads();
  const float rs = rsqrtf((red2[0] + red2[1]) / 128.0f + p.eps);
  const float normed = rbf(rbf(core * rs) * nw);
  p.out[o] = f2bf(normed * rbf(qh_silu(zv)));
}

// 8 channels per thread (16-byte loads and store; C % 8 == 0 and aligned
// rows), the same arithmetic per channel as gdn_conv_kernel.
__global__ __launch_bounds__(256) void gdn_conv8_kernel(QhGdnPrepParams p) {
  const int C8 = p.C >> 3;
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (size_t)p.M * C8) return;
  const int m = (int)(i / (size_t)C8), c0 = (int)(i - (size_t)m * C8) * 8;
  // taps of channels c0 .. c0 + 7: w[c * 4 + j], 64 contiguous bytes
  const u32x4* wq = (const u32x4*)(p.conv_w + (size_t)c0 * 4);
  const u32x4 wv[4] = {wq[0], wq[1], wq[2], wq[3]};
  float x[4][8];  // x[d][k]: token m - d, channel c0 + k
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    const int t = m - d;
    if (t >= 0) {
      const u32x4 v = *(const u32x4*)(p.mixed + (size_t)t * p.C + c0);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        x[d][2 * q] = bf_lo(v[q]);
        x[d][2 * q + 1] = bf_hi(v[q]);
      }
    } else {
#pragma unroll
      for (int k = 0; k < 8; ++k) x[d][k] = bf2f(p.conv_ring[(size_t)(c0 + k) * 4 + ((p.past + t) & 3)]);
    }
  }
  u32x4 out;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    float r2[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int k = 2 * q + h;
      // w of channel k, tap j: word (4 k + j) / 2 of the 16 words
      auto wt = [&](int j) {
        const int e = 4 * k + j;
        const uint32_t word = wv[e >> 3][(e >> 1) & 3];
        return (e & 1) ? bf_hi(word) : bf_lo(word);
      };
      float acc = wt(3) * x[0][k];
      acc = fmaf(wt(2), x[1][k], acc);
      acc = fmaf(wt(1), x[2][k], acc);
      acc = fmaf(wt(0), x[3][k], acc);
      r2[h] = qh_silu(rbf(acc));
    }
    out[q] = (uint32_t)f2bf(r2[0]) | ((uint32_t)f2bf(r2[1]) << 16);
  }
  *(u32x4*)(p.y + (size_t)m * p.C + c0) = out;
}

// 8 elements per thread (16-byte loads and store), same arithmetic.
__global__ __launch_bounds__(256) void silu_mul8_kernel(const uint16_t* g, const uint16_t* u, uint16_t* m,
                                                        size_t n8) {
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n8; i += (size_t)gridDim.x * 256) {
    const u32x4 gv = ((const u32x4*)g)[i], uv = ((const u32x4*)u)[i];
    u32x4 o;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float a = rbf(qh_silu(bf_lo(gv[q]))) * bf_lo(uv[q]);
      const float b = rbf(qh_silu(bf_hi(gv[q]))) * bf_hi(uv[q]);
      o[q] = (uint32_t)f2bf(a) | ((uint32_t)f2bf(b) << 16);
    }
    ((u32x4*)m)[i] = o;
  }
}

__global__ __launch_bounds__(256) void silu_mul_kernel(const uint16_t* g, const uint16_t* u,
                                                       uint16_t* m, size_t n) {
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256)
    m[i] = f2bf(rbf(qh_silu(bf2f(g[i]))) * bf2f(u[i]));
}

bool rot_ok(int rot, int D) {
  const int npl = D / 64;
  return rot >= 0 && rot <= D && rot % 2 == 0 &&
         (rot == 0 || ((rot / 2) % npl == 0 && (((rot / 2 / npl) & (rot / 2 / npl - 1)) == 0)));
}

}  // namespace

int qh_launch_attn_prep(const QhAttnPrepParams& p, hipStream_t st) {
  if ((p.D != 128 && p.D != 256) || !rot_ok(p.rot, p.D) || p.Hkv <= 0 || p.Hq <= 0 || p.Hq % p.Hkv != 0 ||
      p.past < 0 || p.past + p.M > p.max_seq) {
    qh_set_error("attn_prep: unsupported shape (D=%d rot=%d Hq=%d Hkv=%d past=%d M=%d max_seq=%d)",
                 p.D, p.rot, p.Hq, p.Hkv, p.past, p.M, p.max_seq);
    return -1;
  }
  if (p.M <= 0) return 0;
  const dim3 grid((unsigned)(((long)p.M * (p.Hq + p.Hkv) + 3) / 4));
  if (p.D == 256)
    hipLaunchKernelGGL(attn_prep_kernel<256>, grid, dim3(256), 0, st, p);
  else
    hipLaunchKernelGGL(attn_prep_kernel<128>, grid, dim3(256), 0, st, p);
  return 0;
}

int qh_launch_attn_prefill(const QhAttnPrefillParams& p, hipStream_t st) {
  if ((p.D != 128 && p.D != 256) || p.Hkv <= 0 || p.Hq <= 0 || p.Hq % p.Hkv != 0 || p.Hq / p.Hkv > MAXG ||
      p.past < 0 || p.past + p.M > p.max_seq) {
    qh_set_error("attn_prefill: unsupported shape (D=%d Hq=%d Hkv=%d past=%d M=%d)", p.D, p.Hq,
                 p.Hkv, p.past, p.M);
    return -1;
  }
  if (p.M <= 0) return 0;
  // D = 256 with 4 query heads per KV head, 16-byte aligned rows and at
  // least 256 tokens: the matrix-core kernel (one workgroup per 32 tokens);
  // other launches the per-token one.  Measured per layer at 4 KV heads:
  // 128 tokens 15.3 vs 27.5 us, 256 tokens 38 vs 38 us, 512 tokens 116 vs
  // 54 us, 3700 tokens 4.3 ms vs 0.45 ms (per-token vs matrix-core).
  if (p.M >= 256 && p.D == 256 && p.Hq == 4 * p.Hkv && (uintptr_t)p.q % 16 == 0 && (uintptr_t)p.gate % 8 == 0 &&
      p.gate_mstride % 4 == 0 && p.gate_hstride % 4 == 0 && (uintptr_t)p.k_cache % 16 == 0 &&
      (uintptr_t)p.v_cache % 16 == 0 && (uintptr_t)p.out % 8 == 0) {
    hipLaunchKernelGGL(attn_prefill_mfma_kernel, dim3(p.Hkv, (p.M + 31) / 32), dim3(256), (size_t)kFaLds, st, p);
    return 0;
  }
  const dim3 grid(p.Hkv, p.M);
  const bool g4 = p.Hq <= 4 * p.Hkv;  // one query head per wave
  void (*fn)(QhAttnPrefillParams) =
      p.D == 256 ? (g4 ? attn_prefill_kernel<256, 1> : attn_prefill_kernel<256, 2>)
                 : (g4 ? attn_prefill_kernel<128, 1> : attn_prefill_kernel<128, 2>);
  hipLaunchKernelGGL(fn, grid, dim3(256), 0, st, p);
  return 0;
}

int qh_launch_gdn_prep(const QhGdnPrepParams& p, hipStream_t st) {
  if (p.dk != 128 || p.dv != 128 || p.Hk <= 0 || p.Hv <= 0 || p.Hv % p.Hk != 0 || p.Hv > 64 ||
      p.C != 2 * p.Hk * p.dk + p.Hv * p.dv || p.past < 0) {
    qh_set_error("gdn_prep: unsupported shape (dk=%d dv=%d Hk=%d Hv=%d C=%d)", p.dk, p.dv, p.Hk,
                 p.Hv, p.C);
    return -1;
  }
  if (p.M <= 0) return 0;
  const size_t n = (size_t)p.M * p.C;
  // 8 channels per thread from 512 tokens (3700 tokens: 72.8 -> 49.6 us);
  // below that the thread-per-channel kernel's parallelism wins (128 tokens:
  // 4.8 against 6.1 us)
  if (p.M >= 512 && p.C % 8 == 0 && (uintptr_t)p.mixed % 16 == 0 && (uintptr_t)p.y % 16 == 0 &&
      (uintptr_t)p.conv_w % 16 == 0) {
    const size_t n8 = n / 8;
    hipLaunchKernelGGL(gdn_conv8_kernel, dim3((unsigned)((n8 + 255) / 256)), dim3(256), 0, st, p);
  } else {
    hipLaunchKernelGGL(gdn_conv_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, p);
  }
  hipLaunchKernelGGL(gdn_norm_gates_kernel, dim3((unsigned)(((long)p.M * (2 * p.Hk + 1) + 3) / 4)), dim3(256), 0, st,
                     p);
  return 0;
}

int qh_launch_gdn_scan(const QhGdnScanParams& p, hipStream_t st) {
  if (p.dk != 128 || p.dv != 128 || p.Hk <= 0 || p.Hv <= 0 || p.Hv % p.Hk != 0) {
    qh_set_error("gdn_scan: unsupported shape (dk=%d dv=%d Hk=%d Hv=%d)", p.dk, p.dv, p.Hk, p.Hv);
    return -1;
  }
  if (p.M <= 0) return 0;
  // 4 columns per wave (1024 waves at Hv = 32): 128-token prompt 10.32 ms vs
  // 10.44 ms with 8 columns per wave
  hipLaunchKernelGGL(gdn_scan_kernel<4>, dim3(p.Hv * (128 / 4)), dim3(64), 0, st, p);
  return qh_launch_gdn_gated_norm(p, st);
}

int qh_launch_gdn_gated_norm(const QhGdnScanParams& p, hipStream_t st) {
  if (p.M <= 0) return 0;
  if (p.dv == 128) {
    const long n = (long)p.M * p.Hv;
    hipLaunchKernelGGL(gdn_gated_norm_wave_kernel, dim3((unsigned)((n + 3) / 4)), dim3(256), 0, st, p);
  } else {
    hipLaunchKernelGGL(gdn_gated_norm_kernel, dim3(p.M, p.Hv), dim3(128), 0, st, p);
  }
  return 0;
}

int qh_launch_silu_mul(const uint16_t* g, const uint16_t* u, uint16_t* m, size_t n, hipStream_t st) {
  if (n == 0) return 0;
  if (n % 8 == 0 && (uintptr_t)g % 16 == 0 && (uintptr_t)u % 16 == 0 && (uintptr_t)m % 16 == 0) {
    const size_t blocks = std::min<size_t>((n / 8 + 255) / 256, 8192);
    hipLaunchKernelGGL(silu_mul8_kernel, dim3((unsigned)blocks), dim3(256), 0, st, g, u, m, n / 8);
    return 0;
  }
  const size_t blocks = std::min<size_t>((n + 255) / 256, 4096);
  hipLaunchKernelGGL(silu_mul_kernel, dim3((unsigned)blocks), dim3(256), 0, st, g, u, m, n);
  return 0;
}
