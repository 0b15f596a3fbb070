// Chunked (WY) GatedDeltaNet prefill on the bf16 matrix cores (gfx950).
//
// Semantics: the gated delta rule of the batch prefill from the stored state
// (main.py:1139-1149 calls transformers torch_chunk_gated_delta_rule,
// modeling_qwen3_5.py:249-328, chunk 64), q and k l2-normalised in bf16 steps
// (gdn_norm_gates_kernel) and q scaled by dk^-1/2.  Per value head h and chunk
// of 64 tokens, with G the cumulative log decay inside the chunk and beta the
// write strength:
//   A  = -tril_(-1)(diag(beta) K K^T * exp(G_i - G_j)),   T = (I - A)^-1
//   W  = T diag(beta e^G) K,   U = T diag(beta) V                (prep kernel)
//   V' = U - W S,   O = diag(e^G) Q S + tril(Q K^T * exp(G_i - G_j)) V'
//   S <- e^{G_last} S + K^T diag(e^{G_last - G}) V'               (state kernel)
// core = bf16(O); gdn_gated_norm_kernel then applies the gated RMSNorm.
//
// Products run on v_mfma_f32_16x16x16_bf16 (lane l holds A[l%16][4(l/16)+r],
// B[4(l/16)+r][l%16] and D[4(l/16)+r][l%16], r = 0..3).  k, v and the
// l2-normalised q are bf16 values, so K K^T, Q K^T and the products with K, V
// and K^T take them exactly in one pass.  fp32 operands (T, W, S, V', the
// decays) are split into bf16 hi + lo, x = hi + lo + O(2^-17 |x|), and
// multiplied in two or three passes (lo x lo dropped); accumulation is fp32.
//
// Work split: the prep kernel is one workgroup per (chunk, head), all chunks at
// once (it does not read the state); the state kernel is one workgroup per
// (head, 16 value columns), walking the chunks in order with its state slice in
// LDS.  The prep kernel hands W, U, the masked Q K^T, G and K^T to the state
// kernel through a workspace of qh_gdn_chunk_ws_bytes().
#include "qh_common.h"
#include "qh_prefill.h"

namespace {

constexpr int CH = 64;           // tokens per chunk
constexpr int DK = 128, DV = 128;
constexpr int RS = 136;          // bf16 row stride of the token-major K and Q tiles
constexpr int TS = 72;           // bf16 row stride of the dim-major K^T and V^T tiles
constexpr int PS = 68;           // bf16 row stride of the T' (hi, lo) tiles
constexpr int AS = 68;           // fp32 row stride of A
constexpr int NCG = DV / 16;     // state-kernel workgroups per head
constexpr float kQScale = 0.0883883476483184405f;  // 128^-1/2

// Workspace of one (head, chunk) unit, in floats: W [CH][DK], U^T [DV][CH],
// Att [CH][CH] (the masked, scaled Q K^T), G [CH], K^T [DK][CH] bf16, and the
// decays the state kernel applies: E [CH] = e^(G_last - G), QE [CH] =
// 128^-1/2 e^G, and e^(G_last) (padded to CH).
constexpr size_t kW = 0, kU = (size_t)CH * DK, kAtt = kU + (size_t)CH * DV, kG = kAtt + (size_t)CH * CH,
                 kKT = kG + CH, kE = kKT + (size_t)DK * CH / 2, kQE = kE + CH, kEL = kQE + CH,
                 kUnitFloats = kEL + CH;

typedef short bf4 __attribute__((ext_vector_type(4)));
typedef float f4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f4 mma(bf4 a, bf4 b, f4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
}
// x = hi + lo + O(2^-17 |x|), hi and lo bf16 (round to nearest even)
__device__ __forceinline__ void split4(f4 x, bf4& hi, bf4& lo) {
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const uint16_t h = f2bf(x[r]);
    hi[r] = (short)h;
    lo[r] = (short)f2bf(x[r] - bf2f(h));
  }
}
__device__ __forceinline__ f4 zero4() { return f4{0.0f, 0.0f, 0.0f, 0.0f}; }

// acc[q] += sum_m L[4 rg + q][m] R[m][c] over a 16 x 16 fp32 block product in
// LDS (row strides ldl, ldr): the lane's 16 R values and its 4 L rows are read
// first, then 64 multiply-adds.
__device__ __forceinline__ void blk_mac(float (&acc)[4], const float* L, int ldl, const float* R, int ldr,
                                        int rg, int c) {
  float rc[16];
#pragma unroll
  for (int m = 0; m < 16; ++m) rc[m] = R[m * ldr + c];
  f4 lr[4][4];
#pragma unroll
  for (int q = 0; q < 4; ++q)
#pragma unroll
    for (int m4 = 0; m4 < 4; ++m4) lr[q][m4] = *(const f4*)(L + (4 * rg + q) * ldl + 4 * m4);
#pragma unroll
  for (int q = 0; q < 4; ++q)
#pragma unroll
    for (int m4 = 0; m4 < 4; ++m4)
#pragma unroll
      for (int u = 0; u < 4; ++u) acc[q] = fmaf(lr[q][m4][u], rc[4 * m4 + u], acc[q]);
}

// ---- prep: grid (chunks, Hv), 256 threads -----------------------------------
__global__ __launch_bounds__(256) void gdn_chunk_prep_kernel(QhGdnScanParams p, float* ws, int nch) {
  // phase 1 holds K and Q token-major here, phase 3 the T' tiles
  __shared__ __align__(16) uint16_t sKQ[2 * CH * RS];
  __shared__ __align__(16) uint16_t sKT[DK * TS];
  __shared__ __align__(16) uint16_t sVT[DV * TS];
  __shared__ __align__(16) float sA[CH * AS];
  __shared__ __align__(16) float sT[CH * AS];      // T = (I - A)^-1
  __shared__ __align__(16) float sX[4][16 * 17];   // per-wave 16 x 16 block scratch
  __shared__ float sG[CH], sB[CH];
  uint16_t* sK = sKQ;
  uint16_t* sQ = sKQ + CH * RS;
  uint16_t* sTw = sKQ;              // [2][CH][PS]: T diag(beta e^G), hi then lo
  uint16_t* sTu = sKQ + 2 * CH * PS;  // [2][CH][PS]: T diag(beta)
  static_assert(4 * CH * PS <= 2 * CH * RS, "T' tiles fit the K/Q space");

  const int c = blockIdx.x, h = blockIdx.y, kh = h / (p.Hv / p.Hk);
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int t0 = c * CH;
  float* unit = ws + ((size_t)h * nch + c) * kUnitFloats;

  // ---- the chunk's K, Q (token-major) and K, V (dim-major); rows past M are 0.
  // Waves 0-1 take K, waves 2-3 V: a thread holds 8 tokens x 8 dims, stores
  // them token-major (K) and, transposed in registers (v_perm), as 16-byte
  // rows of the dim-major tile (2-byte scatter stores hit 8-way LDS bank
  // conflicts); every thread also copies 4 16-byte pieces of Q.
  // the chunk's log decay and write strength per token, requested with the
  // tiles below (every thread loads; threads tid < CH keep them)
  const bool tok_ok = t0 + lane < p.M;
  const int tok = tok_ok ? t0 + lane : p.M - 1;
  const float g_tok = p.g[(size_t)tok * p.Hv + h];
  const float b_tok = bf2f(p.beta[(size_t)tok * p.Hv + h]);
  {
    const u32x4 zero = {0u, 0u, 0u, 0u};
    const bool is_v = tid >= 128;  // wave-uniform
    const int tt = tid & 127, tg = tt & 7, dg = tt >> 3;  // tokens 8 tg .. + 7, dims 8 dg .. + 7
    u32x4 x[8], qv[4];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int t = min(t0 + 8 * tg + j, p.M - 1);
      x[j] = is_v ? *(const u32x4*)(p.y + (size_t)t * p.C + (size_t)2 * p.Hk * DK + (size_t)h * DV + 8 * dg)
                  : *(const u32x4*)(p.kn + ((size_t)t * p.Hk + kh) * DK + 8 * dg);
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int e = tid + 256 * r, i = e >> 4, c8 = (e & 15) * 8;
      qv[r] = *(const u32x4*)(p.qn + ((size_t)min(t0 + i, p.M - 1) * p.Hk + kh) * DK + c8);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int i = 8 * tg + j;
      if (t0 + i >= p.M) x[j] = zero;
      if (!is_v) *(u32x4*)(sK + i * RS + 8 * dg) = x[j];
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int e = tid + 256 * r, i = e >> 4, c8 = (e & 15) * 8;
      *(u32x4*)(sQ + i * RS + c8) = t0 + i < p.M ? qv[r] : zero;
    }
    uint16_t* dT = is_v ? sVT : sKT;
#pragma unroll
    for (int j = 0; j < 8; ++j) {  // dim 8 dg + j: tokens 8 tg .. + 7, pairs of 16-bit halves
      const uint32_t sel = (j & 1) ? 0x07060302u : 0x05040100u;
      u32x4 col;
#pragma unroll
      for (int q = 0; q < 4; ++q) col[q] = __builtin_amdgcn_perm(x[2 * q + 1][j >> 1], x[2 * q][j >> 1], sel);
      *(u32x4*)(dT + (8 * dg + j) * TS + 8 * tg) = col;
    }
  }
  if (tid < CH) {
    sG[tid] = tok_ok ? g_tok : 0.0f;  // padding: no decay, no write
    sB[tid] = tok_ok ? b_tok : 0.0f;
  }
  __syncthreads();
  if (w == 0) {  // inclusive cumulative sum of the log decays
    float x = sG[lane];
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const float y = __shfl_up(x, off, 64);
      x = lane >= off ? x + y : x;
    }
    sG[lane] = x;
    unit[kG + lane] = x;
    const float glast = __shfl(x, CH - 1, 64);
    unit[kE + lane] = expf(glast - x);
    unit[kQE + lane] = kQScale * expf(x);
    if (lane == 0) unit[kEL] = expf(glast);
  }
  __syncthreads();

  // ---- K K^T and Q K^T, rows 16w .. 16w+15 ------------------------------------
  const int ar = 16 * w + (lane & 15), kc = 4 * (lane >> 4);
  {
    f4 kk[4], qk[4];
#pragma unroll
    for (int tj = 0; tj < 4; ++tj) kk[tj] = qk[tj] = zero4();
#pragma unroll
    for (int s = 0; s < DK / 16; ++s) {
      const bf4 ak = *(const bf4*)(sK + ar * RS + 16 * s + kc);
      const bf4 aq = *(const bf4*)(sQ + ar * RS + 16 * s + kc);
#pragma unroll
      for (int tj = 0; tj < 4; ++tj) {
        const bf4 b = *(const bf4*)(sK + (16 * tj + (lane & 15)) * RS + 16 * s + kc);
        kk[tj] = mma(ak, b, kk[tj]);
        qk[tj] = mma(aq, b, qk[tj]);
      }
    }
#pragma unroll
    for (int tj = 0; tj < 4; ++tj) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = 16 * w + kc + r, j = 16 * tj + (lane & 15);
        const float dec = expf(sG[i] - sG[j]);  // used for j <= i only (G_i <= G_j)
        sA[i * AS + j] = j < i ? -sB[i] * kk[tj][r] * dec : 0.0f;
        unit[kAtt + i * CH + j] = j <= i ? qk[tj][r] * kQScale * dec : 0.0f;
      }
    }
  }
  __syncthreads();  // sA complete; K and Q tiles no longer read

  // ---- T = (I - A)^-1, blocked by 16 ---------------------------------------
  // Diagonal blocks T_bb = (I - A_bb)^-1 by forward substitution, one per wave;
  // then block row by block row, T_ij = T_ii sum_{k=j}^{i-1} A_ik T_kj, wave j
  // computing block (i, j).  The upper blocks of T are zero.
  const int bc = lane & 15, brg = lane >> 4;  // block column; rows 4 brg .. +3
  {
    // lane m (mod 16) holds column m of A_ww; row i reads A[i][m] from lane m
    // into a scalar register (v_readlane)
    float Acol[16], Tc[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) Acol[i] = sA[(16 * w + i) * AS + 16 * w + bc];
#pragma unroll
    for (int m = 0; m < 16; ++m) Tc[m] = m == bc ? 1.0f : 0.0f;
#pragma unroll
    for (int i = 1; i < 16; ++i) {
      float acc[2] = {0.0f, 0.0f};
      const int ai = __builtin_bit_cast(int, Acol[i]);
#pragma unroll
      for (int m = 0; m < i; ++m)
        acc[m & 1] = fmaf(__builtin_bit_cast(float, __builtin_amdgcn_readlane(ai, m)), Tc[m], acc[m & 1]);
      Tc[i] = i > bc ? acc[0] + acc[1] : Tc[i];
    }
    if (lane < 16) {
#pragma unroll
      for (int i = 0; i < 16; ++i) sT[(16 * w + i) * AS + 16 * w + bc] = Tc[i];
    }
    for (int b = w + 1; b < 4; ++b) {  // zero upper blocks of block row w
#pragma unroll
      for (int q = 0; q < 4; ++q) sT[(16 * w + 4 * brg + q) * AS + 16 * b + bc] = 0.0f;
    }
  }
  __syncthreads();
  for (int i = 1; i < 4; ++i) {
    if (w < i) {
      const int j = w;
      float x[4] = {0.0f, 0.0f, 0.0f, 0.0f};
      for (int k = j; k < i; ++k) blk_mac(x, sA + 16 * i * AS + 16 * k, AS, sT + 16 * k * AS + 16 * j, AS, brg, bc);
#pragma unroll
      for (int q = 0; q < 4; ++q) sX[w][(4 * brg + q) * 17 + bc] = x[q];
      float t[4] = {0.0f, 0.0f, 0.0f, 0.0f};
      blk_mac(t, sT + 16 * i * AS + 16 * i, AS, sX[w], 17, brg, bc);
#pragma unroll
      for (int q = 0; q < 4; ++q) sT[(16 * i + 4 * brg + q) * AS + 16 * j + bc] = t[q];
    }
    __syncthreads();
  }
  // T' = T diag(beta e^G) and T diag(beta) as bf16 hi + lo, rows 16w .. 16w+15
  {
    const float sw = sB[lane] * expf(sG[lane]), su = sB[lane];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int i = 16 * w + r;
      const float tv = sT[i * AS + lane];
      const float xw = tv * sw, xu = tv * su;
      const uint16_t hw = f2bf(xw), hu = f2bf(xu);
      sTw[i * PS + lane] = hw;
      sTw[CH * PS + i * PS + lane] = f2bf(xw - bf2f(hw));
      sTu[i * PS + lane] = hu;
      sTu[CH * PS + i * PS + lane] = f2bf(xu - bf2f(hu));
    }
  }
  __syncthreads();

  // ---- W = T' K and U = T' V, rows 16w .. 16w+15 ------------------------------
  {
    f4 wa[DK / 16], ua[DV / 16];
#pragma unroll
    for (int tn = 0; tn < DK / 16; ++tn) wa[tn] = ua[tn] = zero4();
#pragma unroll
    for (int s = 0; s < CH / 16; ++s) {
      const bf4 awh = *(const bf4*)(sTw + ar * PS + 16 * s + kc);
      const bf4 awl = *(const bf4*)(sTw + CH * PS + ar * PS + 16 * s + kc);
      const bf4 auh = *(const bf4*)(sTu + ar * PS + 16 * s + kc);
      const bf4 aul = *(const bf4*)(sTu + CH * PS + ar * PS + 16 * s + kc);
#pragma unroll
      for (int tn = 0; tn < DK / 16; ++tn) {
        const bf4 bk = *(const bf4*)(sKT + (16 * tn + (lane & 15)) * TS + 16 * s + kc);
        const bf4 bv = *(const bf4*)(sVT + (16 * tn + (lane & 15)) * TS + 16 * s + kc);
        wa[tn] = mma(awh, bk, wa[tn]);
        wa[tn] = mma(awl, bk, wa[tn]);
        ua[tn] = mma(auh, bv, ua[tn]);
        ua[tn] = mma(aul, bv, ua[tn]);
      }
    }
#pragma unroll
    for (int tn = 0; tn < DK / 16; ++tn) {
      // U transposed: a lane's 4 tokens of one column are one 16-byte store
      // here and one 16-byte load in the state kernel
      *(f4*)(unit + kU + (size_t)(16 * tn + (lane & 15)) * CH + 16 * w + kc) = ua[tn];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = 16 * w + kc + r, d = 16 * tn + (lane & 15);
        unit[kW + i * DK + d] = wa[tn][r];
      }
    }
  }
  // K^T for the state update, bf16 [DK][CH]
  uint16_t* kt = (uint16_t*)(unit + kKT);
  for (int e = tid; e < DK * CH / 8; e += 256) {
    const int d = e >> 3, c8 = (e & 7) * 8;
    *(u32x4*)(kt + d * CH + c8) = *(const u32x4*)(sKT + d * TS + c8);
  }
}

// ---- state: grid Hv * NCG (head h, value columns 16 cg .. +15), 512 threads --
// Waves 0-3 ("row waves", token rows 16 w .. +15 of the chunk) form V' = U - W S
// and the output O = diag(e^G) Q S + Att V'; waves 4-7 ("state waves", d rows
// 32 (w-4) .. +31) update the state from V', alongside the row waves' Att V'.
// Per chunk: [row: W S, Q S, V'] barrier [row: Att V', O | state: S update]
// barrier.  Each wave requests its next chunk's global operands (two register
// sets, the chunk loop unrolled by two) while the current chunk runs.
struct RowOps {
  f4 w[DK / 16];     // W[ar][16 s + kc .. +3]
  u32x2 q[DK / 16];  // q[ar][16 s + kc .. +3], bf16
  f4 att[CH / 16];   // Att[ar][16 s + kc .. +3]
  f4 u;              // U[16 w + kc + r][16 cg + col], r = 0..3
  float qe;          // 128^-1/2 e^G[ar]
};
struct StateOps {
  bf4 kt[2][CH / 16];    // K^T rows 16 td + col (td = 2 (w-4) + tt), tokens 16 s + kc .. +3
  f4 eb[CH / 16];        // e^(G_last - G[16 s + kc + r])
  float elast;           // e^(G_last)
};

__global__ __launch_bounds__(512) void gdn_chunk_state_kernel(QhGdnScanParams p, const float* ws, int nch) {
  // Column-major, padded: an MFMA operand (4 consecutive d or tokens of one
  // column) is one 16-byte LDS access, conflict-free across a 16-lane row.
  constexpr int SST = DK + 4, VST = CH + 4;
  __shared__ __align__(16) float sS[16 * SST];   // the state slice, sS[column][d]
  __shared__ __align__(16) float sVn[16 * VST];  // V' of the chunk, sVn[column][token]
  // The NCG workgroups of a head share its chunk operands (W, Att, q, K^T):
  // with Hv % 8 == 0 they are placed on one XCD (workgroup i runs on XCD
  // i % 8), so those operands come from memory once per head, not once per
  // column group.
  const int bid = (int)blockIdx.x;
  const bool xcd = p.Hv % 8 == 0;
  const int h = xcd ? ((bid >> 3) / NCG) * 8 + (bid & 7) : bid / NCG;
  const int cg = xcd ? (bid >> 3) % NCG : bid % NCG;
  const int kh = h / (p.Hv / p.Hk);
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int col = lane & 15, kc = 4 * (lane >> 4);
  float* state = p.state + (size_t)h * DK * DV + cg * 16;
  const float* units = ws + (size_t)h * nch * kUnitFloats;
  {  // the state slice: all four loads of a thread in flight before its LDS stores
    float sv[DK * 16 / 512];
#pragma unroll
    for (int k = 0; k < DK * 16 / 512; ++k) {
      const int e = tid + 512 * k;
      sv[k] = state[(size_t)(e >> 4) * DV + (e & 15)];
    }
#pragma unroll
    for (int k = 0; k < DK * 16 / 512; ++k) {
      const int e = tid + 512 * k;
      sS[(e & 15) * SST + (e >> 4)] = sv[k];
    }
  }
  __syncthreads();

  if (w < 4) {
    // ---------------------------------------------------------- row waves
    const int ar = 16 * w + col;  // A-operand row (token) of this lane
    // the workgroup's 16 output columns of every token (a uniform resource;
    // the lane's column goes in the offset): bytes past row M - 1 are out of
    // the resource's range
    const auto rout = __builtin_amdgcn_make_buffer_rsrc(p.out + (size_t)h * DV + cg * 16, (short)0,
                                                        (int)(((size_t)(p.M - 1) * p.Hv * DV + 16) * 2), 0x00020000);
    auto load = [&](RowOps& o, int c) {
      const float* unit = units + (size_t)c * kUnitFloats;
      const int t = min(c * CH + ar, p.M - 1);  // rows past M: any row (outputs dropped)
      const uint16_t* qrow = p.qn + ((size_t)t * p.Hk + kh) * DK;
#pragma unroll
      for (int s = 0; s < DK / 16; ++s) {
        o.w[s] = *(const f4*)(unit + kW + ar * DK + 16 * s + kc);
        o.q[s] = *(const u32x2*)(qrow + 16 * s + kc);
      }
#pragma unroll
      for (int s = 0; s < CH / 16; ++s) o.att[s] = *(const f4*)(unit + kAtt + ar * CH + 16 * s + kc);
      o.u = *(const f4*)(unit + kU + (size_t)(cg * 16 + col) * CH + 16 * w + kc);
      o.qe = unit[kQE + ar];
    };
    auto step = [&](const RowOps& cur, int c) {
      const int t0 = c * CH;
      f4 Sv;
      bf4 Sh[DK / 16], Sl[DK / 16];
#pragma unroll
      for (int s = 0; s < DK / 16; ++s) {
        Sv = *(const f4*)(sS + col * SST + 16 * s + kc);
        split4(Sv, Sh[s], Sl[s]);
      }
      const float qs = cur.qe;
      f4 ws_acc = zero4(), o = zero4();
#pragma unroll
      for (int s = 0; s < DK / 16; ++s) {
        bf4 ah, al;
        split4(cur.w[s], ah, al);
        ws_acc = mma(ah, Sh[s], ws_acc);
        ws_acc = mma(ah, Sl[s], ws_acc);
        ws_acc = mma(al, Sh[s], ws_acc);
        const u32x2 qb = cur.q[s];
        const f4 qv = {bf_lo(qb.x) * qs, bf_hi(qb.x) * qs, bf_lo(qb.y) * qs, bf_hi(qb.y) * qs};
        split4(qv, ah, al);
        o = mma(ah, Sh[s], o);
        o = mma(ah, Sl[s], o);
        o = mma(al, Sh[s], o);
      }
      // V' = U - W S (D layout: token 16w + kc + r, column col)
      *(f4*)(sVn + col * VST + 16 * w + kc) =
          f4{cur.u[0] - ws_acc[0], cur.u[1] - ws_acc[1], cur.u[2] - ws_acc[2], cur.u[3] - ws_acc[3]};
      __syncthreads();  // V' complete; the old state is read
#pragma unroll
      for (int s = 0; s < CH / 16; ++s) {
        bf4 vh, vl, ah, al;
        split4(*(const f4*)(sVn + col * VST + 16 * s + kc), vh, vl);
        split4(cur.att[s], ah, al);
        o = mma(ah, vh, o);
        o = mma(ah, vl, o);
        o = mma(al, vh, o);
      }
      // range-checked stores: rows past M are dropped without a branch (a
      // guarded store in this loop made the compiler wait for every
      // outstanding load, the next chunk's operands included, at its head)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = 16 * w + kc + r;
        __builtin_amdgcn_raw_buffer_store_b16(f2bf(o[r]), rout, (uint32_t)(((t0 + i) * p.Hv * DV + col) * 2), 0, 0);
      }
      __syncthreads();  // V' read; the new state written
    };
    // the next chunk's loads go out before the step (a scheduling barrier
    // keeps the compiler from sinking them into it, where the next step's
    // wait would expose their latency)
    RowOps ra, rb;
    load(ra, 0);
    for (int c = 0; c < nch; c += 2) {
      load(rb, min(c + 1, nch - 1));
      __builtin_amdgcn_sched_barrier(0);
      step(ra, c);
      if (c + 1 >= nch) break;
      load(ra, min(c + 2, nch - 1));
      __builtin_amdgcn_sched_barrier(0);
      step(rb, c + 1);
    }
  } else {
    // -------------------------------------------------------- state waves
    const int sw = w - 4;
    auto load = [&](StateOps& o, int c) {
      const float* unit = units + (size_t)c * kUnitFloats;
      const uint16_t* kt = (const uint16_t*)(unit + kKT);
#pragma unroll
      for (int tt = 0; tt < 2; ++tt)
#pragma unroll
        for (int s = 0; s < CH / 16; ++s)
          o.kt[tt][s] = *(const bf4*)(kt + (16 * (2 * sw + tt) + col) * CH + 16 * s + kc);
      // one 16-byte load per 4 decays: the loads' count, not their bytes,
      // is what the chunk loop's issue waits on
#pragma unroll
      for (int s = 0; s < CH / 16; ++s) o.eb[s] = *(const f4*)(unit + kE + 16 * s + kc);
      o.elast = unit[kEL];
    };
    // S <- e^{G_last} S + K^T diag(e^{G_last - G}) V', d tiles 2 sw, 2 sw + 1
    auto step = [&](const StateOps& cur) {
      __syncthreads();  // V' complete
      const float eg = cur.elast;
      bf4 Bh[CH / 16], Bl[CH / 16];
#pragma unroll
      for (int s = 0; s < CH / 16; ++s) {
        const f4 v = *(const f4*)(sVn + col * VST + 16 * s + kc);
        f4 x;
#pragma unroll
        for (int r = 0; r < 4; ++r) x[r] = cur.eb[s][r] * v[r];
        split4(x, Bh[s], Bl[s]);
      }
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
        float* dst = sS + col * SST + 16 * (2 * sw + tt) + kc;
        f4 acc = *(const f4*)dst * eg;
#pragma unroll
        for (int s = 0; s < CH / 16; ++s) {
          acc = mma(cur.kt[tt][s], Bh[s], acc);
          acc = mma(cur.kt[tt][s], Bl[s], acc);
        }
        *(f4*)dst = acc;  // the row waves read the old state before the first barrier
      }
      __syncthreads();  // new state visible; V' read
    };
    StateOps sa, sb;
    load(sa, 0);
    for (int c = 0; c < nch; c += 2) {
      load(sb, min(c + 1, nch - 1));
      __builtin_amdgcn_sched_barrier(0);
      step(sa);
      if (c + 1 >= nch) break;
      load(sa, min(c + 2, nch - 1));
      __builtin_amdgcn_sched_barrier(0);
      step(sb);
    }
  }
  __syncthreads();
  for (int e = tid; e < DK * 16; e += 512) state[(size_t)(e >> 4) * DV + (e & 15)] = sS[(e & 15) * SST + (e >> 4)];
}

}  // namespace

size_t qh_gdn_chunk_ws_bytes(int M, int Hv) {
  if (M <= 0 || Hv <= 0) return 0;
  return (size_t)Hv * ((M + CH - 1) / CH) * kUnitFloats * sizeof(float);
}

int qh_launch_gdn_chunk(const QhGdnScanParams& p, float* ws, size_t ws_bytes, hipStream_t st) {
  if (p.dk != DK || p.dv != DV || p.Hk <= 0 || p.Hv <= 0 || p.Hv % p.Hk != 0) {
    qh_set_error("gdn_chunk: unsupported shape (dk=%d dv=%d Hk=%d Hv=%d)", p.dk, p.dv, p.Hk, p.Hv);
    return -1;
  }
  if (p.M <= 0) return 0;
  const size_t need = qh_gdn_chunk_ws_bytes(p.M, p.Hv);
  if (!ws || ws_bytes < need || ((uintptr_t)ws & 15u) != 0) {
    qh_set_error("gdn_chunk: workspace of %zu bytes (16-byte aligned) needed, got %zu", need, ws_bytes);
    return -1;
  }
  const int nch = (p.M + CH - 1) / CH;
  hipLaunchKernelGGL(gdn_chunk_prep_kernel, dim3(nch, p.Hv), dim3(256), 0, st, p, ws, nch);
  hipLaunchKernelGGL(gdn_chunk_state_kernel, dim3(p.Hv * NCG), dim3(512), 0, st, p, (const float*)ws, nch);
  return qh_launch_gdn_gated_norm(p, st);
}
