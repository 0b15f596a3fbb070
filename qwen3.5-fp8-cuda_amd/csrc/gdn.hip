// GatedDeltaNet ("linear attention") single-token decode step on gfx950.
//
// Semantics (reference: main.py:1064-1162 linear_attention_forward with s == 1,
// main.py:1165-1199 delta rule, qwen3_infer/csrc/fused_kernels.cu:623-684
// delta_rule_decode_kernel; conv update = transformers causal_conv1d_update,
// modeling_qwen3_5.py:200-217):
//   conv   : y_c = bf16(silu(bf16(sum_i w[c,i] * x_{t-3+i})))  (window of 4)
//   gates  : beta = bf16(sigmoid(b)), g = -exp(A_log) * softplus(a + dt_bias)
//   per value head h (key head h / (Hv/Hk)):
//     q^ = q / sqrt(sum q^2 + 1e-6) / sqrt(dk),  k^ = k / sqrt(sum k^2 + 1e-6)  (fp32)
//     S  <- S * e^g;  d = (v - S^T k^) * beta;  S <- S + k^ d^T;  o = S^T q^
//   core = bf16(o); out = bf16(bf16(bf16(core * rsqrt(mean core^2 + eps)) * w)
//                              * bf16(silu(z)))   (main.py:1152-1158)
//
// Design: the fp32 state S[h] (dk x dv) is split by value columns; one
// 256-thread workgroup owns 32 columns of one head (8 row groups x 32
// columns), so a step reads and writes every state byte exactly once, spread
// over Hv * dv / 32 workgroups.  Each workgroup recomputes the conv + l2norm of
// its key head's q/k (256 channels, cheap) so workgroups never wait on each
// other.  The conv state is a 4-slot ring indexed by position (slot t % 4
// holds x_t): readers of slots t-1..t-3 and the writer of slot t never
// collide.  The gated RMSNorm needs a whole head: the last of a head's column
// workgroups to finish (self-resetting arrival counter) applies it.
#include "qh_common.h"
#include "qh_gdn.h"

namespace {

constexpr int VS = 32;  // value columns per workgroup

// Delta-rule update of 32 value columns.  Thread t: column t & 31, rows
// (t >> 5) * DK/8 .. +DK/8 (S holds them, loaded early by load_columns).
// qn/kn: normalised q, k (fp32, LDS).  Returns the column's output o.
template <int DK>
__device__ __forceinline__ void load_columns(float (&S)[DK / 8], const float* state_cols, int dv) {
  constexpr int RPT = DK / 8;
  const int j = threadIdx.x & 31;
  const int rg = threadIdx.x >> 5;
#pragma unroll
  for (int r = 0; r < RPT; ++r) S[r] = state_cols[(size_t)(rg * RPT + r) * dv + j];
}

template <int DK>
__device__ __forceinline__ float delta_columns(const float (&S)[DK / 8], float* state_cols, int dv,
                                               const float* qn, const float* kn, float vval,
                                               float beta, float decay, float* red) {
  constexpr int RPT = DK / 8;
  const int j = threadIdx.x & 31;
  const int rg = threadIdx.x >> 5;
  float pred = 0.0f;
#pragma unroll
  for (int r = 0; r < RPT; ++r) pred = fmaf(S[r] * decay, kn[rg * RPT + r], pred);
  red[rg * 32 + j] = pred;
  __syncthreads();
  pred = 0.0f;
#pragma unroll
  for (int g = 0; g < 8; ++g) pred += red[g * 32 + j];
  const float delta = (vval - pred) * beta;
  float o = 0.0f;
#pragma unroll
  for (int r = 0; r < RPT; ++r) {
    const float upd = fmaf(kn[rg * RPT + r], delta, S[r] * decay);
    state_cols[(size_t)(rg * RPT + r) * dv + j] = upd;
    o = fmaf(upd, qn[rg * RPT + r], o);
  }
  __syncthreads();
  red[rg * 32 + j] = o;
  __syncthreads();
  o = 0.0f;
#pragma unroll
  for (int g = 0; g < 8; ++g) o += red[g * 32 + j];
  return o;
}

// Sum over the 128 threads [base, base+128) of a 256-thread block.
__device__ __forceinline__ float half_block_sum(float v, float* red2) {
  v = wave_sum(v);
  const int wid = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) red2[wid] = v;
  __syncthreads();
  const int base = (wid >> 1) * 2;
  return red2[base] + red2[base + 1];
}

// One 512-thread workgroup per value head (dk = dv = 128): thread t owns value
// column j = t & 127 and state rows 32 (t >> 7) .. +32 of it, so the head's
// 64 KB of state is requested at once, first thing, and the gated RMSNorm
// over the head's 128 outputs is a block reduction (no cross-workgroup
// hand-off).  The q/k conv + l2norm of the key head is recomputed per value
// head (256 channels, cheap).
constexpr int GDN_THREADS = 512;

template <int DK>
__global__ __launch_bounds__(GDN_THREADS) void gdn_decode_kernel(QhGdnParams p) {
  static_assert(DK == 128, "fused decode step assumes dk = dv = 128");
  constexpr int DV = 128, RG = GDN_THREADS / DV, RPT = DK / RG;  // 4 row groups x 32 rows
  __shared__ float qn[DK], kn[DK], vconv[DV];
  __shared__ float red[RG][DV];
  __shared__ float red2[8];

  const int h = blockIdx.x;
  const int r = p.Hv / p.Hk;
  const int kh = h / r;
  const int t = p.pos_dev ? *p.pos_dev : p.pos;
  const int tid = threadIdx.x;
  const int j = tid & (DV - 1);
  const int rg = tid >> 7;
  const int lane = tid & 63, wid = tid >> 6;

  // Vector-memory loads complete in issue order, so the few small operands go
  // out before the head's 64 KB of state: the conv, norms and gates then run
  // while the state is still arriving.  The conv window is read as the whole
  // 4-slot ring row (one 8-byte load, independent of the position).
  int c = -1;
  if (tid < 2 * DK) {
    const bool is_k = tid >= DK;
    c = (is_k ? p.Hk * DK : 0) + kh * DK + (tid & (DK - 1));
  } else if (tid < 2 * DK + DV) {
    c = 2 * p.Hk * DK + h * DV + (tid - 2 * DK);
  }
  uint16_t x_t = 0;
  u32x2 ring4 = {0u, 0u}, w4 = {0u, 0u};
  if (c >= 0) {
    x_t = p.mixed[c];
    ring4 = *(const u32x2*)(p.conv_ring + (size_t)c * 4);
    w4 = *(const u32x2*)(p.conv_w + (size_t)c * 4);
  }
  const float bh = bf2f(p.b[h]), ah = bf2f(p.a[h]);
  const float A_log = p.A_log[h], dt_bias = p.dt_bias[h];
  // Operands of the output norm, needed last (loaded by every row group so
  // no branch waits on them).
  const uint16_t zraw = p.z[(size_t)h * DV + j], nwraw = p.norm_w[j];
  float* cols = p.state + (size_t)h * DK * DV + j;
  float S[RPT];
#pragma unroll
  for (int i = 0; i < RPT; ++i) S[i] = cols[(size_t)(rg * RPT + i) * DV];

  // ---- causal conv (window of 4) + SiLU: q/k of key head kh (threads
  // 0..255), v of value head h (256..383) ------------------------------------
  float y = 0.0f;
  if (c >= 0) {
    // slot s of the ring holds bf16 lane s of (ring4.x lo, hi, ring4.y lo, hi)
    auto slot = [&](int sidx) {
      const uint32_t wv = (sidx & 2) ? ring4.y : ring4.x;
      return (sidx & 1) ? bf_hi(wv) : bf_lo(wv);
    };
    float acc = bf_hi(w4.y) * bf2f(x_t);
    acc = fmaf(bf_lo(w4.y), slot((t + 3) & 3), acc);
    acc = fmaf(bf_hi(w4.x), slot((t + 2) & 3), acc);
    acc = fmaf(bf_lo(w4.x), slot((t + 1) & 3), acc);
    y = rbf(qh_silu(rbf(acc)));
    // q/k channels are shared by the r value heads of a key head: one writes.
    if (tid >= 2 * DK || (h % r) == 0) p.conv_ring[(size_t)c * 4 + (t & 3)] = x_t;
  }
  // l2norm of q (waves 0-1) and k (waves 2-3)
  float ss = wave_sum(y * y);
  if (lane == 0) red2[wid] = ss;
  __syncthreads();
  if (tid < 2 * DK) {
    const int base = (wid >> 1) * 2;
    const float n = red2[base] + red2[base + 1];
    if (tid >= DK) kn[tid - DK] = y * rsqrtf(n + 1e-6f);
    else qn[tid] = y * rsqrtf(n + 1e-6f) * rsqrtf((float)DK);
  } else if (tid < 2 * DK + DV) {
    vconv[tid - 2 * DK] = y;
  }
  // ---- gates ----------------------------------------------------------------
  const float beta = rbf(qh_sigmoid(bh));
  const float g = -expf(A_log) * qh_softplus(ah + dt_bias);
  const float decay = expf(g);
  __syncthreads();

  // ---- delta rule on column j ---------------------------------------------
  float pred = 0.0f;
#pragma unroll
  for (int i = 0; i < RPT; ++i) pred = fmaf(S[i] * decay, kn[rg * RPT + i], pred);
  red[rg][j] = pred;
  __syncthreads();
  pred = red[0][j] + red[1][j] + red[2][j] + red[3][j];
  const float delta = (vconv[j] - pred) * beta;
  float o = 0.0f;
#pragma unroll
  for (int i = 0; i < RPT; ++i) {
    const float upd = fmaf(kn[rg * RPT + i], delta, S[i] * decay);
    cols[(size_t)(rg * RPT + i) * DV] = upd;
    o = fmaf(upd, qn[rg * RPT + i], o);
  }
  __syncthreads();
  red[rg][j] = o;
  __syncthreads();
  // ---- gated RMSNorm over the head (threads 0..127 = waves 0, 1) ------------
  float core = 0.0f;
  if (rg == 0) {
    core = rbf(red[0][j] + red[1][j] + red[2][j] + red[3][j]);
    if (p.core) p.core[(size_t)h * DV + j] = core;  // optional: the bf16-rounded core
    const float sq = wave_sum(core * core);
    if (lane == 0) red2[wid] = sq;
  }
  __syncthreads();
  if (rg == 0) {
    const float rs = rsqrtf((red2[0] + red2[1]) / (float)DV + p.eps);
    const float normed = rbf(rbf(core * rs) * bf2f(nwraw));
    const float sz = rbf(qh_silu(bf2f(zraw)));
    p.out[(size_t)h * DV + j] = f2bf(normed * sz);
  }
}

// ---- decode step split by value columns: one wave per (value head, 8 columns) --
// Same semantics as gdn_decode_kernel up to the bf16 core output, which goes
// to `out`; the gated RMSNorm (needs a whole head, here spread over 16 waves)
// is the output projection's prologue (qh_gemv_e4m3_gated).  Lane l owns
// value column 8 cg + (l >> 3) and state rows 16 (l & 7) .. +16, so a wave
// reads and writes 4 KB of state and its sums over the key dimension are
// 8-lane DPP butterflies: no workgroup barrier anywhere.  Each wave recomputes
// the conv + l2norm of its key head's q and k (two channels of each per lane,
// full-wave sums).  Block b runs head b % Hv, column group b / Hv: the 16
// waves of a head share the state's 128-byte lines and sit on one XCD (blocks
// are dealt to the XCDs round-robin and Hv is a multiple of 8).
constexpr int GDN_COLS = 8;

__global__ __launch_bounds__(64) void gdn_decode_cols_kernel(QhGdnParams p) {
  constexpr int DK = 128, DV = 128, L = 64 / GDN_COLS, RPT = DK / L;  // 8 lanes x 16 rows per column
  __shared__ __align__(16) float sq[DK];
  __shared__ __align__(16) float sk[DK];
  const int h = (int)blockIdx.x % p.Hv, cg = (int)blockIdx.x / p.Hv;
  const int r = p.Hv / p.Hk, kh = h / r;
  const int lane = threadIdx.x;
  const int rg = lane & (L - 1);
  const int j = cg * GDN_COLS + lane / L;
  const int t = p.pos_dev ? *p.pos_dev : p.pos;

  // Small operands first (vector-memory loads complete in issue order), then
  // the state slice: the conv, norms and gates run while it arrives.
  const int cq = kh * DK + 2 * lane;             // q channels cq, cq + 1
  const int ck = p.Hk * DK + kh * DK + 2 * lane;  // k channels ck, ck + 1
  const int cv = 2 * p.Hk * DK + h * DV + j;      // this lane's v channel
  const uint32_t xq = *(const uint32_t*)(p.mixed + cq), xk = *(const uint32_t*)(p.mixed + ck);
  const uint16_t xv = p.mixed[cv];
  const u32x4 ringq = *(const u32x4*)(p.conv_ring + (size_t)cq * 4);  // 2 channels x 4 slots
  const u32x4 ringk = *(const u32x4*)(p.conv_ring + (size_t)ck * 4);
  const u32x2 ringv = *(const u32x2*)(p.conv_ring + (size_t)cv * 4);
  const u32x4 wq = *(const u32x4*)(p.conv_w + (size_t)cq * 4);
  const u32x4 wk = *(const u32x4*)(p.conv_w + (size_t)ck * 4);
  const u32x2 wv = *(const u32x2*)(p.conv_w + (size_t)cv * 4);
  const float bh = bf2f(p.b[h]), ah = bf2f(p.a[h]);
  const float A_log = p.A_log[h], dt_bias = p.dt_bias[h];
  float* col = p.state + (size_t)h * DK * DV + j;
  float S[RPT];
#pragma unroll
  for (int i = 0; i < RPT; ++i) S[i] = col[(size_t)(rg * RPT + i) * DV];

  // causal conv (window of 4) + SiLU of one channel: ring = its 4 slots (slot
  // s holds x at positions = s mod 4), w = its 4 taps, x = x_t
  auto conv = [&](uint32_t r01, uint32_t r23, uint32_t w01, uint32_t w23, float x) {
    auto slot = [&](int sidx) {
      const uint32_t wv2 = (sidx & 2) ? r23 : r01;
      return (sidx & 1) ? bf_hi(wv2) : bf_lo(wv2);
    };
    float acc = bf_hi(w23) * x;
    acc = fmaf(bf_lo(w23), slot((t + 3) & 3), acc);
    acc = fmaf(bf_hi(w01), slot((t + 2) & 3), acc);
    acc = fmaf(bf_lo(w01), slot((t + 1) & 3), acc);
    return rbf(qh_silu(rbf(acc)));
  };
  const float q0 = conv(ringq.x, ringq.y, wq.x, wq.y, bf_lo(xq));
  const float q1 = conv(ringq.z, ringq.w, wq.z, wq.w, bf_hi(xq));
  const float k0 = conv(ringk.x, ringk.y, wk.x, wk.y, bf_lo(xk));
  const float k1 = conv(ringk.z, ringk.w, wk.z, wk.w, bf_hi(xk));
  const float v = conv(ringv.x, ringv.y, wv.x, wv.y, bf2f(xv));
  // The ring's slot t: q/k channels are shared by the r value heads of a key
  // head (written by column group 0 of its first value head), v by its head.
  if (cg == 0 && h % r == 0) {
    p.conv_ring[(size_t)cq * 4 + (t & 3)] = (uint16_t)(xq & 0xFFFFu);
    p.conv_ring[(size_t)(cq + 1) * 4 + (t & 3)] = (uint16_t)(xq >> 16);
    p.conv_ring[(size_t)ck * 4 + (t & 3)] = (uint16_t)(xk & 0xFFFFu);
    p.conv_ring[(size_t)(ck + 1) * 4 + (t & 3)] = (uint16_t)(xk >> 16);
  }
  if (rg == 0) p.conv_ring[(size_t)cv * 4 + (t & 3)] = xv;

  // l2norm of q and k over the key head (full-wave sums)
  const float nq = wave_total(fmaf(q0, q0, q1 * q1));
  const float nk = wave_total(fmaf(k0, k0, k1 * k1));
  const float iq = rsqrtf(nq + 1e-6f) * rsqrtf((float)DK), ik = rsqrtf(nk + 1e-6f);
  *(qh_f32x2*)(sq + 2 * lane) = qh_f32x2{q0 * iq, q1 * iq};
  *(qh_f32x2*)(sk + 2 * lane) = qh_f32x2{k0 * ik, k1 * ik};
  const float beta = rbf(qh_sigmoid(bh));
  const float decay = expf(-expf(A_log) * qh_softplus(ah + dt_bias));
  __syncthreads();  // one wave: orders the LDS writes before the reads
  float kr[RPT], qr[RPT];
#pragma unroll
  for (int i = 0; i < RPT; i += 4) {
    *(f32x4*)(kr + i) = *(const f32x4*)(sk + rg * RPT + i);
    *(f32x4*)(qr + i) = *(const f32x4*)(sq + rg * RPT + i);
  }

  // delta rule on column j
  float pp[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int i = 0; i < RPT; ++i) {
    S[i] *= decay;
    pp[i & 3] = fmaf(S[i], kr[i], pp[i & 3]);
  }
  const float pred = column_sum<L>((pp[0] + pp[1]) + (pp[2] + pp[3]));
  const float delta = (v - pred) * beta;
  float op[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int i = 0; i < RPT; ++i) {
    S[i] = fmaf(kr[i], delta, S[i]);
    col[(size_t)(rg * RPT + i) * DV] = S[i];
    op[i & 3] = fmaf(S[i], qr[i], op[i & 3]);
  }
  const float o = column_sum<L>((op[0] + op[1]) + (op[2] + op[3]));
  p.out[(size_t)h * DV + j] = f2bf(o);  // the 8 lanes of the column store the same value
}

// Reference ABI delta rule (fused_kernels.cu:623-684): q, k already expanded to
// one row per value head, g fp32, beta bf16, state updated in place, bf16 out.
template <int DK>
__global__ __launch_bounds__(256) void delta_rule_kernel(const uint16_t* q, const uint16_t* k,
                                                         const uint16_t* v, const float* g,
                                                         const uint16_t* beta, float* state,
                                                         uint16_t* out) {
  __shared__ float qn[DK], kn[DK];
  __shared__ float red[8 * 32];
  __shared__ float red2[4];
  const int h = blockIdx.x;
  const int sidx = blockIdx.y;
  const int tid = threadIdx.x;
  // l2norm of q and k: threads [0,128) and [128,256) each own up to DK/128 values
  {
    constexpr int PER = DK > 128 ? DK / 128 : 1;
    const bool is_k = tid >= 128;
    const int i0 = (tid & 127) * PER;
    const uint16_t* src = (is_k ? k : q) + (size_t)h * DK;
    float vals[PER];
    float ss = 0.0f;
#pragma unroll
    for (int e = 0; e < PER; ++e) {
      vals[e] = (i0 + e < DK) ? bf2f(src[i0 + e]) : 0.0f;
      ss = fmaf(vals[e], vals[e], ss);
    }
    ss = half_block_sum(ss, red2);
    const float sc = is_k ? rsqrtf(ss + 1e-6f) : rsqrtf(ss + 1e-6f) * rsqrtf((float)DK);
#pragma unroll
    for (int e = 0; e < PER; ++e)
      if (i0 + e < DK) (is_k ? kn : qn)[i0 + e] = vals[e] * sc;
  }
  __syncthreads();
  const float decay = expf(g[h]);
  const float bt = bf2f(beta[h]);
  const int j = tid & 31;
  const float vval = bf2f(v[(size_t)h * DK + sidx * VS + j]);
  float* cols = state + (size_t)h * DK * DK + sidx * VS;
  float S[DK / 8];
  load_columns<DK>(S, cols, DK);
  const float o = delta_columns<DK>(S, cols, DK, qn, kn, vval, bt, decay, red);
  if (tid < 32) out[(size_t)h * DK + sidx * VS + j] = f2bf(o);
}

}  // namespace

int qh_launch_gdn_decode(const QhGdnParams& p, hipStream_t st) {
  if (p.dk != 128 || p.dv != 128 || p.Hk <= 0 || p.Hv <= 0 || p.Hv % p.Hk != 0) {
    qh_set_error("gdn: unsupported shape (dk=%d dv=%d Hk=%d Hv=%d; need dk = dv = 128)", p.dk, p.dv,
                 p.Hk, p.Hv);
    return -1;
  }
  hipLaunchKernelGGL(gdn_decode_kernel<128>, dim3(p.Hv), dim3(GDN_THREADS), 0, st, p);
  return 0;
}

int qh_launch_gdn_decode_core(const QhGdnParams& p, hipStream_t st) {
  if (p.dk != 128 || p.dv != 128 || p.Hk <= 0 || p.Hv <= 0 || p.Hv % p.Hk != 0 || p.Hv % 8 != 0) {
    qh_set_error("gdn_core: unsupported shape (dk=%d dv=%d Hk=%d Hv=%d; need dk = dv = 128, Hv %% 8 == 0)",
                 p.dk, p.dv, p.Hk, p.Hv);
    return -1;
  }
  hipLaunchKernelGGL(gdn_decode_cols_kernel, dim3(p.Hv * (128 / GDN_COLS)), dim3(64), 0, st, p);
  return 0;
}

int qh_launch_delta_rule(const void* q, const void* k, const void* v, const float* g,
                         const void* beta, float* state, void* out, int n_heads, int head_dim,
                         hipStream_t st) {
  dim3 grid(n_heads, head_dim / VS);
#define QH_DR(DKV)                                                                             \
  hipLaunchKernelGGL(delta_rule_kernel<DKV>, grid, dim3(256), 0, st, (const uint16_t*)q,       \
                     (const uint16_t*)k, (const uint16_t*)v, g, (const uint16_t*)beta, state, \
                     (uint16_t*)out)
  switch (head_dim) {
    case 64: QH_DR(64); break;
    case 128: QH_DR(128); break;
    case 256: QH_DR(256); break;
    default:
      qh_set_error("delta_rule: head_dim=%d unsupported (64, 128, 256)", head_dim);
      return -1;
  }
#undef QH_DR
  return 0;
}
