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
template <int D>
__global__ __launch_bounds__(64) void attn_prep_kernel(QhAttnPrepParams p) {
  constexpr int NPL = D / 64;
  const int m = blockIdx.x, row = blockIdx.y, lane = threadIdx.x;
  const int pos = p.past + m;
  const bool is_q = row < p.Hq;
  const int head = is_q ? row : row - p.Hq;
  const uint16_t* src = is_q ? p.q_all + ((size_t)m * p.Hq + head) * 2 * D
                             : p.k + ((size_t)m * p.Hkv + head) * D;
  const float* nw = is_q ? p.q_norm_w : p.k_norm_w;
  float v[NPL];
#pragma unroll
  for (int i = 0; i < NPL; ++i) v[i] = bf2f(src[lane * NPL + i]);
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
    const float* cr = p.cos_t + (size_t)pos * p.rot;
    const float* sr = p.sin_t + (size_t)pos * p.rot;
#pragma unroll
    for (int i = 0; i < NPL; ++i) {
      const float partner = __shfl_xor(v[i], pm, 64);
      const int c = lane * NPL + i;
      if (c < half) v[i] = v[i] * cr[c] - partner * sr[c];
      else if (c < p.rot) v[i] = v[i] * cr[c] + partner * sr[c];
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
// The 4 waves serve the query heads of the GQA group (heads wid, wid + 4);
// K/V tiles of 32 positions are staged in LDS and shared by those heads.
template <int D>
__global__ __launch_bounds__(256) void attn_prefill_kernel(QhAttnPrefillParams p) {
  constexpr int NPL = D / 64;
  constexpr int KS = D + 8;
  constexpr int HPW = MAXG / 4;
  __shared__ float sQ[MAXG][D];
  __shared__ __align__(16) uint16_t sK[TP * KS];
  __shared__ __align__(16) uint16_t sV[TP * D];
  __shared__ float sP[MAXG][TP];
  const int kvh = blockIdx.x, m = blockIdx.y;
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int G = p.Hq / p.Hkv;
  const int total = p.past + m + 1;
  const uint16_t* kbase = p.k_cache + (size_t)kvh * p.max_seq * D;
  const uint16_t* vbase = p.v_cache + (size_t)kvh * p.max_seq * D;

  float gate_v[HPW][NPL];
  for (int gi = wid; gi < G; gi += 4) {
    const int h = kvh * G + gi;
    const float* q = p.q + ((size_t)m * p.Hq + h) * D;
#pragma unroll
    for (int i = 0; i < NPL; ++i) sQ[gi][lane * NPL + i] = q[lane * NPL + i];
    const uint16_t* gp = p.gate + (size_t)m * p.gate_mstride + (size_t)h * p.gate_hstride;
#pragma unroll
    for (int i = 0; i < NPL; ++i) gate_v[gi >> 2][i] = bf2f(gp[lane * NPL + i]);
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
  for (int t0 = 0; t0 < total; t0 += TP) {
    __syncthreads();
    for (int e = threadIdx.x; e < TP * (D / 8); e += 256) {
      const int row = e / (D / 8), c8 = (e % (D / 8)) * 8;
      const int pos = t0 + row;
      u32x4 kq = {0u, 0u, 0u, 0u}, vq = {0u, 0u, 0u, 0u};
      if (pos < total) {
        kq = *(const u32x4*)(kbase + (size_t)pos * D + c8);
        vq = *(const u32x4*)(vbase + (size_t)pos * D + c8);
      }
      *(u32x4*)(sK + row * KS + c8) = kq;
      *(u32x4*)(sV + row * D + c8) = vq;
    }
    __syncthreads();
    const int prow = lane >> 1, half = lane & 1;
    const bool valid = t0 + prow < total;
#pragma unroll
    for (int hi = 0; hi < HPW; ++hi) {
      const int gi = wid + 4 * hi;
      if (gi < G) {
        float dot = 0.0f;
        for (int c = half * (D / 2); c < (half + 1) * (D / 2); c += 8) {
          const u32x4 k8 = *(const u32x4*)(sK + prow * KS + c);
          const uint32_t kw[4] = {k8.x, k8.y, k8.z, k8.w};
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            dot = fmaf(sQ[gi][c + 2 * u], bf_lo(kw[u]), dot);
            dot = fmaf(sQ[gi][c + 2 * u + 1], bf_hi(kw[u]), dot);
          }
        }
        dot += __shfl_xor(dot, 1, 64);
        const float s = valid ? dot * scale : -INFINITY;
        const float nm = fmaxf(mx[hi], wave_max(s));
        const float corr = __expf(mx[hi] - nm);
        const float pv = valid ? __expf(s - nm) : 0.0f;
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
        for (int j = 0; j < TP; ++j) {
          const float pj = sP[gi][j];
#pragma unroll
          for (int i = 0; i < NPL; ++i) o[hi][i] = fmaf(pj, bf2f(sV[j * D + lane * NPL + i]), o[hi][i]);
        }
      }
    }
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

// ---- GDN conv over the sequence: one thread per channel ---------------------
__global__ __launch_bounds__(256) void gdn_conv_kernel(QhGdnPrepParams p) {
  const int c = blockIdx.x * 256 + threadIdx.x;
  if (c >= p.C) return;
  uint16_t* ring = p.conv_ring + (size_t)c * 4;
  const uint16_t* w = p.conv_w + (size_t)c * 4;
  const float w0 = bf2f(w[0]), w1 = bf2f(w[1]), w2 = bf2f(w[2]), w3 = bf2f(w[3]);
  float x3 = bf2f(ring[(p.past + 1) & 3]);  // x_{past-3}
  float x2 = bf2f(ring[(p.past + 2) & 3]);  // x_{past-2}
  float x1 = bf2f(ring[(p.past + 3) & 3]);  // x_{past-1}
  for (int m = 0; m < p.M; ++m) {
    const uint16_t xb = p.mixed[(size_t)m * p.C + c];
    const float x0 = bf2f(xb);
    float acc = w3 * x0;
    acc = fmaf(w2, x1, acc);
    acc = fmaf(w1, x2, acc);
    acc = fmaf(w0, x3, acc);
    p.y[(size_t)m * p.C + c] = f2bf(qh_silu(rbf(acc)));
    if (m >= p.M - 4) ring[(p.past + m) & 3] = xb;
    x3 = x2;
    x2 = x1;
    x1 = x0;
  }
}

// ---- q/k l2norm (bf16 steps) and gates: grid (M, 2 Hk + 1), one wave each ----
// blockIdx.y < 2 Hk: l2norm of q (y < Hk) or k of key head y % Hk; the last
// row computes the Hv gates of token m.
__global__ __launch_bounds__(64) void gdn_norm_gates_kernel(QhGdnPrepParams p) {
  const int m = blockIdx.x, row = blockIdx.y, lane = threadIdx.x;
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
    p.g[(size_t)m * p.Hv + h] = -__expf(p.A_log[h]) * qh_softplus(a + p.dt_bias[h]);
    p.beta[(size_t)m * p.Hv + h] = f2bf(qh_sigmoid(b));
  }
}

// ---- recurrent scan + gated RMSNorm: one 512-thread workgroup per head --------
// Thread t: value column j = t & 127, state rows 32 (t >> 7) .. +32 (as the
// decode step); the next token's operands are fetched while the current one
// is processed.
constexpr int SCAN_THREADS = 512;

__global__ __launch_bounds__(SCAN_THREADS) void gdn_scan_kernel(QhGdnScanParams p) {
  constexpr int DK = 128, DV = 128, RG = SCAN_THREADS / DV, RPT = DK / RG;
  __shared__ float sq[DK], sk[DK];
  __shared__ float red[RG][DV];
  __shared__ float red2[2];
  const int h = blockIdx.x;
  const int kh = h / (p.Hv / p.Hk);
  const int tid = threadIdx.x, j = tid & (DV - 1), rg = tid >> 7;
  const int lane = tid & 63, wid = tid >> 6;
  float* cols = p.state + (size_t)h * DK * DV + j;
  float S[RPT];
#pragma unroll
  for (int i = 0; i < RPT; ++i) S[i] = cols[(size_t)(rg * RPT + i) * DV];
  const float nw = bf2f(p.norm_w[j]);
  const float qscale = rsqrtf((float)DK);
  const int voff = 2 * p.Hk * DK + h * DV + j;

  auto fetch = [&](int m, float& qk, float& vv, float& zz, float& gg, float& bb) {
    if (tid < DK) qk = bf2f(p.qn[((size_t)m * p.Hk + kh) * DK + tid]);
    else if (tid < 2 * DK) qk = bf2f(p.kn[((size_t)m * p.Hk + kh) * DK + tid - DK]);
    vv = bf2f(p.y[(size_t)m * p.C + voff]);
    zz = bf2f(p.z[(size_t)m * p.Hv * DV + h * DV + j]);
    gg = p.g[(size_t)m * p.Hv + h];
    bb = bf2f(p.beta[(size_t)m * p.Hv + h]);
  };
  float qk = 0.0f, vv = 0.0f, zz = 0.0f, gg = 0.0f, bb = 0.0f;
  if (p.M > 0) fetch(0, qk, vv, zz, gg, bb);
  for (int m = 0; m < p.M; ++m) {
    if (tid < DK) sq[tid] = qk * qscale;
    else if (tid < 2 * DK) sk[tid - DK] = qk;
    const float v = vv, z = zz, decay = __expf(gg), beta = bb;
    if (m + 1 < p.M) fetch(m + 1, qk, vv, zz, gg, bb);
    __syncthreads();
    float pred = 0.0f;
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
      S[i] *= decay;
      pred = fmaf(S[i], sk[rg * RPT + i], pred);
    }
    red[rg][j] = pred;
    __syncthreads();
    pred = red[0][j] + red[1][j] + red[2][j] + red[3][j];
    const float delta = (v - pred) * beta;
    float o = 0.0f;
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
      S[i] = fmaf(sk[rg * RPT + i], delta, S[i]);
      o = fmaf(S[i], sq[rg * RPT + i], o);
    }
    __syncthreads();
    red[rg][j] = o;
    __syncthreads();
    float core = 0.0f;
    if (rg == 0) {
      core = rbf(red[0][j] + red[1][j] + red[2][j] + red[3][j]);
      const float s2 = wave_sum(core * core);
      if (lane == 0) red2[wid] = s2;
    }
    __syncthreads();
    if (rg == 0) {
      const float rs = rsqrtf((red2[0] + red2[1]) / (float)DV + p.eps);
      const float normed = rbf(rbf(core * rs) * nw);
      p.out[(size_t)m * p.Hv * DV + h * DV + j] = f2bf(normed * rbf(qh_silu(z)));
    }
  }
#pragma unroll
  for (int i = 0; i < RPT; ++i) cols[(size_t)(rg * RPT + i) * DV] = S[i];
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
  if ((p.D != 128 && p.D != 256) || !rot_ok(p.rot, p.D) || p.Hkv <= 0 || p.Hq % p.Hkv != 0 ||
      p.past < 0 || p.past + p.M > p.max_seq) {
    qh_set_error("attn_prep: unsupported shape (D=%d rot=%d Hq=%d Hkv=%d past=%d M=%d max_seq=%d)",
                 p.D, p.rot, p.Hq, p.Hkv, p.past, p.M, p.max_seq);
    return -1;
  }
  if (p.M <= 0) return 0;
  const dim3 grid(p.M, p.Hq + p.Hkv);
  if (p.D == 256)
    hipLaunchKernelGGL(attn_prep_kernel<256>, grid, dim3(64), 0, st, p);
  else
    hipLaunchKernelGGL(attn_prep_kernel<128>, grid, dim3(64), 0, st, p);
  return 0;
}

int qh_launch_attn_prefill(const QhAttnPrefillParams& p, hipStream_t st) {
  if ((p.D != 128 && p.D != 256) || p.Hkv <= 0 || p.Hq % p.Hkv != 0 || p.Hq / p.Hkv > MAXG ||
      p.past < 0 || p.past + p.M > p.max_seq) {
    qh_set_error("attn_prefill: unsupported shape (D=%d Hq=%d Hkv=%d past=%d M=%d)", p.D, p.Hq,
                 p.Hkv, p.past, p.M);
    return -1;
  }
  if (p.M <= 0) return 0;
  const dim3 grid(p.Hkv, p.M);
  if (p.D == 256)
    hipLaunchKernelGGL(attn_prefill_kernel<256>, grid, dim3(256), 0, st, p);
  else
    hipLaunchKernelGGL(attn_prefill_kernel<128>, grid, dim3(256), 0, st, p);
  return 0;
}

int qh_launch_gdn_prep(const QhGdnPrepParams& p, hipStream_t st) {
  if (p.dk != 128 || p.dv != 128 || p.Hk <= 0 || p.Hv % p.Hk != 0 || p.Hv > 64 ||
      p.C != 2 * p.Hk * p.dk + p.Hv * p.dv || p.past < 0) {
    qh_set_error("gdn_prep: unsupported shape (dk=%d dv=%d Hk=%d Hv=%d C=%d)", p.dk, p.dv, p.Hk,
                 p.Hv, p.C);
    return -1;
  }
  if (p.M <= 0) return 0;
  hipLaunchKernelGGL(gdn_conv_kernel, dim3((p.C + 255) / 256), dim3(256), 0, st, p);
  hipLaunchKernelGGL(gdn_norm_gates_kernel, dim3(p.M, 2 * p.Hk + 1), dim3(64), 0, st, p);
  return 0;
}

int qh_launch_gdn_scan(const QhGdnScanParams& p, hipStream_t st) {
  if (p.dk != 128 || p.dv != 128 || p.Hk <= 0 || p.Hv % p.Hk != 0) {
    qh_set_error("gdn_scan: unsupported shape (dk=%d dv=%d Hk=%d Hv=%d)", p.dk, p.dv, p.Hk, p.Hv);
    return -1;
  }
  if (p.M <= 0) return 0;
  hipLaunchKernelGGL(gdn_scan_kernel, dim3(p.Hv), dim3(SCAN_THREADS), 0, st, p);
  return 0;
}

int qh_launch_silu_mul(const uint16_t* g, const uint16_t* u, uint16_t* m, size_t n, hipStream_t st) {
  if (n == 0) return 0;
  const size_t blocks = std::min<size_t>((n + 255) / 256, 4096);
  hipLaunchKernelGGL(silu_mul_kernel, dim3((unsigned)blocks), dim3(256), 0, st, g, u, m, n);
  return 0;
}
