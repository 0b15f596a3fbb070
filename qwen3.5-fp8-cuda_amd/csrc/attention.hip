// Batch-1 GQA decode attention for the full-attention layers (gfx950).
//
// Semantics (reference: qwen3_infer/csrc/fused_kernels.cu:1224-1297
// layer_mid_attn, 787-867 fused_attn_v2_kernel, 872-903 rope_decode_kernel,
// 1199-1219 kv_cache_write_kernel; gate: main.py:1059):
//   q_h  = bf16 RMSNorm_(1+w)(q_h)           (per head, D dims, eps 1e-6)
//   k    = bf16 RMSNorm_(1+w)(k)
//   q,k  = bf16 partial RoPE on dims [0, rot): pairs (c, c + rot/2),
//          out0 = x0 cos - x1 sin, out1 = x1 cos + x0 sin  at position `pos`
//   K/V cache[kv, slot] = k, v
//   o_h  = softmax(q_h . K[kv(h)]^T / sqrt(D)) V[kv(h)] over `total` positions,
//          kv(h) = h * n_kv / n_heads, fp32 softmax, bf16 output
//   optional gate: out_h = bf16(o_h) * bf16(sigmoid(gate_h))
//
// Design: one workgroup per (kv head, position split).  The 4 waves share one
// K/V tile (32 positions) staged in LDS, each wave serving one query head of
// the GQA group, so each KV head is read from HBM exactly once per step.  Each
// split keeps an online-softmax state; the last split to finish for a KV head
// (atomic arrival counter, self-resetting) merges the partial states and
// applies the output gate.  Above 8 active splits the merge has two levels:
// the last arriver of each group of 8 splits merges its group, the last group
// merges the group records.  The new token's K/V come from registers, so no
// split ever waits on another.
#include <cstring>
#include <mutex>

#include "qh_common.h"
#include "qh_attn.h"

namespace {

constexpr int TP = 32;  // positions per LDS tile
constexpr int MAXG = 8;  // query heads per KV head supported

template <int NPL>
__device__ __forceinline__ void load_head(float (&v)[NPL], const uint16_t* src) {
  if constexpr (NPL == 4) {
    const u32x2 u = *(const u32x2*)src;
    v[0] = bf_lo(u.x); v[1] = bf_hi(u.x); v[2] = bf_lo(u.y); v[3] = bf_hi(u.y);
  } else {
    const uint32_t u = *(const uint32_t*)src;
    v[0] = bf_lo(u); v[1] = bf_hi(u);
  }
}

// load_head through a buffer resource, for loads that would otherwise sit
// under a branch (the compiler then waits for every earlier load there):
// valid == false gives an empty resource, whose load reads zeros.  `valid`
// must be wave-uniform.
template <int NPL>
__device__ __forceinline__ void load_head_b(float (&v)[NPL], const uint16_t* head, int lane, bool valid) {
  const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(head), (short)0, valid ? (int)(64 * NPL * 2) : 0, 0x00020000);
  const uint32_t off = (uint32_t)lane * NPL * 2u;
  if constexpr (NPL == 4) {
    const u32x2 u = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0);
    v[0] = bf_lo(u.x); v[1] = bf_hi(u.x); v[2] = bf_lo(u.y); v[3] = bf_hi(u.y);
  } else {
    const uint32_t u = __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
    v[0] = bf_lo(u); v[1] = bf_hi(u);
  }
}

template <int NPL>
__device__ __forceinline__ void store_head(uint16_t* dst, const float (&v)[NPL]) {
  if constexpr (NPL == 4) {
    *(u32x2*)dst = u32x2{pack_bf2(v[0], v[1]), pack_bf2(v[2], v[3])};
  } else {
    *(uint32_t*)dst = pack_bf2(v[0], v[1]);
  }
}

// A head's D fp32 values (lane l holds NPL consecutive ones at l * NPL),
// written / read with one device-coherent (sc1) buffer access per lane: split
// partials pass between workgroups that may sit on different XCDs, whose L2
// caches are not coherent.  `head` is wave-uniform (the buffer resource lives
// in scalar registers); the lane offset goes in the vector offset.
template <int NPL>
__device__ __forceinline__ void store_head_f32_coherent(float* head, int lane, const float (&v)[NPL]) {
  const __amdgpu_buffer_rsrc_t r =
      __builtin_amdgcn_make_buffer_rsrc(head, (short)0, (int)(64 * NPL * 4), 0x00020000);
  const uint32_t off = (uint32_t)lane * NPL * 4u;
  if constexpr (NPL == 4) {
    __builtin_amdgcn_raw_buffer_store_b128(
        u32x4{__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]), __float_as_uint(v[3])},
        r, off, 0, 16);
  } else {
    __builtin_amdgcn_raw_buffer_store_b64(u32x2{__float_as_uint(v[0]), __float_as_uint(v[1])}, r, off, 0,
                                          16);
  }
}
template <int NPL>
__device__ __forceinline__ void load_head_f32_coherent(float (&v)[NPL], const float* head, int lane,
                                                       bool valid = true) {
  // valid == false: a zero-range resource, the load returns zeros untouched
  const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float*>(head), (short)0, valid ? (int)(64 * NPL * 4) : 0, 0x00020000);
  const uint32_t off = (uint32_t)lane * NPL * 4u;
  if constexpr (NPL == 4) {
    const u32x4 u = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 16);
    v[0] = __uint_as_float(u.x); v[1] = __uint_as_float(u.y);
    v[2] = __uint_as_float(u.z); v[3] = __uint_as_float(u.w);
  } else {
    const u32x2 u = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 16);
    v[0] = __uint_as_float(u.x); v[1] = __uint_as_float(u.y);
  }
}

// Per-lane operands of the head norm and RoPE: lane l holds dims
// c = l * NPL + i.  They are loaded once, up front, so the norm and rotation
// below never wait on memory.
template <int NPL>
struct NormRopeIn {
  float qw[NPL], kw[NPL];  // (1+w) norm weights of q and k (w)
  float cs[NPL], sn[NPL];  // cos / sin of dim c at the position (c < rot)
};

template <int NPL>
__device__ __forceinline__ void load_norm_w(NormRopeIn<NPL>& in, const float* q_norm_w,
                                            const float* k_norm_w, int lane) {
  // Buffer loads keep this branch-free (a load under a branch makes the
  // compiler wait for every earlier load there): a null pointer gets an empty
  // resource, whose loads read 0.
  constexpr int bytes = NPL * 64 * 4;
  const auto rq = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(q_norm_w), (short)0,
                                                    q_norm_w ? bytes : 0, 0x00020000);
  const auto rk = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(k_norm_w), (short)0,
                                                    k_norm_w ? bytes : 0, 0x00020000);
#pragma unroll
  for (int i = 0; i < NPL; ++i) {
    const int off = (lane * NPL + i) * 4;
    in.qw[i] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rq, off, 0, 0));
    in.kw[i] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rk, off, 0, 0));
  }
}
// cos / sin rows of the tables at the position.  Buffer loads over exactly the
// row keep this branch-free (dims c >= rot read past the range: zeros, replaced
// by cos 1, sin 0), so the loads can be issued ahead of the K/V tile and
// waited for without waiting for the tile.
template <int NPL>
__device__ __forceinline__ void load_rope(NormRopeIn<NPL>& in, const float* cos_row, const float* sin_row,
                                          int rot, int lane) {
  const int bytes = rot > 0 ? rot * 4 : 0;
  const auto rc = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(cos_row), (short)0, bytes, 0x00020000);
  const auto rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(sin_row), (short)0, bytes, 0x00020000);
#pragma unroll
  for (int i = 0; i < NPL; ++i) {
    const int c = lane * NPL + i;
    const float cv = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rc, c * 4, 0, 0));
    const float sv = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, c * 4, 0, 0));
    in.cs[i] = c < rot ? cv : 1.0f;
    in.sn[i] = c < rot ? sv : 0.0f;
  }
}

// bf16 (1+w) RMSNorm over a D-wide head held NPL values per lane, then bf16
// partial RoPE.  All lanes of the wave must call this.
template <int D>
__device__ __forceinline__ void norm_rope(float (&v)[D / 64], bool has_norm, const float (&nw)[D / 64],
                                          const NormRopeIn<D / 64>& r, float eps, int rot, int lane) {
  constexpr int NPL = D / 64;
  if (has_norm) {
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < NPL; ++i) ss = fmaf(v[i], v[i], ss);
    ss = wave_total(ss);
    const float rs = rsqrtf(ss / (float)D + eps);
#pragma unroll
    for (int i = 0; i < NPL; ++i) v[i] = rbf(v[i] * rs * (1.0f + nw[i]));
  }
  if (rot > 0) {
    const int half = rot >> 1;
    const int pm = half / NPL;  // partner lane distance (power of two, checked on the host)
#pragma unroll
    for (int i = 0; i < NPL; ++i) {
      const float partner = __shfl_xor(v[i], pm, 64);
      const int c = lane * NPL + i;
      const float lo = v[i] * r.cs[i] - partner * r.sn[i];   // c < rot/2
      const float hi = v[i] * r.cs[i] + partner * r.sn[i];   // rot/2 <= c < rot
      v[i] = c < half ? rbf(lo) : (c < rot ? rbf(hi) : v[i]);
    }
  }
}

// Merges n <= 8 partial records (o [D] unnormalised against m, then m, l) at
// base + r * stride, r < n: lane r holds record r's (m, l); the n o-vectors
// are requested together (one memory round trip).  Returns the sum of the o
// rescaled to the common maximum M, and L = sum of the l rescaled likewise.
constexpr int kMergeBatch = 8;
template <int NPL>
__device__ __forceinline__ void merge_records(const float* base, size_t stride, int n, int lane,
                                              float (&acc)[NPL], float& Mo, float& Lo) {
  constexpr int D = NPL * 64;
  const bool have = lane < n;
  const float ls = have ? pub_load(base + lane * stride + D + 1) : 0.0f;
  const float ms = have ? pub_load(base + lane * stride + D) : -INFINITY;
  float part[kMergeBatch][NPL];
#pragma unroll
  for (int u = 0; u < kMergeBatch; ++u)
    load_head_f32_coherent<NPL>(part[u], base + (size_t)u * stride, lane, u < n);
  const float M = wave_max_dpp(ls > 0.0f ? ms : -INFINITY);
  const float ws = ls > 0.0f ? __expf(ms - M) : 0.0f;
  Lo = wave_total(ls * ws);
  Mo = M;
#pragma unroll
  for (int i = 0; i < NPL; ++i) acc[i] = 0.0f;
#pragma unroll
  for (int u = 0; u < kMergeBatch; ++u) {
    const float w = __shfl(ws, u, 64);
#pragma unroll
    for (int i = 0; i < NPL; ++i) acc[i] = w != 0.0f ? fmaf(part[u][i], w, acc[i]) : acc[i];
  }
}

// HPW: query heads per wave, ceil(G / 4) for the GQA group size G.
template <int D, int HPW>
__global__ __launch_bounds__(256) void attn_decode_kernel(QhAttnParams p) {
  constexpr int NPL = D / 64;
  constexpr int KS = D + 16;  // padded K row (bf16): conflict-free 16-byte LDS reads
  __shared__ __align__(16) uint16_t sK[TP * KS];
  __shared__ __align__(16) uint16_t sV[TP * D];
  __shared__ __align__(16) uint16_t sQ[MAXG * D];
  __shared__ __align__(16) float sP[MAXG][TP];
  __shared__ __align__(16) uint16_t sKn[D];
  __shared__ __align__(16) uint16_t sVn[D];
  __shared__ int s_last;

  const int kvh = blockIdx.x;
  const int split = blockIdx.y;
  const int lane = threadIdx.x & 63;
  // wave-uniform (scalar) so per-head buffer resources need no waterfall loop
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int G = p.n_heads / p.n_kv;

  // Loads that do not depend on the position go out first: this wave's query
  // heads and output gates, the new token's K/V (wave 0) and the norm weights.
  float qraw[HPW][NPL], gate_v[HPW][NPL];
#pragma unroll
  for (int hi = 0; hi < HPW; ++hi) {
    const int gi = wid + 4 * hi;
    const bool ok = gi < G;
    const size_t h = (size_t)(kvh * G + (ok ? gi : 0));
    load_head_b<NPL>(qraw[hi], p.q + h * p.q_stride, lane, ok);
    load_head_b<NPL>(gate_v[hi], p.gate ? p.gate + h * p.gate_stride : nullptr, lane,
                     ok && p.gate != nullptr);
  }
  float kraw[NPL], vraw[NPL];
  const bool kv_in = wid == 0 && p.k_new != nullptr;
  load_head_b<NPL>(kraw, kv_in ? p.k_new + (size_t)kvh * D : nullptr, lane, kv_in);
  load_head_b<NPL>(vraw, kv_in ? p.v_new + (size_t)kvh * D : nullptr, lane, kv_in);
  NormRopeIn<NPL> nr;
  load_norm_w<NPL>(nr, p.q_norm_w, p.k_norm_w, lane);

  const uint16_t* kbase = p.k_cache + (size_t)kvh * p.max_seq * D;
  const uint16_t* vbase = p.v_cache + (size_t)kvh * p.max_seq * D;
  // K/V tile staging: each thread moves PER 16-byte pieces of K and of V.
  // Loads are branch-free (rows at or past `lim` are clamped to row t0, and
  // lim <= max_seq) so a whole tile is in flight at once; the next tile is
  // requested before the current one is used.
  constexpr int PER = TP * (D / 8) / 256;
  u32x4 kreg[PER], vreg[PER];
  auto fetch = [&](int t0, int lim) {
#pragma unroll
    for (int e = 0; e < PER; ++e) {
      const int idx = threadIdx.x + 256 * e;
      const int pos = t0 + idx / (D / 8);
      const int c8 = (idx % (D / 8)) * 8;
      const int src = pos < lim ? pos : t0;
      kreg[e] = *(const u32x4*)(kbase + (size_t)src * D + c8);
      vreg[e] = *(const u32x4*)(vbase + (size_t)src * D + c8);
    }
  };
  auto span_of = [&](int n) {
    const int s = (n + p.nsplit - 1) / p.nsplit;
    return ((s + TP - 1) / TP) * TP;
  };

  int rope_pos = p.rope_pos, slot = p.slot, total = p.total;
  if (p.pos_dev) {
    const int t = *p.pos_dev;
    rope_pos = t;
    slot = t;
    total = t + 1;
  }
  // A device-resident position past the cache touches nothing (bounds guard).
  if (slot < 0 || slot >= p.max_seq || total > p.max_seq) return;
  // The span is sized to the context.  (A span fixed by the cache length,
  // whose first tile can be requested before the position arrives, leaves
  // fewer active splits at short context and measured slower.)
  const int span = span_of(total);
  const int p0 = split * span;
  const int p1 = min(total, p0 + span);
  // Splits past the context do nothing and do not take part in the merge:
  // the arrival target is the number of splits that hold positions (the same
  // value in every workgroup, computed from the device position).
  const int nactive = (total + span - 1) / span;
  const bool slot_in_range0 = slot >= 0 && slot < total;
  if (p.nsplit > 1 && split >= nactive && !(split == 0 && !slot_in_range0)) return;
  const bool slot_in_range = slot >= 0 && slot < total;
  const bool owner = (slot >= p0 && slot < p1) || (split == 0 && !slot_in_range);
  const float* cos_row = p.cos_t + (size_t)rope_pos * p.rot;
  const float* sin_row = p.sin_t + (size_t)rope_pos * p.rot;
  const float scale = rsqrtf((float)D);
  const bool new_kv = p.k_new != nullptr;

  auto stage = [&](int t0) {
    const u32x4 zero = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int e = 0; e < PER; ++e) {
      const int idx = threadIdx.x + 256 * e;
      const int row = idx / (D / 8);
      const int c8 = (idx % (D / 8)) * 8;
      const int pos = t0 + row;
      u32x4 kq = kreg[e], vq = vreg[e];
      if (new_kv && pos == slot) {
        kq = *(const u32x4*)(sKn + c8);
        vq = *(const u32x4*)(sVn + c8);
      }
      if (pos >= p1) { kq = zero; vq = zero; }
      *(u32x4*)(sK + row * KS + c8) = kq;
      *(u32x4*)(sV + row * D + c8) = vq;
    }
  };
  // cos / sin first: waiting for them (the norm and rotation below) then
  // does not wait for the tile requested after them.  Every workgroup that
  // gets here holds positions (p0 < p1: split 0 starts at 0 < total, the
  // others returned above unless split < nactive), so the fetch needs no
  // branch, which would make the compiler wait for all loads at the join.
  load_rope<NPL>(nr, cos_row, sin_row, p.rot, lane);
  fetch(p0, p1);

  // ---- query heads of this KV group: norm + RoPE, kept as bf16 in LDS ----
#pragma unroll
  for (int hi = 0; hi < HPW; ++hi) {
    const int gi = wid + 4 * hi;
    if (gi >= G) continue;
    const int h = kvh * G + gi;
    norm_rope<D>(qraw[hi], p.q_norm_w != nullptr, nr.qw, nr, p.eps, p.rot, lane);
    store_head<NPL>(sQ + gi * D + lane * NPL, qraw[hi]);
    if (p.q_wb && split == 0) store_head<NPL>(p.q_wb + (size_t)h * D + lane * NPL, qraw[hi]);
  }
  // ---- the new token's K (norm + RoPE) and V -------------------------------
  if (wid == 0 && p.k_new) {
    float (&kv)[NPL] = kraw;
    float (&vv)[NPL] = vraw;
    norm_rope<D>(kv, p.k_norm_w != nullptr, nr.kw, nr, p.eps, p.rot, lane);
    store_head<NPL>(sKn + lane * NPL, kv);
    store_head<NPL>(sVn + lane * NPL, vv);
    if (owner) {
      const size_t off = ((size_t)kvh * p.max_seq + slot) * D + lane * NPL;
      store_head<NPL>(p.k_cache + off, kv);
      store_head<NPL>(p.v_cache + off, vv);
      if (p.k_wb) store_head<NPL>(p.k_wb + (size_t)kvh * D + lane * NPL, kv);
    }
  }
  __syncthreads();

  float m[HPW], l[HPW], o[HPW][NPL];
#pragma unroll
  for (int hi = 0; hi < HPW; ++hi) {
    m[hi] = -INFINITY;
    l[hi] = 0.0f;
#pragma unroll
    for (int i = 0; i < NPL; ++i) o[hi][i] = 0.0f;
  }

  // scores: lane pair (2j, 2j+1) owns position t0+j, each lane half the dims
  // (chunks of 8 dims c = 2 cc + half); the lane's q chunks stay in registers
  // for the whole loop, so only K is read from LDS per position.
  const int prow = lane >> 1, half = lane & 1;
  u32x4 qreg[HPW][D / 16];
#pragma unroll
  for (int hi = 0; hi < HPW; ++hi) {
    const int gi = wid + 4 * hi < G ? wid + 4 * hi : 0;
#pragma unroll
    for (int cc = 0; cc < D / 16; ++cc) qreg[hi][cc] = *(const u32x4*)(sQ + gi * D + (2 * cc + half) * 8);
  }

  for (int t0 = p0; t0 < p1; t0 += TP) {
    stage(t0);
    __syncthreads();
    if (t0 + TP < p1) fetch(t0 + TP, p1);

    const bool valid = t0 + prow < p1;
#pragma unroll
    for (int hi = 0; hi < HPW; ++hi) {
      const int gi = wid + 4 * hi;
      if (gi < G) {
        float dot = 0.0f;
        // constant trip count: unrolled, the LDS reads are issued together
#pragma unroll
        for (int cc = 0; cc < D / 16; ++cc) {
          const int c = 2 * cc + half;
          const u32x4 k8 = *(const u32x4*)(sK + prow * KS + c * 8);
          const u32x4 q8 = qreg[hi][cc];
          dot = __builtin_amdgcn_fdot2_f32_bf16(as_bf2(q8.x), as_bf2(k8.x), dot, false);
          dot = __builtin_amdgcn_fdot2_f32_bf16(as_bf2(q8.y), as_bf2(k8.y), dot, false);
          dot = __builtin_amdgcn_fdot2_f32_bf16(as_bf2(q8.z), as_bf2(k8.z), dot, false);
          dot = __builtin_amdgcn_fdot2_f32_bf16(as_bf2(q8.w), as_bf2(k8.w), dot, false);
        }
        dot += __shfl_xor(dot, 1, 64);
        const float s = valid ? dot * scale : -INFINITY;
        const float tmax = wave_max_dpp(s);
        const float nm = fmaxf(m[hi], tmax);
        const float corr = __expf(m[hi] - nm);
        const float pv = valid ? __expf(s - nm) : 0.0f;
        const float psum = wave_total(half == 0 ? pv : 0.0f);
        l[hi] = l[hi] * corr + psum;
        m[hi] = nm;
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
        // fully unrolled: the V reads and the 4-position p reads issue ahead
#pragma unroll
        for (int j4 = 0; j4 < TP / 4; ++j4) {
          const float4 p4 = *(const float4*)&sP[gi][4 * j4];
          const float pj[4] = {p4.x, p4.y, p4.z, p4.w};
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            float vv[NPL];
            load_head<NPL>(vv, sV + (4 * j4 + u) * D + lane * NPL);
#pragma unroll
            for (int i = 0; i < NPL; ++i) o[hi][i] = fmaf(pj[u], vv[i], o[hi][i]);
          }
        }
      }
    }
    __syncthreads();
  }

  auto emit = [&](int gi, const float (&gv)[NPL], float (&ov)[NPL], float inv) {
    const int h = kvh * G + gi;
    float r[NPL];
#pragma unroll
    for (int i = 0; i < NPL; ++i) {
      float a = ov[i] * inv;
      if (p.gate) a = rbf(a) * rbf(qh_sigmoid(gv[i]));
      r[i] = a;
    }
    store_head<NPL>(p.out + (size_t)h * D + lane * NPL, r);
  };

  if (p.nsplit == 1) {
#pragma unroll
    for (int hi = 0; hi < HPW; ++hi) {
      const int gi = wid + 4 * hi;
      if (gi < G) emit(gi, gate_v[hi], o[hi], 1.0f / l[hi]);
    }
    return;
  }

  // ---- publish this split's partial state; the last split merges ---------
  const int rec = D + 2;
#pragma unroll
  for (int hi = 0; hi < HPW; ++hi) {
    const int gi = wid + 4 * hi;
    if (gi < G) {
      float* dst = p.part + ((size_t)(kvh * p.nsplit + split) * MAXG + gi) * rec;
      store_head_f32_coherent<NPL>(dst, lane, o[hi]);
      if (lane == 0) {
        pub_store(dst + D, m[hi]);
        pub_store(dst + D + 1, l[hi]);
      }
    }
  }
  // Up to 8 active splits: the last to arrive merges them all.  More: two
  // levels, so no workgroup reads more than 8 records per query head (one
  // reading all 64 splits' records through one CU took ~10 us at context
  // 4096): the last split of each group of 8 merges its group into a
  // level-2 record, and the last group merges the groups.
  const size_t sstride = (size_t)MAXG * rec;
  const float* src = p.part + (size_t)kvh * p.nsplit * sstride;  // records of this KV head
  int nsrc = nactive;
  if (nactive > kMergeBatch) {
    const int grp = split / kMergeBatch, ngrp = (nactive + kMergeBatch - 1) / kMergeBatch;
    const int gsize = min(kMergeBatch, nactive - grp * kMergeBatch);
    float* lvl2 = p.part + (size_t)p.n_kv * p.nsplit * sstride + (size_t)kvh * kMergeBatch * sstride;
    unsigned* gc = p.gcounters + kvh * kMergeBatch + grp;
    if (!arrive_last(gc, (unsigned)gsize, &s_last)) return;
#pragma unroll
    for (int hi = 0; hi < HPW; ++hi) {
      const int gi = wid + 4 * hi;
      if (gi >= G) continue;
      float acc[NPL], M, L;
      merge_records<NPL>(src + (size_t)grp * kMergeBatch * sstride + (size_t)gi * rec, sstride, gsize, lane,
                         acc, M, L);
      float* dst = lvl2 + (size_t)grp * sstride + (size_t)gi * rec;
      store_head_f32_coherent<NPL>(dst, lane, acc);
      if (lane == 0) {
        pub_store(dst + D, M);
        pub_store(dst + D + 1, L);
      }
    }
    if (threadIdx.x == 0) reset_counter(gc);
    if (!arrive_last(p.counters + kvh, (unsigned)ngrp, &s_last)) return;
    src = lvl2;
    nsrc = ngrp;
  } else if (!arrive_last(p.counters + kvh, (unsigned)nactive, &s_last)) {
    return;
  }
#pragma unroll
  for (int hi = 0; hi < HPW; ++hi) {
    const int gi = wid + 4 * hi;
    if (gi >= G) continue;
    float acc[NPL], M, L;
    merge_records<NPL>(src + (size_t)gi * rec, sstride, nsrc, lane, acc, M, L);
    emit(gi, gate_v[hi], acc, 1.0f / L);
  }
  if (threadIdx.x == 0) reset_counter(p.counters + kvh);
}

// ---- fixed scratch of qh_attn_decode_noalloc --------------------------------
// Words [0, kStaticCounterWords) are the per-KV-head arrival counters and
// then the group counters [64][8] of the two-level merge (the kernel's last
// arrivers return each to zero), the rest the split partials.
// The array is device memory that each GPU the library runs on holds until
// the process ends; every call on one GPU shares it.
constexpr int kStaticKv = 64;                                 // n_kv <= 64
constexpr int kStaticCounterWords = kStaticKv * (1 + kMergeBatch);
constexpr size_t kStaticPartFloats = (size_t)1 << 21;         // 8 MiB of partials
constexpr size_t kStaticWords = kStaticCounterWords + kStaticPartFloats;
constexpr int kMaxDevices = 64;

__global__ __launch_bounds__(64) void zero_words_kernel(unsigned* w, int n) {
  for (int i = (int)threadIdx.x; i < n; i += 64) w[i] = 0u;
}

}  // namespace

static __device__ __align__(256) uint32_t scratch[kStaticWords];

namespace {

std::mutex g_static_mu;
uint32_t* g_static_ptr[kMaxDevices] = {};

// Device address of this GPU's copy of `scratch`, looked up once per device
// (with that device current) and its counters cleared by a fill kernel on
// the caller's stream.  Host code only ever uses this address: the array's
// name in host code is a stand-in, not a device pointer.
uint32_t* static_scratch(hipStream_t st) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    qh_set_error("attn_decode_noalloc: no current device (or device index >= %d)", kMaxDevices);
    return nullptr;
  }
  std::lock_guard<std::mutex> lk(g_static_mu);
  if (!g_static_ptr[dev]) {
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr) {
      qh_set_error("attn_decode_noalloc: hipGetSymbolAddress failed: %s", hipGetErrorString(e));
      return nullptr;
    }
    hipLaunchKernelGGL(zero_words_kernel, dim3(1), dim3(64), 0, st, (unsigned*)ptr,
                       kStaticCounterWords);
    g_static_ptr[dev] = (uint32_t*)ptr;
  }
  return g_static_ptr[dev];
}

}  // namespace

// Layout (4-byte words): the group arrival counters of the two-level merge
// [n_kv][8] (zero before the first call; they return to zero themselves),
// the splits' records [n_kv][nsplit][MAXG][D + 2] and, above 8 splits, the
// level-2 records [n_kv][8][MAXG][D + 2].
size_t qh_attn_scratch_floats(int n_kv, int nsplit, int head_dim) {
  const size_t rec = (size_t)MAXG * (head_dim + 2);
  return (size_t)n_kv * kMergeBatch + (size_t)n_kv * (nsplit + (nsplit > kMergeBatch ? kMergeBatch : 0)) * rec;
}

int qh_launch_attn(const QhAttnParams& p, int head_dim, hipStream_t st) {
  if (p.n_kv <= 0 || p.n_heads <= 0 || p.n_heads % p.n_kv != 0 || p.n_heads / p.n_kv > MAXG) {
    qh_set_error("attn: n_heads=%d n_kv_heads=%d unsupported (group size must divide and be <= %d)",
                 p.n_heads, p.n_kv, MAXG);
    return -1;
  }
  if (head_dim != 128 && head_dim != 256) {
    qh_set_error("attn: head_dim=%d unsupported (128 or 256)", head_dim);
    return -1;
  }
  const int npl = head_dim / 64;
  if (p.rot < 0 || p.rot > head_dim || (p.rot % 2) != 0 ||
      (p.rot > 0 && (((p.rot / 2) % npl) != 0 || ((p.rot / 2 / npl) & (p.rot / 2 / npl - 1)) != 0))) {
    qh_set_error("attn: rotary_dim=%d unsupported for head_dim=%d", p.rot, head_dim);
    return -1;
  }
  if (p.nsplit < 1 || p.nsplit > 64 || (p.nsplit > 1 && (!p.part || !p.counters)) ||
      (p.nsplit > kMergeBatch && !p.gcounters)) {
    qh_set_error("attn: nsplit=%d must be 1..64; split-K needs scratch and counters", p.nsplit);
    return -1;
  }
  if (!p.pos_dev) {
    if (p.total < 1 || p.total > p.max_seq || p.slot < 0 || p.slot >= p.max_seq || p.rope_pos < 0) {
      qh_set_error("attn: positions out of range (pos=%d slot=%d total=%d max_seq=%d)", p.rope_pos,
                   p.slot, p.total, p.max_seq);
      return -1;
    }
  }
  dim3 grid(p.n_kv, p.nsplit);
  const bool two = p.n_heads / p.n_kv > 4;  // two query heads per wave
  if (head_dim == 256) {
    if (two) hipLaunchKernelGGL((attn_decode_kernel<256, 2>), grid, dim3(256), 0, st, p);
    else hipLaunchKernelGGL((attn_decode_kernel<256, 1>), grid, dim3(256), 0, st, p);
  } else {
    if (two) hipLaunchKernelGGL((attn_decode_kernel<128, 2>), grid, dim3(256), 0, st, p);
    else hipLaunchKernelGGL((attn_decode_kernel<128, 1>), grid, dim3(256), 0, st, p);
  }
  return 0;
}

// Allocation-free variant of qh_attn_decode: the split partials and arrival
// counters live in the file-scope array above instead of caller memory.  No
// counterpart in the reference; for callers that cannot allocate (code under
// graph capture, serving loops that forbid hipMalloc).  Limits: n_kv <= 64
// and qh_attn_scratch_floats(n_kv, nsplit, head_dim) <= 2^21 (8 MiB): the
// split records, plus the level-2 records above 8 splits.
// Calls that overlap on one GPU race on the shared array.
extern "C" __attribute__((visibility("default"))) int qh_attn_decode_noalloc(
    const void* q, int q_stride, const void* gate, int gate_stride, const void* k_new,
    const void* v_new, const float* q_norm_w, const float* k_norm_w, const float* cos_t,
    const float* sin_t, void* k_cache, void* v_cache, int max_seq, int head_dim, int rot,
    int n_heads, int n_kv, const int* pos_dev, int pos, int nsplit, void* out, float eps,
    hipStream_t stream) {
  if (n_kv < 1 || n_kv > kStaticKv || nsplit < 1 || nsplit > 64 ||
      (head_dim != 128 && head_dim != 256) ||
      qh_attn_scratch_floats(n_kv, nsplit, head_dim) > kStaticPartFloats) {
    qh_set_error("qh_attn_decode_noalloc: n_kv=%d, nsplit=%d, head_dim=%d exceed the fixed "
                 "scratch (n_kv <= %d, nsplit 1..64, qh_attn_scratch_floats <= %zu floats: "
                 "n_kv*nsplit*%d*(head_dim+2), plus n_kv*8*%d*(head_dim+2)+n_kv*8 above 8 splits)",
                 n_kv, nsplit, head_dim, kStaticKv, kStaticPartFloats, MAXG, MAXG);
    return -1;
  }
  uint32_t* ws = static_scratch(stream);
  if (!ws) return -1;
  QhAttnParams a;
  memset(&a, 0, sizeof(a));
  a.q = (const uint16_t*)q;
  a.q_stride = q_stride;
  a.gate = (const uint16_t*)gate;
  a.gate_stride = gate_stride;
  a.k_new = (const uint16_t*)k_new;
  a.v_new = (const uint16_t*)v_new;
  a.q_norm_w = q_norm_w;
  a.k_norm_w = k_norm_w;
  a.cos_t = cos_t;
  a.sin_t = sin_t;
  a.k_cache = (uint16_t*)k_cache;
  a.v_cache = (uint16_t*)v_cache;
  a.max_seq = max_seq;
  a.rot = rot;
  a.n_heads = n_heads;
  a.n_kv = n_kv;
  a.pos_dev = pos_dev;
  a.rope_pos = pos;
  a.slot = pos;
  a.total = pos + 1;
  a.nsplit = nsplit;
  a.counters = (unsigned*)ws;
  a.gcounters = (unsigned*)ws + kStaticKv;
  a.part = (float*)(ws + kStaticCounterWords);
  a.out = (uint16_t*)out;
  a.eps = eps;
  if (qh_launch_attn(a, head_dim, stream) != 0) return -1;
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    qh_set_error("qh_attn_decode_noalloc: launch failed: %s", hipGetErrorString(e));
    return -1;
  }
  return 0;
}
