// On-device nucleus sampling (gfx950): the reference's top_p_sample,
// main.py:49-87, for one [V] bf16 logits row.
//
// Semantics followed (reference line numbers in main.py):
//   y   = bf16(logits * (1/T)) if T > 0 (54-55; the reference's CUDA division by
//         a scalar multiplies by the fp32 reciprocal)
//   y_i = bf16(y_i * rp) if y_i < 0 else bf16(y_i * (1/rp)), for each distinct
//         id i of the recent window, when rp > 1 (57-63)
//   p_i = bf16(exp(bf16(y_i - bf16(logsumexp(y)))))  over the tokens sorted by y
//         descending (64-72); if the top-min(2000, V) mass, rounded to bf16, is
//         below bf16(top_p), the full-vocabulary softmax bf16(exp(y - max) / Z)
//         is used instead (73-78)
//   keep the sorted prefix whose running mass, rounded to bf16, is <= bf16(top_p)
//         (at least the first token), renormalise, draw one (79-86).
// Ties in y are ordered by token index (lowest first).  The draw uses SplitMix64
// (Steele, Lea & Flood 2014) of (seed, counter) -- not torch's generator -- so
// a given call reproduces the reference's distribution, not its token.
//
// Design: no sort.  Tokens are ordered by the 16-bit order-preserving key of
// their bf16 y, so four passes suffice, none of which needs a host round trip:
//   1. scale (grid): y -> workspace, online (max, sum exp) per block, merged by
//      the last block to arrive; the key histogram is cleared;
//   2. histogram (grid): per-block key counts in LDS (two 16-bit counters per
//      word), merged into a global [65536] count histogram;
//   3. select (one 1024-thread workgroup): per-key probability masses in 2^-40
//      fixed point (exact, order independent), block scans over the keys in
//      descending order, the top-2000 mass, the top-p cut and the drawn
//      (key, rank among that key's tokens);
//   4. locate (grid): the rank-th token of that key in index order; the last
//      block writes the token, the history slot and the next embedding row.
#include "qh_common.h"
#include "qh_sample.h"

namespace {

constexpr int kPerThread = 8;                  // tokens per thread, passes 1, 2, 4
constexpr int kBlockTokens = 256 * kPerThread;  // tokens per block
constexpr int kKeys = 65536;
constexpr int kTopK = 2000;                    // main.py:66
constexpr double kFxOne = 1099511627776.0;     // 2^40
constexpr double kFxInv = 1.0 / 1099511627776.0;

// Workspace layout (bytes), derived from V.
struct SampleWs {
  uint16_t* y;        // [V] bf16
  unsigned* hist;     // [65536] key counts
  float* part;        // [nblk][2] (max, sum exp) partials
  unsigned* cnt;      // [nblk] per-block match counts (pass 4)
  unsigned* arrive;   // [2] arrival counters (passes 1 and 4), self-resetting
  float* dist;        // [4] max, Z, bf16(logsumexp)
  int64_t* sel;       // [4] drawn key, rank, window size, slot
};

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

int nblocks(int V) { return (V + kBlockTokens - 1) / kBlockTokens; }

size_t layout(int V, uint8_t* base, SampleWs* w) {
  const int nb = nblocks(V);
  size_t off = 0;
  auto take = [&](size_t bytes) { const size_t o = off; off = align256(off + bytes); return base + o; };
  uint8_t* y = take((size_t)V * 2);
  uint8_t* hist = take((size_t)kKeys * 4);
  uint8_t* part = take((size_t)nb * 8);
  uint8_t* cnt = take((size_t)nb * 4);
  uint8_t* arrive = take(2 * 4);
  uint8_t* dist = take(4 * 4);
  uint8_t* sel = take(4 * 8);
  if (w) {
    w->y = (uint16_t*)y;
    w->hist = (unsigned*)hist;
    w->part = (float*)part;
    w->cnt = (unsigned*)cnt;
    w->arrive = (unsigned*)arrive;
    w->dist = (float*)dist;
    w->sel = (int64_t*)sel;
  }
  return off;
}

// bf16 bits -> key, larger key = larger value (-0 sorts just below +0).
__device__ __forceinline__ uint32_t asc_key(uint16_t b) {
  return (b & 0x8000u) ? (~(uint32_t)b & 0xFFFFu) : ((uint32_t)b | 0x8000u);
}
__device__ __forceinline__ float key_value(uint32_t k) {
  const uint16_t b = (k & 0x8000u) ? (uint16_t)(k & 0x7FFFu) : (uint16_t)(~k & 0xFFFFu);
  return bf2f(b);
}

__device__ __forceinline__ uint64_t to_fx(float p) {
  // p in [0, 1]; non-finite or negative (only from non-finite logits) -> 0
  return (p >= 0.0f && p <= 1.0f) ? (uint64_t)((double)p * kFxOne) : 0ull;
}
// A running mass as the reference materialises it: fp32, then bf16.
__device__ __forceinline__ float fx_bf16(uint64_t c) { return rbf((float)((double)c * kFxInv)); }

__device__ __forceinline__ float p_ref(float y, float logz_b) { return rbf(expf(rbf(y - logz_b))); }
__device__ __forceinline__ float p_soft(float y, float M, float Z) { return rbf(expf(y - M) / Z); }

__device__ __forceinline__ uint64_t splitmix64(uint64_t x) {
  x += 0x9E3779B97F4A7C15ull;
  x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
  x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
  return x ^ (x >> 31);
}

struct Window {
  int slot;  // where the new token goes
  int lo;    // first window slot
  int n;     // window size
};
__device__ __forceinline__ Window window_of(const QhSampleParams& p) {
  Window w;
  w.slot = (p.pos_dev ? *p.pos_dev : p.pos) + p.pos_offset;
  const int lo0 = p.lo_dev ? *p.lo_dev : 0;
  w.lo = max(max(lo0, 0), w.slot - p.window);
  const int end = min(w.slot, p.hist_len);  // window slots stay inside hist
  w.n = (p.hist && p.window > 0) ? max(0, min(end - w.lo, p.window)) : 0;
  return w;
}

// ---- pass 1: scale + penalty, (max, sum exp), histogram clear ---------------
__global__ __launch_bounds__(256) void sample_scale_kernel(QhSampleParams p, SampleWs w, int nb) {
  __shared__ int64_t s_win[kSampleMaxWindow];
  __shared__ float s_m[4], s_s[4];
  __shared__ int s_last;
  const int tid = threadIdx.x;
  const Window win = window_of(p);
  const bool penal = p.rep_penalty > 1.0f && win.n > 0;
  if (penal && tid < win.n) s_win[tid] = p.hist[win.lo + tid];
  // clear this block's share of the key histogram (read by pass 2)
  for (int k = blockIdx.x * 256 + tid; k < kKeys; k += nb * 256) w.hist[k] = 0u;
  __syncthreads();

  const float inv_t = p.temperature > 0.0f ? 1.0f / p.temperature : 1.0f;
  const float inv_rp = 1.0f / p.rep_penalty;
  const int base = blockIdx.x * kBlockTokens + tid * kPerThread;
  float m = -INFINITY, s = 0.0f;
  uint16_t yb[kPerThread];
#pragma unroll
  for (int e = 0; e < kPerThread; ++e) {
    const int i = base + e;
    float y = -INFINITY;
    if (i < p.V) {
      y = bf2f(p.logits[i]);
      if (p.temperature > 0.0f) y = rbf(y * inv_t);
      if (penal) {
        bool hit = false;
        for (int r = 0; r < win.n; ++r) hit |= s_win[r] == (int64_t)i;
        if (hit) y = y < 0.0f ? rbf(y * p.rep_penalty) : rbf(y * inv_rp);
      }
      if (y > -INFINITY) {
        const float nm = fmaxf(m, y);
        s = s * expf(m - nm) + expf(y - nm);
        m = nm;
      }
    }
    yb[e] = f2bf(y);
  }
#pragma unroll
  for (int e = 0; e < kPerThread; ++e)
    if (base + e < p.V) w.y[base + e] = yb[e];
  // block (max, sum): wave reduce, then 4 waves
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float m2 = __shfl_xor(m, o, 64), s2 = __shfl_xor(s, o, 64);
    const float nm = fmaxf(m, m2);
    s = (m == -INFINITY ? 0.0f : s * expf(m - nm)) + (m2 == -INFINITY ? 0.0f : s2 * expf(m2 - nm));
    m = nm;
  }
  if ((tid & 63) == 0) {
    s_m[tid >> 6] = m;
    s_s[tid >> 6] = s;
  }
  __syncthreads();
  if (tid == 0) {
    float bm = -INFINITY, bs = 0.0f;
    for (int q = 0; q < 4; ++q) {
      const float nm = fmaxf(bm, s_m[q]);
      bs = (bm == -INFINITY ? 0.0f : bs * expf(bm - nm)) + (s_m[q] == -INFINITY ? 0.0f : s_s[q] * expf(s_m[q] - nm));
      bm = nm;
    }
    pub_store(&w.part[2 * blockIdx.x], bm);
    pub_store(&w.part[2 * blockIdx.x + 1], bs);
  }
  if (!arrive_last(&w.arrive[0], (unsigned)nb, &s_last)) return;
  if (tid == 0) {
    // merge the block partials in block order (deterministic)
    float M = -INFINITY, Z = 0.0f;
    for (int b = 0; b < nb; ++b) {
      const float bm = pub_load(&w.part[2 * b]), bs = pub_load(&w.part[2 * b + 1]);
      const float nm = fmaxf(M, bm);
      Z = (M == -INFINITY ? 0.0f : Z * expf(M - nm)) + (bm == -INFINITY ? 0.0f : bs * expf(bm - nm));
      M = nm;
    }
    w.dist[0] = M;
    w.dist[1] = Z;
    w.dist[2] = rbf(M + logf(Z));  // torch.logsumexp of a bf16 tensor, main.py:70
    reset_counter(&w.arrive[0]);
  }
}

// ---- pass 2: key histogram ----------------------------------------------------
__global__ __launch_bounds__(256) void sample_hist_kernel(QhSampleParams p, SampleWs w) {
  // two 16-bit counters per word (a block counts at most 2048 tokens)
  __shared__ unsigned s_h[kKeys / 2];
  const int tid = threadIdx.x;
  for (int k = tid; k < kKeys / 2; k += 256) s_h[k] = 0u;
  __syncthreads();
  const int base = blockIdx.x * kBlockTokens + tid * kPerThread;
#pragma unroll
  for (int e = 0; e < kPerThread; ++e) {
    const int i = base + e;
    if (i < p.V) {
      const uint32_t k = asc_key(w.y[i]);
      atomicAdd(&s_h[k >> 1], (k & 1u) ? 65536u : 1u);
    }
  }
  __syncthreads();
  for (int q = tid; q < kKeys / 2; q += 256) {
    const unsigned v = s_h[q];
    if (v & 0xFFFFu)
      __hip_atomic_fetch_add(&w.hist[2 * q], v & 0xFFFFu, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (v >> 16)
      __hip_atomic_fetch_add(&w.hist[2 * q + 1], v >> 16, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// ---- pass 3: selection ---------------------------------------------------------
constexpr int SNT = 1024;
constexpr int KPT = kKeys / SNT;  // keys per thread (64), in descending key order

// Exclusive prefix over the 1024 threads (thread order); also the total.
__device__ __forceinline__ uint64_t block_excl_u64(uint64_t v, uint64_t* s_w, uint64_t& total) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  uint64_t x = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint64_t y = __shfl_up(x, o, 64);
    if (lane >= o) x += y;
  }
  if (lane == 63) s_w[wid] = x;
  __syncthreads();
  uint64_t before = 0, tot = 0;
  for (int q = 0; q < SNT / 64; ++q) {
    const uint64_t t = s_w[q];
    if (q < wid) before += t;
    tot += t;
  }
  __syncthreads();
  total = tot;
  return before + x - v;
}

__global__ __launch_bounds__(SNT) void sample_select_kernel(QhSampleParams p, SampleWs w) {
  __shared__ uint64_t s_w[SNT / 64];
  __shared__ uint64_t s_c2k;
  __shared__ int s_flags[2];  // [0] fallback, [1] boundary found
  __shared__ uint64_t s_cut[4];  // boundary key, kept at the key, kept count, kept mass
  __shared__ int64_t s_pick[2];
  __shared__ uint64_t s_ctr;
  const int tid = threadIdx.x;
  if (tid == 0) s_ctr = *p.counter;  // published by the scans' barriers below
  const float M = w.dist[0], Z = w.dist[1], logz_b = w.dist[2];
  const float tp_b = rbf(p.top_p);  // the comparison runs in bf16 (main.py:73, 79)
  auto kept = [&](uint64_t cum) { return fx_bf16(cum) <= tp_b; };

  // this thread's keys: k = kKeys - 1 - (KPT * tid + i), i = 0 .. KPT-1, whose
  // counts are read four at a time (ascending in memory) whenever they are
  // walked; fn(k, count) returns true to stop.
  const uint32_t k0 = (uint32_t)(kKeys - 1 - KPT * tid);
  const u32x4* seg = (const u32x4*)(w.hist + (k0 - (KPT - 1)));  // 16-byte aligned
  auto walk = [&](auto fn) {
    for (int q = KPT / 4 - 1; q >= 0; --q) {
      const u32x4 v = seg[q];
      const unsigned cs[4] = {v.w, v.z, v.y, v.x};
      for (int j = 0; j < 4; ++j) {
        const uint32_t k = k0 - (uint32_t)((KPT / 4 - 1 - q) * 4 + j);
        if (cs[j] && fn(k, (uint64_t)cs[j])) return;
      }
    }
  };
  uint64_t n_t = 0, mr_t = 0, ms_t = 0;
  walk([&](uint32_t k, uint64_t cnt) {
    const float y = key_value(k);
    n_t += cnt;
    mr_t += cnt * to_fx(p_ref(y, logz_b));
    ms_t += cnt * to_fx(p_soft(y, M, Z));
    return false;
  });
  uint64_t n_all, mr_all, ms_all;
  const uint64_t n_b = block_excl_u64(n_t, s_w, n_all);
  const uint64_t mr_b = block_excl_u64(mr_t, s_w, mr_all);
  const uint64_t ms_b = block_excl_u64(ms_t, s_w, ms_all);

  // (1) mass of the top min(2000, V) tokens under the reference's p (main.py:66-72)
  const uint64_t ktop = (uint64_t)min(kTopK, p.V);
  if (tid == 0) {
    s_c2k = mr_all;
    s_flags[1] = 0;
  }
  __syncthreads();
  if (n_b < ktop && n_b + n_t >= ktop) {
    uint64_t cnt = n_b, mass = mr_b;
    walk([&](uint32_t k, uint64_t ck) {
      const uint64_t pf = to_fx(p_ref(key_value(k), logz_b));
      if (cnt + ck >= ktop) {
        mass += (ktop - cnt) * pf;
        return true;
      }
      cnt += ck;
      mass += ck * pf;
      return false;
    });
    s_c2k = mass;
  }
  __syncthreads();
  // (2) fallback to the full softmax when the top-k mass is below top_p (main.py:73-78)
  const bool soft = fx_bf16(s_c2k) < tp_b;
  const uint64_t m_t = soft ? ms_t : mr_t, m_b = soft ? ms_b : mr_b, m_all = soft ? ms_all : mr_all;
  auto p_of = [&](uint32_t k) {
    const float y = key_value(k);
    return to_fx(soft ? p_soft(y, M, Z) : p_ref(y, logz_b));
  };

  // (3) the top-p cut: the sorted prefix whose running mass stays <= top_p (main.py:79)
  if (tid == 0) {
    s_flags[0] = soft;
    s_cut[0] = 0; s_cut[1] = 0; s_cut[2] = n_all; s_cut[3] = m_all;  // all kept
  }
  __syncthreads();
  if (kept(m_b) && !kept(m_b + m_t)) {
    uint64_t cum = m_b, cnt = n_b;
    walk([&](uint32_t k, uint64_t ck) {
      const uint64_t pf = p_of(k);
      if (kept(cum + ck * pf)) {
        cum += ck * pf;
        cnt += ck;
        return false;
      }
      // largest j in [0, ck) with kept(cum + j * pf)
      uint64_t lo = 0, hi = ck;
      while (hi - lo > 1) {
        const uint64_t mid = (lo + hi) >> 1;
        if (kept(cum + mid * pf)) lo = mid;
        else hi = mid;
      }
      s_cut[0] = k;
      s_cut[1] = lo;
      s_cut[2] = cnt + lo;
      s_cut[3] = cum + lo * pf;
      s_flags[1] = 1;
      return true;
    });
  }
  __syncthreads();
  const bool cut = s_flags[1] != 0;
  const uint32_t kcut = (uint32_t)s_cut[0];
  const uint64_t mcut = s_cut[1];
  uint64_t S = s_cut[3];
  const bool forced = s_cut[2] == 0;  // nothing kept: the first token alone (main.py:80-81)

  // (4) the draw: target t in [0, S) over the kept prefix
  const uint64_t draw_ctr = s_ctr;
  const uint64_t r24 = splitmix64(p.seed ^ splitmix64(draw_ctr)) >> 40;
  if (tid == 0) {
    s_pick[0] = -1;
    s_pick[1] = 0;
  }
  __syncthreads();
  if (forced) {
    // the top key's first token
    if (n_t > 0 && n_b == 0) {
      walk([&](uint32_t k, uint64_t) {
        s_pick[0] = k;
        s_pick[1] = 0;
        return true;
      });
    }
  } else {
    // t = floor(S * r24 / 2^24) < S; the thread whose mass range holds t is at
    // or before the cut (every later thread has m_b >= S)
    const uint64_t t = (S >> 24) * r24 + (((S & 0xFFFFFFull) * r24) >> 24);
    if (m_b <= t && t < m_b + m_t) {
      uint64_t cum = m_b;
      walk([&](uint32_t k, uint64_t c_all) {
        const uint64_t pf = p_of(k);
        const uint64_t ck = (cut && k == kcut) ? mcut : c_all;
        if (pf > 0 && t < cum + ck * pf) {
          s_pick[0] = k;
          s_pick[1] = (int64_t)((t - cum) / pf);
          return true;
        }
        cum += ck * pf;
        return cut && k == kcut;
      });
    }
  }
  __syncthreads();
  if (tid == 0) {
    const Window win = window_of(p);
    w.sel[0] = s_pick[0];
    w.sel[1] = s_pick[1];
    w.sel[2] = win.n;
    w.sel[3] = win.slot;
    *p.counter = draw_ctr + 1;
    if (p.info) {
      p.info[0] = cut ? (int64_t)kcut : -1;
      p.info[1] = (int64_t)mcut;
      p.info[2] = forced ? 1 : (int64_t)s_cut[2];
      p.info[3] = soft;
      p.info[4] = (int64_t)S;
      p.info[5] = (int64_t)r24;
      p.info[6] = s_pick[0];
      p.info[7] = s_pick[1];
      p.info[8] = (int64_t)s_c2k;
      p.info[9] = (int64_t)__float_as_uint(M);
      p.info[10] = (int64_t)__float_as_uint(Z);
      p.info[11] = (int64_t)__float_as_uint(logz_b);
      p.info[13] = (int64_t)draw_ctr;
      p.info[14] = win.n;
    }
  }
}

// ---- pass 4: locate the drawn token, write the outputs ------------------------
__global__ __launch_bounds__(256) void sample_locate_kernel(QhSampleParams p, SampleWs w, int nb) {
  __shared__ unsigned s_c[4];
  __shared__ int s_last;
  __shared__ int s_blk, s_rank;
  __shared__ int s_tok;
  const int tid = threadIdx.x;
  const int64_t key = w.sel[0];
  const int64_t rank = w.sel[1];
  auto count_in = [&](int blk) {
    const int base = blk * kBlockTokens + tid * kPerThread;
    unsigned n = 0;
#pragma unroll
    for (int e = 0; e < kPerThread; ++e)
      if (base + e < p.V && (int64_t)asc_key(w.y[base + e]) == key) ++n;
    return n;
  };
  auto block_excl = [&](unsigned v, unsigned& total) {
    unsigned x = v;
    const int lane = tid & 63, wid = tid >> 6;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const unsigned y = __shfl_up(x, o, 64);
      if (lane >= o) x += y;
    }
    __syncthreads();
    if (lane == 63) s_c[wid] = x;
    __syncthreads();
    unsigned before = 0;
    total = 0;
    for (int q = 0; q < 4; ++q) {
      if (q < wid) before += s_c[q];
      total += s_c[q];
    }
    return before + x - v;
  };
  unsigned tot;
  const unsigned mine = count_in(blockIdx.x);
  block_excl(mine, tot);
  if (tid == 0) pub_store((int*)&w.cnt[blockIdx.x], (int)tot);
  if (!arrive_last(&w.arrive[1], (unsigned)nb, &s_last)) return;
  if (tid == 0) {
    // the block holding the rank-th match, in block order
    int64_t before = 0;
    int blk = -1, r = 0;
    for (int b = 0; b < nb; ++b) {
      const int n = pub_load((const int*)&w.cnt[b]);
      if (blk < 0 && rank < before + n) {
        blk = b;
        r = (int)(rank - before);
      }
      before += n;
    }
    s_blk = blk;
    s_rank = r;
    s_tok = -1;
    reset_counter(&w.arrive[1]);
  }
  __syncthreads();
  if (s_blk >= 0 && key >= 0) {
    const unsigned n = count_in(s_blk);
    unsigned t2;
    const unsigned before = block_excl(n, t2);
    if ((unsigned)s_rank >= before && (unsigned)s_rank < before + n) {
      int r = s_rank - (int)before;
      const int base = s_blk * kBlockTokens + tid * kPerThread;
      for (int e = 0; e < kPerThread; ++e) {
        const int i = base + e;
        if (i < p.V && (int64_t)asc_key(w.y[i]) == key) {
          if (r == 0) {
            s_tok = i;
            break;
          }
          --r;
        }
      }
    }
  }
  __syncthreads();
  const int tok = s_tok >= 0 ? s_tok : 0;  // not reached for finite logits
  if (tid == 0) {
    *p.tok_out = tok;
    const int slot = (int)w.sel[3];
    if (p.hist && slot >= 0 && slot < p.hist_len) p.hist[slot] = tok;
    if (p.info) p.info[12] = s_tok;
  }
  if (p.embed && p.h) {
    const uint16_t* src = p.embed + (size_t)tok * p.D;
    for (int k = tid; k < p.D; k += 256) p.h[k] = src[k];
  }
}

}  // namespace

size_t qh_sample_workspace_bytes(int V) { return V > 0 ? layout(V, nullptr, nullptr) : 0; }

int qh_launch_sample(const QhSampleParams& p, hipStream_t st) {
  if (!p.logits || p.V <= 0 || !p.ws || !p.counter || !p.tok_out) {
    qh_set_error("sample: logits, V > 0, workspace, counter and tok_out are required");
    return -1;
  }
  if (p.window < 0 || p.window > kSampleMaxWindow) {
    qh_set_error("sample: window=%d outside [0, %d]", p.window, kSampleMaxWindow);
    return -1;
  }
  if (!(p.top_p > 0.0f) || !(p.rep_penalty > 0.0f)) {
    qh_set_error("sample: top_p=%g and rep_penalty=%g must be positive", p.top_p, p.rep_penalty);
    return -1;
  }
  if (p.hist && p.hist_len <= 0) {
    qh_set_error("sample: a token history needs hist_len > 0");
    return -1;
  }
  if (p.embed && (!p.h || p.D <= 0)) {
    qh_set_error("sample: an embedding table needs h and D > 0");
    return -1;
  }
  if ((uintptr_t)p.ws % 256 != 0) {
    qh_set_error("sample: workspace must be 256-byte aligned");
    return -1;
  }
  SampleWs w;
  layout(p.V, p.ws, &w);
  const int nb = nblocks(p.V);
  hipLaunchKernelGGL(sample_scale_kernel, dim3(nb), dim3(256), 0, st, p, w, nb);
  hipLaunchKernelGGL(sample_hist_kernel, dim3(nb), dim3(256), 0, st, p, w);
  hipLaunchKernelGGL(sample_select_kernel, dim3(1), dim3(SNT), 0, st, p, w);
  hipLaunchKernelGGL(sample_locate_kernel, dim3(nb), dim3(256), 0, st, p, w, nb);
  return 0;
}
