// Shared device helpers for the gfx950 (MI355X) decode kernels.
//
// Conventions used by every kernel in this library:
//   * activations are bf16 stored as raw uint16_t bits (round-to-nearest-even
//     on every float -> bf16 conversion, like torch's .to(torch.bfloat16));
//   * FP8 weights are OCP E4M3FN bytes (bias 7, no inf, 0x7F/0xFF = NaN,
//     max 448), which gfx950 converts natively;
//   * a wavefront is 64 lanes; workgroups are 256 threads (4 waves) unless a
//     kernel says otherwise.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define QH_WAVE 64

typedef __bf16 qh_bf16x2 __attribute__((ext_vector_type(2)));
typedef float qh_f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// ---- bf16 <-> f32 ----------------------------------------------------------
__device__ __forceinline__ float bf2f(uint16_t b) {
  return __uint_as_float(((uint32_t)b) << 16);
}
__device__ __forceinline__ float bf_lo(uint32_t p) { return __uint_as_float(p << 16); }
__device__ __forceinline__ float bf_hi(uint32_t p) { return __uint_as_float(p & 0xFFFF0000u); }

// Round-to-nearest-even f32 -> bf16 (hardware v_cvt_pk_bf16_f32 on gfx950).
__device__ __forceinline__ uint16_t f2bf(float f) {
  __bf16 h = (__bf16)f;
  return __builtin_bit_cast(uint16_t, h);
}
__device__ __forceinline__ uint32_t pack_bf2(float lo, float hi) {
  return (uint32_t)f2bf(lo) | ((uint32_t)f2bf(hi) << 16);
}
// Round a float through bf16 and back (models a bf16 tensor materialisation).
__device__ __forceinline__ float rbf(float f) { return bf2f(f2bf(f)); }

__device__ __forceinline__ qh_bf16x2 as_bf2(uint32_t u) {
  return __builtin_bit_cast(qh_bf16x2, u);
}

// ---- E4M3FN -> bf16 / f32 --------------------------------------------------
// Two E4M3 bytes (word 0 = bytes 0,1; word 1 = bytes 2,3) -> two bf16, exact
// (every E4M3 value is representable in bf16).  Scale 1.0 = plain conversion.
__device__ __forceinline__ qh_bf16x2 e4m3x2_lo_bf16(uint32_t p) {
  return __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(p, 1.0f, false);
}
__device__ __forceinline__ qh_bf16x2 e4m3x2_hi_bf16(uint32_t p) {
  return __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(p, 1.0f, true);
}
__device__ __forceinline__ qh_f32x2 e4m3x2_lo_f32(uint32_t p) {
  return __builtin_amdgcn_cvt_pk_f32_fp8(p, false);
}
__device__ __forceinline__ qh_f32x2 e4m3x2_hi_f32(uint32_t p) {
  return __builtin_amdgcn_cvt_pk_f32_fp8(p, true);
}

// Dot product of 8 E4M3 weights (two dwords) with 8 bf16 activations (one
// u32x4), fp32 accumulate via v_dot2_f32_bf16.
__device__ __forceinline__ float dot8_e4m3_bf16(uint32_t w0, uint32_t w1, u32x4 x, float acc) {
  acc = __builtin_amdgcn_fdot2_f32_bf16(e4m3x2_lo_bf16(w0), as_bf2(x.x), acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(e4m3x2_hi_bf16(w0), as_bf2(x.y), acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(e4m3x2_lo_bf16(w1), as_bf2(x.z), acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(e4m3x2_hi_bf16(w1), as_bf2(x.w), acc, false);
  return acc;
}
// Dot product of 8 bf16 weights with 8 bf16 activations.
__device__ __forceinline__ float dot8_bf16(u32x4 w, u32x4 x, float acc) {
  acc = __builtin_amdgcn_fdot2_f32_bf16(as_bf2(w.x), as_bf2(x.x), acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(as_bf2(w.y), as_bf2(x.y), acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(as_bf2(w.z), as_bf2(x.z), acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(as_bf2(w.w), as_bf2(x.w), acc, false);
  return acc;
}

// ---- reductions -------------------------------------------------------------
// wave_sum / wave_max (defined after the DPP helpers below) reduce over all 64
// lanes and return the result in every lane; the whole wave must be active.
// Sum of the 64 lanes' values as a wave-uniform result, with DPP moves only
// (no LDS traffic): pairs (quad_perm xor 1, xor 2), then row_half_mirror and
// row_mirror give every lane its 16-lane row sum, then row_bcast:15 and
// row_bcast:31 fold the four rows into lane 63, which is read back.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_src(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL,
                                                               ROW_MASK, 0xF, false));
}
__device__ __forceinline__ float wave_total(float v) {
  v += dpp_src<0xB1, 0xF>(v);   // quad_perm [1,0,3,2]
  v += dpp_src<0x4E, 0xF>(v);   // quad_perm [2,3,0,1]
  v += dpp_src<0x141, 0xF>(v);  // row_half_mirror
  v += dpp_src<0x140, 0xF>(v);  // row_mirror
  v += dpp_src<0x142, 0xA>(v);  // row_bcast:15 into rows 1 and 3
  v += dpp_src<0x143, 0xC>(v);  // row_bcast:31 into rows 2 and 3
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}
// Maximum over the wave by the same DPP steps as wave_total; lanes the two
// row broadcasts leave out take -inf (the identity), not 0.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_src_or(float v, float old) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, old),
                                                               __builtin_bit_cast(int, v), CTRL,
                                                               ROW_MASK, 0xF, false));
}
__device__ __forceinline__ float wave_max_dpp(float v) {
  const float ninf = -__builtin_inff();
  v = fmaxf(v, dpp_src_or<0xB1, 0xF>(v, ninf));
  v = fmaxf(v, dpp_src_or<0x4E, 0xF>(v, ninf));
  v = fmaxf(v, dpp_src_or<0x141, 0xF>(v, ninf));
  v = fmaxf(v, dpp_src_or<0x140, 0xF>(v, ninf));
  v = fmaxf(v, dpp_src_or<0x142, 0xA>(v, ninf));
  v = fmaxf(v, dpp_src_or<0x143, 0xC>(v, ninf));
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}
// Sum over aligned groups of L consecutive lanes (L = 8 or 16), in every lane
// of the group: DPP quad swaps, then half-row and row mirrors.
template <int L>
__device__ __forceinline__ float column_sum(float x) {
  static_assert(L == 8 || L == 16, "group of 8 or 16 lanes");
  x += dpp_src<0xB1, 0xF>(x);   // quad_perm [1,0,3,2]
  x += dpp_src<0x4E, 0xF>(x);   // quad_perm [2,3,0,1]
  x += dpp_src<0x141, 0xF>(x);  // row_half_mirror
  if constexpr (L == 16) x += dpp_src<0x140, 0xF>(x);  // row_mirror
  return x;
}
// Full-wave sum and maximum through DPP: each step is a modifier on the add or
// max, where a butterfly of __shfl_xor calls costs six dependent LDS-crossbar
// permutes (measured: decode attention at context 4096 21.3 -> 20.0 us).
__device__ __forceinline__ float wave_sum(float v) { return wave_total(v); }
__device__ __forceinline__ float wave_max(float v) { return wave_max_dpp(v); }
// Sum over aligned groups of `G` lanes (G a power of two <= 64).
template <int G>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
  for (int o = G / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, QH_WAVE);
  return v;
}

// Block-wide sum for an NT-thread block; `red` must hold >= NT/64 floats of LDS.
// One barrier: the caller must pass a workgroup barrier after reading the
// result and before the next block_sum / block_sum_256 on the same `red`.
template <int NT>
__device__ __forceinline__ float block_sum(float v, float* red) {
  v = wave_sum(v);
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  if (lane == 0) red[wid] = v;
  __syncthreads();
  float s = 0.0f;
#pragma unroll
  for (int w = 0; w < NT / 64; ++w) s += red[w];
  return s;
}

// Block-wide sum for a 256-thread block; `red` must hold >= 4 floats of LDS.
// Same single-barrier contract as block_sum.
__device__ __forceinline__ float block_sum_256(float v, float* red) {
  v = wave_sum(v);
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  if (lane == 0) red[wid] = v;
  __syncthreads();
  return red[0] + red[1] + red[2] + red[3];
}

// ---- cross-workgroup hand-off ---------------------------------------------
// A kernel's workgroups publish partial results to the last one to finish.
// __threadfence() would write back and invalidate the whole L2 of the XCD
// (buffer_wbl2 / buffer_inv) in every workgroup.  Instead the published values
// are device-scope atomic stores and loads (coherent across XCDs without any
// cache maintenance); the publisher waits for its stores to complete before
// it increments the arrival counter, so the last arriver reads them all.
__device__ __forceinline__ void pub_store(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void pub_store(int* p, int v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float pub_load(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int pub_load(const int* p) {
  return __hip_atomic_load(const_cast<int*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Wait until this wave's outstanding memory operations have completed.
__device__ __forceinline__ void wait_mem() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }
// Called by every thread of the block after it published its values: returns
// true in the last block to arrive.  The counter returns to zero for the next
// launch (the last block resets it).
__device__ __forceinline__ bool arrive_last(unsigned* counter, unsigned n_blocks, int* s_flag) {
  wait_mem();
  __syncthreads();
  if (threadIdx.x == 0) {
    const unsigned prev = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *s_flag = prev == n_blocks - 1;
  }
  __syncthreads();
  return *s_flag != 0;
}
__device__ __forceinline__ void reset_counter(unsigned* counter) {
  __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---- math --------------------------------------------------------------------
// The logistic functions use the accurate exponential (expf, about one ulp):
// their results feed bf16 roundings and the GatedDeltaNet recurrent state,
// where the fast hardware exponential's larger error shows up as rounding
// flips and a per-step bias against the reference's fp32 torch ops.
__device__ __forceinline__ float qh_sigmoid(float x) { return 1.0f / (1.0f + expf(-x)); }
__device__ __forceinline__ float qh_silu(float x) { return x / (1.0f + expf(-x)); }
// SiLU on the fast exponential, for per-element loops on a kernel's critical
// path (the gated RMSNorm prologue of the decode output projection).
// The reciprocal is the hardware v_rcp_f32 (about 1 ulp) in place of the IEEE
// division's ten-instruction sequence; callers round the result to bf16.
__device__ __forceinline__ float qh_silu_fast(float x) {
  return x * __builtin_amdgcn_rcpf(1.0f + __expf(-x));
}
// torch.nn.functional.softplus(beta=1, threshold=20)
__device__ __forceinline__ float qh_softplus(float x) {
  return x > 20.0f ? x : log1pf(expf(x));
}

// ---- scale addressing ----------------------------------------------------
// Scale-mode encoding of the reference ABI (`K_blocks` argument):
//   kb > 1  : 128x128 block scales, shape [ceil(N/128), kb]
//   kb == 1 : one scale per output row, shape [N]
//   kb < 0  : per-row-per-block scales, shape [N, -kb]
__device__ __forceinline__ int scale_index(int kb_code, int row, int kblk) {
  if (kb_code > 1) return (row >> 7) * kb_code + kblk;
  if (kb_code == 1) return row;
  return row * (-kb_code) + kblk;
}
template <typename ScaleT> __device__ __forceinline__ float load_scale(const ScaleT* s, int i);
template <> __device__ __forceinline__ float load_scale<float>(const float* s, int i) { return s[i]; }
template <> __device__ __forceinline__ float load_scale<uint16_t>(const uint16_t* s, int i) {
  return bf2f(s[i]);
}
