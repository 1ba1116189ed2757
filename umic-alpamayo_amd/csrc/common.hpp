// Shared device helpers for the UMIC gfx950 kernels: bf16 bit handling,
// 16-byte vector access, wavefront reductions and launch-time argument
// checks.  Everything here is written for CDNA4 (64-lane wavefronts).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/umic_hip.h"

namespace umic {

constexpr int kWave = 64;

// Native 16-byte vector (clang ext_vector) -- the unit of every coalesced
// global access below (one global_load/store_dwordx4 per lane).
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));  // 8-byte accesses

// ---- bf16 <-> fp32 --------------------------------------------------------
// bf16 values travel as raw 16-bit patterns packed two per 32-bit word
// (element 2i in the low half, 2i+1 in the high half, little-endian order).

__device__ __forceinline__ float bf_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ float bf2f(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

// Round-to-nearest-even fp32 -> bf16 -- the rounding every eager bf16 op
// ends with (torch's c10::BFloat16 conversion).  gfx950 does it in hardware:
// v_cvt_pk_bf16_f32 converts two floats per instruction under the default
// round-to-nearest-even mode with fp32 denormals preserved, which is what
// clang emits for a float -> __bf16 conversion.  (A NaN input yields a quiet
// NaN; only its payload bits may differ from torch's.)
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  const f32x2_t v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

__device__ __forceinline__ uint32_t f2bf(float f) {
  return (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)f);
}

// fp32 value of bf16(f)
__device__ __forceinline__ float rbf(float f) { return (float)(__bf16)f; }

// rbf of two values through one paired conversion (v_cvt_pk_bf16_f32 and two
// extractions: three VALU instructions where two rbf take four)
__device__ __forceinline__ void rbf2(float& a, float& b) {
  const uint32_t w = pack2(a, b);
  a = bf_lo(w);
  b = bf_hi(w);
}

// 4 bf16 values <-> 4 floats
__device__ __forceinline__ void unpack4(const u32x2& v, float f[4]) {
  f[0] = bf_lo(v.x); f[1] = bf_hi(v.x);
  f[2] = bf_lo(v.y); f[3] = bf_hi(v.y);
}

__device__ __forceinline__ u32x2 pack4(const float f[4]) {
  u32x2 v;
  v.x = pack2(f[0], f[1]);
  v.y = pack2(f[2], f[3]);
  return v;
}

// 8 bf16 values <-> 8 floats
__device__ __forceinline__ void unpack8(const u32x4& v, float f[8]) {
  f[0] = bf_lo(v.x); f[1] = bf_hi(v.x);
  f[2] = bf_lo(v.y); f[3] = bf_hi(v.y);
  f[4] = bf_lo(v.z); f[5] = bf_hi(v.z);
  f[6] = bf_lo(v.w); f[7] = bf_hi(v.w);
}

__device__ __forceinline__ u32x4 pack8(const float f[8]) {
  u32x4 v;
  v.x = pack2(f[0], f[1]);
  v.y = pack2(f[2], f[3]);
  v.z = pack2(f[4], f[5]);
  v.w = pack2(f[6], f[7]);
  return v;
}

// ---- division by a launch-uniform divisor ---------------------------------
// q = n / d and r = n - q * d for 0 <= n < 2^22 and 1 <= d < 2^22, with
// inv = 1.0f / d rounded on the host: (float)n * inv differs from n / d by
// two roundings of relative size <= 2^-24, so by less than n * 2^-23 < 0.5,
// and truncating it gives q - 1, q or q + 1; one correction step makes it
// exact.  About eight VALU instructions, against a few dozen for a 32-bit
// and many more for a 64-bit integer division.
struct SmallDiv {
  int d;
  float inv;
};

inline SmallDiv small_div(int d) { return SmallDiv{d, 1.0f / (float)d}; }

__device__ __forceinline__ int div_small(const SmallDiv& s, int n, int& r) {
  int q = (int)((float)n * s.inv);
  r = n - q * s.d;
  if (r < 0) {
    q -= 1;
    r += s.d;
  }
  if (r >= s.d) {
    q += 1;
    r -= s.d;
  }
  return q;
}

// ---- streaming global access ---------------------------------------------
// Activations are touched exactly once per kernel: load/store them with the
// non-temporal hint so they do not evict reused data (weights, cos/sin).

__device__ __forceinline__ u32x4 ld_stream(const u32x4* p) {
  return __builtin_nontemporal_load(p);
}
__device__ __forceinline__ void st_stream(u32x4* p, const u32x4& v) {
  __builtin_nontemporal_store(v, p);
}

// ---- wavefront reductions -------------------------------------------------
// Butterfly sum over aligned groups of G lanes (G a power of two <= 64);
// every lane of the group ends with the group total.

// Inside a 16-lane row the steps are DPP moves (full-rate VALU, no LDS
// crossbar): quad_perm lane ^ 1 and ^ 2; after those every lane of a quad
// holds the quad sum, so row_half_mirror (lane -> 7 - lane) and row_mirror
// (lane -> 15 - lane) add the partner quad and half-row.  G = 32, 64 finish
// with shuffles.  The result is the same sum combined in another order.
template <int CTRL>
__device__ __forceinline__ float dpp_move(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
template <int CTRL>
__device__ __forceinline__ double dpp_move(double v) {
  const int lo = __builtin_amdgcn_update_dpp(0, __double2loint(v), CTRL, 0xF, 0xF, false);
  const int hi = __builtin_amdgcn_update_dpp(0, __double2hiint(v), CTRL, 0xF, 0xF, false);
  return __hiloint2double(hi, lo);
}

template <int G, typename T>
__device__ __forceinline__ T group_sum_dpp(T v) {
  static_assert(G >= 1 && G <= 64 && (G & (G - 1)) == 0, "G: a power of two up to 64");
  if constexpr (G >= 2) v += dpp_move<0xB1>(v);   // quad_perm [1,0,3,2]
  if constexpr (G >= 4) v += dpp_move<0x4E>(v);   // quad_perm [2,3,0,1]
  if constexpr (G >= 8) v += dpp_move<0x141>(v);  // row_half_mirror
  if constexpr (G >= 16) v += dpp_move<0x140>(v); // row_mirror
#pragma unroll
  for (int m = 16; m < G; m <<= 1) v += __shfl_xor(v, m, kWave);
  return v;
}

template <int G>
__device__ __forceinline__ double group_sum(double v) { return group_sum_dpp<G>(v); }

template <int G>
__device__ __forceinline__ float group_sum(float v) { return group_sum_dpp<G>(v); }

// Correctly rounded fp32 1/sqrt(v).  For a positive normal v the hardware
// estimate y = v_rsq_f32(v) is within an ulp, so the result is y or a
// neighbour, and the midpoint m between y and a neighbour decides:
// 1/sqrt(v) > m exactly when v * m^2 < 1, and fma(v, m * m, -1) in double has
// that sign exactly (m has at most 25 significant bits, so m * m is exact, and
// the fma rounds once).  1/sqrt(v) never equals a midpoint (v would be 1/m^2,
// not a float).  Inputs below the normal range are scaled by 2^64 and the
// result by 2^32 (both exact); zero, infinities, NaN and negatives come out of
// the estimate unchanged.  Selects, no branches: a branch here sat between a
// row's stores and cost add+RMSNorm 4%.  Checked on MI355X against
// (float)(1.0 / sqrt((double)v)) for every non-negative finite float and the
// special values: identical, at about a third of that quotient's fp64 work.
__device__ __forceinline__ float rsqrt_cr(float v) {
  const bool tiny = v < 0x1p-126f;
  const float vs = tiny ? v * 0x1p64f : v;
  const float y = __builtin_amdgcn_rsqf(vs);
  const uint32_t yb = __float_as_uint(y);
  const float up = __uint_as_float(yb + 1u), dn = __uint_as_float(yb - 1u);
  const double vd = vs, yd = y;
  const double mu = 0.5 * (yd + (double)up), md = 0.5 * (yd + (double)dn);
  const bool go_up = __builtin_fma(vd, mu * mu, -1.0) < 0.0;
  const bool go_dn = __builtin_fma(vd, md * md, -1.0) > 0.0;
  const float r = go_up ? up : go_dn ? dn : y;
  return tiny ? r * 0x1p32f : r;
}

// ---- torch's reduction plan for the RMSNorm statistic (host side) --------

// setReduceConfig (Reduce.cuh) for a contiguous fp32 [rows, n] tensor reduced
// over its last dim on a 64-lane, 512-threads-per-block device: vec = the
// threads read 4-element vectors (n >= 128), bw threads across a row, bh the
// block height, split = the row is also divided over the bh wavefronts.
struct RmsPlan {
  int vec, bw, bh, split;
};

inline int last_pow2(int64_t v) {
  int p = 1;
  while ((int64_t)p * 2 <= v) p *= 2;
  return p;
}

// false when torch would also split rows across blocks (n >= 131072)
inline bool rms_plan(int64_t rows, int64_t n, RmsPlan& p) {
  constexpr int kMaxThreads = 512;
  int64_t dim0 = n;
  p.vec = dim0 >= 128;
  if (p.vec) dim0 /= 4;
  const int d0 = dim0 < kMaxThreads ? last_pow2(dim0) : kMaxThreads;
  const int d1 = rows < kMaxThreads ? last_pow2(rows) : kMaxThreads;
  int bw = d0 < kWave ? d0 : kWave;
  const int bh = d1 < kMaxThreads / bw ? d1 : kMaxThreads / bw;
  bw = d0 < kMaxThreads / bh ? d0 : kMaxThreads / bh;
  const int64_t vpt = (n + bw - 1) / bw;
  p.bw = bw;
  p.bh = bh;
  p.split = vpt >= (bh * 16 < 256 ? bh * 16 : 256);
  return !(p.split && (n + (int64_t)bw * bh - 1) / ((int64_t)bw * bh) >= 256);
}

// ---- host-side argument checks -------------------------------------------

inline bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }
inline bool aligned8(const void* p) { return ((uintptr_t)p & 7u) == 0; }

// Byte ranges [a, a + na) and [b, b + nb) share a byte.
inline bool overlaps(const void* a, int64_t na, const void* b, int64_t nb) {
  const uintptr_t x = (uintptr_t)a, y = (uintptr_t)b;
  return na > 0 && nb > 0 && x < y + (uintptr_t)nb && y < x + (uintptr_t)na;
}

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// Status of the launch just enqueued (0 on success).
inline int launch_status() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? UMIC_OK : (int)e;
}

}  // namespace umic
