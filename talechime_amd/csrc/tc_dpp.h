// tc_dpp.h -- wave64 cross-lane primitives built on DPP and ds_swizzle.
//
// __shfl_* lowers to ds_bpermute, an LDS round trip per step; long chains of
// them (scans, sorts) dominate a latency-bound row kernel.  Within a row of
// 16 lanes DPP moves operands for free as an instruction modifier; across
// rows the scans use row_bcast15/row_bcast31, reductions read the four row
// results with v_readlane, and the xor exchanges of 4/8/16 lanes use
// ds_swizzle (no address operand).  Only the xor-32 exchange of the sorts
// remains a ds_bpermute.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tc {

// DPP controls (GFX9 encoding)
constexpr int kDppXor1 = 0xB1;   // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;   // quad_perm [2,3,0,1]
constexpr int kDppRowShr1 = 0x111, kDppRowShr2 = 0x112, kDppRowShr4 = 0x114, kDppRowShr8 = 0x118;
constexpr int kDppWaveShr1 = 0x138;
constexpr int kDppRowMirror = 0x140, kDppRowHalfMirror = 0x141;
constexpr int kDppBcast15 = 0x142, kDppBcast31 = 0x143;

template <int CTRL, int ROW_MASK = 0xf, bool BC = true>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
  // lanes whose source is outside the pattern (or whose row is masked off) read 0
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, ROW_MASK, 0xf, BC);
}
template <int CTRL, int ROW_MASK = 0xf, bool BC = true>
__device__ __forceinline__ float dpp_f32(float v) {
  return __uint_as_float(dpp_u32<CTRL, ROW_MASK, BC>(__float_as_uint(v)));
}
template <int CTRL, int ROW_MASK = 0xf, bool BC = true>
__device__ __forceinline__ double dpp_f64(double v) {
  const uint64_t b = (uint64_t)__double_as_longlong(v);
  const uint32_t lo = dpp_u32<CTRL, ROW_MASK, BC>((uint32_t)b), hi = dpp_u32<CTRL, ROW_MASK, BC>((uint32_t)(b >> 32));
  return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}

__device__ __forceinline__ uint32_t rl_u32(uint32_t v, int l) { return (uint32_t)__builtin_amdgcn_readlane((int)v, l); }
__device__ __forceinline__ float rl_f32(float v, int l) { return __uint_as_float(rl_u32(__float_as_uint(v), l)); }
__device__ __forceinline__ uint64_t rl_u64(uint64_t v, int l) {
  return ((uint64_t)rl_u32((uint32_t)(v >> 32), l) << 32) | rl_u32((uint32_t)v, l);
}
__device__ __forceinline__ double rl_f64(double v, int l) {
  const uint64_t b = (uint64_t)__double_as_longlong(v);
  return __longlong_as_double((long long)(((uint64_t)rl_u32((uint32_t)(b >> 32), l) << 32) | rl_u32((uint32_t)b, l)));
}

// ---------------------------------------------------------------- reductions (every lane gets the result)
// Inside each row of 16: xor 1, xor 2, half mirror, mirror; then the four row
// results combine in row order.
#define TC_ROW_REDUCE(T, v, OP, DPP)                 \
  v = OP(v, DPP<kDppXor1, 0xf, false>(v));           \
  v = OP(v, DPP<kDppXor2, 0xf, false>(v));           \
  v = OP(v, DPP<kDppRowHalfMirror, 0xf, false>(v));  \
  v = OP(v, DPP<kDppRowMirror, 0xf, false>(v));

__device__ __forceinline__ float fmax_nan_last(float a, float b) { return a > b ? a : b; }
__device__ __forceinline__ float dpp_wave_max(float v) {
  TC_ROW_REDUCE(float, v, fmax_nan_last, dpp_f32)
  const float a = fmax_nan_last(rl_f32(v, 0), rl_f32(v, 16)), b = fmax_nan_last(rl_f32(v, 32), rl_f32(v, 48));
  return fmax_nan_last(a, b);
}
__device__ __forceinline__ float add_f(float a, float b) { return a + b; }
__device__ __forceinline__ float dpp_wave_sum(float v) {
  TC_ROW_REDUCE(float, v, add_f, dpp_f32)
  return (rl_f32(v, 0) + rl_f32(v, 16)) + (rl_f32(v, 32) + rl_f32(v, 48));
}
__device__ __forceinline__ double add_d(double a, double b) { return a + b; }
__device__ __forceinline__ double dpp_wave_sum_d(double v) {
  TC_ROW_REDUCE(double, v, add_d, dpp_f64)
  return (rl_f64(v, 0) + rl_f64(v, 16)) + (rl_f64(v, 32) + rl_f64(v, 48));
}
__device__ __forceinline__ double max_d(double a, double b) { return a > b ? a : b; }
__device__ __forceinline__ double dpp_wave_max_d(double v) {
  TC_ROW_REDUCE(double, v, max_d, dpp_f64)
  return max_d(max_d(rl_f64(v, 0), rl_f64(v, 16)), max_d(rl_f64(v, 32), rl_f64(v, 48)));
}
__device__ __forceinline__ uint32_t or_u(uint32_t a, uint32_t b) { return a | b; }
__device__ __forceinline__ uint32_t dpp_wave_or(uint32_t v) {
  TC_ROW_REDUCE(uint32_t, v, or_u, dpp_u32)
  return (rl_u32(v, 0) | rl_u32(v, 16)) | (rl_u32(v, 32) | rl_u32(v, 48));
}
#undef TC_ROW_REDUCE

// ---------------------------------------------------------------- inclusive scans (lane order)
__device__ __forceinline__ uint32_t dpp_scan_u32(uint32_t v) {
  v += dpp_u32<kDppRowShr1>(v);
  v += dpp_u32<kDppRowShr2>(v);
  v += dpp_u32<kDppRowShr4>(v);
  v += dpp_u32<kDppRowShr8>(v);
  v += dpp_u32<kDppBcast15, 0xa, false>(v);
  v += dpp_u32<kDppBcast31, 0xc, false>(v);
  return v;
}
__device__ __forceinline__ float dpp_scan_f32(float v) {
  v += dpp_f32<kDppRowShr1>(v);
  v += dpp_f32<kDppRowShr2>(v);
  v += dpp_f32<kDppRowShr4>(v);
  v += dpp_f32<kDppRowShr8>(v);
  v += dpp_f32<kDppBcast15, 0xa, false>(v);
  v += dpp_f32<kDppBcast31, 0xc, false>(v);
  return v;
}
__device__ __forceinline__ double dpp_scan_f64(double v) {
  v += dpp_f64<kDppRowShr1>(v);
  v += dpp_f64<kDppRowShr2>(v);
  v += dpp_f64<kDppRowShr4>(v);
  v += dpp_f64<kDppRowShr8>(v);
  v += dpp_f64<kDppBcast15, 0xa, false>(v);
  v += dpp_f64<kDppBcast31, 0xc, false>(v);
  return v;
}
// The value of the previous lane (lane 0 reads 0).
__device__ __forceinline__ uint32_t dpp_prev_u32(uint32_t v) { return dpp_u32<kDppWaveShr1>(v); }
__device__ __forceinline__ float dpp_prev_f32(float v) { return dpp_f32<kDppWaveShr1>(v); }

// ---------------------------------------------------------------- xor exchanges
template <int J>
__device__ __forceinline__ uint32_t xchg_u32(uint32_t v) {
  static_assert(J == 1 || J == 2 || J == 4 || J == 8 || J == 16 || J == 32, "xor distance");
  if constexpr (J == 1) return dpp_u32<kDppXor1, 0xf, false>(v);
  else if constexpr (J == 2) return dpp_u32<kDppXor2, 0xf, false>(v);
  else if constexpr (J == 32) return (uint32_t)__builtin_amdgcn_ds_bpermute((int)((threadIdx.x ^ 32u) << 2), (int)v);
  else return (uint32_t)__builtin_amdgcn_ds_swizzle((int)v, (J << 10) | 0x1f);
}
template <int J>
__device__ __forceinline__ uint64_t xchg_u64(uint64_t v) {
  return ((uint64_t)xchg_u32<J>((uint32_t)(v >> 32)) << 32) | xchg_u32<J>((uint32_t)v);
}

// Bitonic sort of 64*S 64-bit keys into descending order; element i lives in
// lane i % 64 of slot i / 64.
template <int S, int K, int J>
__device__ __forceinline__ void bitonic_step(uint64_t (&v)[S]) {
  const int lane = threadIdx.x & 63;
  if constexpr (J >= 64) {
    constexpr int js = J / 64;
#pragma unroll
    for (int sl = 0; sl < S; ++sl) {
      if (sl & js) continue;
      const int i = sl * 64 + lane;
      const bool desc = (i & K) == 0;
      const uint64_t x = v[sl], y = v[sl + js];
      const uint64_t hi = x > y ? x : y, lo = x > y ? y : x;
      v[sl] = desc ? hi : lo;
      v[sl + js] = desc ? lo : hi;
    }
  } else {
#pragma unroll
    for (int sl = 0; sl < S; ++sl) {
      const int i = sl * 64 + lane;
      const uint64_t o = xchg_u64<J>(v[sl]);
      const bool take_max = ((i & J) == 0) == ((i & K) == 0);
      v[sl] = take_max ? (o > v[sl] ? o : v[sl]) : (o < v[sl] ? o : v[sl]);
    }
  }
}
template <int S, int K, int J>
__device__ __forceinline__ void bitonic_merge_steps(uint64_t (&v)[S]) {
  bitonic_step<S, K, J>(v);
  if constexpr (J > 1) bitonic_merge_steps<S, K, J / 2>(v);
}
template <int S, int K>
__device__ __forceinline__ void bitonic_stages(uint64_t (&v)[S]) {
  bitonic_merge_steps<S, K, K / 2>(v);
  if constexpr (K < 64 * S) bitonic_stages<S, K * 2>(v);
}
template <int S>
__device__ __forceinline__ void dpp_sort_desc_u64(uint64_t (&v)[S]) {
  bitonic_stages<S, 2>(v);
}

}  // namespace tc
