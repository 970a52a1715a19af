// tc_seqsum.h -- exact emulation, across a workgroup, of a sequential f32 sum
// of non-negative terms (s = -0.0; for each term in order: s = s + t).
//
// The reference samplers accumulate softmax denominators and CDFs with one
// f32 add per element in element order; every add rounds.  Doing the adds one
// by one on the GPU costs one dependent add per element.  This header gets
// the identical bits with a scan:
//
//   * While the running sum s lies in one binade [2^e, 2^(e+1)), every
//     representable value there is a multiple of u = 2^(e-23), so adding a
//     term t rounds to s + r*u with r = round(t / u) -- unless t/u ends in
//     exactly .5 (a tie, settled by the parity of s), or the result leaves
//     the binade.
//   * A double prefix sum P_j of the terms predicts where s_j lies.  The
//     sequential sum after j+1 adds differs from the exact one by less than
//     (j+1) * 2^-24 relative (each add errs by at most half an ulp of its
//     result, which is at most 2^-24 of the final sum), and the terms the
//     prediction uses are themselves within a known number of ulps.  An
//     element is "safe" when both the sum before it and after it are proven
//     to lie inside one binade; its contribution is then the integer r.
//   * Unsafe elements (the first positive term, elements near a binade
//     crossing, ties) are collected in element order.  Between two unsafe
//     elements all safe elements share one binade, so one lane walks the
//     unsafe list: s += (sum of r since the last unsafe element) ulps, which
//     is an integer add on the bit pattern, then s = s + t in f32.
//
// Approximate terms are allowed: an approximate term decides r only when the
// exact term cannot lie across a rounding midpoint of the grid; otherwise,
// and for every unsafe element, the exact term is computed.
#pragma once

#include "tc_device.h"

namespace tc {

struct SeqLds {
  static constexpr int kCap = 512;
  float a[kCap];        // exact term of each unsafe element, in element order
  float s_after[kCap];  // running sum after each unsafe element (walk output)
  long long q[kCap];    // sum of r over the safe elements before it
  long long qtot;
  uint32_t n;
  uint32_t bad;
  float S;
};

// Per-thread state kept for prefix queries after the walk.
template <int ITEMS>
struct SeqThread {
  uint32_t unsafe;    // bit i: element i is in the unsafe list
  int r[ITEMS];       // contribution of each safe element, in ulps of its binade
  uint32_t u_base;    // index in the unsafe list of this thread's first unsafe element
  long long q_base;   // sum of r over the safe elements before this thread
};

__device__ __forceinline__ float add_ulps(float s, long long d) {
  return d == 0 ? s : u2f(f2u(s) + (uint32_t)d);
}

// r = round(a / 2^g) when it is not a tie; returns false on a tie.
__device__ __forceinline__ bool grid_round(float a, int g, int* r) {
  double q = ldexp((double)a, -g);
  double fl = floor(q);
  double fr = q - fl;
  if (fr == 0.5) return false;
  *r = (int)fl + (fr > 0.5 ? 1 : 0);
  return true;
}

// Index-selected read and write of a register array without dynamic
// indexing (which would move the array to scratch memory).  Masks on the bit
// patterns rather than selects: a chain of selects between array elements
// can be folded into one load from a computed address, which forces the
// whole array into scratch for every path of the kernel.
template <int ITEMS>
__device__ __forceinline__ float pick_item(const float (&v)[ITEMS], int i) {
  uint32_t r = 0;
#pragma unroll
  for (int j = 0; j < ITEMS; ++j) r |= f2u(v[j]) & (0u - (uint32_t)(i == j));
  return u2f(r);
}
template <int ITEMS>
__device__ __forceinline__ void put_item(float (&v)[ITEMS], int i, float x) {
#pragma unroll
  for (int j = 0; j < ITEMS; ++j) {
    const uint32_t m = 0u - (uint32_t)(i == j);
    v[j] = u2f((f2u(v[j]) & ~m) | (f2u(x) & m));
  }
}

// Binade test and grid rounding of one element: returns 0 = safe (r set),
// 1 = the approximate term cannot decide r, 2 = unsafe.
__device__ __forceinline__ int classify_term(double P, double Pa, float a, bool exact, double tau, int err_ulps,
                                             int* r) {
  if (a == 0.0f && exact) {
    *r = 0;
    return 0;  // adding an exact zero never changes the sum
  }
  if (!(P > 0.0)) return 2;
  const int e = ilogb(P);
  const double lo = ldexp(1.0, e), hi = ldexp(1.0, e + 1);
  if (!(e >= -126 && P * (1.0 - tau) >= lo && Pa * (1.0 + tau) < hi * (1.0 - 0x1p-25))) return 2;
  const int g = e - 23;
  const double q = ldexp((double)a, -g);
  const double fl = floor(q);
  const double fr = q - fl;
  if (!exact) {
    // can the exact term lie across a midpoint of the grid?
    const int ea = a > 0.0f ? (ilogb(a) > -126 ? ilogb(a) : -126) : 0;
    const double rad = a > 0.0f ? ldexp((double)(2 * err_ulps + 2), ea - 23 - g) : 1.0;
    if (fabs(fr - 0.5) <= rad) return 1;
  }
  if (fr == 0.5) return 2;  // a tie: settled by the parity of the running sum
  *r = (int)fl + (fr > 0.5 ? 1 : 0);
  return 0;
}

// The exact sequential sum of the terms.  Thread t holds ITEMS terms at
// element positions pos0 + i (pos0 = t * ITEMS - shift; threads in order).
// ap[i]: the term, exact where bit i of `exact_mask` is set, otherwise within
// `err_ulps` ulps of f(in[i]), the exact term.  Invalid positions hold an
// exact 0.  On return ap holds the exact term of every element the sum
// needed exactly.  Returns false when more than SeqLds::kCap elements are
// unsafe (the caller then sums sequentially).
template <int ITEMS, class F>
__device__ __forceinline__ bool block_seqsum(float (&ap)[ITEMS], uint32_t exact_mask, const float (&in)[ITEMS], F f,
                                             int pos0, int err_ulps, SeqThread<ITEMS>& th, SeqLds& L, ScanLds& sc,
                                             float* S_out) {
  // 1. prediction: exclusive double prefix over threads
  double D = 0.0;
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) D += (double)ap[i];
  double Ptot;
  const double P0 = block_excl_scan_d(D, sc, &Ptot);
  // bound on the relative distance between the prediction and the running
  // sum, for every element of this thread
  const double tau = (double)(pos0 + ITEMS + 4) * 0x1p-24 * 1.001 + (double)(err_ulps + 2) * 0x1p-23;
  // 2. classify with the terms at hand
  uint32_t unsafe = 0, amb = 0;
  {
    double P = P0;
#pragma unroll
    for (int i = 0; i < ITEMS; ++i) {
      const double Pa = P + (double)ap[i];
      int r = 0;
      const int c = classify_term(P, Pa, ap[i], (exact_mask >> i) & 1u, tau, err_ulps, &r);
      th.r[i] = r;
      if (c == 1) amb |= 1u << i;
      if (c == 2) unsafe |= 1u << i;
      P = Pa;
    }
  }
  // 3. exact terms where the approximate ones cannot decide, and for every
  // unsafe element (one flagged item per lane per pass)
  uint32_t need = (amb | unsafe) & ~exact_mask;
  while (__ballot(need != 0u)) {
    if (need) {
      const int i = __builtin_ctz(need);
      put_item<ITEMS>(ap, i, f(pick_item<ITEMS>(in, i)));
      need &= need - 1u;
    }
  }
  exact_mask |= amb | unsafe;
  if (__ballot(amb != 0u)) {
    double P = P0;
#pragma unroll
    for (int i = 0; i < ITEMS; ++i) {
      const double Pa = P + (double)ap[i];
      if ((amb >> i) & 1u) {
        int r = 0;
        if (classify_term(P, Pa, ap[i], true, tau, err_ulps, &r) != 0) unsafe |= 1u << i;
        th.r[i] = r;
      }
      P = Pa;
    }
  }
  long long rsum = 0;
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) {
    if ((unsafe >> i) & 1u) th.r[i] = 0;
    rsum += th.r[i];
  }
  th.unsafe = unsafe;
  // 4. list the unsafe elements in element order
  uint32_t u_off, u_tot;
  long long q_off, q_tot;
  block_excl_scan_cq(__builtin_popcount(unsafe), rsum, sc, &u_off, &q_off, &u_tot, &q_tot);
  th.u_base = u_off;
  th.q_base = q_off;
  u_tot = (uint32_t)__builtin_amdgcn_readfirstlane((int)u_tot);
  if (u_tot > (uint32_t)SeqLds::kCap) return false;
  {
    uint32_t k = u_off;
    long long q = q_off;
#pragma unroll
    for (int i = 0; i < ITEMS; ++i) {
      if ((unsafe >> i) & 1u) {
        L.a[k] = ap[i];
        L.q[k] = q;
        ++k;
      } else {
        q += th.r[i];
      }
    }
  }
  __syncthreads();
  // 5. the walk (wave 0; every lane carries the same running sum)
  if (wave_id() == 0) {
    const int lane = lane_id();
    float s = -0.0f;
    long long qp = 0;
    uint32_t bad = 0;
    for (uint32_t base = 0; base < u_tot; base += kWave) {
      const uint32_t k = base + lane;
      const float ak = k < u_tot ? L.a[k] : 0.0f;
      const long long qk = k < u_tot ? L.q[k] : 0;
      float sk = 0.0f;
      const uint32_t m = u_tot - base < (uint32_t)kWave ? u_tot - base : (uint32_t)kWave;
      for (uint32_t j = 0; j < m; ++j) {
        const long long qj = (long long)readlane_u64((uint64_t)qk, j);
        const long long d = qj - qp;
        if (d != 0) {
          const float s2 = add_ulps(s, d);
          if (!(s > 0.0f) || (f2u(s2) >> 23) != (f2u(s) >> 23)) bad = 1;
          s = s2;
        }
        s = s + readlane_f32(ak, j);
        qp = qj;
        if ((uint32_t)lane == j) sk = s;
      }
      if (k < u_tot) L.s_after[k] = sk;
    }
    const long long d = q_tot - qp;
    if (d != 0) {
      const float s2 = add_ulps(s, d);
      if (!(s > 0.0f) || (f2u(s2) >> 23) != (f2u(s) >> 23)) bad = 1;
      s = s2;
    }
    if (lane == 0) {
      L.S = s;
      L.n = u_tot;
      L.qtot = q_tot;
      L.bad = bad;
    }
  }
  __syncthreads();
  *S_out = L.S;
  return true;
}

// Running sum after each of the thread's elements (inclusive prefix), from
// the state block_seqsum left behind.
template <int ITEMS>
__device__ __forceinline__ void seq_prefix(const SeqThread<ITEMS>& th, const SeqLds& L, float (&pre)[ITEMS]) {
  uint32_t k = th.u_base;
  long long q = th.q_base;
  float base = k == 0 ? -0.0f : L.s_after[k - 1];
  long long qb = k == 0 ? 0 : L.q[k - 1];
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) {
    if ((th.unsafe >> i) & 1u) {
      base = L.s_after[k];
      qb = L.q[k];
      ++k;
      pre[i] = base;
    } else {
      q += th.r[i];
      pre[i] = add_ulps(base, q - qb);
    }
  }
}

// Fallback: the sequential sum done literally by one lane over LDS-staged
// chunks of exact terms.  `stage` holds at least kChunk floats.
template <int ITEMS>
__device__ __forceinline__ float block_seqsum_slow(const float (&ex)[ITEMS], int pos0, int n, float* stage, int kChunk,
                                   volatile float* out) {
  float s = -0.0f;
  if (threadIdx.x == 0) *out = s;
  for (int c0 = 0; c0 < n; c0 += kChunk) {
#pragma unroll
    for (int i = 0; i < ITEMS; ++i) {
      const int p = pos0 + i;
      if (p >= c0 && p < c0 + kChunk && p < n) stage[p - c0] = ex[i];
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      const int c1 = c0 + kChunk < n ? c0 + kChunk : n;
      for (int p = c0; p < c1; ++p) s = s + stage[p - c0];
      *out = s;
    }
    __syncthreads();
  }
  __syncthreads();
  return *out;
}

}  // namespace tc
