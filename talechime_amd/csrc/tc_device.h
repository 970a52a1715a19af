// tc_device.h -- device building blocks for the row sampler kernels (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "tc_math.h"
#include "_gen/expf_glibc_exc.inc"
#include "_gen/logf_glibc_exc.inc"

namespace tc {

constexpr int kWave = 64;
constexpr int kMaxThreads = 1024;
constexpr int kMaxWaves = kMaxThreads / kWave;

__device__ __forceinline__ uint32_t f2u(float f) { return __float_as_uint(f); }
__device__ __forceinline__ float u2f(uint32_t u) { return __uint_as_float(u); }

// Unsigned key ordered like Rust's f32::total_cmp.
__device__ __forceinline__ uint32_t tkey(float f) {
  uint32_t b = f2u(f);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float untkey(uint32_t k) {
  return u2f((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}
// Key ordered like IEEE `<` on non-NaN floats (-0 and +0 share a key).
__device__ __forceinline__ uint32_t ckey(float f) { return f == 0.0f ? 0x80000000u : tkey(f); }

// Rust f32::max / f64::max (NaN operands ignored).
__device__ __forceinline__ float rmaxf(float a, float b) {
  return __builtin_isnan(a) ? b : (__builtin_isnan(b) ? a : (a > b ? a : b));
}
__device__ __forceinline__ double rmaxd(double a, double b) {
  return __builtin_isnan(a) ? b : (__builtin_isnan(b) ? a : (a > b ? a : b));
}

// exp(d) for d in [-87, 0], approximate: d * log2(e), with log2(e) in two
// floats, is p + e (p = the rounded product, e the rest to about 2^-48
// relative, by two fmas); v_exp_f32(p) corrected to first order by
// 1 + e ln 2.  Within 3 ulps of the correctly rounded value on every input of
// the range (checked on the device by tc_selftest_exp_approx; the result is
// normal, >= 2^-125.5), so within 4 ulps, 2^-21 relative, of glibc's expf.
__device__ __forceinline__ float exp_approx(float d) {
  constexpr float kL2eHi = 0x1.715476p+0f, kL2eLo = 0x1.4ae0cp-26f;
  const float p = d * kL2eHi;
  const float e = __builtin_fmaf(d, kL2eLo, __builtin_fmaf(d, kL2eHi, -p));
  return __builtin_amdgcn_exp2f(p) * __builtin_fmaf(e, 0.693147180559945309f, 1.0f);
}

// ---------------------------------------------------------------- glibc expf
// glibc's expf differs from the correctly rounded value only on the inputs in
// tc_expf_exc_keys, all of which sit within TC_EXPF_BAND ulp of a rounding
// midpoint; there it returns the neighbour on the far side of the midpoint.
__device__ __forceinline__ bool expf_is_exception(uint32_t b) {
  uint32_t h = b >> 16;
  uint32_t lo = tc_expf_exc_index[h], hi = tc_expf_exc_index[h + 1];
  while (lo < hi) {
    uint32_t mid = (lo + hi) >> 1;
    uint32_t k = tc_expf_exc_keys[mid];
    if (k == b) return true;
    if (k < b) lo = mid + 1;
    else hi = mid;
  }
  return false;
}

__device__ __forceinline__ float expf_glibc(float x) {
  if (__builtin_isnan(x)) return x;
  if (x < -104.0f) return 0.0f;
  if (x > 88.72283935546875f) return __builtin_inff();
  double y = tc_exp_d((double)x);
  float r = (float)y;
  if (tc_mid_dist(y, r) < TC_EXPF_BAND) {
    if (expf_is_exception(f2u(x))) r = u2f(tc_toward(y, r));
  }
  return r;
}

// expf_glibc of every lane's x, the lanes whose value lies in the band looked
// up one at a time by the whole wave: the bucket's index entries (one uniform
// load), then all of its keys at once (one load per lane) against the key,
// instead of a binary search of dependent loads.  Every lane active.
__device__ __forceinline__ float expf_glibc_wave(float x) {
  const bool mid = !__builtin_isnan(x) && x >= -104.0f && x <= 88.72283935546875f;
  const double y = tc_exp_d(mid ? (double)x : 0.0);
  float r = (float)y;
  const bool inb = mid && tc_mid_dist(y, r) < TC_EXPF_BAND;
  uint64_t need = __ballot(inb);
  const uint32_t lane = threadIdx.x & 63u;
  while (need) {
    const int l = __builtin_ctzll(need);
    need &= need - 1ull;
    const uint32_t b = (uint32_t)__builtin_amdgcn_readlane((int)f2u(x), l);
    const uint32_t lo = tc_expf_exc_index[b >> 16], hi = tc_expf_exc_index[(b >> 16) + 1u];
    bool exc = false;
    for (uint32_t base = lo; base < hi; base += 64u) {
      const uint32_t j = base + lane;
      const uint32_t k = j < hi ? tc_expf_exc_keys[j] : ~b;
      exc = exc || __ballot(k == b) != 0ull;
    }
    if (exc && lane == (uint32_t)l) r = u2f(tc_toward(y, r));
  }
  if (!mid) r = __builtin_isnan(x) ? x : (x < -104.0f ? 0.0f : __builtin_inff());
  return r;
}

// ---------------------------------------------------------------- glibc logf
// glibc's logf on [1, 2^24) differs from tc_logf_cr only on the inputs in
// tc_logf_exc_keys, all within TC_LOGF_BAND ulp of a rounding midpoint, where
// it returns the neighbour across the midpoint.  Keys are bucketed by
// (bits - bits(1.0f)) >> TC_LOGF_BUCKET_SHIFT.
__device__ __forceinline__ bool logf_is_exception(uint32_t b) {
  const uint32_t off = b - 0x3f800000u;
  const uint32_t bk = off >> TC_LOGF_BUCKET_SHIFT;
  if (bk >= TC_LOGF_NBUCKETS) return false;
  uint32_t lo = tc_logf_exc_index[bk], hi = tc_logf_exc_index[bk + 1];
  while (lo < hi) {
    uint32_t mid = (lo + hi) >> 1;
    uint32_t k = tc_logf_exc_keys[mid];
    if (k == b) return true;
    if (k < b) lo = mid + 1;
    else hi = mid;
  }
  return false;
}

// The exception keys of the buckets holding [s_lo, s_hi] in lane registers of
// one wave (lane j: key lo + j), fetched ahead of a logf_glibc_keys call
// whose argument is expected in that range: the index entries first
// (logf_keys_index), the keys once those have arrived (logf_keys_load).
// Every lane of the wave active throughout.
struct LogfKeys {
  uint32_t b0, nb, lo, n;  // wave-uniform
  uint32_t idx, key;       // per lane
  bool ok;
};
__device__ __forceinline__ void logf_keys_index(LogfKeys& K, float s_lo, float s_hi) {
  s_lo = s_lo > 1.0f ? s_lo : 1.0f;
  const uint32_t b0 = (f2u(s_lo) - 0x3f800000u) >> TC_LOGF_BUCKET_SHIFT;
  const uint32_t b1 = (f2u(s_hi) - 0x3f800000u) >> TC_LOGF_BUCKET_SHIFT;
  K.ok = s_hi >= s_lo && s_hi < 16777216.0f && b1 < TC_LOGF_NBUCKETS && b1 - b0 < 63u;
  K.b0 = b0;
  K.nb = b1 - b0 + 1u;
  const uint32_t j = threadIdx.x & 63u;
  K.idx = (K.ok && j <= K.nb) ? tc_logf_exc_index[b0 + j] : 0u;
}
__device__ __forceinline__ void logf_keys_load(LogfKeys& K) {
  if (K.ok) {
    K.lo = (uint32_t)__builtin_amdgcn_readlane((int)K.idx, 0);
    K.n = (uint32_t)__builtin_amdgcn_readlane((int)K.idx, (int)K.nb) - K.lo;
    K.ok = K.n <= 64u;
  }
  const uint32_t j = threadIdx.x & 63u;
  K.key = (K.ok && j < K.n) ? tc_logf_exc_keys[K.lo + j] : 0xffffffffu;  // a NaN: never a key
}

// Rust's f32::ln (glibc logf) for x in [1, 2^24); other inputs get the
// correctly rounded value.
__device__ __forceinline__ float logf_glibc(float x) {
  if (!(x >= 1.0f && x < 16777216.0f)) return tc_logf_cr(x);
  if (x == 1.0f) return 0.0f;
  double y = tc_log_d((double)x);
  float r = (float)y;
  if (tc_mid_dist(y, r) < TC_LOGF_BAND && logf_is_exception(f2u(x))) r = u2f(tc_toward(y, r));
  return r;
}
// The same with x wave-uniform and the keys of its bucket, when K covers it,
// read from K (every lane of the wave active).
__device__ __forceinline__ float logf_glibc_keys(float x, const LogfKeys& K) {
  if (!(x >= 1.0f && x < 16777216.0f)) return tc_logf_cr(x);
  if (x == 1.0f) return 0.0f;
  double y = tc_log_d((double)x);
  float r = (float)y;
  if (tc_mid_dist(y, r) < TC_LOGF_BAND) {
    const uint32_t b = f2u(x), bk = (b - 0x3f800000u) >> TC_LOGF_BUCKET_SHIFT;
    const bool exc = (K.ok && bk >= K.b0 && bk - K.b0 < K.nb) ? __ballot(K.key == b) != 0ull : logf_is_exception(b);
    if (exc) r = u2f(tc_toward(y, r));
  }
  return r;
}

// logf_glibc_keys(x, K) from ln_ref = tc_log_d(ref) and inv_ref = 1 / ref
// for a float ref near x: log x = ln_ref + log1p((x - ref) / ref), the series
// to the fifth power (|d| < 2^-10: the rest is below 2^-60).  This y and
// tc_log_d(x) are both within a few 2^-53 relative of log x, so they differ
// by less than err = 2^-48 (|ln_ref| + |log1p|): farther than err from a
// rounding midpoint both round alike, and every input whose tc_log_d lies
// inside the exception band lies within band + err here.  Near a midpoint,
// or with ref far from x, the reference computation.  x wave-uniform, every
// lane active.
__device__ __forceinline__ float logf_glibc_near(float x, float ref, double ln_ref, double inv_ref,
                                                 const LogfKeys& K) {
  if (!(x > 1.0f && x < 16777216.0f)) return logf_glibc_keys(x, K);
  const double dd = ((double)x - (double)ref) * inv_ref;
  if (!(__builtin_fabs(dd) < 0x1p-10)) return logf_glibc_keys(x, K);
  const double lp = dd * (1.0 - dd * (0.5 - dd * (1.0 / 3.0 - dd * (0.25 - dd * 0.2))));
  const double y = ln_ref + lp;
  const float r = (float)y;
  const uint32_t nbb = tc_toward(y, r);
  const double gap = __builtin_fabs((double)u2f(nbb) - (double)r), mid = 0.5 * ((double)u2f(nbb) + (double)r);
  const double dist = __builtin_fabs(y - mid), err = 0x1p-48 * (__builtin_fabs(ln_ref) + __builtin_fabs(lp));
  if (!(dist > err)) return logf_glibc_keys(x, K);
  if (dist < TC_LOGF_BAND * gap + err) {
    const uint32_t b = f2u(x), bk = (b - 0x3f800000u) >> TC_LOGF_BUCKET_SHIFT;
    const bool exc = (K.ok && bk >= K.b0 && bk - K.b0 < K.nb) ? __ballot(K.key == b) != 0ull : logf_is_exception(b);
    if (exc) return u2f(nbb);
  }
  return r;
}

// ---------------------------------------------------------------- wave / block
__device__ __forceinline__ int lane_id() { return threadIdx.x & (kWave - 1); }
__device__ __forceinline__ int wave_id() { return threadIdx.x >> 6; }
__device__ __forceinline__ int num_waves() { return blockDim.x >> 6; }

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = rmaxf(v, __shfl_xor(v, o));
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = v + __shfl_xor(v, o);
  return v;
}
__device__ __forceinline__ uint32_t wave_sum_u(uint32_t v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}
__device__ __forceinline__ uint32_t wave_or_u(uint32_t v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v |= __shfl_xor(v, o);
  return v;
}
__device__ __forceinline__ uint32_t wave_incl_scan(uint32_t v) {
  const int lane = lane_id();
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
    uint32_t t = __shfl_up(v, o);
    if (lane >= o) v += t;
  }
  return v;
}

struct BlockScratch {
  float f[kMaxWaves];
  uint32_t u[kMaxWaves + 16];
  double d[kMaxWaves];
};

// Max over the block (NaN ignored); every thread gets the result.
__device__ __forceinline__ float block_max(float v, BlockScratch& s) {
  v = wave_max(v);
  if (lane_id() == 0) s.f[wave_id()] = v;
  __syncthreads();
  float r = s.f[0];
  for (int w = 1; w < num_waves(); ++w) r = rmaxf(r, s.f[w]);
  __syncthreads();
  return r;
}

// Sum over the block: in-thread order, then a butterfly inside each wave, then
// the wave sums in wave order.  Deterministic for a fixed block shape.
__device__ __forceinline__ float block_sum(float v, BlockScratch& s) {
  v = wave_sum(v);
  if (lane_id() == 0) s.f[wave_id()] = v;
  __syncthreads();
  float r = s.f[0];
  for (int w = 1; w < num_waves(); ++w) r = r + s.f[w];
  __syncthreads();
  return r;
}

__device__ __forceinline__ double block_max_d(double v, BlockScratch& s) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = rmaxd(v, __shfl_xor(v, o));
  if (lane_id() == 0) s.d[wave_id()] = v;
  __syncthreads();
  double r = s.d[0];
  for (int w = 1; w < num_waves(); ++w) r = rmaxd(r, s.d[w]);
  __syncthreads();
  return r;
}

__device__ __forceinline__ uint32_t block_sum_u(uint32_t v, BlockScratch& s) {
  v = wave_sum_u(v);
  if (lane_id() == 0) s.u[wave_id()] = v;
  __syncthreads();
  uint32_t r = 0;
  for (int w = 0; w < num_waves(); ++w) r += s.u[w];
  __syncthreads();
  return r;
}

__device__ __forceinline__ uint32_t block_or_u(uint32_t v, BlockScratch& s) {
  v = wave_or_u(v);
  if (lane_id() == 0) s.u[wave_id()] = v;
  __syncthreads();
  uint32_t r = 0;
  for (int w = 0; w < num_waves(); ++w) r |= s.u[w];
  __syncthreads();
  return r;
}

// Exclusive prefix sum over threads in thread order; *total gets the sum.
__device__ __forceinline__ uint32_t block_excl_scan(uint32_t v, BlockScratch& s, uint32_t* total) {
  uint32_t inc = wave_incl_scan(v);
  if (lane_id() == kWave - 1) s.u[wave_id()] = inc;
  __syncthreads();
  uint32_t off = 0, tot = 0;
  for (int w = 0; w < num_waves(); ++w) {
    uint32_t t = s.u[w];
    if (w < wave_id()) off += t;
    tot += t;
  }
  __syncthreads();
  *total = tot;
  return off + inc - v;
}

__device__ __forceinline__ uint32_t block_min_u(uint32_t v, BlockScratch& s) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const uint32_t w = __shfl_xor(v, o);
    v = w < v ? w : v;
  }
  if (lane_id() == 0) s.u[wave_id()] = v;
  __syncthreads();
  uint32_t r = 0xffffffffu;
  for (int w = 0; w < num_waves(); ++w) r = s.u[w] < r ? s.u[w] : r;
  __syncthreads();
  return r;
}

__device__ __forceinline__ uint32_t block_max_u(uint32_t v, BlockScratch& s) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const uint32_t w = __shfl_xor(v, o);
    v = w > v ? w : v;
  }
  if (lane_id() == 0) s.u[wave_id()] = v;
  __syncthreads();
  uint32_t r = 0u;
  for (int w = 0; w < num_waves(); ++w) r = s.u[w] > r ? s.u[w] : r;
  __syncthreads();
  return r;
}

// The K elements that come first under (key descending, element position
// ascending), given kk = the K-th largest key: every key above kk, then the
// keys equal to kk in element order until K are taken.  Returns the mask of
// taken items.
template <int ITEMS>
__device__ __forceinline__ uint32_t block_first_k(const uint32_t (&key)[ITEMS], uint32_t sel, uint32_t kk, uint32_t K,
                                                  BlockScratch& s) {
  uint32_t gt = 0, eq = 0;
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) {
    if (!((sel >> i) & 1u)) continue;
    gt += key[i] > kk ? 1u : 0u;
    eq += key[i] == kk ? 1u : 0u;
  }
  const uint32_t need = K - block_sum_u(gt, s);
  uint32_t eq_tot;
  uint32_t pos = block_excl_scan(eq, s, &eq_tot);
  uint32_t out = 0;
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) {
    if (!((sel >> i) & 1u)) continue;
    if (key[i] > kk) {
      out |= 1u << i;
    } else if (key[i] == kk) {
      if (pos < need) out |= 1u << i;
      ++pos;
    }
  }
  return out;
}

// K-th largest (K >= 1) of the 32-bit keys selected by bit i of `sel`.
// Four MSB-first 8-bit radix passes with LDS histograms.  Returns false when
// fewer than K keys are selected.
template <int ITEMS>
__device__ __forceinline__ bool block_kth_largest(const uint32_t (&key)[ITEMS], uint32_t sel, uint32_t K,
                                  uint32_t* hist /*[256]*/, BlockScratch& s, uint32_t* out) {
  uint32_t prefix = 0, pmask = 0;
  const int t = threadIdx.x;
  for (int pass = 0; pass < 4; ++pass) {
    const int shift = 24 - 8 * pass;
    for (int i = t; i < 256; i += blockDim.x) hist[i] = 0u;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < ITEMS; ++i)
      if (((sel >> i) & 1u) && (key[i] & pmask) == prefix)
        atomicAdd(&hist[(key[i] >> shift) & 255u], 1u);
    __syncthreads();
    // threads 0..255 hold bins 255..0; an inclusive scan gives the count of
    // keys whose digit is >= the bin.
    uint32_t v = t < 256 ? hist[255 - t] : 0u;
    uint32_t inc = wave_incl_scan(v);
    if (t < 256 && lane_id() == kWave - 1) s.u[wave_id()] = inc;
    __syncthreads();
    if (t < 256) {
      uint32_t off = 0;
      for (int w = 0; w < wave_id(); ++w) off += s.u[w];
      uint32_t P = off + inc, Pex = P - v;
      if (P >= K && Pex < K) {
        s.u[kMaxWaves + 0] = 255u - (uint32_t)t;
        s.u[kMaxWaves + 1] = K - Pex;
      }
      if (t == 255) s.u[kMaxWaves + 2] = P;
    }
    __syncthreads();
    if (pass == 0 && s.u[kMaxWaves + 2] < K) {
      __syncthreads();
      return false;
    }
    uint32_t d = s.u[kMaxWaves + 0];
    K = s.u[kMaxWaves + 1];
    prefix |= d << shift;
    pmask |= 255u << shift;
    __syncthreads();
  }
  *out = prefix;
  return true;
}

// In-place ascending bitonic sort of n_pad (a power of two) 64-bit keys in LDS
// by the whole block.  Each stage (k, j) gives thread p the pairs
// p + r * blockDim, pair p ordering elements i = 2 (p & ~(j-1)) + (p & (j-1)) and i + j.  While j <= 64
// the pairs 64w .. 64w+63 touch only elements 128w .. 128w+127, so with
// blockDim a multiple of 64 each such segment belongs to one wave.  Between
// two stages that both stay inside segments the wave orders its own LDS
// accesses (one wave's LDS operations complete in order; the fences keep the
// compiler from moving them); any other boundary takes a block barrier.
template <typename KeyT>
__device__ __forceinline__ void block_bitonic_sort(KeyT* a, int n_pad) {
  const int half = n_pad >> 1;
  const bool segs = (blockDim.x & 63u) == 0u;
  for (int k = 2; k <= n_pad; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int p = threadIdx.x; p < half; p += blockDim.x) {
        const int i = ((p & ~(j - 1)) << 1) | (p & (j - 1));
        const int ixj = i + j;
        const KeyT x = a[i], y = a[ixj];
        const bool up = (i & k) == 0;
        if ((x > y) == up) {
          a[i] = y;
          a[ixj] = x;
        }
      }
      // the next stage is (k, j/2), or (2k, k) after j == 1
      const bool next_in_seg = j > 1 ? true : (2 * k <= n_pad && k <= 64);
      if (segs && j <= 64 && next_in_seg) {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      } else {
        __syncthreads();
      }
    }
  }
}

__device__ __forceinline__ int next_pow2(int n) {
  int p = 1;
  while (p < n) p <<= 1;
  return p;
}

// ---------------------------------------------------------------- wave sorts
__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int m) {
  uint32_t lo = __shfl_xor((uint32_t)v, m), hi = __shfl_xor((uint32_t)(v >> 32), m);
  return ((uint64_t)hi << 32) | lo;
}

// ---------------------------------------------------------------- 2048-key sort
// One compare-exchange of the bitonic network against lane t ^ d: the lower
// position keeps the minimum when the run ascends.
__device__ __forceinline__ uint64_t bitonic_lane(uint64_t x, int d, bool lower, bool up) {
  const uint64_t y = shfl_xor_u64(x, d);
  const uint64_t mn = x < y ? x : y, mx = x < y ? y : x;
  return lower == up ? mn : mx;
}
__device__ __forceinline__ void bitonic_pair(uint64_t& x0, uint64_t& x1, bool up) {
  const uint64_t lo = x0 < x1 ? x0 : x1, hi = x0 < x1 ? x1 : x0;
  x0 = up ? lo : hi;
  x1 = up ? hi : lo;
}
// LDS slot of position e in the transposition buffer: bits 8-9 folded into
// bits 3-4, so that the column reads (positions c + 256 s) of a wave fall in
// distinct bank pairs two lanes at a time.
__device__ __forceinline__ int sort_slot(int e) { return e ^ (((e >> 8) & 3) << 3); }

// Ascending sort of the 2048 keys at a (LDS) by a workgroup of exactly 1024
// threads.  Thread t keeps positions 2t and 2t + 1 in registers; the network's
// stages of stride 64 and below pair lanes of one wave (lane exchanges, no
// barrier).  For merges of 256 keys and up, the stages of stride 128 and above
// run in a transposed layout -- thread t holds positions c + 128 (2s) and
// c + 128 (2s + 1), c = t / 8, s = t % 8 -- in which those partners are again
// lanes of one wave; each switch of layout is one LDS round trip with one
// barrier (each slot is read and later written by one thread only).  The
// sorted keys are back at a, in order, when the call returns.
__device__ __forceinline__ void block_sort2048(uint64_t* a) {
  const int t = threadIdx.x, c = t >> 3, s = t & 7;
  uint64_t x0 = a[2 * t], x1 = a[2 * t + 1];
  __syncthreads();  // every key read before the buffer is reused
  for (int k = 2, q = -6; k <= 2048; k <<= 1, ++q) {  // k = 128 * 2^q
    if (k >= 256) {
      a[sort_slot(2 * t)] = x0;
      a[sort_slot(2 * t + 1)] = x1;
      __syncthreads();
      x0 = a[sort_slot(c + 256 * s)];
      x1 = a[sort_slot(c + 256 * s + 128)];
      const bool up = ((s >> (q - 1)) & 1) == 0;
      for (int j = k >> 1; j >= 256; j >>= 1) {
        const int d = j >> 8;
        const bool lower = (s & d) == 0;
        x0 = bitonic_lane(x0, d, lower, up);
        x1 = bitonic_lane(x1, d, lower, up);
      }
      bitonic_pair(x0, x1, up);  // stride 128
      a[sort_slot(c + 256 * s)] = x0;
      a[sort_slot(c + 256 * s + 128)] = x1;
      __syncthreads();
      x0 = a[sort_slot(2 * t)];
      x1 = a[sort_slot(2 * t + 1)];
    }
    const bool up = ((2 * t) & k) == 0;
    for (int j = (k >> 1) < 64 ? (k >> 1) : 64; j >= 2; j >>= 1) {
      const int d = j >> 1;
      const bool lower = (t & d) == 0;
      x0 = bitonic_lane(x0, d, lower, up);
      x1 = bitonic_lane(x1, d, lower, up);
    }
    bitonic_pair(x0, x1, up);  // stride 1
  }
  __syncthreads();  // the last transposed reads done before the ordered writes
  a[2 * t] = x0;
  a[2 * t + 1] = x1;
  __syncthreads();
}
// __builtin_amdgcn_readlane returns a signed int: go through uint32_t before
// widening so the low word is not sign-extended.
__device__ __forceinline__ uint32_t readlane_u32(uint32_t v, int l) {
  return (uint32_t)__builtin_amdgcn_readlane((int)v, l);
}
__device__ __forceinline__ uint64_t readlane_u64(uint64_t v, int l) {
  return ((uint64_t)readlane_u32((uint32_t)(v >> 32), l) << 32) | (uint64_t)readlane_u32((uint32_t)v, l);
}
__device__ __forceinline__ float readlane_f32(float v, int l) { return u2f(__builtin_amdgcn_readlane(f2u(v), l)); }
__device__ __forceinline__ double readlane_f64(double v, int l) {
  return __longlong_as_double((long long)readlane_u64((uint64_t)__double_as_longlong(v), l));
}

// Bitonic sort of one key per lane into descending lane order.
__device__ __forceinline__ uint32_t wave_sort_desc_u32(uint32_t v) {
  const int lane = lane_id();
#pragma unroll
  for (int k = 2; k <= kWave; k <<= 1) {
#pragma unroll
    for (int j = k >> 1; j > 0; j >>= 1) {
      uint32_t o = __shfl_xor(v, j);
      bool take_max = ((lane & j) == 0) == ((lane & k) == 0);
      v = take_max ? (o > v ? o : v) : (o < v ? o : v);
    }
  }
  return v;
}

// Lane l holds element l of a bitonic sequence; returns it sorted descending.
__device__ __forceinline__ uint32_t wave_bitonic_clean_desc_u32(uint32_t v) {
  const int lane = lane_id();
#pragma unroll
  for (int j = kWave >> 1; j > 0; j >>= 1) {
    uint32_t o = __shfl_xor(v, j);
    v = ((lane & j) == 0) ? (o > v ? o : v) : (o < v ? o : v);
  }
  return v;
}

// Bitonic sort of 64*S 64-bit keys into descending order; element i lives in
// lane i % 64 of slot i / 64.
template <int S>
__device__ __forceinline__ void wave_sort_desc_u64(uint64_t (&v)[S]) {
  const int lane = lane_id();
#pragma unroll
  for (int k = 2; k <= kWave * S; k <<= 1) {
#pragma unroll
    for (int j = k >> 1; j > 0; j >>= 1) {
      if (j >= kWave) {
        const int js = j / kWave;
#pragma unroll
        for (int sl = 0; sl < S; ++sl) {
          if (sl & js) continue;
          const int i = sl * kWave + lane;
          const bool desc = (i & k) == 0;
          uint64_t x = v[sl], y = v[sl + js];
          uint64_t hi = x > y ? x : y, lo = x > y ? y : x;
          v[sl] = desc ? hi : lo;
          v[sl + js] = desc ? lo : hi;
        }
      } else {
#pragma unroll
        for (int sl = 0; sl < S; ++sl) {
          const int i = sl * kWave + lane;
          uint64_t o = shfl_xor_u64(v[sl], j);
          bool take_max = ((i & j) == 0) == ((i & k) == 0);
          v[sl] = take_max ? (o > v[sl] ? o : v[sl]) : (o < v[sl] ? o : v[sl]);
        }
      }
    }
  }
}

// ---------------------------------------------------------------- scans
__device__ __forceinline__ double wave_incl_scan_d(double v) {
  const int lane = lane_id();
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
    double t = __shfl_up(v, o);
    if (lane >= o) v += t;
  }
  return v;
}
__device__ __forceinline__ long long wave_incl_scan_ll(long long v) {
  const int lane = lane_id();
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
    long long t = __shfl_up(v, o);
    if (lane >= o) v += t;
  }
  return v;
}

// Exclusive prefix over threads (thread order) of a double and of a
// (count, int64) pair; *tot gets the totals.  One barrier each.
struct ScanLds {
  double d[kMaxWaves];
  long long q[kMaxWaves];
  uint32_t c[kMaxWaves];
};

__device__ __forceinline__ double block_excl_scan_d(double v, ScanLds& L, double* tot) {
  double inc = wave_incl_scan_d(v);
  if (lane_id() == kWave - 1) L.d[wave_id()] = inc;
  __syncthreads();
  double off = 0.0, all = 0.0;
  for (int w = 0; w < num_waves(); ++w) {
    double t = L.d[w];
    if (w < wave_id()) off += t;
    all += t;
  }
  __syncthreads();
  *tot = all;
  return off + (inc - v);
}

__device__ __forceinline__ void block_excl_scan_cq(uint32_t c, long long q, ScanLds& L, uint32_t* c_off, long long* q_off,
                                   uint32_t* c_tot, long long* q_tot) {
  uint32_t ci = wave_incl_scan(c);
  long long qi = wave_incl_scan_ll(q);
  if (lane_id() == kWave - 1) {
    L.c[wave_id()] = ci;
    L.q[wave_id()] = qi;
  }
  __syncthreads();
  uint32_t co = 0, ca = 0;
  long long qo = 0, qa = 0;
  for (int w = 0; w < num_waves(); ++w) {
    uint32_t tc = L.c[w];
    long long tq = L.q[w];
    if (w < wave_id()) {
      co += tc;
      qo += tq;
    }
    ca += tc;
    qa += tq;
  }
  __syncthreads();
  *c_off = co + ci - c;
  *q_off = qo + qi - q;
  *c_tot = ca;
  *q_tot = qa;
}

// ---------------------------------------------------------------- row loads
// Thread t holds the ITEMS consecutive elements e = t*ITEMS + i - shift of the
// row, where `shift` aligns the row start down to 16 bytes.  Only 16-byte
// chunks that contain at least one element of the row are read; a 16-byte
// aligned chunk never crosses a page, so no read can fault.  Elements outside
// [0, V) are reported invalid.
template <int ITEMS>
__device__ __forceinline__ void load_row(const float* row, int V, float (&x)[ITEMS], int* shift_out) {
  static_assert(ITEMS % 4 == 0, "f32 rows load 4 elements per 16 bytes");
  const int shift = (int)((reinterpret_cast<uintptr_t>(row) >> 2) & 3u);
  const float4* base = reinterpret_cast<const float4*>(row - shift);
  const int t = threadIdx.x;
#pragma unroll
  for (int c = 0; c < ITEMS / 4; ++c) {
    const int q = t * (ITEMS / 4) + c;
    const int e0 = q * 4 - shift;
    if (e0 + 3 >= 0 && e0 < V) {
      float4 v = base[q];
      x[4 * c + 0] = v.x;
      x[4 * c + 1] = v.y;
      x[4 * c + 2] = v.z;
      x[4 * c + 3] = v.w;
    } else {
      x[4 * c + 0] = x[4 * c + 1] = x[4 * c + 2] = x[4 * c + 3] = -__builtin_inff();
    }
  }
  *shift_out = shift;
}

template <int ITEMS>
__device__ __forceinline__ void load_row(const uint16_t* row, int V, float (&x)[ITEMS], int* shift_out) {
  static_assert(ITEMS % 8 == 0, "bf16 rows load 8 elements per 16 bytes");
  const int shift = (int)((reinterpret_cast<uintptr_t>(row) >> 1) & 7u);
  const uint4* base = reinterpret_cast<const uint4*>(row - shift);
  const int t = threadIdx.x;
#pragma unroll
  for (int c = 0; c < ITEMS / 8; ++c) {
    const int q = t * (ITEMS / 8) + c;
    const int e0 = q * 8 - shift;
    if (e0 + 7 >= 0 && e0 < V) {
      uint4 v = base[q];
      uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        x[8 * c + 2 * j + 0] = u2f(w[j] << 16);
        x[8 * c + 2 * j + 1] = u2f(w[j] & 0xffff0000u);
      }
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) x[8 * c + j] = -__builtin_inff();
    }
  }
  *shift_out = shift;
}

template <int ITEMS>
__device__ __forceinline__ uint32_t valid_mask(int V, int shift) {
  uint32_t m = 0;
  const int e0 = (int)threadIdx.x * ITEMS - shift;
#pragma unroll
  for (int i = 0; i < ITEMS; ++i)
    if (e0 + i >= 0 && e0 + i < V) m |= 1u << i;
  return m;
}

}  // namespace tc
