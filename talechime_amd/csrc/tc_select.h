// tc_select.h -- top-k candidate selection for register-resident rows.
//
// Each thread holds ITEMS order keys (larger = better; 0 for invalid slots).
// The k-th largest key of the row is at least the k-th largest of the
// per-thread maxima (those k maxima are k distinct elements), so every
// element at or above the k-th key is found among the elements at or above
// that bound.  On logits that bound admits only a few elements beyond k:
//   * each wave sorts its 64 thread maxima (bitonic, in registers);
//   * after one barrier every wave merges the sorted lists of all waves
//     (top-64 of two sorted lists = bitonic merge) and reads the k-th;
//   * elements at or above the bound are written to per-wave LDS regions in
//     element order, so the regions read in wave order are in vocabulary
//     order.
// k must be at most 64.  The caller finishes in one wave when the candidate
// count is small and falls back to a general selection otherwise.
#pragma once

#include "tc_device.h"

namespace tc {

struct SelLds {
  static constexpr int kCapW = 128;  // candidates per wave region
  static constexpr int kCapF = 128;  // candidates the one-wave finish takes
  uint32_t lists[kMaxWaves][kWave];
  uint64_t cand[kMaxWaves][kCapW];   // (key << 32) | position
  uint32_t cnt[kMaxWaves];
  uint32_t flg[kMaxWaves];
};

// Lower bound on the K-th largest key (1 <= K <= 64); 0 when fewer than K
// threads hold a valid key.  Contains one barrier.
template <int ITEMS>
__device__ __forceinline__ uint32_t block_topk_bound(const uint32_t (&key)[ITEMS], uint32_t vm, int K, SelLds& L) {
  uint32_t m = 0;
#pragma unroll
  for (int i = 0; i < ITEMS; ++i)
    if (((vm >> i) & 1u) && key[i] > m) m = key[i];
  m = wave_sort_desc_u32(m);
  L.lists[wave_id()][lane_id()] = m;
  __syncthreads();
  uint32_t acc = L.lists[0][lane_id()];
  for (int w = 1; w < num_waves(); ++w) {
    uint32_t b = L.lists[w][kWave - 1 - lane_id()];
    acc = wave_bitonic_clean_desc_u32(acc > b ? acc : b);
  }
  return readlane_u32(acc, K - 1);
}

// Writes the elements whose bit is set in `sel` to the wave's region as
// (key << 32) | position.  Contains one barrier; returns the total count
// (valid for every thread), sets *overflow when a region overflowed and
// *flag_or to the OR of `flag` over the block.
template <int ITEMS>
__device__ __forceinline__ uint32_t block_compact_candidates(const uint32_t (&key)[ITEMS], uint32_t sel, int pos0, SelLds& L,
                                             bool flag, bool* overflow, uint32_t* flag_or) {
  const uint32_t c = __builtin_popcount(sel);
  const uint32_t inc = wave_incl_scan(c);
  const uint32_t tot = readlane_u32(inc, kWave - 1);
  uint32_t p = inc - c;
  const int w = wave_id();
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) {
    if ((sel >> i) & 1u) {
      if (p < (uint32_t)SelLds::kCapW) L.cand[w][p] = ((uint64_t)key[i] << 32) | (uint32_t)(pos0 + i);
      ++p;
    }
  }
  const bool fw = __ballot(flag) != 0ull;
  if (lane_id() == 0) {
    L.cnt[w] = tot;
    L.flg[w] = fw ? 1u : 0u;
  }
  __syncthreads();
  uint32_t n = 0, f = 0;
  bool of = false;
  for (int v = 0; v < num_waves(); ++v) {
    uint32_t cv = L.cnt[v];
    n += cv;
    f |= L.flg[v];
    of |= cv > (uint32_t)SelLds::kCapW;
  }
  *overflow = of;
  *flag_or = f;
  return n;
}

// Candidate i (0 <= i < n, vocabulary order) from the wave regions.
__device__ __forceinline__ uint64_t candidate_at(const SelLds& L, uint32_t i) {
  int w = 0;
  uint32_t base = 0;
  while (i >= base + L.cnt[w]) {
    base += L.cnt[w];
    ++w;
  }
  return L.cand[w][i - base];
}

}  // namespace tc
