// tc_row.h -- what the sampler kernels share: the per-launch arguments
// (RowArgs), the survivor stage in LDS, the steps every variant takes
// (history map, compaction, results), and the launch functions each
// kernel source file defines for the C ABI in sampler.hip.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/talechime_hip.h"
#include "tc_device.h"
#include "tc_seqsum.h"

namespace tc {

constexpr int kSurvCap = 1024;      // survivors held in LDS per row

// Register-resident row shapes: ITEMS elements per thread, at most
// max_threads(ITEMS) threads (which sets the register budget per thread).
constexpr int max_threads(int items) { return items <= 8 ? 1024 : (items <= 16 ? 768 : 704); }


constexpr int kMaxVocabReg = 16384; // register-resident rows: V + alignment <= 1024 * 16

struct RowArgs {
  const void* logits;
  long long ld;
  int V;
  int rows;
  const uint32_t* hist_off;
  const uint32_t* hist_ids;
  int hist_mode;
  const float* pen_mask;
  const float* add_mask;
  const void* uniforms;
  uint32_t* out_ids;
  int32_t* out_status;
  uint32_t* out_flags;
  uint32_t cap;
  uint32_t* topk_count;
  uint32_t* topk_ids;
  uint32_t* keep_count;
  uint32_t* keep_ids;
  float* keep_probs;
  float* norm;  // optional [rows] normaliser output
  // parameters, prepared on the host
  int do_pen;
  float pen_f;    // penalty as f32
  float inv_pen;  // qwen: 1.0f / pen_f
  int do_temp;    // qwen: affine temperature on; others: divide by t_f
  float tmul;     // qwen: (f32)(1 / T)
  float t_f;      // (f32)T
  int greedy;     // qwen: T < 0.01
  int K;          // top-k selection size (0 = none)
  int top_k;      // raw top_k
  int do_topp;
  float top_p_f;
  double top_p_d;
  int min_keep;
  int eos_id;
  int exclude_id;
  int ras_win;
  float ras_thresh;  // (f32)win * tau
  int fast;          // indextts, qwen: the streaming fast path applies (1 <= K <= 64 < V, sampling)
  float* mark;       // optional [V] penalty mask: set to 1.0 at each row's sampled id
  float* keep_scores;  // indextts beam step: the final score of each kept id, beside keep_ids
  double typical_mass; // indextts: the typical warper's mass (k_idx_typical); 0 = off
};

// Writes a row's result.  A row sampled cleanly also marks its token in the
// penalty mask the next step reads (synthesis.rs:568-579 update_penalty_mask,
// fused: ids >= V are ignored there too).  Called by one lane per row, after
// every read of the row's inputs.
__device__ __forceinline__ void put_result(const RowArgs& a, int row, uint32_t tok, int32_t st, uint32_t flags) {
  a.out_ids[row] = tok;
  if (a.out_status) a.out_status[row] = st;
  if (a.out_flags) a.out_flags[row] = flags;
  if (a.mark && st == 0 && tok < (uint32_t)a.V) a.mark[tok] = 1.0f;
}

struct SurvLds {
  uint64_t key[kSurvCap];
  double w[kSurvCap];
  float val[kSurvCap];
  float e[kSurvCap];
  uint32_t idx[kSurvCap];
  uint8_t flag[kSurvCap];
};


}  // namespace tc

#include "tc_fast.h"

namespace tc {

// ---------------------------------------------------------------- shared steps

__device__ __forceinline__ void hist_range(const RowArgs& a, int row, uint32_t* h0, uint32_t* h1) {
  if (a.hist_ids == nullptr || a.hist_off == nullptr) {
    *h0 = *h1 = 0;
  } else if (a.hist_mode == TC_HIST_BROADCAST) {
    *h0 = a.hist_off[0];
    *h1 = a.hist_off[1];
  } else {
    *h0 = a.hist_off[row];
    *h1 = a.hist_off[row + 1];
  }
}

// Byte map of the ids in the row's history (ids >= V ignored).  Returns true if
// some id was >= V.
__device__ __forceinline__ bool build_seen(const RowArgs& a, int row, uint8_t* seen, BlockScratch& s) {
  const int V = a.V;
  uint32_t* w = reinterpret_cast<uint32_t*>(seen);
  for (int i = threadIdx.x; i < (V + 3) / 4; i += blockDim.x) w[i] = 0u;
  __syncthreads();
  uint32_t h0, h1;
  hist_range(a, row, &h0, &h1);
  uint32_t oob = 0;
  for (uint32_t j = h0 + threadIdx.x; j < h1; j += blockDim.x) {
    uint32_t id = a.hist_ids[j];
    if (id < (uint32_t)V) seen[id] = 1;
    else oob = 1;
  }
  __syncthreads();
  return block_or_u(oob, s) != 0u;
}

// Ordered compaction of the selected elements into LDS (vocabulary order).
// Returns the number selected (may exceed kSurvCap; then only the count is valid).
template <int ITEMS>
__device__ __forceinline__ uint32_t compact(const float (&x)[ITEMS], uint32_t sel, int e0, SurvLds& sv, BlockScratch& s) {
  uint32_t c = __builtin_popcount(sel);
  uint32_t total;
  uint32_t pos = block_excl_scan(c, s, &total);
  if (total <= (uint32_t)kSurvCap) {
#pragma unroll
    for (int i = 0; i < ITEMS; ++i)
      if ((sel >> i) & 1u) {
        sv.val[pos] = x[i];
        sv.idx[pos] = (uint32_t)(e0 + i);
        ++pos;
      }
  }
  __syncthreads();
  return total;
}

__device__ __forceinline__ void write_topk(const RowArgs& a, int row, const SurvLds& sv, uint32_t n) {
  if (a.topk_count == nullptr) return;
  if (threadIdx.x == 0) a.topk_count[row] = n;
  if (n > (uint32_t)kSurvCap) return;  // only the count is known
  uint32_t m = n < a.cap ? n : a.cap;
  for (uint32_t j = threadIdx.x; j < m; j += blockDim.x) a.topk_ids[(size_t)row * a.cap + j] = sv.idx[j];
}

// Rank-order sort of the n survivors: keys built by the caller in sv.key[0..n),
// padded to a power of two.
__device__ __forceinline__ void sort_survivors(SurvLds& sv, uint32_t n) {
  int n_pad = next_pow2((int)n < 2 ? 2 : (int)n);
  for (int j = (int)n + threadIdx.x; j < n_pad; j += blockDim.x) sv.key[j] = ~0ull;
  __syncthreads();
  block_bitonic_sort(sv.key, n_pad);
}

__device__ __forceinline__ void finish_row(const RowArgs& a, int row, uint32_t tok, int32_t st, uint32_t flags) {
  if (threadIdx.x == 0) {
    put_result(a, row, tok, st, flags);
  }
}

__device__ __forceinline__ void put_norm(const RowArgs& a, int row, float v) {
  if (a.norm && threadIdx.x == 0) a.norm[row] = v;
}

__device__ __forceinline__ void no_verify(const RowArgs& a, int row) {
  if (threadIdx.x == 0 && a.norm) a.norm[row] = __builtin_nanf("");
  if (threadIdx.x == 0) {
    if (a.topk_count) a.topk_count[row] = 0;
    if (a.keep_count) a.keep_count[row] = 0;
  }
}

// ---------------------------------------------------------------- many survivors
// Rows with more survivors than the LDS stage holds (top-k off or above
// kSurvCap, or ties at the k-th value) keep them in the register-resident row;
// the rank order comes from their 32-bit keys sorted in LDS, where equal
// values are equal terms, so the order-dependent sums need no ids.

// A copy of v the compiler cannot see through: a weight recomputed from it at
// each use stays a recomputation, instead of one value per item held live in
// registers across the row's passes (which spills the wide shapes).
__device__ __forceinline__ float opaque(float v) {
  asm volatile("" : "+v"(v));
  return v;
}
__device__ __forceinline__ uint32_t opaque(uint32_t v) {
  asm volatile("" : "+v"(v));
  return v;
}

// The survivor stage, or the sorted keys of every survivor of the row.
union SurvWide {
  SurvLds sv;
  uint32_t wide[kMaxVocabReg];
};

// Sorts the keys of the selected items (n of them, n <= ITEMS * blockDim)
// ascending in buf (complemented with `desc`: descending) and gives thread t
// the sorted words at positions ITEMS * t + i (0xffffffff at and past n).
// buf stays sorted (padded to a power of two).
template <int ITEMS>
__device__ __forceinline__ void block_rank_keys(const uint32_t (&key)[ITEMS], uint32_t sel, uint32_t n, bool desc,
                                                uint32_t* buf, BlockScratch& s, uint32_t (&rk)[ITEMS]) {
  uint32_t tot;
  uint32_t pos = block_excl_scan((uint32_t)__builtin_popcount(sel), s, &tot);
  const uint32_t flip = desc ? 0xffffffffu : 0u;
#pragma unroll
  for (int i = 0; i < ITEMS; ++i)
    if ((sel >> i) & 1u) buf[pos++] = key[i] ^ flip;
  const int n_pad = next_pow2((int)n < 2 ? 2 : (int)n);
  for (int j = (int)n + (int)threadIdx.x; j < n_pad; j += blockDim.x) buf[j] = 0xffffffffu;
  __syncthreads();
  block_bitonic_sort(buf, n_pad);
  const int p0 = ITEMS * (int)threadIdx.x;
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) rk[i] = p0 + i < (int)n ? buf[p0 + i] : 0xffffffffu;
}

// The selected items whose key is above kc, and of those equal to it the ones
// whose place among them (vocabulary order) lies in [lo, hi).
template <int ITEMS>
__device__ __forceinline__ uint32_t select_above_and_ties(const uint32_t (&key)[ITEMS], uint32_t sel, uint32_t kc,
                                                          uint32_t lo, uint32_t hi, BlockScratch& s) {
  uint32_t eq = 0;
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) eq += (((sel >> i) & 1u) && key[i] == kc) ? 1u : 0u;
  uint32_t tot;
  uint32_t r = block_excl_scan(eq, s, &tot);
  uint32_t out = 0;
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) {
    if (!((sel >> i) & 1u)) continue;
    if (key[i] > kc) {
      out |= 1u << i;
    } else if (key[i] == kc) {
      if (r >= lo && r < hi) out |= 1u << i;
      ++r;
    }
  }
  return out;
}

// The first cap ids of the selected items, in vocabulary order, to ids[row *
// cap ...]; returns their number (all of them, also past cap).
template <int ITEMS>
__device__ __forceinline__ uint32_t write_ids(uint32_t* ids, uint32_t cap, int row, uint32_t sel, int e0,
                                              BlockScratch& s) {
  uint32_t tot;
  uint32_t p = block_excl_scan((uint32_t)__builtin_popcount(sel), s, &tot);
  if (ids) {
#pragma unroll
    for (int i = 0; i < ITEMS; ++i)
      if ((sel >> i) & 1u) {
        if (p < cap) ids[(size_t)row * cap + p] = (uint32_t)(e0 + i);
        ++p;
      }
  }
  return tot;
}

// A decision of the reference taken on sums the block computes in another
// order: x against y (both sums of non-negative terms, or fixed limits) is
// settled when they differ by more than order_margin(n) of the larger.
__device__ __forceinline__ bool settled(double x, double y, uint32_t n) {
  const double m = __builtin_fmax(__builtin_fabs(x), __builtin_fabs(y));
  return __builtin_fabs(x - y) > order_margin(n) * m;
}
// The same decision taken in the reference's own order, where only the f64
// exp of this library can differ from its libm's.
__device__ __forceinline__ bool settled_exp(double x, double y) {
  const double m = __builtin_fmax(__builtin_fabs(x), __builtin_fabs(y));
  return __builtin_fabs(x - y) > exp_margin() * m;
}

// Where the block sums leave a decision open: the reference's sequential loop
// itself.  One lane runs step(j, v) over positions j = 0 .. n-1 in order, v
// being the value the thread holding position j supplies (val(i) for its item
// i at position pos(i); pos(i) >= n: none), staged kWalkChunk at a time in
// buf; step returns false to stop.  Every thread returns after the walk.
constexpr uint32_t kWalkChunk = kMaxVocabReg / 2;  // doubles in a 64 KB stage
struct WalkLds {
  double d[4];
  uint32_t u[4];
};
template <int ITEMS, typename Pos, typename Val, typename Step>
__device__ __forceinline__ void staged_walk(uint32_t n, Pos pos, Val val, double* buf, WalkLds& W, Step step) {
  for (uint32_t c0 = 0; c0 < n; c0 += kWalkChunk) {
    const uint32_t c1 = c0 + kWalkChunk < n ? c0 + kWalkChunk : n;
#pragma unroll
    for (int i = 0; i < ITEMS; ++i) {
      const uint32_t p = pos(i);
      if (p >= c0 && p < c1) buf[p - c0] = val(i);
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      uint32_t stop = 0;
      for (uint32_t j = c0; j < c1; ++j)
        if (!step(j, buf[j - c0])) {
          stop = 1;
          break;
        }
      W.u[3] = stop;
    }
    __syncthreads();
    const bool stop = W.u[3] != 0;
    __syncthreads();
    if (stop) break;
  }
}

// Positions of the selected items in vocabulary order (pos(i) for item i;
// 0xffffffff when not selected), from the block's exclusive scan.
template <int ITEMS>
struct VocabPos {
  uint32_t off, sel;
  __device__ __forceinline__ uint32_t operator()(int i) const {
    return ((sel >> i) & 1u) ? off + (uint32_t)__builtin_popcount(sel & ((1u << i) - 1u)) : 0xffffffffu;
  }
};
template <int ITEMS>
__device__ __forceinline__ VocabPos<ITEMS> vocab_pos(uint32_t sel, BlockScratch& s) {
  uint32_t tot;
  return VocabPos<ITEMS>{block_excl_scan((uint32_t)__builtin_popcount(sel), s, &tot), sel};
}

// Launches of the register-resident kernels (one workgroup per row, `threads`
// threads of `items` elements), one per kernel source file.
hipError_t launch_k_qwen(int dtype, int items, int threads, int rows, hipStream_t st, const RowArgs& a);
hipError_t launch_k_indextts(int dtype, int items, int threads, int rows, hipStream_t st, const RowArgs& a);
hipError_t launch_k_idx_typical(int dtype, int items, int threads, int rows, hipStream_t st, const RowArgs& a);
hipError_t launch_k_cosy(int dtype, int items, int threads, int rows, hipStream_t st, const RowArgs& a);
hipError_t launch_k_moss(int dtype, int items, int threads, int rows, hipStream_t st, const RowArgs& a);
hipError_t launch_k_nano(int dtype, int items, int threads, int rows, hipStream_t st, const RowArgs& a);
// The large-vocabulary qwen kernels (1024 threads per row): the packed bf16
// passes, or the general form over f32/bf16 rows and the masks.
constexpr int kLargeThreads = 1024;
constexpr int kLargeCand = 2048;
constexpr int kLargeVocab = 262144;
hipError_t launch_k_large(bool packed, int dtype, int rows, hipStream_t st, const RowArgs& a);

#define TC_DEFINE_LAUNCH(NAME)                                                                   \
  hipError_t launch_##NAME(int dtype, int items, int threads, int rows, hipStream_t st,          \
                           const tc::RowArgs& a) {                                               \
    dim3 g(rows), b(threads);                                                                    \
    if (dtype == TC_F32) {                                                                       \
      if (items == 8) hipLaunchKernelGGL((NAME<float, 8>), g, b, 0, st, a);                  \
      else if (items == 12) hipLaunchKernelGGL((NAME<float, 12>), g, b, 0, st, a);           \
      else if (items == 16) hipLaunchKernelGGL((NAME<float, 16>), g, b, 0, st, a);           \
      else hipLaunchKernelGGL((NAME<float, 24>), g, b, 0, st, a);                            \
    } else {                                                                                     \
      if (items == 8) hipLaunchKernelGGL((NAME<uint16_t, 8>), g, b, 0, st, a);               \
      else if (items == 16) hipLaunchKernelGGL((NAME<uint16_t, 16>), g, b, 0, st, a);        \
      else hipLaunchKernelGGL((NAME<uint16_t, 24>), g, b, 0, st, a);                         \
    }                                                                                            \
    return hipGetLastError();                                                                    \
  }

}  // namespace tc
