// k_large.hip -- qwen sampling over large vocabularies (up to 262,144 logits,
// one 1024-thread workgroup per row).

#include <type_traits>

#include "tc_row.h"

namespace tc {

// ================================================================ qwen, large vocabulary
// qwen semantics (sampling.rs:169-328 with the per-row penalty of 334-395) for
// bf16 rows of up to kLargeVocab logits, one 1024-thread workgroup per row.
// The row is walked three times in tiles of 16-byte chunks; the first
// kLargeR tiles stay in registers and the next one in LDS from pass A on, so
// at a 151,936 vocabulary only the last 14 % of the row is read again.
//  * Pass A: finiteness, the greedy argmax, and the largest bf16 key over ids
//    outside the history.  Those ids keep the order of their raw keys (the
//    transform multiplies by positive constants and distinct bf16 values
//    cannot meet in f32).
//  * Pass B: an exact histogram of the 256 keys at and below the largest,
//    which gives the K-th largest such key: a lower bound on the k-th logit.
//  * Pass C: candidates (ids outside the history at or above that key, ids in
//    it whose penalised logit reaches the bound, found as a second key
//    threshold; at most kLargeCand), staged in vocabulary order a tile at a
//    time.
//  * Rows these passes do not decide (non-finite logits, a negative penalty,
//    a K-th key more than 256 keys below the largest) take large_candidates,
//    which streams the row from memory again and selects on the final logits.
//  * A bitonic sort gives the reference's rank order (value descending, id
//    ascending); top-k keeps every value >= the k-th (ties kept).
//  * top-p: exact terms, the reference's sequential f32 sum in rank order and
//    its running sum (block_seqsum, seq_prefix), the first crossing kept.
//  * softmax and the CDF in vocabulary order over the kept ids, again as the
//    reference's sequential sums; the first index whose running sum reaches u.
constexpr int kLargeU = 4;  // 16-byte chunks in flight per thread in the streaming passes
constexpr int kLargeR = 3;  // tiles of kLargeU * blockDim chunks kept in registers across the passes
constexpr int kLargePer = kLargeCand / kLargeThreads;  // candidate slots per thread
constexpr int kLargeWords = kLargeVocab / 32;
static_assert(kLargeCand == 2048 && kLargeThreads == 1024, "block_sort2048 sorts 2048 keys over 1024 threads");

struct QLargeLds {
  uint4 ltile[kLargeU * kLargeThreads];  // the row's tile kLargeR (chunk kLargeU * t + u at u * blockDim + t)
  uint32_t bits[kLargeWords + 1];  // history ids (k_qwen_large: bit id + shift)
  uint32_t hist[256];
  uint64_t cand[kLargeCand];   // rank order after the sort
  uint64_t candv[kLargeCand];  // vocabulary order
  float stage[kLargeCand];
  uint32_t wtot[2][kMaxWaves];
  double wd[2][kMaxWaves];
  SeqLds sq;
  ScanLds sc;
  BlockScratch s;
  uint32_t misc[8];
};

// The reference's sequential sum of kLargeCand terms held kLargePer per thread
// (positions kLargePer * t + q) and its inclusive running sums.
__device__ __forceinline__ float small_seq_prefix(const float (&tm)[kLargePer], float (&pre)[kLargePer], QLargeLds& S) {
  SeqThread<kLargePer> th;
  float t2[kLargePer];
#pragma unroll
  for (int q = 0; q < kLargePer; ++q) t2[q] = tm[q];
  auto same = [](float v) { return v; };
  float tot;
  if (block_seqsum<kLargePer>(t2, ~0u, t2, same, kLargePer * (int)threadIdx.x, 0, th, S.sq, S.sc, &tot)) {
    seq_prefix<kLargePer>(th, S.sq, pre);
    return tot;
  }
  // one lane walks the staged terms
#pragma unroll
  for (int q = 0; q < kLargePer; ++q) S.stage[kLargePer * threadIdx.x + q] = tm[q];
  __syncthreads();
  if (threadIdx.x == 0) {
    float s = -0.0f;
    for (int p = 0; p < kLargeCand; ++p) {
      s = s + S.stage[p];
      S.stage[p] = s;
    }
  }
  __syncthreads();
#pragma unroll
  for (int q = 0; q < kLargePer; ++q) pre[q] = S.stage[kLargePer * threadIdx.x + q];
  tot = S.stage[kLargeCand - 1];
  __syncthreads();
  return tot;
}

// The reference's draw decisions without its sums, when they are clear.  The
// reference computes terms e_k = expf(d_k) at positions k < n (kLargePer per
// thread, position kLargePer * t + q; zero where it has none), their
// sequential f32 total S, p_k = e_k / S, and the first eligible position
// whose sequential f32 running sum C_k of the p's exceeds thr (reaches it when
// kGE).  Here the terms are exp_approx(d_k) (within 2^-20 of e_k; 0 below
// -87, where e_k < 2^-125 and S >= 1), summed in f64 (thread, wave and block
// scans).  The approximate total's distance dS from the reference's S comes
// from the terms' error and S's own rounding, at most
// 2^-24 * 1.02 * sum_k (n - k) e_k.  So
// each p_k lies within eps = 2^-19 + 1.01 dS / S of its approximation, and
// C_k within 2^-24 * 1.03 * Q_k of the exact running sum, Q_k the sum of the
// running sums up to k.  The first position whose running sum may cross and
// the first whose crossing is certain agree: that position.  No position may
// cross: 0xffffffff.  Otherwise kUndecided.  Every thread calls it.
constexpr uint32_t kUndecided = 0xfffffffeu;
template <bool kGE>
__device__ __forceinline__ uint32_t certified_first(const float (&d)[kLargePer], uint32_t live, uint32_t elig, int n,
                                                    float thr, QLargeLds& S) {
  const int t = threadIdx.x, lane = lane_id(), wv = wave_id(), nw = num_waves();
  float ea[kLargePer];
  double tp = 0.0, tm = 0.0;
#pragma unroll
  for (int q = 0; q < kLargePer; ++q) {
    ea[q] = ((live >> q) & 1u) && d[q] >= -87.0f ? exp_approx(d[q]) : 0.0f;
    tp += (double)ea[q];
    tm += (double)(kLargePer * t + q) * (double)ea[q];
  }
  const double ip = dpp_scan_f64(tp), im = dpp_scan_f64(tm);
  if (lane == kWave - 1) {
    S.wd[0][wv] = ip;
    S.wd[1][wv] = im;
  }
  __syncthreads();
  double pb = 0.0, mb = 0.0, Sh, Mh;
  {
    const double vp = lane < nw ? S.wd[0][lane] : 0.0, vq = lane < nw ? S.wd[1][lane] : 0.0;
    const double cp = dpp_scan_f64(vp), cm = dpp_scan_f64(vq);
    const int w = __builtin_amdgcn_readfirstlane(wv);
    if (w > 0) {
      pb = rl_f64(cp, w - 1);
      mb = rl_f64(cm, w - 1);
    }
    Sh = rl_f64(cp, kWave - 1);
    Mh = rl_f64(cm, kWave - 1);
  }
  const double dS = 0x1p-20 * Sh + 0x1p-24 * 1.02 * ((double)n * Sh - Mh) + 0x1p-40 * Sh;
  const bool ok = Sh >= 1.0;  // the largest term is expf(0) = 1
  const double inv = ok ? 1.0 / Sh : 0.0, eps = 0x1p-19 + 1.01 * dS * inv;
  double A = pb + (ip - tp), M = mb + (im - tm);
  uint32_t lo = 0xffffffffu, hi = 0xffffffffu;
#pragma unroll
  for (int q = 0; q < kLargePer; ++q) {
    const int k = kLargePer * t + q;
    A += (double)ea[q];
    M += (double)k * (double)ea[q];
    const double P = A * inv, Q = ((double)(k + 1) * A - M) * inv;
    const double E = (eps + 0x1p-40) * P + 0x1p-24 * 1.03 * Q + 0x1p-60;
    const bool e = (elig >> q) & 1u;
    const bool may = kGE ? P + E >= (double)thr : P + E > (double)thr;
    const bool cert = kGE ? P - E >= (double)thr : P - E > (double)thr;
    if (lo == 0xffffffffu && e && may) lo = (uint32_t)k;
    if (hi == 0xffffffffu && e && cert) hi = (uint32_t)k;
  }
  // positions are in lane order: the wave's first is its first lane's
  // (read with every lane active)
  const uint64_t bl = __ballot(lo != 0xffffffffu), bh = __ballot(hi != 0xffffffffu);
  const uint32_t wl = bl ? rl_u32(lo, __builtin_ctzll(bl)) : 0xffffffffu;
  const uint32_t wh = bh ? rl_u32(hi, __builtin_ctzll(bh)) : 0xffffffffu;
  if (lane == 0) {
    S.wtot[0][wv] = wl;
    S.wtot[1][wv] = wh;
  }
  __syncthreads();
  lo = hi = 0xffffffffu;
  for (int w = 0; w < nw; ++w) {
    lo = S.wtot[0][w] < lo ? S.wtot[0][w] : lo;
    hi = S.wtot[1][w] < hi ? S.wtot[1][w] : hi;
  }
  __syncthreads();  // S.wtot and S.wd are free again
  if (!ok) return kUndecided;
  if (lo == 0xffffffffu) return 0xffffffffu;
  return lo == hi ? lo : kUndecided;
}

// Bits [p, p + 32) of an LDS bitmap of nwords words (p may be negative; bits
// outside the map read 0).
__device__ __forceinline__ uint32_t bits_at_fn(const uint32_t* bm, int nwords, int p) {
  const int w = p >> 5, sh = p & 31;
  const uint32_t lo = (w >= 0 && w < nwords) ? bm[w] : 0u;
  const uint32_t hi = (w + 1 >= 0 && w + 1 < nwords) ? bm[w + 1] : 0u;
  return sh ? ((lo >> sh) | (hi << (32 - sh))) : lo;
}

// One 16-byte chunk of a bf16 row: the 8 logits of elements q*8 - shift + h
// as f32 (elements outside [0, V): the most negative finite value), their
// history/EOS bits, and whether a logit inside the row is non-finite.
struct LChunk {
  float x[8];
  uint32_t sn;  // bit h: in the history or the EOS id
  bool bad;
};
__device__ __forceinline__ LChunk decode_lchunk(const uint4 v, int q, int shift, int V, const uint32_t* bits,
                                                int nwords, int eos) {
  LChunk c;
  const int e0 = q * 8 - shift;
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
  const uint32_t hb = bits_at_fn(bits, nwords, q * 8);  // the bitmap holds id + shift
  c.bad = false;
  c.sn = 0;
#pragma unroll
  for (int h = 0; h < 8; ++h) {
    const int e = e0 + h;
    const bool in = e >= 0 && e < V;
    const uint32_t b = (h & 1) ? (w[h >> 1] & 0xffff0000u) : (w[h >> 1] << 16);
    c.bad |= in && (b & 0x7f800000u) == 0x7f800000u;
    c.x[h] = in ? __uint_as_float(b) : -3.3895313892515355e38f;
    const bool s = ((hb >> h) & 1u) != 0u || e == eos;
    c.sn |= (s ? 1u : 0u) << h;
  }
  return c;
}

__device__ __forceinline__ uint32_t pick_u32(bool c, uint32_t a, uint32_t b) { return c ? a : b; }
__device__ __forceinline__ uint32_t u4_word(const uint4& v, int i) { return i == 0 ? v.x : (i == 1 ? v.y : (i == 2 ? v.z : v.w)); }
__device__ __forceinline__ void u4_set(uint4& v, int i, uint32_t x) {
  if (i == 0) v.x = x;
  else if (i == 1) v.y = x;
  else if (i == 2) v.z = x;
  else v.w = x;
}

// ckey(x) >> 16 for the f32 widening of the two bf16 values of a 32-bit word:
// negative halves complemented, positive ones with the top bit set, -0
// raised to +0's key (both zeros give 0x8000).
__device__ __forceinline__ uint32_t bkey16x2(uint32_t w) {
  const uint32_t sgn = w & 0x80008000u;
  const uint32_t m = (sgn - (sgn >> 15)) | sgn;  // 0xffff in each negative half
  const uint32_t k = w ^ (m | 0x80008000u);
  const uint32_t nz = ((w & 0x7fff7fffu) + 0x7fff7fffu) & 0x80008000u;  // low 15 bits nonzero, per half
  return k + ((sgn & ~nz) >> 15);
}
// The bf16 bits of a 16-bit key (key 0x8000, shared by both zeros: +0)
__device__ __forceinline__ uint32_t unkey16(uint32_t k) { return (k & 0x8000u) ? (k & 0x7fffu) : (k ^ 0xffffu); }
// 0x8000 in each half whose exponent bits are all ones (inf or NaN)
__device__ __forceinline__ uint32_t nonfinite16x2(uint32_t w) {
  const uint32_t e = (w & 0x7f807f80u) ^ 0x7f807f80u;
  return ~((e + 0x7fff7fffu) & 0x80008000u) & 0x80008000u;
}
// 0xffff in the halves of word j whose bit (2j, 2j+1) of m8 is set
__device__ __forceinline__ uint32_t half_mask(uint32_t m8, int j) {
  const uint32_t t = (m8 >> (2 * j)) & 3u;
  return __umul24((t & 1u) | ((t & 2u) << 15), 0xffffu);
}
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

// The reference's logit of element e after the caller chain and temperature
// (synthesis.rs:1238-1276, sampling.rs:175-184): the per-row penalty on ids in
// the history (sn), the EOS id forced to -inf, then the multiply by f32(1/T).
__device__ __forceinline__ float qlogit(const RowArgs& a, float x, bool sn, int e, int eos) {
  float v = x;
  if (a.do_pen && sn && e != eos) v = v * (v > 0.0f ? a.inv_pen : a.pen_f);
  if (e == eos) v = -__builtin_inff();
  if (a.do_temp) v = v * a.tmul + 0.0f;
  return v;
}

// The logit of element e with every option of the caller chain
// (synthesis.rs:1238-1276) and the temperature (sampling.rs:175-184): the
// penalty on ids in the history bitmap (hist_bit) or, in TC_HIST_MASK mode,
// on ids whose [V] mask entry is > 0; the additive mask; the EOS id forced
// to -inf; the multiply by f32(1/T).
__device__ __forceinline__ float qlogit_all(const RowArgs& a, float x, bool hist_bit, int e, int eos) {
  float v = x;
  if (a.do_pen) {
    const bool pen = a.hist_mode == TC_HIST_MASK ? a.pen_mask[e] > 0.0f : hist_bit;
    if (pen) v = v * (v > 0.0f ? a.inv_pen : a.pen_f);
  }
  if (a.add_mask) v = v + a.add_mask[e];
  if (e == eos) v = -__builtin_inff();
  if (a.do_temp) v = v * a.tmul + 0.0f;
  return v;
}

// Element h of a 16-byte chunk of a bf16 or f32 row, as f32.
template <typename InT>
__device__ __forceinline__ float chunk_val(const uint4& v, int h) {
  if constexpr (sizeof(InT) == 2) {
    const uint32_t w = u4_word(v, h >> 1);
    return __uint_as_float((h & 1) ? (w & 0xffff0000u) : (w << 16));
  } else {
    return __uint_as_float(u4_word(v, h));
  }
}

// A row of a large-vocabulary launch as 16-byte chunks: chunk q holds
// elements q * kEpc - shift .. q * kEpc - shift + kEpc - 1.
template <typename InT>
struct LargeRow {
  static constexpr int kEpc = 16 / (int)sizeof(InT);
  const uint4* base;
  int shift, nchunks;
  __device__ __forceinline__ LargeRow(const RowArgs& a, int row) {
    const InT* rp = reinterpret_cast<const InT*>(a.logits) + (size_t)row * (size_t)a.ld;
    shift = (int)((reinterpret_cast<uintptr_t>(rp) / sizeof(InT)) & (uintptr_t)(kEpc - 1));
    base = reinterpret_cast<const uint4*>(rp - shift);
    nchunks = (a.V + shift + kEpc - 1) / kEpc;
  }
};

// The 16-bit key of a logit (ckey's high half): monotone non-decreasing in
// the value, both zeros at 0x8000, -inf at 0x007f.
__device__ __forceinline__ uint32_t key16(float v) { return ckey(v) >> 16; }

// Candidates of a large-vocabulary qwen row selected on its final logits:
// every option of the caller chain (penalty from the history or a mask, the
// additive mask, EOS, temperature, a penalty of either sign), bf16 or f32
// rows, non-finite values.  The row is streamed from memory, four passes:
//  1. NaN and +inf logits, and the largest key16 over the logits not NaN;
//  2.-3. a radix select of the K-th largest key16 over its 16-bit distance
//     below the largest, high byte first (runs of equal bins added at once),
//     then the low byte inside the chosen bin;
//  4. every id whose logit is not NaN and reaches the smallest value of the
//     K-th key's bin (at most the K-th largest logit: a superset of the
//     reference's top-k survivors), staged in vocabulary order in S.cand and
//     S.candv.
// With fewer than K logits not NaN every one of them is a candidate.
// Returns the candidate count (the first kLargeCand staged), or 0xffffffff
// when a logit is +inf.  NaN logits are left out and the row flagged
// TC_FLAG_NAN_ROW: the reference's order for them at top-k is unspecified.
// The history bitmap (S.bits, bit id + boff) must be built when the penalty
// reads it.
template <typename InT>
__device__ __forceinline__ uint32_t large_candidates(const RowArgs& a, QLargeLds& S, int row, int eos,
                                                     uint32_t* row_flags, int boff) {
  constexpr int E = LargeRow<InT>::kEpc;
  const LargeRow<InT> R(a, row);
  const int t = threadIdx.x, V = a.V, nwords = (V + boff + 31) >> 5;
  const int tile = kLargeU * (int)blockDim.x;
  const uint32_t K = (uint32_t)a.K;
  const bool use_bits = a.do_pen && a.hist_mode != TC_HIST_MASK;
  // every chunk once, thread t taking chunks tb + kLargeU * t + u of each tile
  // (vocabulary order within the tile); the tile count is the same for all
  auto walk = [&](auto&& body) __attribute__((always_inline)) {
    for (int tb = 0; tb < R.nchunks; tb += tile) {
      uint4 raw[kLargeU];
#pragma unroll
      for (int u = 0; u < kLargeU; ++u) raw[u] = R.base[min(tb + kLargeU * t + u, R.nchunks - 1)];
      body(raw, tb);
    }
  };
  // the logits of chunk q (bit h of the result: element h lies in the row)
  auto logits = [&](const uint4& v, int q, float (&lv)[E]) __attribute__((always_inline)) -> uint32_t {
    const int c0 = q * E - R.shift;
    const uint32_t hb = use_bits ? bits_at_fn(S.bits, nwords, c0 + boff) : 0u;
    uint32_t in = 0;
#pragma unroll
    for (int h = 0; h < E; ++h) {
      const int e = c0 + h;
      const bool ok = e >= 0 && e < V;
      in |= (ok ? 1u : 0u) << h;
      lv[h] = ok ? qlogit_all(a, chunk_val<InT>(v, h), ((hb >> h) & 1u) != 0u, e, eos) : 0.0f;
    }
    return in;
  };
  // pass 1
  uint32_t nan = 0, pinf = 0, km = 0;
  walk([&](const uint4 (&raw)[kLargeU], int tb) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < kLargeU; ++u) {
      const int q = tb + kLargeU * t + u;
      if (q >= R.nchunks) break;
      float lv[E];
      const uint32_t in = logits(raw[u], q, lv);
#pragma unroll
      for (int h = 0; h < E; ++h) {
        if (!((in >> h) & 1u)) continue;
        if (__builtin_isnan(lv[h])) {
          nan = 1u;
          continue;
        }
        pinf |= lv[h] == __builtin_inff() ? 1u : 0u;
        km = max(km, key16(lv[h]));
      }
    }
  });
  const bool any_nan = block_or_u(nan, S.s) != 0u;
  pinf = block_or_u(pinf, S.s);
  const uint32_t kmax = block_max_u(km, S.s);
  if (any_nan) *row_flags |= TC_FLAG_NAN_ROW;
  if (pinf) return 0xffffffffu;
  // passes 2-3
  uint32_t bK = 0xffffffffu, hi = 0;
  for (int lvl = 0; lvl < 2; ++lvl) {
    if (t < 256) S.hist[t] = 0u;
    __syncthreads();
    walk([&](const uint4 (&raw)[kLargeU], int tb) __attribute__((always_inline)) {
      uint32_t run_bin = 0xffffffffu, run_n = 0;
#pragma unroll
      for (int u = 0; u < kLargeU; ++u) {
        const int q = tb + kLargeU * t + u;
        if (q >= R.nchunks) break;
        float lv[E];
        const uint32_t in = logits(raw[u], q, lv);
#pragma unroll
        for (int h = 0; h < E; ++h) {
          if (!((in >> h) & 1u) || __builtin_isnan(lv[h])) continue;
          const uint32_t dist = kmax - key16(lv[h]);
          if (lvl == 1 && (dist >> 8) != hi) continue;
          const uint32_t bin = lvl == 0 ? (dist >> 8) : (dist & 0xffu);
          if (bin != run_bin) {
            if (run_n) atomicAdd(&S.hist[run_bin], run_n);
            run_bin = bin;
            run_n = 0;
          }
          ++run_n;
        }
      }
      if (run_n) atomicAdd(&S.hist[run_bin], run_n);
    });
    __syncthreads();
    // the bin holding the K-th: the high level counts from the largest key,
    // the low level what the higher bins left
    const uint32_t need = lvl == 0 ? K : S.misc[1];
    if (wave_id() == 0) {
      const int l = lane_id();
      const uint32_t h0 = S.hist[4 * l], h1 = S.hist[4 * l + 1], h2 = S.hist[4 * l + 2], h3 = S.hist[4 * l + 3];
      const uint32_t inc = dpp_scan_u32(h0 + h1 + h2 + h3), ex = inc - (h0 + h1 + h2 + h3);
      uint32_t b = 0xffffffffu, before = 0;
      if (ex + h0 >= need) { b = 4 * l; before = ex; }
      else if (ex + h0 + h1 >= need) { b = 4 * l + 1; before = ex + h0; }
      else if (ex + h0 + h1 + h2 >= need) { b = 4 * l + 2; before = ex + h0 + h1; }
      else if (inc >= need) { b = 4 * l + 3; before = ex + h0 + h1 + h2; }
      const uint64_t m = __ballot(b != 0xffffffffu && ex < need);
      const int w = m ? __builtin_ctzll(m) : 0;
      const uint32_t bw = rl_u32(b, w), bef = rl_u32(before, w);  // every lane active
      if (l == 0) {
        S.misc[0] = m ? bw : 0xffffffffu;
        S.misc[1] = m ? need - bef : 0u;
      }
    }
    __syncthreads();
    const uint32_t found = S.misc[0];
    __syncthreads();
    if (found == 0xffffffffu) break;  // fewer than K logits not NaN: all are candidates
    if (lvl == 0) hi = found;
    else bK = (hi << 8) | found;
  }
  float thr = -__builtin_inff();
  if (bK != 0xffffffffu) {
    const uint32_t keyK = kmax - bK;
    thr = keyK <= 0x007fu ? -__builtin_inff() : untkey(keyK << 16);  // the smallest value with that key
  }
  // pass 4
  uint32_t n_c = 0;
  walk([&](const uint4 (&raw)[kLargeU], int tb) __attribute__((always_inline)) {
    uint32_t sel[kLargeU], cnt = 0;
#pragma unroll
    for (int u = 0; u < kLargeU; ++u) {
      sel[u] = 0u;
      const int q = tb + kLargeU * t + u;
      if (q < R.nchunks) {
        float lv[E];
        const uint32_t in = logits(raw[u], q, lv);
#pragma unroll
        for (int h = 0; h < E; ++h)
          sel[u] |= (((in >> h) & 1u) && !__builtin_isnan(lv[h]) && lv[h] >= thr) ? 1u << h : 0u;
      }
      cnt += (uint32_t)__builtin_popcount(sel[u]);
    }
    uint32_t tot;
    uint32_t off = n_c + block_excl_scan(cnt, S.s, &tot);
#pragma unroll
    for (int u = 0; u < kLargeU; ++u) {
      if (!sel[u]) continue;
      const int q = tb + kLargeU * t + u;
      float lv[E];
      (void)logits(raw[u], q, lv);
#pragma unroll
      for (int h = 0; h < E; ++h) {
        if (!((sel[u] >> h) & 1u)) continue;
        if (off < (uint32_t)kLargeCand) {
          const uint64_t kv = ((uint64_t)(~ckey(lv[h])) << 32) | (uint32_t)(q * E - R.shift + h);
          S.cand[off] = kv;
          S.candv[off] = kv;
        }
        ++off;
      }
    }
    n_c += tot;
  });
  return n_c;
}


// The finish of a large-vocabulary qwen row from its n_c candidates (S.cand
// and S.candv in vocabulary order): the rank sort (value descending, id
// ascending), top-k with ties kept (sampling.rs:224-249), top-p on exact terms
// with the reference's sequential sums in rank order (:255-299), softmax and
// the CDF in vocabulary order over the kept ids (:302-328).
__device__ __forceinline__ void large_finish(const RowArgs& a, QLargeLds& S, int row, uint32_t n_c, uint32_t row_flags) {
  const int t = threadIdx.x;
  const uint32_t K = (uint32_t)a.K;
  __syncthreads();
  if (n_c > (uint32_t)kLargeCand) {
    finish_row(a, row, 0u, TC_EUNSUPPORTED, row_flags);
    no_verify(a, row);
    return;
  }
  // rank order: more than 256 candidates sort as 2048 keys in registers
  const int n_pad = n_c > 256u ? kLargeCand : next_pow2((int)n_c < 2 ? 2 : (int)n_c);
  for (int j = (int)n_c + t; j < n_pad; j += blockDim.x) S.cand[j] = ~0ull;
  __syncthreads();
  if (n_pad == kLargeCand) block_sort2048(S.cand);
  else block_bitonic_sort(S.cand, n_pad);
  // top-k (sampling.rs:224-249): every value >= the K-th largest
  const uint32_t kth_hi = (uint32_t)(S.cand[K - 1] >> 32);  // ~ckey of the K-th value
  auto val_of = [](uint64_t kv) { return untkey(~(uint32_t)(kv >> 32)); };
  uint32_t ns_part = 0;
  for (int j = t; j < (int)n_c; j += blockDim.x) ns_part += (uint32_t)(S.cand[j] >> 32) <= kth_hi ? 1u : 0u;
  const uint32_t ns = block_sum_u(ns_part, S.s);
  const float vmax = val_of(S.cand[0]);
  if (vmax == __builtin_inff()) {  // a finite value overflowing to +inf: as above
    finish_row(a, row, 0u, TC_OK, row_flags);
    no_verify(a, row);
    return;
  }
  uint32_t flags = row_flags, cut = ns;
  // without verification outputs the draw's sums themselves are not needed:
  // the token is taken from a certified approximation where it is clear
  const bool quick = !a.topk_count && !a.norm;
  if (a.do_topp) {
    // top-p (sampling.rs:255-299) in rank order: e = exp(v - max), S = sequential
    // sum, running sum of e / S, cutoff at the first crossing (kept)
    float e[kLargePer], pre[kLargePer];
#pragma unroll
    for (int q = 0; q < kLargePer; ++q) {
      const uint32_t r = kLargePer * t + q;
      e[q] = r < ns ? expf_glibc(val_of(S.cand[r]) - vmax) : 0.0f;
    }
    float Sr = small_seq_prefix(e, pre, S);
    float pq[kLargePer];
#pragma unroll
    for (int q = 0; q < kLargePer; ++q) pq[q] = (kLargePer * t + q) < ns ? e[q] / Sr : 0.0f;
    small_seq_prefix(pq, pre, S);
    uint32_t first = 0xffffffffu;
#pragma unroll
    for (int q = kLargePer - 1; q >= 0; --q)
      if ((kLargePer * t + q) < ns && pre[q] > a.top_p_f) first = kLargePer * t + q;
    first = block_min_u(first, S.s);
    if (first != 0xffffffffu) cut = first + 1;
    if (cut < ns && (uint32_t)(S.cand[cut - 1] >> 32) == (uint32_t)(S.cand[cut] >> 32)) flags |= TC_FLAG_TIE_CUT;
  }
  const uint64_t last_kept = S.cand[cut - 1];
  const float u = reinterpret_cast<const float*>(a.uniforms)[row];
  if (quick) {
    // the draw: the first kept id whose running sum reaches u (none for u <= 0)
    uint32_t tok = 0xffffffffu;
    if (u > 0.0f) {
      float dq[kLargePer];
      uint32_t kp = 0;
#pragma unroll
      for (int q = 0; q < kLargePer; ++q) {
        const uint32_t j = kLargePer * t + q;
        const bool k = j < n_c && S.candv[j] <= last_kept;
        dq[q] = k ? val_of(S.candv[j]) - vmax : 0.0f;
        kp |= (k ? 1u : 0u) << q;
      }
      const uint32_t f = certified_first<true>(dq, kp, kp, (int)n_c, u, S);
      if (f != kUndecided) tok = f == 0xffffffffu ? 0u : (uint32_t)S.candv[f];
    } else {
      tok = 0u;
    }
    if (tok != 0xffffffffu) {
      finish_row(a, row, tok, TC_OK, flags);
      return;
    }
  }
  // softmax + multinomial in vocabulary order over the kept ids (sampling.rs:302-328)
  float ev[kLargePer], pre2[kLargePer];
  bool kept[kLargePer];
#pragma unroll
  for (int q = 0; q < kLargePer; ++q) {
    const uint32_t j = kLargePer * t + q;
    kept[q] = j < n_c && S.candv[j] <= last_kept;
    ev[q] = kept[q] ? expf_glibc(val_of(S.candv[j]) - vmax) : 0.0f;
  }
  const float S2 = small_seq_prefix(ev, pre2, S);
  float pv[kLargePer];
#pragma unroll
  for (int q = 0; q < kLargePer; ++q) pv[q] = kept[q] ? ev[q] / S2 : 0.0f;
  small_seq_prefix(pv, pre2, S);
  uint32_t first = 0xffffffffu;
  if (u > 0.0f) {
#pragma unroll
    for (int q = kLargePer - 1; q >= 0; --q)
      if (kept[q] && pre2[q] >= u) first = kLargePer * t + q;
  }
  first = block_min_u(first, S.s);
  const uint32_t tok = (u > 0.0f && first != 0xffffffffu) ? (uint32_t)S.candv[first] : 0u;
  finish_row(a, row, tok, TC_OK, flags);
  put_norm(a, row, S2);
  if (a.topk_count) {
    // survivors and kept ids in vocabulary order
    uint32_t cs = 0, ck = 0;
#pragma unroll
    for (int q = 0; q < kLargePer; ++q) {
      const uint32_t j = kLargePer * t + q;
      cs += (j < n_c && (uint32_t)(S.candv[j] >> 32) <= kth_hi) ? 1u : 0u;
      ck += kept[q] ? 1u : 0u;
    }
    uint32_t ts, tk;
    uint32_t os = block_excl_scan(cs, S.s, &ts);
    uint32_t ok = block_excl_scan(ck, S.s, &tk);
#pragma unroll
    for (int q = 0; q < kLargePer; ++q) {
      const uint32_t j = kLargePer * t + q;
      if (j < n_c && (uint32_t)(S.candv[j] >> 32) <= kth_hi) {
        if (os < a.cap) a.topk_ids[(size_t)row * a.cap + os] = (uint32_t)S.candv[j];
        ++os;
      }
      if (kept[q]) {
        if (ok < a.cap) {
          a.keep_ids[(size_t)row * a.cap + ok] = (uint32_t)S.candv[j];
          a.keep_probs[(size_t)row * a.cap + ok] = pv[q];
        }
        ++ok;
      }
    }
    if (t == 0) {
      a.topk_count[row] = ts;
      a.keep_count[row] = tk;
    }
  }
}


__global__ void __launch_bounds__(kLargeThreads) k_qwen_large(RowArgs a) {
  __shared__ QLargeLds S;
  const int row = blockIdx.x, t = threadIdx.x, V = a.V;
  const uint16_t* rp = reinterpret_cast<const uint16_t*>(a.logits) + (size_t)row * (size_t)a.ld;
  const int shift = (int)((reinterpret_cast<uintptr_t>(rp) >> 1) & 7u);
  const uint4* base = reinterpret_cast<const uint4*>(rp - shift);
  const int nchunks = (V + shift + 7) >> 3;
  const int eos = (a.eos_id >= 0 && a.eos_id < V) ? a.eos_id : -1;
  // history bitmap, bit id + shift: the bits of chunk q are byte q
  const int nwords = (V + shift + 31) >> 5;
  for (int w = t; w < nwords; w += blockDim.x) S.bits[w] = 0u;
  if (t < 256) S.hist[t] = 0u;
  __syncthreads();
  if (a.do_pen) {
    uint32_t h0, h1;
    hist_range(a, row, &h0, &h1);
    for (uint32_t k = h0 + (uint32_t)t; k < h1; k += blockDim.x) {
      const uint32_t id = a.hist_ids[k];
      const uint32_t b = id + (uint32_t)shift;
      if (id < (uint32_t)V) atomicOr(&S.bits[b >> 5], 1u << (b & 31u));
    }
  }
  __syncthreads();
  const uint8_t* hbytes = reinterpret_cast<const uint8_t*>(S.bits);
  // the chunks holding elements outside the row (q_lo, q_hi) or the EOS id
  // (-1: none); in_bits and eos_bits give their masks, 0xff and 0 elsewhere
  const int q_lo = shift ? 0 : -1, q_hi = ((V + shift) & 7) ? nchunks - 1 : -1;
  const int q_eos = eos >= 0 ? (eos + shift) >> 3 : -1;
  auto in_bits = [&](int q) __attribute__((always_inline)) -> uint32_t {
    if (q != q_lo && q != q_hi) return 0xffu;
    const int c0 = q * 8 - shift;  // in [-7, V)
    uint32_t inm = 0xffu;
    if (c0 < 0) inm &= 0xffu << (uint32_t)(-c0);
    if (c0 + 8 > V) inm &= (1u << (uint32_t)(V - c0)) - 1u;
    return inm;
  };
  auto eos_bits = [&](int q) __attribute__((always_inline)) -> uint32_t {
    return q == q_eos ? 1u << (uint32_t)(eos + shift - q * 8) : 0u;
  };
  // the reference's logit after the caller chain and temperature
  // (synthesis.rs:1238-1276, sampling.rs:175-184)
  auto logit = [&](float x, bool sn, int e) { return qlogit(a, x, sn, e, eos); };
  // Each streaming pass keeps kLargeU 16-byte loads in flight per thread (one
  // at a time leaves the pass bound by load latency, not by HBM).
  const int bd = (int)blockDim.x;
  // The passes walk the row a tile of kLargeU * blockDim chunks at a time,
  // thread t holding the tile's chunks kLargeU * t + u.  The first kLargeR
  // tiles are loaded once (pass A) and stay in registers for passes B and C;
  // tile kLargeR is loaded once and kept in LDS, each thread reading back only
  // the slots it wrote; the rest are streamed in every pass, the next tile's
  // loads issued before the current tile's body.  The tile count depends on V
  // only, so every thread runs every body (pass C's holds barriers).  Pass A
  // (fill) turns each word of the register and LDS tiles into its two order
  // keys (bkey16x2); the body's third argument says whether its chunks hold
  // keys (std::true_type) or the row's bits.
  const int tile = kLargeU * bd;
  uint4 cache[kLargeR][kLargeU];
  auto tiles = [&](bool fill, auto&& body) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < kLargeR; ++i)
      if (i * tile < nchunks) {
        if (fill) body(cache[i], i * tile, std::false_type{});
        else body(cache[i], i * tile, std::true_type{});
      }
    int tb = kLargeR * tile;
    uint4 raw[kLargeU], nxt[kLargeU];
    if (tb < nchunks) {
#pragma unroll
      for (int u = 0; u < kLargeU; ++u) raw[u] = fill ? base[min(tb + kLargeU * t + u, nchunks - 1)] : S.ltile[u * bd + t];
#pragma unroll
      for (int u = 0; u < kLargeU; ++u) nxt[u] = base[min(tb + tile + kLargeU * t + u, nchunks - 1)];
      if (fill) {
        body(raw, tb, std::false_type{});
#pragma unroll
        for (int u = 0; u < kLargeU; ++u) S.ltile[u * bd + t] = raw[u];
      } else {
        body(raw, tb, std::true_type{});
      }
      tb += tile;
#pragma unroll
      for (int u = 0; u < kLargeU; ++u) raw[u] = nxt[u];
    }
    for (; tb < nchunks; tb += tile) {
#pragma unroll
      for (int u = 0; u < kLargeU; ++u) nxt[u] = base[min(tb + tile + kLargeU * t + u, nchunks - 1)];
      body(raw, tb, std::false_type{});
#pragma unroll
      for (int u = 0; u < kLargeU; ++u) raw[u] = nxt[u];
    }
  };
  // pass A
  uint32_t bad = 0, kmax = 0;
  uint64_t best = 0;
  if (a.greedy) {
    uint4 raw[kLargeU], nxt[kLargeU];
#pragma unroll
    for (int u = 0; u < kLargeU; ++u) raw[u] = base[min(t + u * bd, nchunks - 1)];
    for (int q0 = t; q0 < nchunks; q0 += kLargeU * bd) {
#pragma unroll
      for (int u = 0; u < kLargeU; ++u) nxt[u] = base[min(q0 + (kLargeU + u) * bd, nchunks - 1)];
#pragma unroll
      for (int u = 0; u < kLargeU; ++u) {
        const int q = q0 + u * bd;
        if (q >= nchunks) break;
        const LChunk c = decode_lchunk(raw[u], q, shift, V, S.bits, nwords, eos);
#pragma unroll
        for (int h = 0; h < 8; ++h) {
          const int e = q * 8 - shift + h;
          const float lv = logit(c.x[h], (c.sn >> h) & 1u, e);
          const bool in = e >= 0 && e < V;
          // candle argmax skips NaN; a NaN at index 0 is never replaced
          if (in && __builtin_isnan(lv)) bad |= e == 0 ? 2u : 1u;
          const uint64_t k = ((uint64_t)ckey(lv) << 32) | (uint64_t)(~(uint32_t)e);
          best = (in && !__builtin_isnan(lv) && k > best) ? k : best;
        }
      }
#pragma unroll
      for (int u = 0; u < kLargeU; ++u) raw[u] = nxt[u];
    }
  } else {
    // the largest key outside the history, from the bf16 bits alone, two
    // values per instruction (v_pk_max_u16 over masked key pairs)
    u16x2 km2 = {0, 0};
    uint32_t bad2 = 0;
#pragma unroll
    for (int i = 0; i < kLargeR; ++i)
#pragma unroll
      for (int u = 0; u < kLargeU; ++u) cache[i][u] = base[min(i * tile + kLargeU * t + u, nchunks - 1)];
    tiles(true, [&](uint4 (&raw)[kLargeU], int tb, auto) __attribute__((always_inline)) {
#pragma unroll
      for (int u = 0; u < kLargeU; ++u) {
        const int q = tb + kLargeU * t + u;
        if (q >= nchunks) break;
        const uint32_t hb = hbytes[q];
        const uint32_t inm = in_bits(q), em = eos_bits(q);
        const uint32_t live = inm & ~hb & ~em;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint32_t w = u4_word(raw[u], j);
          const uint32_t kw = bkey16x2(w);
          km2 = __builtin_elementwise_max(km2, __builtin_bit_cast(u16x2, kw & half_mask(live, j)));
          bad2 |= nonfinite16x2(w) & half_mask(inm, j);
          u4_set(raw[u], j, kw);
        }
      }
    });
    kmax = km2.x > km2.y ? (uint32_t)km2.x : (uint32_t)km2.y;
    bad = bad2 ? 1u : 0u;
  }
  bad = block_or_u(bad, S.s);
  if (a.greedy) {  // candle argmax: first index whose value is strictly greater
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      const uint64_t other = __shfl_xor(best, o);
      best = other > best ? other : best;
    }
    if (lane_id() == 0) S.cand[wave_id()] = best;
    __syncthreads();
    if (t == 0) {
      uint64_t b = 0;
      for (int w = 0; w < num_waves(); ++w) b = S.cand[w] > b ? S.cand[w] : b;
      finish_row(a, row, (b && !(bad & 2u)) ? ~(uint32_t)(b & 0xffffffffu) : 0u, TC_OK, TC_FLAG_GREEDY);
    }
    no_verify(a, row);
    return;
  }
  // Rows the streaming passes below do not decide -- non-finite logits, a
  // negative penalty, a K-th key more than 256 keys below the largest, a K-th
  // logit overflowing to -inf -- get their candidates from large_candidates,
  // which streams the row again from memory; the common rows keep the row
  // tiles in registers throughout.
  const uint32_t K = (uint32_t)a.K;
  uint32_t row_flags = 0, n_c = 0;
  uint32_t bK = 0xffffffffu;
  if (!bad) {
    kmax = block_max_u(kmax, S.s);
    // pass B: exact histogram of the 256 keys at and below the largest
    // (two keys per 32-bit operation; a live key is at most kmax, so its
    // 16-bit distance below kmax does not wrap)
    const u16x2 kmax2 = {(unsigned short)kmax, (unsigned short)kmax};
    tiles(false, [&](const uint4 (&raw)[kLargeU], int tb, auto keyed) __attribute__((always_inline)) {
      constexpr bool kKeyed = decltype(keyed)::value;
  #pragma unroll
      for (int u = 0; u < kLargeU; ++u) {
        const int q = tb + kLargeU * t + u;
        if (q >= nchunks) break;
        const uint32_t hb = hbytes[q];
        const uint32_t inm = in_bits(q), em = eos_bits(q);
        const uint32_t live = inm & ~hb & ~em;
  #pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint32_t w = u4_word(raw[u], j);
          const uint32_t d2 = __builtin_bit_cast(uint32_t, kmax2 - __builtin_bit_cast(u16x2, kKeyed ? w : bkey16x2(w)));
          if (((live >> (2 * j)) & 1u) && (d2 & 0xff00u) == 0u) atomicAdd(&S.hist[d2 & 0xffu], 1u);
          if (((live >> (2 * j + 1)) & 1u) && (d2 >> 24) == 0u) atomicAdd(&S.hist[(d2 >> 16) & 0xffu], 1u);
        }
      }
    });
    __syncthreads();
    if (wave_id() == 0) {
      const int l = lane_id();
      const uint32_t h0 = S.hist[4 * l], h1 = S.hist[4 * l + 1], h2 = S.hist[4 * l + 2], h3 = S.hist[4 * l + 3];
      const uint32_t inc = dpp_scan_u32(h0 + h1 + h2 + h3), ex = inc - (h0 + h1 + h2 + h3);
      uint32_t b = 0xffffffffu;
      if (ex + h0 >= K) b = 4 * l;
      else if (ex + h0 + h1 >= K) b = 4 * l + 1;
      else if (ex + h0 + h1 + h2 >= K) b = 4 * l + 2;
      else if (inc >= K) b = 4 * l + 3;
      const uint64_t m = __ballot(b != 0xffffffffu && ex < K);
      const uint32_t bw = m ? rl_u32(b, __builtin_ctzll(m)) : 0xffffffffu;  // every lane active
      if (l == 0) S.misc[0] = bw;
    }
    __syncthreads();
    bK = S.misc[0];
  }
  const uint32_t keyK = kmax - bK;
  const float xK = untkey(keyK << 16 | ((keyK & 0x8000u) ? 0u : 0xffffu));
  const float thr = a.do_temp ? xK * a.tmul + 0.0f : xK;  // its logit (not in the history)
  if (bad || bK == 0xffffffffu || (a.do_pen && a.pen_f < 0.0f) || thr == -__builtin_inff()) {
    n_c = large_candidates<uint16_t>(a, S, row, eos, &row_flags, shift);
    if (n_c == 0xffffffffu) {  // a +inf logit: the reference's CDF is NaN -> index 0
      finish_row(a, row, 0u, TC_OK, row_flags);
      no_verify(a, row);
      return;
    }
  } else {
    // Penalised ids (in the history, not the EOS id) whose logit reaches thr.
    // Their logit is a non-decreasing function of the bf16 value (a multiply by
    // a positive factor, then by f32(1/T), each rounded), so they are the ids
    // whose key reaches keyP, the smallest finite key whose penalised logit
    // reaches thr (0xff80, above every finite key, when none does).  Both zeros
    // share key 0x8000 and both give a logit of zero.  Every thread finds keyP
    // by the same bisection over the finite keys [0x0080, 0xff7f].
    uint32_t keyP = 0xff80u;
    if (a.do_pen) {
      uint32_t lo = 0x0080u, hi = 0xff80u;
      while (lo < hi) {
        const uint32_t mid = (lo + hi) >> 1;
        const uint32_t b = (mid & 0x8000u) ? (mid & 0x7fffu) : (~mid & 0xffffu);
        const float x = __uint_as_float(b << 16);
        float v = x * (x > 0.0f ? a.inv_pen : a.pen_f);  // logit() for a penalised id that is not EOS
        if (a.do_temp) v = v * a.tmul + 0.0f;
        if (v >= thr) hi = mid;
        else lo = mid + 1u;
      }
      keyP = lo;
    }
    // pass C: candidates in vocabulary order, a tile at a time.  Live ids are
    // selected by key (two per instruction), penalised ones by the bitmap
    // above.
    int parity = 0;
    const uint32_t kK32 = keyK * 0x00010001u, kP32 = keyP * 0x00010001u;  // the thresholds in both halves
    tiles(false, [&](const uint4 (&raw)[kLargeU], int tb, auto keyed) __attribute__((always_inline)) {
      constexpr bool kKeyed = decltype(keyed)::value;
      uint64_t sel = 0, pens = 0;  // bit 8u + h
  #pragma unroll
      for (int u = 0; u < kLargeU; ++u) {
        const int q = tb + kLargeU * t + u;
        if (q < nchunks) {
          const uint32_t hb = hbytes[q];
          const uint32_t inm = in_bits(q), em = eos_bits(q);
          const uint32_t live = inm & ~hb & ~em, pen = inm & hb & ~em;
          uint32_t ge = 0;  // bit h: key >= keyK (live ids) or keyP (the others)
  #pragma unroll
          for (int j = 0; j < 4; ++j) {
            const uint32_t w = u4_word(raw[u], j);
            const uint32_t k2 = kKeyed ? w : bkey16x2(w);
            const uint32_t th2 = kP32 ^ ((kK32 ^ kP32) & half_mask(live, j));
            const uint32_t m2 = __builtin_bit_cast(uint32_t, __builtin_elementwise_max(__builtin_bit_cast(u16x2, k2),
                                                                                       __builtin_bit_cast(u16x2, th2)));
            const uint32_t d = m2 ^ k2;  // 0 in a half where the key reaches its threshold
            const uint32_t nz = (((d & 0x7fff7fffu) + 0x7fff7fffu) | d) & 0x80008000u;
            ge |= (((~nz >> 15) & 1u) | ((~nz >> 30) & 2u)) << (2 * j);
          }
          sel |= (uint64_t)((live | pen) & ge) << (8 * u);
          pens |= (uint64_t)pen << (8 * u);
        }
      }
      const uint32_t cnt = (uint32_t)__popcll(sel);
      const uint32_t ci = dpp_scan_u32(cnt);
      if (lane_id() == kWave - 1) S.wtot[parity][wave_id()] = ci;
      __syncthreads();
      uint32_t off, ntile;
      wave_table_u32(S.wtot[parity], &off, &ntile);
      off += n_c + ci - cnt;
      if (sel && n_c + ntile <= (uint32_t)kLargeCand) {
        // the set bits only (a few per lane); the chunk index stays static so
        // that the chunk registers are never indexed at run time
  #pragma unroll
        for (int u = 0; u < kLargeU; ++u) {
          const uint32_t x = raw[u].x, y = raw[u].y, z = raw[u].z, w = raw[u].w;
          const uint32_t pu = (uint32_t)(pens >> (8 * u));
          for (uint32_t m = (uint32_t)(sel >> (8 * u)) & 0xffu; m; m &= m - 1u) {
            const int h = __builtin_ctz(m);
            const uint32_t wv = pick_u32((h & 4) != 0, pick_u32((h & 2) != 0, w, z), pick_u32((h & 2) != 0, y, x));
            const uint32_t hw = (h & 1) ? (wv >> 16) : (wv & 0xffffu);
            const uint32_t b = (kKeyed ? unkey16(hw) : hw) << 16;
            const int e = (tb + kLargeU * t + u) * 8 - shift + h;
            const float vv = logit(__uint_as_float(b), ((pu >> h) & 1u) != 0u, e);
            const uint64_t kv = ((uint64_t)(~ckey(vv)) << 32) | (uint32_t)e;
            S.cand[off] = kv;
            S.candv[off] = kv;
            ++off;
          }
        }
      }
      n_c += ntile;
      parity ^= 1;
    });
  }
  large_finish(a, S, row, n_c, row_flags);
}

// qwen at large vocabularies for what k_qwen_large's packed bf16 passes do not
// take: f32 rows, the penalty mask (TC_HIST_MASK) and the additive mask.
// Greedy rows take candle's argmax over the final logits (the first index of
// the largest, NaN skipped, a NaN at index 0 never replaced); the others
// stream their candidates (large_candidates) and share k_qwen_large's finish.
template <typename InT>
__global__ void __launch_bounds__(kLargeThreads) k_qwen_large_gen(RowArgs a) {
  __shared__ QLargeLds S;
  const int row = blockIdx.x, t = threadIdx.x, V = a.V;
  const int eos = (a.eos_id >= 0 && a.eos_id < V) ? a.eos_id : -1;
  const int nwords = (V + 31) >> 5;
  const bool use_bits = a.do_pen && a.hist_mode != TC_HIST_MASK;
  if (use_bits) {
    for (int w = t; w < nwords; w += blockDim.x) S.bits[w] = 0u;
    __syncthreads();
    uint32_t h0, h1;
    hist_range(a, row, &h0, &h1);
    for (uint32_t k = h0 + (uint32_t)t; k < h1; k += blockDim.x) {
      const uint32_t id = a.hist_ids[k];
      if (id < (uint32_t)V) atomicOr(&S.bits[id >> 5], 1u << (id & 31u));
    }
  }
  __syncthreads();
  if (a.greedy) {
    constexpr int E = LargeRow<InT>::kEpc;
    const LargeRow<InT> R(a, row);
    uint64_t best = 0;
    uint32_t bad = 0;
    for (int q = t; q < R.nchunks; q += blockDim.x) {
      const uint4 v = R.base[q];
      const int c0 = q * E - R.shift;
      const uint32_t hb = use_bits ? bits_at_fn(S.bits, nwords, c0) : 0u;
#pragma unroll
      for (int h = 0; h < E; ++h) {
        const int e = c0 + h;
        if (e < 0 || e >= V) continue;
        const float lv = qlogit_all(a, chunk_val<InT>(v, h), ((hb >> h) & 1u) != 0u, e, eos);
        if (__builtin_isnan(lv)) {
          bad |= e == 0 ? 2u : 1u;
          continue;
        }
        const uint64_t k = ((uint64_t)ckey(lv) << 32) | (uint64_t)(~(uint32_t)e);
        best = k > best ? k : best;
      }
    }
    bad = block_or_u(bad, S.s);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      const uint64_t other = __shfl_xor(best, o);
      best = other > best ? other : best;
    }
    if (lane_id() == 0) S.cand[wave_id()] = best;
    __syncthreads();
    if (t == 0) {
      uint64_t b = 0;
      for (int w = 0; w < num_waves(); ++w) b = S.cand[w] > b ? S.cand[w] : b;
      finish_row(a, row, (b && !(bad & 2u)) ? ~(uint32_t)(b & 0xffffffffu) : 0u, TC_OK, TC_FLAG_GREEDY);
    }
    no_verify(a, row);
    return;
  }
  uint32_t row_flags = 0;
  const uint32_t n_c = large_candidates<InT>(a, S, row, eos, &row_flags, 0);
  if (n_c == 0xffffffffu) {  // a +inf logit: the reference's CDF is NaN -> index 0
    finish_row(a, row, 0u, TC_OK, row_flags);
    no_verify(a, row);
    return;
  }
  large_finish(a, S, row, n_c, row_flags);
}


hipError_t launch_k_large(bool packed, int dtype, int rows, hipStream_t st, const RowArgs& a) {
  const dim3 gr((unsigned)rows), bl(kLargeThreads);
  if (packed) hipLaunchKernelGGL(k_qwen_large, gr, bl, 0, st, a);
  else if (dtype == TC_BF16) hipLaunchKernelGGL(k_qwen_large_gen<uint16_t>, gr, bl, 0, st, a);
  else hipLaunchKernelGGL(k_qwen_large_gen<float>, gr, bl, 0, st, a);
  return hipGetLastError();
}

}  // namespace tc
