// tc_fast.h -- the streaming fast path of the indextts sampler: an LDS-only
// barrier, an exact emulation of a sequential f32 sum classified in f32
// arithmetic (SeqSum), and a one-wave finish whose order-dependent sums are
// wave scans checked against a rigorous error margin: f32 first, then f64,
// then the reference's sequential loops when a decision lies inside the f64
// margin.  Cross-lane traffic uses DPP (tc_dpp.h).
#pragma once

#include "tc_device.h"
#include "tc_dpp.h"

namespace tc {

// Barrier that waits only for this thread's LDS operations: global loads
// issued before it stay in flight.
__device__ __forceinline__ void lds_barrier() {
  __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
  __asm__ volatile("" ::: "memory");
}
__device__ __forceinline__ void lds_wait() { __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// A per-wave table of num_waves() entries in LDS: the sum over the waves
// before this one and over all of them.  Lane w reads entry w; a DPP scan
// and two readlanes (one LDS round trip, no per-wave loop).  Cross-lane:
// call with every lane of the wave active.
__device__ __forceinline__ void wave_table_u32(const uint32_t* tab, uint32_t* before, uint32_t* all) {
  const uint32_t v = lane_id() < num_waves() ? tab[lane_id()] : 0u;
  const uint32_t inc = dpp_scan_u32(v);
  const int wv = __builtin_amdgcn_readfirstlane(wave_id());
  *before = wv > 0 ? rl_u32(inc, wv - 1) : 0u;
  *all = rl_u32(inc, kWave - 1);
}
__device__ __forceinline__ void wave_table_f32(const float* tab, float* before, float* all) {
  const float v = lane_id() < num_waves() ? tab[lane_id()] : 0.0f;
  const float inc = dpp_scan_f32(v);
  const int wv = __builtin_amdgcn_readfirstlane(wave_id());
  *before = wv > 0 ? rl_f32(inc, wv - 1) : 0.0f;
  *all = rl_f32(inc, kWave - 1);
}


// ---------------------------------------------------------------- exact sequential sum
// The bits of s = -0.0f; for each term in element order: s = s + t (the
// reference's softmax denominators).  The running sum is predicted from
// approximate terms (relative error <= kSeqErr) with a bound `tau` on its
// distance from the true sequential sum.  An element whose sum before and
// after provably stays in one binade [2^e, 2^(e+1)) adds round(t / 2^(e-23))
// ulps, an integer; when the approximate term cannot settle that rounding
// the exact term is computed.  Ties, binade crossings and the first positive
// term go to a list that is replayed exactly.  The integer
// contributions are summed modulo 2^32: between two listed elements they stay
// inside one binade, so every difference the replay takes is below 2^24.
// exp_approx keeps its terms within 4 ulps (2^-21 relative) of glibc's expf.
constexpr float kSeqErr = 0x1p-21f;

// A listed element, one 16-byte LDS store and load.
struct alignas(16) ListEntry {
  float x;        // its input (exact term not yet known) or its exact term
  float P;        // the refined prediction of the running sum before it
  uint32_t q;     // integer contributions of the safe elements before it (mod 2^32)
  uint32_t info;  // bit 0: x is the exact term; bit 1: undecided (not a crossing); bits 8+: uncertainty count
};

struct SeqFastLds {
  static constexpr int kCap = 1024;
  ListEntry e[kCap];
  float ua[kCap];     // the replay's walk: exact terms of the elements that stay listed,
  uint32_t uq[kCap];  // compacted inside each chunk of 64, and the integer
                      // contributions before each (less the earlier chunks' folds)
  uint32_t cf[kCap / kWave];  // per chunk: the integer contributions folded in
  uint32_t ck[kCap / kWave];  // and the number of elements kept
  float wsum[kMaxWaves];
  float wp2[kMaxWaves];  // wave totals of the refined prediction
  uint32_t wcnt[kMaxWaves];
  uint32_t wq[kMaxWaves];
  float S;
  uint32_t bad;
};

// Classification of one element, without branches: 0 = safe (*r set: the
// element adds *r ulps of its binade), 1 = the approximate term cannot decide
// the rounding, 2 = listed (first positive term, binade crossing, tie, or a
// running sum outside [2^-90, 2^23): below 2^-90 the terms under the
// approximation's range, each within 2^-125 of theirs, could matter).
__device__ __forceinline__ uint32_t seq_classify(float P, float Pn, float a, bool exact, float m_lo, float m_hi,
                                                 uint32_t* r) {
  const uint32_t pb = __float_as_uint(P);
  const bool ok_p = P > 0.0f && pb >= 0x12800000u && pb < 0x4b000000u;
  const uint32_t eb = ok_p ? (pb & 0x7f800000u) : 0x3f800000u;
  const float lo = __uint_as_float(eb), hi = __uint_as_float(eb + 0x00800000u);
  const bool inb = ok_p && P * m_lo >= lo && Pn * m_hi < hi;
  const float q = a * __uint_as_float(0x8a800000u - eb);  // a / 2^(e-23), exact
  const float fl = __builtin_floorf(q), fr = q - fl;
  const bool amb = !exact && __builtin_fabsf(fr - 0.5f) <= q * (2.0f * kSeqErr) + 0x1p-24f;
  const bool zero = exact && a == 0.0f;
  *r = zero ? 0u : (uint32_t)fl + (fr > 0.5f ? 1u : 0u);
  return zero ? 0u : (!inb ? 2u : (amb ? 1u : (fr == 0.5f ? 2u : 0u)));
}

// |true sequential sum - prediction| <= tau * prediction for an element at
// position pos: sequential rounding (pos * 2^-24), the approximate terms
// (kSeqErr), the prediction's own f32 adds (at most ITEMS + 6 + 16) and the
// f32 products in the binade tests.
__device__ __forceinline__ float seq_tau(int pos) {
  return (float)(pos + 64) * 0x1p-24f * 1.01f + kSeqErr + 0x1p-21f;
}

// The exact sequential sum in stages, so that a kernel can put its own work
// on the same barriers:
//   predict()     f32 partial sums, their wave scan; writes L.wsum
//   -- barrier --
//   classify()    the prediction P0 of each thread; grid rounding of every
//                 element; the list of undecided and listed elements and its
//                 (count, integer sum, refined prediction) wave scans;
//                 writes L.wcnt / L.wq / L.wp2
//   -- barrier --
//   write_list()  list offsets; writes the list (false: more than kCap)
//   -- barrier --
//   replay_terms() every wave, a chunk of 64 listed elements each: their
//                 exact terms, each classified again against the refined
//                 prediction (safe ones fold into the integer sums)
//   -- barrier --
//   replay_walk() wave 0: one walk over the rest; writes L.S / L.bad
// The refined prediction P2 before a listed element is the sum of what the
// elements before it add: r ulps of the binade for a safe element of a
// short-form thread (exactly what the sequential sum adds) and the
// approximate term for every other element.  Its distance from the
// sequential sum comes from the u elements of the second kind before it
// (each rounds by at most half an ulp of the sum, 2^-24 relative, and its
// term is within kSeqErr) and at most 48 f32 adds, so seq_tau(u) bounds it as
// seq_tau(pos) bounds the first prediction.
// Thread t holds ITEMS terms at element positions pos0 + i (threads in
// order, positions increasing).  ap[i]: the term, an exact +0 where bit i of
// exact_mask is set (positions outside the row), otherwise within kSeqErr of
// the exact term f(x[i]); bits of `force` are undecided whatever ap holds.
template <int ITEMS>
struct SeqSum {
  float D, ex;
  float P0;
  uint32_t r[ITEMS];
  uint32_t listed, amb, exact;
  uint32_t cnt, rsum, ci, qi;
  float T, ex2;  // refined prediction: this thread's share and its wave-exclusive prefix
  float p2_tot;    // refined prediction of the whole sum (after write_list)
  uint32_t u_tot;  // and its uncertainty count: seq_tau(u_tot) bounds it
  float ulp0;    // short form: the ulp of the thread's binade (0: elements checked one by one)
  uint32_t c_tot, q_tot;

  __device__ __forceinline__ void predict(const float (&ap)[ITEMS], SeqFastLds& L) {
    // pairwise: a short dependent chain (any order of non-negative terms
    // keeps the bound of ITEMS - 1 roundings)
    float t[ITEMS];
#pragma unroll
    for (int i = 0; i < ITEMS; ++i) t[i] = ap[i];
#pragma unroll
    for (int h = 1; h < ITEMS; h *= 2)
#pragma unroll
      for (int i = 0; i + h < ITEMS; i += 2 * h) t[i] += t[i + h];
    D = t[0];
    const float inc = dpp_scan_f32(D);
    ex = dpp_prev_f32(inc);  // earlier lanes of this wave
    if (lane_id() == kWave - 1) L.wsum[wave_id()] = inc;
  }

  // The prediction of the whole sum (valid after the first barrier; every
  // lane of the wave active).
  __device__ __forceinline__ float total(const SeqFastLds& L) const {
    float b, t;
    wave_table_f32(L.wsum, &b, &t);
    return t;
  }

  __device__ __forceinline__ void classify(const float (&ap)[ITEMS], uint32_t exact_mask, uint32_t force, int pos0,
                                           SeqFastLds& L) {
    const int wv = wave_id();
    float off, all;
    wave_table_f32(L.wsum, &off, &all);
    P0 = off + ex;
    exact = exact_mask;
    const float tau = seq_tau(pos0 + ITEMS);
    const float m_lo = 1.0f - tau, m_hi = 1.0f + tau;
    uint32_t unsafe = 0;
    amb = force;
    // a thread whose whole range provably stays in one binade rounds every
    // term on that binade's grid; a wave takes the short form when all of its
    // threads can (no divergence inside a wave)
    const uint32_t pb0 = __float_as_uint(P0);
    const uint32_t eb0 = pb0 & 0x7f800000u;
    const bool uni = P0 > 0.0f && pb0 >= 0x12800000u && pb0 < 0x4b000000u && P0 * m_lo >= __uint_as_float(eb0) &&
                     (P0 + D) * (m_hi + 0x1p-20f) < __uint_as_float(eb0 + 0x00800000u);
    ulp0 = 0.0f;
    T = D;
    const uint64_t nub = __ballot(!uni);
    if (__popcll(nub) <= 16) {
      // the short form; a thread whose range may cross a binade (those near a
      // crossing of the running sum, at most 16 per wave here) lists every
      // element instead, r = 0 (scale 0), and the replay classifies them again
      // against the refined prediction
      ulp0 = uni ? __uint_as_float(eb0 - 0x0b800000u) : 0.0f;
      if (!uni) unsafe = (1u << ITEMS) - 1u;
      // r = round-half-even(t / 2^(e-23)) is read from the bits of the f32 sum
      // 2^23 + t * 2^(23-e) (2^23 plus that integer; 2^24 reads as 2^23).  The
      // exact term lies strictly between ap * (1 -+ 2^-20) after the product's
      // own rounding (kSeqErr is 2^-21), so both ends giving the same bits
      // settle the rounding; a tie always lies between ends that differ.  The
      // range stays below 2^e, so t * 2^(23-e) < 2^23.
      const float scale = uni ? __uint_as_float(0x8a800000u - eb0) : 0.0f;  // 2^(23-e)
      const float c_lo = scale * (1.0f - 2.0f * kSeqErr), c_hi = scale * (1.0f + 2.0f * kSeqErr);
      uint32_t dif = 0;
#pragma unroll
      for (int i = 0; i < ITEMS; ++i) {
        const uint32_t th = f2u(0x1p23f + ap[i] * c_hi), tl = f2u(0x1p23f + ap[i] * c_lo);
        dif += th ^ tl;
        r[i] = th - 0x4b000000u;
      }
      if (__ballot(dif != 0u) != 0ull) {
#pragma unroll
        for (int i = 0; i < ITEMS; ++i)
          amb |= (f2u(0x1p23f + ap[i] * c_lo) - 0x4b000000u != r[i] ? 1u : 0u) << i;
      }
    } else if (P0 > 0.0f && pb0 >= 0x12800000u && (P0 + D) * m_hi < 0x1p23f) {
      // element by element: the binade of the prediction P before it must
      // hold P and the sum after it for every value tau allows (+0 terms
      // never move the sum); the rounding as in the short form
      float P = P0;
#pragma unroll
      for (int i = 0; i < ITEMS; ++i) {
        const float Pn = P + ap[i];
        const uint32_t eb = f2u(P) & 0x7f800000u;
        const bool inb = (P * m_lo >= u2f(eb) && Pn * m_hi < u2f(eb + 0x00800000u)) || ap[i] == 0.0f;
        const float scale = u2f(0x8a800000u - eb);
        const uint32_t th = f2u(0x1p23f + ap[i] * (scale * (1.0f + 2.0f * kSeqErr)));
        const uint32_t tl = f2u(0x1p23f + ap[i] * (scale * (1.0f - 2.0f * kSeqErr)));
        r[i] = th - 0x4b000000u;
        unsafe |= (inb ? 0u : 1u) << i;
        amb |= (th != tl ? 1u : 0u) << i;
        P = Pn;
      }
    } else {
      // a zero or out-of-range prediction: every element is listed
#pragma unroll
      for (int i = 0; i < ITEMS; ++i) r[i] = 0u;
      unsafe = (1u << ITEMS) - 1u;
    }
    amb &= ~unsafe;
    listed = unsafe | amb;
    rsum = 0;
#pragma unroll
    for (int i = 0; i < ITEMS; ++i) rsum += r[i];
    if (listed) {
#pragma unroll
      for (int i = 0; i < ITEMS; ++i) rsum -= ((listed >> i) & 1u) ? r[i] : 0u;
    }
    // The refined prediction: in the short form safe elements add exactly r
    // ulps of the binade to the sequential sum and listed ones their
    // approximate term; elements checked one by one enter with their
    // approximate terms, and each counts in the bound like a listed one
    // (bits 16+ of cnt; the list count is bits 0-15).
    uint32_t slack = 0;
    if (ulp0 != 0.0f) {
      T = (float)rsum * ulp0;
      if (listed) {
#pragma unroll
        for (int i = 0; i < ITEMS; ++i) T += ((listed >> i) & 1u) ? ap[i] : 0.0f;
      }
    } else if (listed != (1u << ITEMS) - 1u) {
      slack = ITEMS;
    }
    const float t2 = dpp_scan_f32(T);
    ex2 = dpp_prev_f32(t2);
    cnt = (uint32_t)__builtin_popcount(listed) | (slack << 16);
    ci = dpp_scan_u32(cnt);
    qi = dpp_scan_u32(rsum);
    if (lane_id() == kWave - 1) {
      L.wcnt[wv] = ci;
      L.wq[wv] = qi;
      L.wp2[wv] = t2;
    }
  }

  // One pass over the elements: the list entries of the bits of lm (from
  // position k0, integer sums from q0, refined prediction from p2) and
  // stage(i) for the bits of smask.  SF: every lane of the wave in the short
  // form (safe elements add r ulps of one binade; the others their terms).
  template <bool SF, class G>
  __device__ __forceinline__ void list_pass(const float (&ap)[ITEMS], const float (&x)[ITEMS], SeqFastLds& L,
                                            uint32_t smask, G stage, uint32_t lm, uint32_t k0, uint32_t q0,
                                            uint32_t g, float p2) const {
    uint32_t k = k0, q = q0;
    float acc = 0.0f;  // SF: the listed terms before; otherwise all terms before
#pragma unroll
    for (int i = 0; i < ITEMS; ++i) {
      if ((lm >> i) & 1u) {
        const bool exa = (exact >> i) & 1u;
        ListEntry en;
        en.x = exa ? ap[i] : x[i];
        en.P = SF ? p2 + ((float)(q - q0) * ulp0 + acc) : p2 + acc;
        en.q = q;
        // bits 8+: the uncertainty count of the refined prediction
        en.info = (exa ? 1u : 0u) | (((amb >> i) & 1u) << 1) | ((k + g + (SF ? 0u : (uint32_t)i)) << 8);
        L.e[k] = en;
        ++k;
        if (SF) acc += ap[i];
      } else {
        q += r[i];
      }
      if (!SF) acc += ap[i];
      if ((smask >> i) & 1u) stage(i);
    }
  }

  // Also calls stage(i) for every element i whose bit is set in smask, in the
  // same pass (a kernel's own per-element staging).  false: more than kCap
  // listed (nothing listed is written; stage still runs).
  template <class G>
  __device__ __forceinline__ bool write_list(const float (&ap)[ITEMS], const float (&x)[ITEMS], int pos0,
                                             SeqFastLds& L, uint32_t smask, G stage) {
    uint32_t c_off, q_off;
    float p2, p2_all;
    wave_table_u32(L.wcnt, &c_off, &c_tot);
    wave_table_u32(L.wq, &q_off, &q_tot);
    wave_table_f32(L.wp2, &p2, &p2_all);
    c_off += ci - cnt;
    q_off += qi - rsum;
    p2 += ex2;
    const uint32_t g = c_off >> 16;  // uncertainty count of the threads before
    c_off &= 0xffffu;
    u_tot = (c_tot & 0xffffu) + (c_tot >> 16);
    c_tot &= 0xffffu;
    p2_tot = p2_all;
    const bool ok = c_tot <= (uint32_t)SeqFastLds::kCap;
    const uint32_t lm = ok ? listed : 0u;
    if (lm | smask) {
      // the short form is wave-uniform: one pass per form, each computing only
      // its own refined prediction
      if (__ballot(ulp0 == 0.0f) == 0ull)
        list_pass<true>(ap, x, L, smask, stage, lm, c_off, q_off, g, p2);
      else
        list_pass<false>(ap, x, L, smask, stage, lm, c_off, q_off, g, p2);
    }
    return ok;
  }

  // Every wave, chunks wave, wave + num_waves(), ... of 64 listed elements,
  // all lanes active: the exact terms, each element classified again against
  // the refined prediction (safe ones fold into the integer sums), the rest
  // compacted inside the chunk into ua/uq.
  template <class F>
  __device__ __forceinline__ void replay_terms(F f, SeqFastLds& L) const {
    const int lane = lane_id();
    const uint32_t nw = (uint32_t)num_waves(), wv = (uint32_t)__builtin_amdgcn_readfirstlane(wave_id());
    for (uint32_t c = wv; c * kWave < c_tot; c += nw) {
      const uint32_t k = c * kWave + (uint32_t)lane;
      const bool in = k < c_tot;
      ListEntry en;
      if (in) {
        en = L.e[k];
      } else {
        en.x = 0.0f;
        en.P = 0.0f;
        en.q = 0u;
        en.info = 1u;
      }
      const uint32_t info = en.info;
      const float xin = en.x;
      const float Pk = en.P;
      const float fx = f(xin);  // outside the select: f may need every lane
      const float a = (info & 1u) ? xin : fx;
      uint32_t rk = 0;
      const float tk = seq_tau((int)(info >> 8));
      const bool safe = in && seq_classify(Pk, Pk + a, a, true, 1.0f - tk, 1.0f + tk, &rk) == 0u;
      const uint32_t rs = safe ? rk : 0u;
      const uint32_t R = dpp_scan_u32(rs);  // folded contributions of the chunk up to and including k
      const bool keep = in && !safe;
      const uint64_t km = __ballot(keep);
      if (keep) {
        const uint32_t j = c * kWave + (uint32_t)__popcll(km & ((1ull << lane) - 1ull));
        L.ua[j] = a;
        L.uq[j] = en.q + (R - rs);
      }
      if (lane == kWave - 1) {
        L.cf[c] = R;
        L.ck[c] = (uint32_t)__popcll(km);
      }
    }
  }

  // Wave 0 only, after replay_terms on every wave: one walk over the kept
  // elements in element order.
  __device__ __forceinline__ void replay_walk(SeqFastLds& L) const {
    const int lane = lane_id();
    // the walk: s = s + d ulps (same binade), then s = s + a, for every kept
    // element.  Each chunk of 64 sits in lane registers (d as differences of
    // uq, 0 and +0 past the end: adding them changes nothing) and the chain
    // reads them with readlane, two dependent adds per element.
    // The checks run without branches: xb = max over the elements of
    // sb ^ (sb + d), at least 2^23 when an ulp step leaves the binade (0 for
    // d = 0).  The terms are +0 or positive, so a step from a zero sum is one
    // whose d is the first nonzero d with no positive term before it: two
    // ballots per chunk find it.
    float s = -0.0f;
    uint32_t qp = 0, bad = 0, xb = 0, fold = 0;
    bool pos = false;  // a positive term or a nonzero d seen in an earlier chunk
    const uint32_t nch = (c_tot + kWave - 1) / kWave;
    // Several chunks whose kept elements fit one wave are gathered into one
    // (lane j: kept element j, its integer sum with the folds of the chunks
    // before its own) and walked once.
    bool gather = false;
    if (nch > 1u) {
      const bool lc = (uint32_t)lane < nch;
      const uint32_t ckl = lc ? L.ck[lane] : 0u, cfl = lc ? L.cf[lane] : 0u;
      const uint32_t cki = dpp_scan_u32(ckl), cfi = dpp_scan_u32(cfl);
      const uint32_t kept = rl_u32(cki, kWave - 1);
      gather = kept <= (uint32_t)kWave;
      if (gather) {
        uint32_t src = 0, fadd = 0;
        for (uint32_t c = 0; c < nch; ++c) {
          const uint32_t n_c = rl_u32(ckl, (int)c), b = rl_u32(cki, (int)c) - n_c, f = rl_u32(cfi, (int)c) - rl_u32(cfl, (int)c);
          if ((uint32_t)lane >= b && (uint32_t)lane < b + n_c) {
            src = c * kWave + ((uint32_t)lane - b);
            fadd = f;
          }
        }
        const bool in = (uint32_t)lane < kept;
        const uint32_t qk = in ? L.uq[src] + fadd : 0u;
        const uint32_t qprev = dpp_prev_u32(qk);
        const uint32_t dv = in ? qk - qprev : 0u;
        const float av = in ? L.ua[src] : 0.0f;
        qp = kept ? rl_u32(qk, (int)kept - 1) : 0u;
        fold = rl_u32(cfi, kWave - 1);  // the folds of every chunk
        const uint64_t md = __ballot(dv != 0u), ma = __ballot(av > 0.0f);
        if (md != 0ull && (ma & ((md & (0ull - md)) - 1ull)) == 0ull) bad = 1u;
#pragma unroll
        for (int g = 0; g < kWave / 16; ++g) {
          if ((uint32_t)(g * 16) >= kept) break;
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const uint32_t di = rl_u32(dv, g * 16 + i);
            const float ai = rl_f32(av, g * 16 + i);
            const uint32_t sb = f2u(s), sb2 = sb + di;
            xb = max(xb, sb ^ sb2);
            s = u2f(sb2) + ai;
          }
        }
      }
    }
    for (uint32_t c = 0; c < (gather ? 0u : nch); ++c) {
      const uint32_t nu = (uint32_t)__builtin_amdgcn_readfirstlane((int)L.ck[c]);
      const uint32_t cfc = (uint32_t)__builtin_amdgcn_readfirstlane((int)L.cf[c]);
      if (nu == 0u) {
        fold += cfc;
        continue;
      }
      const uint32_t k = c * kWave + (uint32_t)lane;
      const bool in = (uint32_t)lane < nu;
      const uint32_t qk = in ? L.uq[k] + fold : 0u;
      const uint32_t qprev = in ? (lane == 0 ? qp : L.uq[k - 1] + fold) : 0u;
      const uint32_t dv = in ? qk - qprev : 0u;
      const float av = in ? L.ua[k] : 0.0f;
      qp = rl_u32(qk, (int)nu - 1);
      fold += cfc;
      const uint64_t md = __ballot(dv != 0u), ma = __ballot(av > 0.0f);
      if (!pos && md != 0ull && (ma & ((md & (0ull - md)) - 1ull)) == 0ull) bad = 1u;
      pos = pos || md != 0ull || ma != 0ull;
#pragma unroll
      for (int g = 0; g < kWave / 16; ++g) {
        if ((uint32_t)(g * 16) >= nu) break;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const uint32_t di = rl_u32(dv, g * 16 + i);
          const float ai = rl_f32(av, g * 16 + i);
          const uint32_t sb = f2u(s), sb2 = sb + di;
          xb = max(xb, sb ^ sb2);
          s = u2f(sb2) + ai;
        }
      }
    }
    if (xb >= (1u << 23)) bad = 1u;
    const uint32_t d = q_tot + fold - qp;
    if (d != 0u) {
      const float s2 = u2f(f2u(s) + d);
      if (!(s > 0.0f) || (f2u(s2) >> 23) != (f2u(s) >> 23)) bad = 1u;
      s = s2;
    }
    if (lane == 0) {
      L.S = s == 0.0f ? 0.0f : s;  // the terms are +0 or positive: a zero sum is +0
      L.bad = bad;
    }
  }
};

// ---------------------------------------------------------------- one-wave finish (indextts)
// Relative distance within which a comparison of two f64 sums of n
// non-negative terms may differ between a tree order and the reference's
// sequential order (n * 2^-52 for the orders, a few roundings for the
// divisions and the scan's own error), plus the difference the f64 exp of this
// library may have from the reference's libm (tc_exp_d is within 2^-49).
__device__ __forceinline__ double order_margin(uint32_t n) { return (double)(8u * n + 96u) * 0x1p-53 + 0x1p-46; }
__device__ __forceinline__ double exp_margin() { return 0x1p-46; }

struct FinLds {
  static constexpr int kCap = 128;
  uint64_t cand[kCap];      // (bits of d, history bit 31 | id) in vocabulary order
  uint64_t rkey[kCap + 4];  // rank keys, zero padded
  double wr[kCap];          // top-p weights by ascending position (rank ns-1-p)
  float wr32[kCap];         // the same in f32 (the first, f32 decisions)
  // by rank, for the interval finish: d, the separation its order needs
  // (in wr32) and the history bit
  float cd[kCap];
  alignas(16) uint32_t k32[kCap + 4];  // 32-bit score keys by candidate, zero padded
  uint8_t cpen[kCap];
  uint32_t done;  // the interval finish decided the row
};

// Rank of each lane's key among n keys in LDS (zero padded to a multiple of
// 4): the number of keys larger than it.
template <int NS>
__device__ __forceinline__ void fin_ranks(const uint64_t* rkey, uint32_t n, const uint64_t (&key)[2], uint32_t* rk0,
                                          uint32_t* rk1) {
  const uint32_t nr = (n + 3u) & ~3u;
  uint32_t a0 = 0, a1 = 0, a2 = 0, a3 = 0;
  if (NS == 1) {
    for (uint32_t j = 0; j < nr; j += 4) {
      a0 += rkey[j] > key[0] ? 1u : 0u;
      a1 += rkey[j + 1] > key[0] ? 1u : 0u;
      a2 += rkey[j + 2] > key[0] ? 1u : 0u;
      a3 += rkey[j + 3] > key[0] ? 1u : 0u;
    }
    *rk0 = (a0 + a1) + (a2 + a3);
    *rk1 = 0;
  } else {
    uint32_t b0 = 0, b1 = 0, b2 = 0, b3 = 0;
    for (uint32_t j = 0; j < nr; j += 4) {
      const uint64_t k0 = rkey[j], k1 = rkey[j + 1], k2 = rkey[j + 2], k3 = rkey[j + 3];
      a0 += k0 > key[0] ? 1u : 0u;
      a1 += k1 > key[0] ? 1u : 0u;
      a2 += k2 > key[0] ? 1u : 0u;
      a3 += k3 > key[0] ? 1u : 0u;
      b0 += k0 > key[1] ? 1u : 0u;
      b1 += k1 > key[1] ? 1u : 0u;
      b2 += k2 > key[1] ? 1u : 0u;
      b3 += k3 > key[1] ? 1u : 0u;
    }
    *rk0 = (a0 + a1) + (a2 + a3);
    *rk1 = (b0 + b1) + (b2 + b3);
  }
}

// Ranks from 32-bit keys (4 per LDS read): the number of larger keys and the
// number of equal ones (itself included; a repeated key needs the 64-bit
// ranks, which break the tie by position).
template <int NS>
__device__ __forceinline__ void fin_ranks32(const uint32_t* k32, uint32_t n, const uint32_t (&key)[2], uint32_t* rk0,
                                            uint32_t* rk1, uint32_t* eq0, uint32_t* eq1) {
  const uint32_t nr = (n + 3u) & ~3u;
  const uint4* k4 = reinterpret_cast<const uint4*>(k32);
  uint32_t g0 = 0, g1 = 0, e0 = 0, e1 = 0;
  for (uint32_t j = 0; j < nr; j += 4) {
    const uint4 v = k4[j >> 2];
    g0 += (v.x > key[0] ? 1u : 0u) + (v.y > key[0] ? 1u : 0u) + (v.z > key[0] ? 1u : 0u) + (v.w > key[0] ? 1u : 0u);
    e0 += (v.x == key[0] ? 1u : 0u) + (v.y == key[0] ? 1u : 0u) + (v.z == key[0] ? 1u : 0u) + (v.w == key[0] ? 1u : 0u);
    if (NS == 2) {
      g1 += (v.x > key[1] ? 1u : 0u) + (v.y > key[1] ? 1u : 0u) + (v.z > key[1] ? 1u : 0u) + (v.w > key[1] ? 1u : 0u);
      e1 += (v.x == key[1] ? 1u : 0u) + (v.y == key[1] ? 1u : 0u) + (v.z == key[1] ? 1u : 0u) + (v.w == key[1] ? 1u : 0u);
    }
  }
  *rk0 = g0;
  *rk1 = g1;
  *eq0 = e0;
  *eq1 = e1;
}

// One-wave finish of an indextts row from its n (K <= n <= 128) candidates
// (F.cand, vocabulary order, each with d = x - max and whether its id is in
// the history): x' = d - L, the penalty, x'' = x' / T, the top-k cut
// (generation.rs:148-161), top-p (169-194) and one draw of
// sample_without_replacement (280-303).  Every element whose score can reach
// the k-th largest is a candidate; all scores are finite.
//
// Ranks are counted against every candidate's key, broadcast from LDS.  The
// f64 weights exp(x'' - max) serve both top-p and the draw (their maxima
// coincide: the top score is never removed while min_keep >= 1, and with
// min_keep = 0 the walk keeps it too unless top_p <= 0, where the row has no
// live entry and the reference fails the same way).  The cumulative tests
// compare unnormalised tree sums against lim * sum and u * sum2;
// order_margin bounds everything that separates them from the reference's
// sequential, normalised sums, and the reference's loops run whenever a
// decision falls inside it.
// NS: the candidate slots per lane (1 when n <= 64; slot 1 then folds away).
template <int NS>
__device__ __forceinline__ void idx_fast_finish_t(const RowArgs& a, int row, uint32_t n, float L, FinLds& F,
                                                  uint32_t flags0) {
  const int lane = lane_id();
  float sc[2];
  uint32_t id[2];
  bool has[2];
  uint64_t key[2];
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const uint32_t c = (uint32_t)(q * kWave + lane);
    has[q] = q < NS && c < n;
    const uint64_t v = has[q] ? F.cand[c] : 0ull;
    id[q] = (uint32_t)v & 0x7fffffffu;
    // log_softmax, then the penalty on the log-prob (x' <= 0: s * pen), then T
    float xp = u2f((uint32_t)(v >> 32)) - L;
    xp = ((uint32_t)v & 0x80000000u) ? xp * a.pen_f : xp;
    sc[q] = a.do_temp ? xp / a.t_f : xp;
    // rank order: value descending, then the later id first (the reverse of
    // the reference's ascending stable order)
    key[q] = has[q] ? (((uint64_t)tkey(sc[q]) << 32) | c) : 0ull;
    if (q < NS) F.rkey[c] = key[q];  // zero past n: never larger than a key
  }
  lds_wait();
  // rank = number of candidates with a larger key
  uint32_t rk0 = 0, rk1 = 0;
  fin_ranks<NS>(F.rkey, n, key, &rk0, &rk1);
  const uint32_t rk[2] = {has[0] ? rk0 : 0xffffffffu, has[1] ? rk1 : 0xffffffffu};
  const uint32_t K = (uint32_t)a.K;
  const uint64_t bk0 = __ballot(rk[0] == K - 1), bk1 = __ballot(rk[1] == K - 1);
  const float kth = bk0 ? rl_f32(sc[0], __builtin_ctzll(bk0)) : (bk1 ? rl_f32(sc[1], __builtin_ctzll(bk1)) : -__builtin_inff());
  const uint64_t bm0 = __ballot(rk[0] == 0u), bm1 = __ballot(rk[1] == 0u);
  const float vmax = bm0 ? rl_f32(sc[0], __builtin_ctzll(bm0)) : rl_f32(sc[1], __builtin_ctzll(bm1));
  bool surv[2];
#pragma unroll
  for (int q = 0; q < 2; ++q) surv[q] = has[q] && !(sc[q] < kth);
  const uint64_t sm0 = __ballot(surv[0]), sm1 = __ballot(surv[1]);
  const uint32_t ns = (uint32_t)(__popcll(sm0) + __popcll(sm1));
  // ---- f32 decisions first (when no verification outputs are asked for):
  // weights exp(x'' - max) by exp_approx, within 3 ulps of the reference's
  // f64 values (below 2^-87 they are taken as 0: under 2^-125 of the sum),
  // f32 tree sums and scans.  (ns + 32) * 2^-21 of a sum bounds the f32
  // weights, sums and scans and the reference's f64 sequential normalised
  // sums together; a decision inside that margin goes to the f64 path below.
  if (!a.topk_count) {
    float w32[2];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const float dq = sc[q] - vmax;
      w32[q] = (surv[q] && dq >= -87.0f) ? exp_approx(dq) : 0.0f;
    }
    bool ok = true;
    uint32_t rc = ns;
    if (a.do_topp) {
      const float sum32 = dpp_wave_sum(w32[0] + w32[1]);
#pragma unroll
      for (int q = 0; q < 2; ++q)
        if (surv[q]) F.wr32[ns - 1u - rk[q]] = w32[q];
      lds_wait();
      float wa[2];
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const uint32_t ap = (uint32_t)(q * kWave + lane);
        wa[q] = (q < NS && ap < ns) ? F.wr32[ap] : 0.0f;
      }
      const float c0 = dpp_scan_f32(wa[0]);
      const float c1 = NS == 2 ? dpp_scan_f32(wa[1]) + rl_f32(c0, kWave - 1) : 0.0f;
      const float limS = (float)(1.0 - a.top_p_d) * sum32;
      const uint64_t rm0 = __ballot((uint32_t)lane < ns && c0 <= limS);
      const uint64_t rm1 = __ballot((uint32_t)(kWave + lane) < ns && c1 <= limS);
      const uint32_t n_rm = (uint32_t)(__popcll(rm0) + __popcll(rm1));
      rc = ns - n_rm;
      const float mg = (float)(ns + 32u) * 0x1p-21f * sum32;
      bool close = false;
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const uint32_t ap = (uint32_t)(q * kWave + lane);
        const float cq = q == 0 ? c0 : c1;
        close = close || (ap < ns && (ap + 1u == n_rm || ap == n_rm) && __builtin_fabsf(cq - limS) <= mg);
      }
      ok = __ballot(close) == 0ull;
    }
    if (ok) {
      const uint32_t live_r = rc > (uint32_t)a.min_keep ? rc : (uint32_t)a.min_keep;
      bool lv[2];
#pragma unroll
      for (int q = 0; q < 2; ++q) lv[q] = surv[q] && rk[q] < live_r;
      const uint64_t lm0 = __ballot(lv[0]), lm1 = __ballot(lv[1]);
      const uint32_t nl = (uint32_t)(__popcll(lm0) + __popcll(lm1));
      float e32[2];
#pragma unroll
      for (int q = 0; q < 2; ++q) e32[q] = lv[q] ? w32[q] : 0.0f;
      const float acc0 = dpp_scan_f32(e32[0]);
      const float acc1 = NS == 2 ? dpp_scan_f32(e32[1]) + rl_f32(acc0, kWave - 1) : acc0;
      const float sum2 = rl_f32(acc1, kWave - 1);
      const float target = (float)reinterpret_cast<const double*>(a.uniforms)[row] * sum2;
      const uint64_t pz0 = __ballot(lv[0] && e32[0] > 0.0f), pz1 = __ballot(lv[1] && e32[1] > 0.0f);
      const uint64_t hit0 = __ballot(lv[0] && e32[0] > 0.0f && acc0 > target);
      const uint64_t hit1 = __ballot(lv[1] && e32[1] > 0.0f && acc1 > target);
      ok = nl != 0u && (pz0 | pz1) != 0ull;
      uint32_t pick = 0;
      bool found = true;
      if (hit0) pick = (uint32_t)__builtin_ctzll(hit0);
      else if (hit1) pick = 64u + (uint32_t)__builtin_ctzll(hit1);
      else {
        found = false;
        pick = pz1 ? 64u + 63u - (uint32_t)__builtin_clzll(pz1) : (pz0 ? 63u - (uint32_t)__builtin_clzll(pz0) : 0u);
      }
      const float mg2 = (float)(nl + 32u) * 0x1p-21f * sum2;
      const float a_pick = rl_f32(pick < 64 ? acc0 : acc1, (int)(pick & 63u));
      bool close = __builtin_fabsf(a_pick - target) <= mg2;
      if (found) {
        const uint64_t below0 = pick < 64 ? (pz0 & ((1ull << pick) - 1ull)) : pz0;
        const uint64_t below1 = pick < 64 ? 0ull : (pz1 & ((1ull << (pick - 64u)) - 1ull));
        if (below1 || below0) {
          const uint32_t prev = below1 ? 64u + 63u - (uint32_t)__builtin_clzll(below1) : 63u - (uint32_t)__builtin_clzll(below0);
          const float a_prev = rl_f32(prev < 64 ? acc0 : acc1, (int)(prev & 63u));
          close = close || __builtin_fabsf(a_prev - target) <= mg2;
        }
      }
      if (ok && !close) {
        const uint32_t tok = rl_u32(pick < 64 ? id[0] : id[1], (int)(pick & 63u));
        if (lane == 0) {
          put_result(a, row, tok, TC_OK, flags0);
        }
        return;
      }
    }
  }
  // f64 weights (generation.rs:108-116 for top-p, 289-293 for the draw)
  const double mxd = (double)vmax;
  double w[2];
#pragma unroll
  for (int q = 0; q < 2; ++q) w[q] = surv[q] ? tc_exp_d((double)sc[q] - mxd) : 0.0;
  uint32_t flags = flags0;
  // ---- top-p: ranks [r_cut, ns) are removed, except the min_keep first
  uint32_t r_cut = ns;
  if (a.do_topp) {
    const double sum = dpp_wave_sum_d(w[0] + w[1]);
#pragma unroll
    for (int q = 0; q < 2; ++q)
      if (surv[q]) F.wr[ns - 1u - rk[q]] = w[q];
    lds_wait();
    double wa[2];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const uint32_t ap = (uint32_t)(q * kWave + lane);
      wa[q] = ap < ns ? F.wr[ap] : 0.0;
    }
    // cum(position) / sum is the reference's running sum after adding it
    const double c0 = dpp_scan_f64(wa[0]);
    const double c1 = NS == 2 ? dpp_scan_f64(wa[1]) + rl_f64(c0, kWave - 1) : 0.0;
    const double lim = 1.0 - a.top_p_d;
    const double limS = lim * sum;
    const uint64_t rm0 = __ballot((uint32_t)lane < ns && c0 <= limS);
    const uint64_t rm1 = __ballot((uint32_t)(kWave + lane) < ns && c1 <= limS);
    const uint32_t n_rm = (uint32_t)(__popcll(rm0) + __popcll(rm1));
    r_cut = ns - n_rm;
    // the decisions at the last removed and the first kept positions
    const double mg = order_margin(ns) * sum;
    bool close = false;
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const uint32_t ap = (uint32_t)(q * kWave + lane);
      const double cq = q == 0 ? c0 : c1;
      close = close || (ap < ns && (ap + 1u == n_rm || ap == n_rm) && __builtin_fabs(cq - limS) <= mg);
    }
    if (__ballot(close)) {
      // the reference's order: the sum in vocabulary order, then the ascending walk
      double sr = -0.0;
      for (uint64_t m = sm0; m; m &= m - 1) sr += rl_f64(w[0], __builtin_ctzll(m));
      for (uint64_t m = sm1; m; m &= m - 1) sr += rl_f64(w[1], __builtin_ctzll(m));
      double cum = 0.0;
      uint32_t rc = ns;
      bool near = false;
      for (int p = (int)ns - 1; p >= 0; --p) {
        const uint64_t b0 = __ballot(surv[0] && rk[0] == (uint32_t)p), b1 = __ballot(surv[1] && rk[1] == (uint32_t)p);
        const double wc = b0 ? rl_f64(w[0], __builtin_ctzll(b0)) : rl_f64(w[1], __builtin_ctzll(b1));
        cum += wc / sr;
        near = near || __builtin_fabs(cum - lim) <= exp_margin() * (cum > lim ? cum : lim);
        if (cum <= lim) rc = (uint32_t)p;
      }
      r_cut = rc;
      if (near) flags |= TC_FLAG_NEAR_TIE;
    }
  }
  const uint32_t live_r = r_cut > (uint32_t)a.min_keep ? r_cut : (uint32_t)a.min_keep;
  bool live[2];
#pragma unroll
  for (int q = 0; q < 2; ++q) live[q] = surv[q] && rk[q] < live_r;
  const uint64_t lm0 = __ballot(live[0]), lm1 = __ballot(live[1]);
  const uint32_t nl = (uint32_t)(__popcll(lm0) + __popcll(lm1));
  // ---- the draw: exp(x'' + 0.0 - max over live) = w (rank 0 is live), inverse CDF
  double e[2];
#pragma unroll
  for (int q = 0; q < 2; ++q) e[q] = live[q] ? w[q] : 0.0;
  const double acc0 = dpp_scan_f64(e[0]);
  const double acc1 = NS == 2 ? dpp_scan_f64(e[1]) + rl_f64(acc0, kWave - 1) : acc0;
  const double sum2 = rl_f64(acc1, kWave - 1);
  const double u = reinterpret_cast<const double*>(a.uniforms)[row];
  const double target = u * sum2;
  const uint64_t pz0 = __ballot(live[0] && e[0] > 0.0), pz1 = __ballot(live[1] && e[1] > 0.0);
  const uint64_t hit0 = __ballot(live[0] && e[0] > 0.0 && acc0 > target);
  const uint64_t hit1 = __ballot(live[1] && e[1] > 0.0 && acc1 > target);
  uint32_t pick;
  bool found = true;
  if (hit0) {
    pick = (uint32_t)__builtin_ctzll(hit0);
  } else if (hit1) {
    pick = 64u + (uint32_t)__builtin_ctzll(hit1);
  } else {
    found = false;  // the last positive weight
    pick = pz1 ? 64u + 63u - (uint32_t)__builtin_clzll(pz1) : (pz0 ? 63u - (uint32_t)__builtin_clzll(pz0) : 0u);
  }
  {
    // robustness: the running sums of the pick and of the positive element
    // before it against the target
    const double mg = order_margin(nl) * sum2;
    const double a_pick = rl_f64(pick < 64 ? acc0 : acc1, (int)(pick & 63u));
    // (a beam step draws later, over the joint kept sets: this draw is unused)
    bool close = !a.keep_scores && __builtin_fabs(a_pick - target) <= mg;
    if (found) {
      const uint64_t below0 = pick < 64 ? (pz0 & ((1ull << pick) - 1ull)) : pz0;
      const uint64_t below1 = pick < 64 ? 0ull : (pz1 & ((1ull << (pick - 64u)) - 1ull));
      if (below1 || below0) {
        const uint32_t prev = below1 ? 64u + 63u - (uint32_t)__builtin_clzll(below1) : 63u - (uint32_t)__builtin_clzll(below0);
        const double a_prev = rl_f64(prev < 64 ? acc0 : acc1, (int)(prev & 63u));
        close = close || (!a.keep_scores && __builtin_fabs(a_prev - target) <= mg);
      }
    }
    if (close) {
      // the reference's order: sequential sums in vocabulary order
      double s2 = -0.0;
      for (uint64_t m = lm0; m; m &= m - 1) s2 += rl_f64(e[0], __builtin_ctzll(m));
      for (uint64_t m = lm1; m; m &= m - 1) s2 += rl_f64(e[1], __builtin_ctzll(m));
      double wv[2];
#pragma unroll
      for (int q = 0; q < 2; ++q) wv[q] = live[q] ? e[q] / s2 : 0.0;
      double tot = -0.0;
      for (uint64_t m = lm0; m; m &= m - 1) tot += rl_f64(wv[0], __builtin_ctzll(m));
      for (uint64_t m = lm1; m; m &= m - 1) tot += rl_f64(wv[1], __builtin_ctzll(m));
      const double ue = u * tot;
      double acc = 0.0;
      uint32_t last = 0xffffffffu, pk = 0xffffffffu;
      bool near = false;
      for (int c = 0; c < (int)n && pk == 0xffffffffu; ++c) {
        const uint64_t lm = c < 64 ? lm0 : lm1;
        if (!((lm >> (c & 63)) & 1ull)) continue;
        if (last == 0xffffffffu) last = (uint32_t)c;  // last_positive starts at live[0]
        const double wc = rl_f64(c < 64 ? wv[0] : wv[1], c & 63);
        if (wc <= 0.0) continue;
        last = (uint32_t)c;
        acc += wc;
        near = near || __builtin_fabs(acc - ue) <= exp_margin() * tot;
        if (acc > ue) pk = (uint32_t)c;
      }
      pick = pk != 0xffffffffu ? pk : last;
      if (near) flags |= TC_FLAG_NEAR_TIE;
    }
  }
  const uint32_t tok = nl ? rl_u32(pick < 64 ? id[0] : id[1], (int)(pick & 63u)) : 0u;
  if (lane == 0) {
    put_result(a, row, tok, nl ? TC_OK : TC_ETOOFEW, flags);
    if (a.topk_count) {
      a.topk_count[row] = ns;
      a.keep_count[row] = nl;
    }
  }
  if (a.topk_count) {
    const uint64_t below = (1ull << lane) - 1ull;
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const uint64_t smq = q == 0 ? sm0 : sm1, lmq = q == 0 ? lm0 : lm1;
      const uint32_t so = q == 0 ? 0u : (uint32_t)__popcll(sm0), lo = q == 0 ? 0u : (uint32_t)__popcll(lm0);
      if (surv[q]) {
        const uint32_t j = so + (uint32_t)__popcll(smq & below);
        if (j < a.cap) a.topk_ids[(size_t)row * a.cap + j] = id[q];
      }
      if (live[q]) {
        const uint32_t j = lo + (uint32_t)__popcll(lmq & below);
        if (j < a.cap) {
          a.keep_ids[(size_t)row * a.cap + j] = id[q];
          a.keep_probs[(size_t)row * a.cap + j] = (float)(e[q] / sum2);
          if (a.keep_scores) a.keep_scores[(size_t)row * a.cap + j] = sc[q];
        }
      }
    }
  }
}

// The spacing of the floats in the binade of v (v > 0, normal): every real
// of magnitude <= v rounds to a float within half of it.
__device__ __forceinline__ float spacing_at(float v) { return u2f(f2u(v) & 0x7f800000u) * 0x1p-23f; }

// The indextts finish decided without the exact log-sum: every L in
// [Llo, Lhi] (an interval that holds the reference's log_sum) is shown to give
// the same top-k set, the same top-p cut and the same draw, and the id is
// written; false leaves the row to the exact path (nothing written).
//
// A candidate's score is s = fl(fl(fl(d - L) * c) / T) (c = pen for an id in
// the history, else 1 and no multiply), so s = c (d - L) / T + eta with
// |eta| <= r, r from the float spacings of |x'|, |x' pen| and |s| over the
// interval; s is non-increasing in L.
//   - Order.  Two ids outside the history whose d differ by more than
//     ux + T us keep their order strictly for every L, and equal d stay
//     tied; the sets cut at the top-k boundary and at the edge of the kept set
//     are the same for every L when the pair across the cut is separated by
//     three times that (an element on either side is within one separation of
//     its neighbour at the cut).  An id in the history must keep its rank
//     against every candidate: its score range [s(Lhi), s(Llo)] meets no other
//     candidate's.
//   - Weights.  With rank 0 as anchor, log w = s - s0 is
//     (c (d - L) - c0 (d0 - L)) / T + eta - eta0: taken at La it is within
//     delta = r + r0 + |c - c0| |L - La| / T of the reference's, plus the f32
//     exp and the rounding of the log weight.  A top-p or draw test compares
//     (1 - lim) A with lim B (A, B sums of weights); its margin is
//     (1 - lim) sum(w delta) over A + lim sum(w delta) over B, plus the f32
//     scans' rounding (2^-20 of the sums).
template <int NS>
__device__ __forceinline__ bool idx_cert_finish_t(const RowArgs& a, int row, uint32_t n, float La, float Llo,
                                                  float Lhi, FinLds& F) {
  const int lane = lane_id();
  float sc[2], dd[2], slo[2] = {0.0f, 0.0f}, shi[2] = {0.0f, 0.0f};
  uint32_t id[2];
  bool has[2], pen[2];
  uint64_t key[2];
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const uint32_t c = (uint32_t)(q * kWave + lane);
    has[q] = q < NS && c < n;
    const uint64_t v = has[q] ? F.cand[c] : 0ull;
    id[q] = (uint32_t)v & 0x7fffffffu;
    pen[q] = ((uint32_t)v & 0x80000000u) != 0u;
    dd[q] = u2f((uint32_t)(v >> 32));
    float xp = dd[q] - La;
    xp = pen[q] ? xp * a.pen_f : xp;
    sc[q] = a.do_temp ? xp / a.t_f : xp;
    key[q] = has[q] ? (((uint64_t)tkey(sc[q]) << 32) | c) : 0ull;
    if (q < NS) F.k32[c] = (uint32_t)(key[q] >> 32);
  }
  if (lane < 4) F.k32[NS * kWave + lane] = 0u;
  // the score range over the interval, needed only when an id in the
  // history is among the candidates
  const bool anypen = __ballot((has[0] && pen[0]) || (has[1] && pen[1])) != 0ull;
  if (anypen) {
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const uint32_t c = (uint32_t)(q * kWave + lane);
      float xh = dd[q] - Llo, xl = dd[q] - Lhi;
      xh = pen[q] ? xh * a.pen_f : xh;
      xl = pen[q] ? xl * a.pen_f : xl;
      shi[q] = has[q] ? (a.do_temp ? xh / a.t_f : xh) : -__builtin_inff();
      slo[q] = has[q] ? (a.do_temp ? xl / a.t_f : xl) : -__builtin_inff();
      (void)c;
    }
  }
  lds_wait();
  uint32_t rk0 = 0, rk1 = 0, eq0 = 0, eq1 = 0;
  {
    const uint32_t k2[2] = {(uint32_t)(key[0] >> 32), (uint32_t)(key[1] >> 32)};
    fin_ranks32<NS>(F.k32, n, k2, &rk0, &rk1, &eq0, &eq1);
  }
  if (__ballot((has[0] && eq0 > 1u) || (has[1] && eq1 > 1u))) {
    // equal scores: ranks from the 64-bit keys (the later slot first)
#pragma unroll
    for (int q = 0; q < 2; ++q)
      if (q < NS) F.rkey[q * kWave + lane] = key[q];
    if (lane < 4) F.rkey[NS * kWave + lane] = 0ull;
    lds_wait();
    fin_ranks<NS>(F.rkey, n, key, &rk0, &rk1);
  }
  const uint32_t rk[2] = {has[0] ? rk0 : 0xffffffffu, has[1] ? rk1 : 0xffffffffu};
  // ids in the history keep their rank for every L: each one's score range,
  // broadcast, meets no other candidate's
  if (anypen) {
    bool bad = false;
#pragma unroll
    for (int qp = 0; qp < 2; ++qp) {
      for (uint64_t m = __ballot(has[qp] && pen[qp]); m; m &= m - 1ull) {
        const int l = __builtin_ctzll(m);
        const float plo = rl_f32(slo[qp], l), phi = rl_f32(shi[qp], l);
#pragma unroll
        for (int q = 0; q < 2; ++q)
          bad = bad || (has[q] && !(q == qp && lane == l) && !(slo[q] > phi || shi[q] < plo));
      }
    }
    if (__ballot(bad)) return false;
  }
  const uint32_t K = (uint32_t)a.K;
  const uint64_t bk0 = __ballot(rk[0] == K - 1), bk1 = __ballot(rk[1] == K - 1);
  const float kth = bk0 ? rl_f32(sc[0], __builtin_ctzll(bk0)) : (bk1 ? rl_f32(sc[1], __builtin_ctzll(bk1)) : -__builtin_inff());
  bool surv[2];
#pragma unroll
  for (int q = 0; q < 2; ++q) surv[q] = has[q] && !(sc[q] < kth);
  const uint64_t sm0 = __ballot(surv[0]), sm1 = __ballot(surv[1]);
  const uint32_t ns = (uint32_t)(__popcll(sm0) + __popcll(sm1));
  const float T = a.do_temp ? a.t_f : 1.0f;
  const float iT = (1.0f / T) * (1.0f + 0x1p-20f);  // >= 1/T: for bounds only
  const float pn = a.pen_f;
  // per candidate: the rounding bound r and the separation its order needs
  float r[2], sep[2];
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const float bx = (Lhi - dd[q]) * (1.0f + 0x1p-20f);
    const float ux = spacing_at(bx);
    float bs = bx, rx = 0.5f * ux;
    if (pen[q]) {
      bs = bx * pn * (1.0f + 0x1p-20f);
      rx = 0.5f * (pn * ux + spacing_at(bs));
    }
    const float us = a.do_temp ? spacing_at(bs * iT * (1.0f + 0x1p-20f)) : 0.0f;
    r[q] = (rx * iT + 0.5f * us) * (1.0f + 0x1p-20f);
    sep[q] = 3.0f * (ux + T * us) * (1.0f + 0x1p-20f);
    if (has[q] && rk[q] <= ns) {
      F.cd[rk[q]] = dd[q];
      F.cpen[rk[q]] = pen[q] ? 1 : 0;
      F.wr32[rk[q]] = sep[q];
    }
  }
  lds_wait();
  // ok: the lane's candidate and the one ranked after it keep their order for
  // every L, or either is an id in the history (whose rank was checked above)
  bool ok[2];
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    ok[q] = true;
    if (has[q] && rk[q] < ns && rk[q] + 1u < n) {
      const uint32_t p = rk[q] + 1u;
      const float d1 = F.cd[p];
      ok[q] = pen[q] || F.cpen[p] != 0 || dd[q] == d1 || dd[q] - d1 > F.wr32[p];
    }
  }
  // the top-k cut: ranks K-1 .. ns-1 against their successors
  if (__ballot((has[0] && rk[0] + 1u >= K && rk[0] < ns && !ok[0]) ||
               (has[1] && rk[1] + 1u >= K && rk[1] < ns && !ok[1])))
    return false;
  // log weights against rank 0, in f64 from d (exact inputs), and their
  // uncertainty delta
  const uint64_t bm0 = __ballot(rk[0] == 0u), bm1 = __ballot(rk[1] == 0u);
  const int l0 = bm0 ? __builtin_ctzll(bm0) : __builtin_ctzll(bm1);
  const float d0 = bm0 ? rl_f32(dd[0], l0) : rl_f32(dd[1], l0);
  const float r0 = bm0 ? rl_f32(r[0], l0) : rl_f32(r[1], l0);
  const bool p0 = __builtin_amdgcn_readfirstlane(bm0 ? (pen[0] ? 1 : 0) : (pen[1] ? 1 : 0)) != 0;
  const double c0 = p0 ? (double)pn : 1.0;
  const double invT = 1.0 / (double)T;
  const float hL = __builtin_fmaxf(La - Llo, Lhi - La);
  float w[2], wd[2];
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const double ci = pen[q] ? (double)pn : 1.0;
    const double lw = (ci * ((double)dd[q] - (double)La) - c0 * ((double)d0 - (double)La)) * invT;
    const float lf = (float)lw;
    const float dlt = r[q] + r0 + (float)__builtin_fabs(ci - c0) * hL * iT + __builtin_fabsf(lf) * 0x1p-23f + 0x1p-20f;
    w[q] = (surv[q] && lf >= -87.0f) ? exp_approx(lf) : 0.0f;
    wd[q] = w[q] * dlt;
  }
  uint32_t rc = ns;
  if (a.do_topp) {
    // weights by ascending position ns-1-rank
    float wa[2], da[2];
    if (NS == 1) {
      // one forward permute per value: survivors to their positions, the
      // others to distinct lanes at or past ns
      const int dst = (surv[0] ? (int)(ns - 1u - rk[0]) : (has[0] ? (int)rk[0] : lane)) << 2;
      const float pw = __int_as_float(__builtin_amdgcn_ds_permute(dst, __float_as_int(w[0])));
      const float pd = __int_as_float(__builtin_amdgcn_ds_permute(dst, __float_as_int(wd[0])));
      wa[0] = (uint32_t)lane < ns ? pw : 0.0f;
      da[0] = (uint32_t)lane < ns ? pd : 0.0f;
      wa[1] = da[1] = 0.0f;
    } else {
#pragma unroll
      for (int q = 0; q < 2; ++q)
        if (surv[q]) {
          F.wr[ns - 1u - rk[q]] = (double)w[q];
          F.rkey[ns - 1u - rk[q]] = (uint64_t)f2u(wd[q]);
        }
      lds_wait();
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const uint32_t ap = (uint32_t)(q * kWave + lane);
        const bool in = ap < ns;
        wa[q] = in ? (float)F.wr[ap] : 0.0f;
        da[q] = in ? u2f((uint32_t)F.rkey[ap]) : 0.0f;
      }
    }
    const float cs0 = dpp_scan_f32(wa[0]);
    const float ds0 = dpp_scan_f32(da[0]);
    const float cs1 = NS == 2 ? dpp_scan_f32(wa[1]) + rl_f32(cs0, kWave - 1) : 0.0f;
    const float ds1 = NS == 2 ? dpp_scan_f32(da[1]) + rl_f32(ds0, kWave - 1) : 0.0f;
    const float sum = rl_f32(NS == 2 ? cs1 : cs0, kWave - 1);
    const float dsum = rl_f32(NS == 2 ? ds1 : ds0, kWave - 1);
    const float lim = (float)(1.0 - a.top_p_d);
    const float limS = lim * sum;
    const uint64_t rm0 = __ballot((uint32_t)lane < ns && cs0 <= limS);
    const uint64_t rm1 = __ballot((uint32_t)(kWave + lane) < ns && cs1 <= limS);
    const uint32_t n_rm = (uint32_t)(__popcll(rm0) + __popcll(rm1));
    rc = ns - n_rm;
    bool close = false;
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const uint32_t ap = (uint32_t)(q * kWave + lane);
      const float cq = q == 0 ? cs0 : cs1, eq = q == 0 ? ds0 : ds1;
      const float mg = ((1.0f - lim) * eq + lim * (dsum - eq) + 0x1p-20f * (cq + limS)) * 1.01f;
      close = close || (ap < ns && (ap + 1u == n_rm || ap == n_rm) && __builtin_fabsf(cq - limS) <= mg);
    }
    if (__ballot(close)) return false;
  }
  const uint32_t live_r = rc > (uint32_t)a.min_keep ? rc : (uint32_t)a.min_keep;
  // the edge of the kept set
  if (live_r < ns && __ballot((has[0] && rk[0] + 1u == live_r && !ok[0]) || (has[1] && rk[1] + 1u == live_r && !ok[1])))
    return false;
  bool lv[2];
#pragma unroll
  for (int q = 0; q < 2; ++q) lv[q] = surv[q] && rk[q] < live_r;
  const uint64_t lm0 = __ballot(lv[0]), lm1 = __ballot(lv[1]);
  const uint32_t nl = (uint32_t)(__popcll(lm0) + __popcll(lm1));
  float e[2], ed[2];
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    e[q] = lv[q] ? w[q] : 0.0f;
    ed[q] = lv[q] ? wd[q] : 0.0f;
  }
  const float acc0 = dpp_scan_f32(e[0]);
  const float acc1 = NS == 2 ? dpp_scan_f32(e[1]) + rl_f32(acc0, kWave - 1) : acc0;
  const float sum2 = rl_f32(acc1, kWave - 1);
  const float dacc0 = dpp_scan_f32(ed[0]);
  const float dacc1 = NS == 2 ? dpp_scan_f32(ed[1]) + rl_f32(dacc0, kWave - 1) : dacc0;
  const float dsum2 = rl_f32(dacc1, kWave - 1);
  const float u = (float)reinterpret_cast<const double*>(a.uniforms)[row];
  const float target = u * sum2;
  const uint64_t pz0 = __ballot(lv[0] && e[0] > 0.0f), pz1 = __ballot(lv[1] && e[1] > 0.0f);
  const uint64_t hit0 = __ballot(lv[0] && e[0] > 0.0f && acc0 > target);
  const uint64_t hit1 = __ballot(lv[1] && e[1] > 0.0f && acc1 > target);
  if (nl == 0u || (pz0 | pz1) == 0ull) return false;
  uint32_t pick = 0;
  bool found = true;
  if (hit0) pick = (uint32_t)__builtin_ctzll(hit0);
  else if (hit1) pick = 64u + (uint32_t)__builtin_ctzll(hit1);
  else {
    found = false;
    pick = pz1 ? 64u + 63u - (uint32_t)__builtin_clzll(pz1) : 63u - (uint32_t)__builtin_clzll(pz0);
  }
  // acc_j > u sum2 is (1 - u) acc_j - u (sum2 - acc_j) > 0: its margin weighs
  // the deltas of the two parts the same way
  auto close_at = [&](uint32_t j) -> bool {
    const float aj = rl_f32(j < 64 ? acc0 : acc1, (int)(j & 63u));
    const float dj = rl_f32(j < 64 ? dacc0 : dacc1, (int)(j & 63u));
    const float mg = ((1.0f - u) * dj + u * (dsum2 - dj) + 0x1p-20f * (aj + target)) * 1.01f;
    return __builtin_fabsf(aj - target) <= mg;
  };
  bool close = close_at(pick);
  if (found) {
    const uint64_t below0 = pick < 64 ? (pz0 & ((1ull << pick) - 1ull)) : pz0;
    const uint64_t below1 = pick < 64 ? 0ull : (pz1 & ((1ull << (pick - 64u)) - 1ull));
    if (below1 || below0) {
      const uint32_t prev = below1 ? 64u + 63u - (uint32_t)__builtin_clzll(below1) : 63u - (uint32_t)__builtin_clzll(below0);
      close = close || close_at(prev);
    }
  }
  if (close) return false;
  const uint32_t tok = rl_u32(pick < 64 ? id[0] : id[1], (int)(pick & 63u));
  if (lane == 0) put_result(a, row, tok, TC_OK, 0u);
  return true;
}

__device__ __forceinline__ bool idx_cert_finish(const RowArgs& a, int row, uint32_t n, float La, float Llo, float Lhi,
                                                FinLds& F) {
  if (n <= (uint32_t)kWave) return idx_cert_finish_t<1>(a, row, n, La, Llo, Lhi, F);
  return idx_cert_finish_t<2>(a, row, n, La, Llo, Lhi, F);
}

__device__ __forceinline__ void idx_fast_finish(const RowArgs& a, int row, uint32_t n, float L, FinLds& F,
                                                uint32_t flags0 = 0u) {
  if (n <= (uint32_t)kWave) idx_fast_finish_t<1>(a, row, n, L, F, flags0);
  else idx_fast_finish_t<2>(a, row, n, L, F, flags0);
}

}  // namespace tc
