// tc_idx_general.h -- the indextts general path (crates/indextts/src/generation.rs:95-303):
// exact log_softmax, the typical warper, the radix-selected top-k, top-p and
// the draw over the survivors staged in LDS or, past them, over the
// register-resident row.  Used by k_indextts (rows its fast path does not
// take) and k_idx_typical.
#pragma once

#include "tc_row.h"

namespace tc {

// ================================================================ indextts
// log_softmax (generation.rs:95-105) with the reference's sequential f32
// denominator reproduced exactly; returns log_sum, or NaN when a NaN logit
// makes the sum NaN.  Leaves x untouched when the row max is not finite.
template <int ITEMS>
__device__ __forceinline__ float exact_log_softmax(float (&x)[ITEMS], uint32_t vm, int e0, SeqLds& sq, ScanLds& sc,
                                                   BlockScratch& s, float* stage, int V) {
  float m = -__builtin_inff();
  uint32_t nan_any = 0;
#pragma unroll
  for (int i = 0; i < ITEMS; ++i)
    if ((vm >> i) & 1u) {
      m = rmaxf(m, x[i]);
      nan_any |= __builtin_isnan(x[i]) ? 1u : 0u;
    }
  const float mx = block_max(m, s);
  nan_any = block_or_u(nan_any, s);
  if (!__builtin_isfinite(mx)) return __builtin_nanf("");
  float S;
  if (nan_any) {
    S = __builtin_nanf("");
  } else {
    // terms exp(x - max): approximate (tc_expf_fast) where that is safe to
    // test against; the sum computes the exact glibc bits where it needs them
    float ap[ITEMS];
    uint32_t exm = 0, slow = 0;
#pragma unroll
    for (int i = 0; i < ITEMS; ++i) {
      const float d = x[i] - mx;
      const bool v = (vm >> i) & 1u;
      ap[i] = (v && d >= -87.0f) ? tc_expf_fast(d) : 0.0f;
      if (!v) exm |= 1u << i;
      if (v && !(d >= -87.0f)) slow |= 1u << i;
    }
    auto exact = [mx](float xi) { return expf_glibc(xi - mx); };
    while (__ballot(slow != 0u)) {  // tiny terms: the exact value up front
      if (slow) {
        const int i = __builtin_ctz(slow);
        put_item<ITEMS>(ap, i, exact(pick_item<ITEMS>(x, i)));
        exm |= 1u << i;
        slow &= slow - 1u;
      }
    }
    SeqThread<ITEMS> th;
    if (!block_seqsum<ITEMS>(ap, exm, x, exact, e0, TC_EXPF_FAST_ULPS, th, sq, sc, &S)) {
      float ex[ITEMS];
#pragma unroll
      for (int i = 0; i < ITEMS; ++i) ex[i] = ((vm >> i) & 1u) ? expf_glibc(x[i] - mx) : 0.0f;
      S = block_seqsum_slow<ITEMS>(ex, e0, V, stage, kMaxVocabReg / 4, &sq.S);
    }
  }
  const float L = logf_glibc(S);
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) x[i] = (x[i] - mx) - L;
  return L;
}

struct IdxGenLds {
  uint8_t seen[kMaxVocabReg];
  union {
    SurvLds sv;
    uint32_t wide[kMaxVocabReg];  // idx_wide: the survivors' keys in rank order
  };
  uint32_t hist[256];
  BlockScratch s;
  ScanLds sc;
  SeqLds sq;
  WalkLds walk;
  uint32_t out[4];
};

// The typical warper (generation.rs:196-248, TypicalLogitsWarper) on the
// penalised log-probs x, in place: ids whose |(-nz) - ent| exceeds that of
// the first id (in ascending order of it, ties by id) at which the running
// softmax mass reaches `mass` are set to -inf.  nz = log_softmax(x) and the
// expf in ent's terms are the reference's bits (exact_log_softmax,
// expf_glibc); each term -(double)nz * (double)expf(nz) is exact in f64.
//
// The reference's f64 sums (ent in index order; the softmax denominator and
// the running mass in the sorted order) are not reproduced; the cut is
// certified instead.  ent is a block sum within E = (2V + 64) 2^-53 ent of the
// reference's sequential one (non-negative terms), so each |(-nz) - ent|
// is known within E plus an ulp.  The cut key theta comes from a radix
// select over the bit patterns of |(-nz) - ent| (non-negative doubles order
// as integers), weighted by exp(x - max): at each level the key range is cut
// into 1024 bins, the bin where the weight below reaches mass * sum is kept.
// The row is certified when (a) no id outside theta's group lies within the
// uncertainty of theta and theta's group holds one nz value, and (b) the
// weight strictly below theta is under mass * sum and the weight through
// theta's group above it, each by (4V + 64) 2^-53 + 2^-46 of the sum (the
// reference's f64 exp and sequential sums against these).  Otherwise the
// cut is taken as computed and TC_FLAG_NEAR_TIE is returned.
//
// Rows with a NaN or +inf score keep every id: the reference's softmax is
// NaN or all zero there, so its running mass never reaches `mass` and the
// cut falls on the last id.  Returns the flags to add.
template <int ITEMS>
__device__ __forceinline__ uint32_t idx_typical(const RowArgs& a, float (&x)[ITEMS], uint32_t vm, int e0,
                                             IdxGenLds& G) {
  BlockScratch& s = G.s;
  double* bw = G.sv.w;      // [1024] bin weights (the survivor stage is free until compaction)
  uint32_t* bc = G.sv.idx;  // [1024] bin counts
  uint64_t* m64 = G.sv.key; // [0] range low, [1] range high, [2] chosen bin, [3] nz bits min, [4] max
  double* md = reinterpret_cast<double*>(G.sv.key + 8);  // [0] weight below the chosen bin
  const int t = threadIdx.x, bd = (int)blockDim.x, V = a.V;
  uint32_t bad = 0, fin = 0;
#pragma unroll
  for (int i = 0; i < ITEMS; ++i)
    if ((vm >> i) & 1u) {
      bad |= (__builtin_isnan(x[i]) || x[i] == __builtin_inff()) ? 1u : 0u;
      fin |= x[i] != -__builtin_inff() ? 1u : 0u;
    }
  bad = block_or_u(bad, s);
  fin = block_or_u(fin, s);
  if (bad || !fin) return 0u;
  // nz and the entropy's terms
  float nz[ITEMS];
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) nz[i] = x[i];
  exact_log_softmax<ITEMS>(nz, vm, e0, G.sq, G.sc, s, reinterpret_cast<float*>(&G.sv), V);
  double part = 0.0;
#pragma unroll
  for (int i = 0; i < ITEMS; ++i)
    if (((vm >> i) & 1u) && nz[i] != -__builtin_inff()) part += -(double)nz[i] * (double)expf_glibc(nz[i]);
  double ent;
  (void)block_excl_scan_d(part, G.sc, &ent);
  const double e_ent = (double)(2 * V + 64) * 0x1p-53 * ent + 0x1p-1000;
  auto key_of = [&](float z) { return (uint64_t)__double_as_longlong(fabs(-(double)z - ent)); };
  // weights exp(x - max) in f64 (the reference's softmax_f64 numerators)
  double w[ITEMS];
  double mx = -__builtin_inf();
#pragma unroll
  for (int i = 0; i < ITEMS; ++i)
    if ((vm >> i) & 1u) mx = rmaxd(mx, (double)x[i]);
  mx = block_max_d(mx, s);
  double wpart = 0.0;
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) {
    w[i] = ((vm >> i) & 1u) ? tc_exp_d((double)x[i] - mx) : 0.0;
    wpart += w[i];
  }
  double wsum;
  (void)block_excl_scan_d(wpart, G.sc, &wsum);
  const double target = a.typical_mass * wsum;
  // the range of the keys
  uint64_t klo = ~0ull, khi = 0;
#pragma unroll
  for (int i = 0; i < ITEMS; ++i)
    if ((vm >> i) & 1u) {
      const uint64_t k = key_of(nz[i]);
      klo = k < klo ? k : klo;
      khi = k > khi ? k : khi;
    }
  if (t == 0) {
    m64[0] = ~0ull;
    m64[1] = 0;
    md[0] = 0.0;
  }
  __syncthreads();
  if (klo != ~0ull) {
    atomicMin(reinterpret_cast<unsigned long long*>(&m64[0]), (unsigned long long)klo);
    atomicMax(reinterpret_cast<unsigned long long*>(&m64[1]), (unsigned long long)khi);
  }
  __syncthreads();
  const uint64_t kmax_all = m64[1];
  uint64_t theta = kmax_all;  // no crossing: the cut falls on the last id
  for (int level = 0; level < 8; ++level) {
    const uint64_t lo = m64[0], hi = m64[1];
    const double below = md[0];
    if (lo == hi) {
      theta = lo;
      break;
    }
    const uint64_t span = hi - lo;
    const int sh = (64 - __builtin_clzll(span)) > 10 ? (64 - __builtin_clzll(span)) - 10 : 0;
    for (int b = t; b < 1024; b += bd) {
      bw[b] = 0.0;
      bc[b] = 0u;
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < ITEMS; ++i) {
      if (!((vm >> i) & 1u)) continue;
      const uint64_t k = key_of(nz[i]);
      if (k < lo || k > hi) continue;
      const uint32_t b = (uint32_t)((k - lo) >> sh);
      atomicAdd(&bw[b], w[i]);
      atomicAdd(&bc[b], 1u);
    }
    __syncthreads();
    if (wave_id() == 0) {
      // lane l takes bins 16 l .. 16 l + 15
      const int l = lane_id();
      double lw = 0.0;
#pragma unroll
      for (int j = 0; j < 16; ++j) lw += bw[16 * l + j];
      const double inc = wave_incl_scan_d(lw);
      double run = below + (inc - lw);
      int found = -1;
      double before = 0.0;
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const double nr = run + bw[16 * l + j];
        if (found < 0 && bc[16 * l + j] > 0u && nr >= target) {
          found = 16 * l + j;
          before = run;
        }
        run = nr;
      }
      const uint64_t hit = __ballot(found >= 0);
      if (l == 0) m64[2] = hit ? (uint64_t)0 : ~0ull;
      if (hit && l == __builtin_ctzll(hit)) {
        m64[2] = (uint64_t)found;
        md[0] = before;
      }
    }
    __syncthreads();
    const uint64_t bsel = m64[2];
    if (bsel == ~0ull) {  // the whole row stays below the mass
      theta = kmax_all;
      break;
    }
    const uint64_t nlo = lo + (bsel << sh);
    const uint64_t nhi = (sh + 10 >= 64 || ((bsel + 1) << sh) - 1 > hi - lo) ? hi : lo + ((bsel + 1) << sh) - 1;
    __syncthreads();
    if (t == 0) {
      m64[0] = ~0ull;
      m64[1] = 0;
    }
    __syncthreads();
    klo = ~0ull;
    khi = 0;
#pragma unroll
    for (int i = 0; i < ITEMS; ++i)
      if ((vm >> i) & 1u) {
        const uint64_t k = key_of(nz[i]);
        if (k >= nlo && k <= nhi) {
          klo = k < klo ? k : klo;
          khi = k > khi ? k : khi;
        }
      }
    if (klo != ~0ull) {
      atomicMin(reinterpret_cast<unsigned long long*>(&m64[0]), (unsigned long long)klo);
      atomicMax(reinterpret_cast<unsigned long long*>(&m64[1]), (unsigned long long)khi);
    }
    __syncthreads();
  }
  // certification: the weights below and through theta's group, the ids near
  // theta, the nz values inside the group
  const double th = __longlong_as_double((long long)theta);
  const double band = 2.0 * (e_ent + th * 0x1p-52) + 0x1p-1000;
  double wlt = 0.0, weq = 0.0;
  uint32_t amb = 0, zlo = ~0u, zhi = 0u;
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) {
    if (!((vm >> i) & 1u)) continue;
    const uint64_t k = key_of(nz[i]);
    const double sh_i = __longlong_as_double((long long)k);
    if (k < theta) wlt += w[i];
    if (k == theta) {
      weq += w[i];
      const uint32_t zb = __float_as_uint(nz[i]);
      zlo = zb < zlo ? zb : zlo;
      zhi = zb > zhi ? zb : zhi;
    } else if (fabs(sh_i - th) <= band) {
      amb = 1u;
    }
  }
  if (t == 0) {
    m64[3] = ~0ull;
    m64[4] = 0;
  }
  double wlt_all, weq_all;
  (void)block_excl_scan_d(wlt, G.sc, &wlt_all);
  (void)block_excl_scan_d(weq, G.sc, &weq_all);
  if (zlo != ~0u) {
    atomicMin(reinterpret_cast<unsigned long long*>(&m64[3]), (unsigned long long)zlo);
    atomicMax(reinterpret_cast<unsigned long long*>(&m64[4]), (unsigned long long)zhi);
  }
  amb = block_or_u(amb, s);
  const double marg = ((double)(4 * V + 64) * 0x1p-53 + 0x1p-46) * wsum;
  bool certain = !amb && m64[3] == m64[4];
  if (theta == kmax_all && wlt_all + weq_all < target) {
    certain = certain && wlt_all + weq_all <= target - marg;  // no crossing
  } else {
    certain = certain && wlt_all <= target - marg && wlt_all + weq_all >= target + marg;
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < ITEMS; ++i)
    if (((vm >> i) & 1u) && key_of(nz[i]) > theta) x[i] = -__builtin_inff();
  return certain ? 0u : (uint32_t)TC_FLAG_NEAR_TIE;
}

// top-p (generation.rs:169-194) and the draw (280-303) over more survivors
// than the LDS stage holds (top_k off or above kSurvCap, or ties at the k-th
// score), from the register-resident row x of final scores (surv: the n
// survivors of the top-k cut).
//  * top-p: the survivors' keys are sorted ascending (total_cmp; the
//    reference's stable sort keeps equal scores in id order).  Equal scores
//    are equal terms, so the running sum over rank positions needs no ids:
//    positions ITEMS * t + i in registers, f64 weights exp(v - max) and their
//    block prefix W, the cut at the first position whose W / S exceeds
//    1 - top_p, kept from min(cut, n - min_keep) on.  The kept ids are the
//    scores above the cut position's and, of those equal to it, the highest
//    ids, as many as the positions from the cut to the end of its group.
//    A row whose max is not finite keeps only its min_keep largest (the
//    reference's probabilities are all zero); a NaN score keeps every
//    survivor (its sum is NaN, so no running sum is <= 1 - top_p).
//  * the draw: over the kept finite scores in vocabulary order, the first id
//    whose prefix of exp(v + 0 - max) exceeds u times the total.
// The reference's sums are sequential in their own orders; these are block
// sums.  A decision whose sides lie within order_margin(n) of each other
// (n * 2^-50 relative, and the f64 exp's 2^-46) is taken again by the
// reference's loops in its own order (staged_walk: the softmax denominator in
// vocabulary order and the running sum in rank order; the draw's three
// loops), and the row flagged TC_FLAG_NEAR_TIE when even that decision lies
// within the f64 exp's error of its limit and some weight is not exact
// (exp(0) and underflowed zeros are).
template <int ITEMS>
__device__ __forceinline__ void idx_wide(const RowArgs& a, const float (&x)[ITEMS], uint32_t surv, uint32_t vm, int e0,
                                         uint32_t n, uint32_t flags, IdxGenLds& G) {
  BlockScratch& s = G.s;
  ScanLds& sc = G.sc;
  WalkLds& WL = G.walk;
  double* stage = reinterpret_cast<double*>(G.wide);
  const int row = blockIdx.x, t = threadIdx.x;
  if (a.topk_count) {
    write_ids<ITEMS>(a.topk_ids, a.cap, row, surv, e0, s);
    if (t == 0) a.topk_count[row] = n;
  }
  uint32_t key[ITEMS];
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) key[i] = tkey(x[i]);
  uint32_t kept = surv;
  if (a.do_topp) {
    uint32_t rk[ITEMS];
    block_rank_keys<ITEMS>(key, surv, n, false, G.wide, s, rk);
    double md = -__builtin_inf();
    uint32_t nan_any = 0;
#pragma unroll
    for (int i = 0; i < ITEMS; ++i)
      if ((surv >> i) & 1u) {
        md = rmaxd(md, (double)x[i]);
        nan_any |= __builtin_isnan(x[i]) ? 1u : 0u;
      }
    md = block_max_d(md, s);
    nan_any = block_or_u(nan_any, s);
    const uint32_t floor_keep = n > (uint32_t)a.min_keep ? n - (uint32_t)a.min_keep : 0u;
    uint32_t c = n;  // first kept position
    uint32_t kc = 0;
    if (!__builtin_isfinite(md)) {
      c = floor_keep;
    } else if (!nan_any) {
      const int p0 = ITEMS * t;
      auto wt = [&](int i) { return p0 + i < (int)n ? tc_exp_d((double)untkey(opaque(rk[i])) - md) : 0.0; };
      double part = 0.0;
#pragma unroll
      for (int i = 0; i < ITEMS; ++i) part += wt(i);
      double S;
      const double W0 = block_excl_scan_d(part, sc, &S);
      const double lim = 1.0 - a.top_p_d;
      // removed: the positions whose running sum is <= lim (a prefix)
      uint32_t rm = 0;
      double W = W0;
#pragma unroll
      for (int i = 0; i < ITEMS; ++i) {
        W += wt(i);
        rm += (p0 + i < (int)n && W / S <= lim) ? 1u : 0u;
      }
      uint32_t r_star = block_sum_u(rm, s);
      // the positions either side of the cut must be clear of lim
      uint32_t near = 0, inexact = 0;
      W = W0;
#pragma unroll
      for (int i = 0; i < ITEMS; ++i) {
        W += wt(i);
        const uint32_t p = (uint32_t)(p0 + i);
        if (p < n && (p + 1u == r_star || p == r_star) && !settled(W / S, lim, n)) near = 1;
        if (p < n && untkey(rk[i]) != md && wt(i) > 0.0) inexact = 1;
      }
      if (block_or_u(near, s)) {
        inexact = block_or_u(inexact, s);
        // the reference's loops: the denominator in vocabulary order, then
        // the running sum in rank order up to its first value above lim
        const VocabPos<ITEMS> vp = vocab_pos<ITEMS>(surv, s);
        auto wx = [&](int i) { return tc_exp_d((double)opaque(x[i]) - md); };
        double Sq = -0.0;
        staged_walk<ITEMS>(n, vp, wx, stage, WL, [&](uint32_t, double v) {
          Sq += v;
          return true;
        });
        if (t == 0) WL.d[0] = Sq;
        __syncthreads();
        Sq = WL.d[0];
        double cum = 0.0, c_lo = -1.0, c_hi = 2.0;
        uint32_t r = 0;
        auto rpos = [&](int i) { return p0 + i < (int)n ? (uint32_t)(p0 + i) : 0xffffffffu; };
        staged_walk<ITEMS>(n, rpos, wt, stage, WL, [&](uint32_t, double v) {
          cum += v / Sq;
          if (cum <= lim) {
            ++r;
            c_lo = cum;
            return true;
          }
          c_hi = cum;
          return false;
        });
        if (t == 0) {
          WL.u[0] = r;
          WL.u[1] = (inexact && ((r > 0u && !settled_exp(c_lo, lim)) || (r < n && !settled_exp(c_hi, lim)))) ? 1u : 0u;
        }
        __syncthreads();
        r_star = WL.u[0];
        if (WL.u[1]) flags |= TC_FLAG_NEAR_TIE;
        __syncthreads();
      }
      c = r_star < floor_keep ? r_star : floor_keep;
    } else {
      c = 0;
    }
    // the key at position c, from the registers (the stage may be in use)
#pragma unroll
    for (int i = 0; i < ITEMS; ++i)
      if ((uint32_t)(ITEMS * t + i) == c) WL.u[2] = rk[i];
    __syncthreads();
    kc = WL.u[2];
    __syncthreads();
    if (c < n) {
      uint32_t lt = 0;
#pragma unroll
      for (int i = 0; i < ITEMS; ++i) lt += (((surv >> i) & 1u) && key[i] < kc) ? 1u : 0u;
      const uint32_t g0 = block_sum_u(lt, s);
      kept = select_above_and_ties<ITEMS>(key, surv, kc, c - g0, 0xffffffffu, s);
    } else {
      kept = 0;
    }
  }
  // sample_without_replacement with one draw over the kept finite scores
  uint32_t live = 0;
#pragma unroll
  for (int i = 0; i < ITEMS; ++i)
    if (((kept >> i) & 1u) && __builtin_isfinite(x[i])) live |= 1u << i;
  const uint32_t nl = block_sum_u((uint32_t)__builtin_popcount(live), s);
  if (nl < 1u) {
    finish_row(a, row, 0u, TC_ETOOFEW, flags);
    if (t == 0 && a.keep_count) a.keep_count[row] = 0;
    return;
  }
  double ml = -__builtin_inf();
#pragma unroll
  for (int i = 0; i < ITEMS; ++i)
    if ((live >> i) & 1u) ml = rmaxd(ml, (double)x[i] + 0.0);
  ml = block_max_d(ml, s);
  auto ew = [&](int i) { return ((live >> i) & 1u) ? tc_exp_d(((double)opaque(x[i]) + 0.0) - ml) : 0.0; };
  double part = 0.0;
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) part += ew(i);
  double E;
  double P = block_excl_scan_d(part, sc, &E);
  const double u = reinterpret_cast<const double*>(a.uniforms)[row];
  const double uE = u * E;
  uint32_t first = 0xffffffffu, last = 0u, inexact = 0u;
  double f_in = 0.0, f_ex = 0.0;
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) {
    const double ei = ew(i);
    if (!((live >> i) & 1u) || !(ei > 0.0)) continue;
    const double prev = P;
    P += ei;
    last = (uint32_t)(e0 + i) + 1u;
    inexact |= ((double)x[i] + 0.0) != ml ? 1u : 0u;
    if (first == 0xffffffffu && P > uE) {
      first = (uint32_t)(e0 + i);
      f_in = P;
      f_ex = prev;
    }
  }
  uint32_t tok = block_min_u(first, s);
  const uint32_t lastp = block_max_u(last, s);
  uint32_t near = tok == 0xffffffffu ? 1u : 0u;
  // (no positive weight before the pick: the reference's running sum there is
  // exactly 0, never above u * total)
  if (first == tok && tok != 0xffffffffu && (!settled(f_in, uE, nl) || (f_ex > 0.0 && !settled(f_ex, uE, nl))))
    near = 1u;
  if (block_or_u(near, s)) {
    inexact = block_or_u(inexact, s);
    // the reference's loops over the live ids in vocabulary order: sum,
    // total of the quotients, the walk
    const VocabPos<ITEMS> vp = vocab_pos<ITEMS>(live, s);
    double sum = -0.0;
    staged_walk<ITEMS>(nl, vp, ew, stage, WL, [&](uint32_t, double v) {
      sum += v;
      return true;
    });
    if (t == 0) WL.d[0] = sum;
    __syncthreads();
    sum = WL.d[0];
    auto qw = [&](int i) { return ew(i) / sum; };
    double total = -0.0;
    staged_walk<ITEMS>(nl, vp, qw, stage, WL, [&](uint32_t, double v) {
      total += v;
      return true;
    });
    if (t == 0) WL.d[1] = total;
    __syncthreads();
    total = WL.d[1];
    const double uu = u * total;
    double acc = 0.0;
    uint32_t lastj = 0, pick = 0xffffffffu;
    double a_in = 0.0, a_ex = 0.0;
    staged_walk<ITEMS>(nl, vp, qw, stage, WL, [&](uint32_t j, double v) {
      if (!(v > 0.0)) return true;
      lastj = j;
      a_ex = acc;
      acc += v;
      if (acc > uu) {
        pick = j;
        a_in = acc;
        return false;
      }
      return true;
    });
    if (t == 0) {
      WL.u[0] = pick != 0xffffffffu ? pick : lastj;
      WL.u[1] = (inexact && (pick == 0xffffffffu || !settled_exp(a_in, uu) || (a_ex > 0.0 && !settled_exp(a_ex, uu))))
                    ? 1u : 0u;
    }
    __syncthreads();
    const uint32_t jp = WL.u[0];
    if (WL.u[1]) flags |= TC_FLAG_NEAR_TIE;
    __syncthreads();
    uint32_t id = 0xffffffffu;
#pragma unroll
    for (int i = 0; i < ITEMS; ++i)
      if (vp(i) == jp) id = (uint32_t)(e0 + i);
    tok = block_min_u(id, s);
  } else if (tok == 0xffffffffu) {
    tok = lastp - 1u;
  }
  finish_row(a, row, tok, TC_OK, flags);
  if (a.keep_count) {
    uint32_t tot;
    uint32_t p = block_excl_scan((uint32_t)__builtin_popcount(live), s, &tot);
#pragma unroll
    for (int i = 0; i < ITEMS; ++i)
      if ((live >> i) & 1u) {
        if (p < a.cap) {
          a.keep_ids[(size_t)row * a.cap + p] = (uint32_t)(e0 + i);
          a.keep_probs[(size_t)row * a.cap + p] = (float)(ew(i) / E);
          if (a.keep_scores) a.keep_scores[(size_t)row * a.cap + p] = x[i];
        }
        ++p;
      }
    if (t == 0) a.keep_count[row] = nl;
  }
}

// General path: any K, non-finite scores, more candidates than the fast path
// stages, the typical warper (TYPICAL: k_idx_typical).  Survivors of the
// top-k cut are staged in LDS (at most kSurvCap); more take idx_wide.
template <typename InT, int ITEMS, bool TYPICAL = false>
__device__ __forceinline__ void idx_general(const RowArgs& a, IdxGenLds& G) {
  uint8_t* s_seen = G.seen;
  SurvLds& sv = G.sv;
  uint32_t* s_hist = G.hist;
  BlockScratch& s = G.s;
  ScanLds& sc = G.sc;
  SeqLds& sq = G.sq;
  uint32_t* s_out = G.out;
  const int row = blockIdx.x, t = threadIdx.x, V = a.V;
  const InT* rp = reinterpret_cast<const InT*>(a.logits) + (size_t)row * (size_t)a.ld;
  float x[ITEMS];
  int shift;
  load_row<ITEMS>(rp, V, x, &shift);
  const uint32_t vm = valid_mask<ITEMS>(V, shift);
  const int e0 = t * ITEMS - shift;
  if (a.do_pen) build_seen(a, row, s_seen, s);
  const float log_sum = exact_log_softmax<ITEMS>(x, vm, e0, sq, sc, s, reinterpret_cast<float*>(&sv), V);
  put_norm(a, row, log_sum);
  // repetition penalty on the log-probs (generation.rs:122-134), the typical
  // warper (:649-651), temperature (137-142)
#pragma unroll
  for (int i = 0; i < ITEMS; ++i)
    if (((vm >> i) & 1u) && a.do_pen && s_seen[e0 + i]) x[i] = x[i] < 0.0f ? x[i] * a.pen_f : x[i] / a.pen_f;
  uint32_t row_flags = 0;
  if constexpr (TYPICAL) {
    __syncthreads();
    row_flags = idx_typical<ITEMS>(a, x, vm, e0, G);
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < ITEMS; ++i)
    if (((vm >> i) & 1u) && a.do_temp) x[i] = x[i] / a.t_f;
  // general path: radix select over the whole row, survivors staged in LDS
  float kth = -__builtin_inff();
  bool cut = false;
  if (a.K > 0 && a.K < V) {
    uint32_t key[ITEMS];
#pragma unroll
    for (int i = 0; i < ITEMS; ++i) key[i] = tkey(x[i]);
    uint32_t kk;
    if (block_kth_largest<ITEMS>(key, vm, (uint32_t)a.K, s_hist, s, &kk)) {
      kth = untkey(kk);
      cut = true;
    }
  }
  uint32_t surv = 0;
#pragma unroll
  for (int i = 0; i < ITEMS; ++i)
    if (((vm >> i) & 1u) && !(cut && x[i] < kth) && x[i] != -__builtin_inff()) surv |= 1u << i;
  const uint32_t n = compact<ITEMS>(x, surv, e0, sv, s);
  if (n > (uint32_t)kSurvCap) {
    idx_wide<ITEMS>(a, x, surv, vm, e0, n, row_flags, G);
    return;
  }
  // verification set: finite-or-not survivors of top-k, excluding -inf
  write_topk(a, row, sv, n);
  for (uint32_t j = t; j < n; j += blockDim.x) sv.flag[j] = 1;  // 1 = still present
  __syncthreads();
  if (a.do_topp && n > 0) {
    // top-p (generation.rs:169-194): f64 softmax over the row (dropped entries are
    // exactly zero), ascending stable order by total_cmp, remove cum <= 1 - p,
    // keep the min_keep largest.
    double md = -__builtin_inf();
    for (uint32_t j = t; j < n; j += blockDim.x) md = rmaxd(md, (double)sv.val[j]);
    const double mxd = block_max_d(md, s);
    const bool fin = __builtin_isfinite(mxd);
    for (uint32_t j = t; j < n; j += blockDim.x) {
      sv.w[j] = fin ? tc_exp_d((double)sv.val[j] - mxd) : 0.0;
      sv.key[j] = ((uint64_t)tkey(sv.val[j]) << 32) | (uint64_t)j;
    }
    __syncthreads();
    sort_survivors(sv, n);
    if (t == 0) {
      double sum = -0.0;
      if (fin)
        for (uint32_t j = 0; j < n; ++j) sum += sv.w[j];
      double cum = 0.0;
      const double lim = 1.0 - a.top_p_d;
      for (uint32_t r = 0; r < n; ++r) {
        const uint32_t j = (uint32_t)sv.key[r];
        const double p = fin ? sv.w[j] / sum : 0.0;
        cum += p;
        if (cum <= lim) sv.flag[j] = 0;
      }
      for (uint32_t r = 0; r < n && r < (uint32_t)a.min_keep; ++r) sv.flag[(uint32_t)sv.key[n - 1 - r]] = 1;
    }
    __syncthreads();
  }
  // sample_without_replacement, one draw (generation.rs:280-303), vocab order over live
  if (t == 0) {
    uint32_t nl = 0;
    double mxl = -__builtin_inf();
    for (uint32_t j = 0; j < n; ++j) {
      if (sv.flag[j] && __builtin_isfinite(sv.val[j])) {
        sv.flag[j] = 2;
        ++nl;
        mxl = rmaxd(mxl, (double)sv.val[j] + 0.0);
      }
    }
    uint32_t tok = 0;
    int32_t st = TC_OK;
    if (nl < 1) {
      st = TC_ETOOFEW;
    } else {
      double sum = -0.0;
      for (uint32_t j = 0; j < n; ++j)
        if (sv.flag[j] == 2) { sv.w[j] = tc_exp_d(((double)sv.val[j] + 0.0) - mxl); sum += sv.w[j]; }
      double total = -0.0;
      for (uint32_t j = 0; j < n; ++j)
        if (sv.flag[j] == 2) { sv.w[j] = sv.w[j] / sum; total += sv.w[j]; }
      const double uu = reinterpret_cast<const double*>(a.uniforms)[row] * total;
      double acc = 0.0;
      uint32_t last = 0xffffffffu, pick = 0xffffffffu;
      for (uint32_t j = 0; j < n; ++j) {
        if (sv.flag[j] != 2) continue;
        if (last == 0xffffffffu) last = j;  // last_positive starts at live[0]
        const double w = sv.w[j];
        if (w <= 0.0) continue;
        last = j;
        acc += w;
        if (acc > uu) { pick = j; break; }
      }
      tok = sv.idx[pick != 0xffffffffu ? pick : last];
    }
    put_result(a, row, tok, st, row_flags);
    s_out[0] = nl;
  }
  if (a.keep_count) {
    __syncthreads();
    if (t == 0) {
      uint32_t c = 0;
      for (uint32_t j = 0; j < n; ++j)
        if (sv.flag[j] == 2) {
          if (c < a.cap) {
            a.keep_ids[(size_t)row * a.cap + c] = sv.idx[j];
            a.keep_probs[(size_t)row * a.cap + c] = (float)sv.w[j];
            if (a.keep_scores) a.keep_scores[(size_t)row * a.cap + c] = sv.val[j];
          }
          ++c;
        }
      a.keep_count[row] = c;
    }
  }
}

}  // namespace tc
