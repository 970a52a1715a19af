// k_moss.hip -- moss-tts sampling (crates/moss-tts/src/sampling.rs:22-85) and
// moss-nano's inverse-CDF sampler (crates/moss-tts/src/nano/sampling.rs:11-75).

#include "tc_row.h"

namespace tc {

// The id of the item at place j among the selected items whose key equals kc
// (vocabulary order), on every thread; 0xffffffff when there is none.
template <int ITEMS>
__device__ __forceinline__ uint32_t nth_tie_id(const uint32_t (&key)[ITEMS], uint32_t sel, uint32_t kc, uint32_t j,
                                               int e0, BlockScratch& s) {
  uint32_t eq = 0;
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) eq += (((sel >> i) & 1u) && key[i] == kc) ? 1u : 0u;
  uint32_t tot;
  uint32_t r = block_excl_scan(eq, s, &tot);
  uint32_t id = 0xffffffffu;
#pragma unroll
  for (int i = 0; i < ITEMS; ++i)
    if (((sel >> i) & 1u) && key[i] == kc) {
      if (r == j) id = (uint32_t)(e0 + i);
      ++r;
    }
  return block_min_u(id, s);
}

// The number of selected items whose key is above kc.
template <int ITEMS>
__device__ __forceinline__ uint32_t count_above(const uint32_t (&key)[ITEMS], uint32_t sel, uint32_t kc,
                                                BlockScratch& s) {
  uint32_t c = 0;
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) c += (((sel >> i) & 1u) && key[i] > kc) ? 1u : 0u;
  return block_sum_u(c, s);
}

// ================================================================ moss
// moss over more than kSurvCap ranks (top_k above it): ranked[0..K) are the
// survivors surv (block_first_k), their keys sorted descending in LDS and
// held by position (ITEMS * t + i) in registers.  Their weights
// expf((v - max) / T) are the reference's bits; the sums (total, the running
// sum of w / total against top_p, the kept weights' sum and the draw's
// running difference, sampling.rs:63-83) are sequential in rank order, which
// depends only on the sorted values.  Block prefix sums decide each step when
// it is clear of the rounding both orders allow (settled); otherwise one lane
// runs the reference's loops over the weights staged by rank.  The token is
// the id at the drawn rank: among equal values, ids ascending.
template <int ITEMS>
__device__ __forceinline__ void moss_wide(const RowArgs& a, const float (&x)[ITEMS], const uint32_t (&key)[ITEMS],
                                          uint32_t surv, int e0, uint32_t K, uint32_t flags, SurvWide& U,
                                          BlockScratch& s, ScanLds& sc, uint32_t* s_out, double* s_sw) {
  const int row = blockIdx.x, t = threadIdx.x;
  uint32_t rk[ITEMS];
  block_rank_keys<ITEMS>(key, surv, K, true, U.wide, s, rk);
  const float maximum = untkey(~U.wide[0]);
  const int p0 = ITEMS * t;
  // the weight at rank position p0 + i, recomputed where needed (fewer live
  // registers than holding it)
  auto wfv = [&](int i) { return p0 + i < (int)K ? expf_glibc((untkey(~opaque(rk[i])) - maximum) / a.t_f) : 0.0f; };
  double part = 0.0;
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) part += (double)wfv(i);
  double T;
  const double W0 = block_excl_scan_d(part, sc, &T);
  // keep: the first rank whose running sum of w / total exceeds top_p, plus one
  uint32_t le = 0;
  double W = W0;
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) {
    W += (double)wfv(i);
    le += (p0 + i < (int)K && !(W / T > a.top_p_d)) ? 1u : 0u;
  }
  const uint32_t n_le = block_sum_u(le, s);
  const uint32_t keep = n_le < K ? n_le + 1u : K;
  uint32_t near = 0;
  W = W0;
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) {
    W += (double)wfv(i);
    const uint32_t p = (uint32_t)(p0 + i);
    if (p < K && (p + 1u == n_le || p == n_le) && !settled(W / T, a.top_p_d, K)) near = 1;
    if (p + 1u == keep) *s_sw = W;  // the kept weights' sum
  }
  near = block_or_u(near, s);
  const double sw = *s_sw;
  __syncthreads();
  // draw = u sw - (running sum) <= 0 first at rank `pick`
  const double usw = reinterpret_cast<const double*>(a.uniforms)[row] * sw;
  uint32_t lt = 0;
  W = W0;
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) {
    W += (double)wfv(i);
    lt += ((uint32_t)(p0 + i) < keep && W < usw) ? 1u : 0u;
  }
  const uint32_t n_lt = block_sum_u(lt, s);
  uint32_t pick = n_lt < keep ? n_lt : keep - 1u;
  W = W0;
  uint32_t near2 = 0;
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) {
    W += (double)wfv(i);
    const uint32_t p = (uint32_t)(p0 + i);
    if (p < keep && (p + 1u == n_lt || p == n_lt) && !settled(W, usw, K)) near2 = 1;
  }
  near = block_or_u(near | near2, s) | (n_lt >= keep ? 1u : 0u);
  uint32_t keep_r = keep;
  double sw_r = sw;
  if (near) {
    // the reference's loops, one lane over the weights staged by rank
    float* wr = reinterpret_cast<float*>(U.wide);
#pragma unroll
    for (int i = 0; i < ITEMS; ++i)
      if (p0 + i < (int)K) wr[p0 + i] = wfv(i);
    __syncthreads();
    if (t == 0) {
      double total = -0.0;
      for (uint32_t r = 0; r < K; ++r) total += (double)wr[r];
      double cum = 0.0;
      uint32_t kp = K;
      for (uint32_t r = 0; r < K; ++r) {
        cum += (double)wr[r] / total;
        if (cum > a.top_p_d) {
          kp = r + 1u;
          break;
        }
      }
      double sm = -0.0;
      for (uint32_t r = 0; r < kp; ++r) sm += (double)wr[r];
      double draw = reinterpret_cast<const double*>(a.uniforms)[row] * sm;
      uint32_t pk = kp - 1u;
      for (uint32_t r = 0; r < kp; ++r) {
        draw -= (double)wr[r];
        if (draw <= 0.0) {
          pk = r;
          break;
        }
      }
      s_out[0] = kp;
      s_out[1] = pk;
      *s_sw = sm;
    }
    __syncthreads();
    keep_r = s_out[0];
    pick = s_out[1];
    sw_r = *s_sw;
    __syncthreads();
  }
  // keys at the drawn rank and either side of the kept set's edge
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) {
    const uint32_t p = (uint32_t)(p0 + i);
    if (p == pick) s_out[0] = ~rk[i];
    if (p + 1u == keep_r) s_out[1] = ~rk[i];
    if (p == keep_r) s_out[2] = ~rk[i];
  }
  __syncthreads();
  const uint32_t kpick = s_out[0], kedge = s_out[1], knext = s_out[2];
  __syncthreads();
  if (keep_r < K && kedge == knext) flags |= TC_FLAG_TIE_CUT;
  const uint32_t tok = nth_tie_id<ITEMS>(key, surv, kpick, pick - count_above<ITEMS>(key, surv, kpick, s), e0, s);
  finish_row(a, row, tok, TC_OK, flags);
  if (a.topk_count) {
    const uint32_t c1 = write_ids<ITEMS>(a.topk_ids, a.cap, row, surv, e0, s);
    const uint32_t g0 = count_above<ITEMS>(key, surv, kedge, s);
    const uint32_t kept = select_above_and_ties<ITEMS>(key, surv, kedge, 0u, keep_r - g0, s);
    uint32_t tot;
    uint32_t p = block_excl_scan((uint32_t)__builtin_popcount(kept), s, &tot);
#pragma unroll
    for (int i = 0; i < ITEMS; ++i)
      if ((kept >> i) & 1u) {
        if (p < a.cap) {
          a.keep_ids[(size_t)row * a.cap + p] = (uint32_t)(e0 + i);
          a.keep_probs[(size_t)row * a.cap + p] = (float)((double)expf_glibc((x[i] - maximum) / a.t_f) / sw_r);
        }
        ++p;
      }
    if (t == 0) {
      a.topk_count[row] = c1;
      a.keep_count[row] = tot;
    }
  }
}

template <typename InT, int ITEMS>
__global__ void __launch_bounds__(max_threads(ITEMS)) k_moss(RowArgs a) {
  __shared__ uint8_t s_seen[kMaxVocabReg];
  __shared__ SurvWide U;
  SurvLds& sv = U.sv;
  __shared__ ScanLds sc;
  __shared__ uint32_t s_hist[256];
  __shared__ BlockScratch s;
  __shared__ uint32_t s_out[4];
  __shared__ double s_sw;
  const int row = blockIdx.x, t = threadIdx.x, V = a.V;
  const InT* rp = reinterpret_cast<const InT*>(a.logits) + (size_t)row * (size_t)a.ld;
  float x[ITEMS];
  int shift;
  put_norm(a, row, __builtin_nanf(""));
  load_row<ITEMS>(rp, V, x, &shift);
  const uint32_t vm = valid_mask<ITEMS>(V, shift);
  const int e0 = t * ITEMS - shift;
  if (a.do_pen) build_seen(a, row, s_seen, s);
  uint32_t bad = 0, fin = 0;
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) {
    if (!((vm >> i) & 1u)) continue;
    const int e = e0 + i;
    float v = x[i];
    if (a.do_pen && s_seen[e]) v = v < 0.0f ? v * a.pen_f : v / a.pen_f;
    if (e == a.exclude_id) v = -__builtin_inff();
    x[i] = v;
    bad |= __builtin_isnan(v) ? 1u : 0u;
    fin |= __builtin_isfinite(v) ? 1u : 0u;
  }
  bad = block_or_u(bad, s);
  fin = block_or_u(fin, s);
  if (bad || !fin) {  // sampling.rs:51-54
    finish_row(a, row, 0u, TC_ENONFINITE, 0u);
    no_verify(a, row);
    return;
  }
  const uint32_t K = a.greedy ? 1u : (uint32_t)(a.top_k < V ? a.top_k : V);
  uint32_t key[ITEMS];
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) key[i] = tkey(x[i]);
  uint32_t kk = 0;
  block_kth_largest<ITEMS>(key, vm, K, s_hist, s, &kk);
  // ranked[0..K) under (value descending, id ascending); more keys equal to
  // the K-th mean the reference's unstable sort could have kept another id
  uint32_t ge = 0;
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) ge += (((vm >> i) & 1u) && key[i] >= kk) ? 1u : 0u;
  const uint32_t n_ge = block_sum_u(ge, s);
  const uint32_t surv = block_first_k<ITEMS>(key, vm, kk, K, s);
  const uint32_t n = compact<ITEMS>(x, surv, e0, sv, s);
  if (n > (uint32_t)kSurvCap) {
    moss_wide<ITEMS>(a, x, key, surv, e0, K, n_ge > K ? (uint32_t)TC_FLAG_TIE_CUT : 0u, U, s, sc, s_out, &s_sw);
    return;
  }
  for (uint32_t j = t; j < n; j += blockDim.x) sv.key[j] = ((uint64_t)(~tkey(sv.val[j])) << 32) | (uint64_t)j;
  __syncthreads();
  sort_survivors(sv, n);
  uint32_t flags = n_ge > K ? (uint32_t)TC_FLAG_TIE_CUT : 0u;
  if (a.greedy) {  // temperature == 0: ranked[0]
    finish_row(a, row, sv.idx[(uint32_t)sv.key[0]], TC_OK, flags);
    no_verify(a, row);
    return;
  }
  const float maximum = sv.val[(uint32_t)sv.key[0]];
  for (uint32_t r = t; r < K; r += blockDim.x)
    sv.w[r] = (double)expf_glibc((sv.val[(uint32_t)sv.key[r]] - maximum) / a.t_f);
  __syncthreads();
  if (t == 0) {
    double total = -0.0;
    for (uint32_t r = 0; r < K; ++r) total += sv.w[r];
    double cum = 0.0;
    uint32_t keep = K;
    for (uint32_t r = 0; r < K; ++r) {
      cum += sv.w[r] / total;
      if (cum > a.top_p_d) { keep = r + 1; break; }
    }
    if (keep < K && sv.key[keep - 1] >> 32 == sv.key[keep] >> 32) flags |= TC_FLAG_TIE_CUT;
    double sw = -0.0;
    for (uint32_t r = 0; r < keep; ++r) sw += sv.w[r];
    double draw = reinterpret_cast<const double*>(a.uniforms)[row] * sw;
    uint32_t tok = sv.idx[(uint32_t)sv.key[keep - 1]];
    for (uint32_t r = 0; r < keep; ++r) {
      draw -= sv.w[r];
      if (draw <= 0.0) { tok = sv.idx[(uint32_t)sv.key[r]]; break; }
    }
    put_result(a, row, tok, TC_OK, flags);
    s_out[0] = keep;
    s.d[0] = sw;
  }
  if (a.topk_count) {
    __syncthreads();
    const uint32_t keep = s_out[0];
    const double sw = s.d[0];
    // ids in ascending order: mark ranks, then walk the vocab-ordered survivors
    for (uint32_t r = t; r < n; r += blockDim.x) sv.flag[(uint32_t)sv.key[r]] = r < K ? (r < keep ? 2 : 1) : 0;
    __syncthreads();
    for (uint32_t r = t; r < K; r += blockDim.x) sv.e[(uint32_t)sv.key[r]] = (float)(sv.w[r] / sw);
    __syncthreads();
    if (t == 0) {
      uint32_t c1 = 0, c2 = 0;
      for (uint32_t j = 0; j < n; ++j) {
        if (sv.flag[j] >= 1) { if (c1 < a.cap) a.topk_ids[(size_t)row * a.cap + c1] = sv.idx[j]; ++c1; }
        if (sv.flag[j] == 2) {
          if (c2 < a.cap) {
            a.keep_ids[(size_t)row * a.cap + c2] = sv.idx[j];
            a.keep_probs[(size_t)row * a.cap + c2] = sv.e[j];
          }
          ++c2;
        }
      }
      a.topk_count[row] = c1;
      a.keep_count[row] = c2;
    }
  }
}

// ================================================================ moss-nano
// nano over more than kSurvCap ids at or above the threshold (top_k above it,
// or ties at the k-th value).  Weights exp((v - max) as f64) of the survivors
// surv; top-p (nano/sampling.rs:52-62) walks the stable rank order (value
// descending, ids ascending), which zeroes every rank after the first whose
// running sum of w / total exceeds top_p: positions ITEMS * t + i of the
// sorted keys hold it in registers, equal values being equal terms.  The draw
// (63-70) subtracts the weights in vocabulary order: the first positive one
// at which the running sum reaches u * sum.  Block sums decide both; a
// decision within order_margin of the rounding the reference's sequential
// orders allow is taken again by its own loops (staged_walk), and the row
// flagged TC_FLAG_NEAR_TIE when that decision lies within the f64 exp's error
// and some weight is not exact.
template <int ITEMS>
__device__ __forceinline__ void nano_wide(const RowArgs& a, const float (&x)[ITEMS], uint32_t surv, int e0,
                                          uint32_t n, float maximum, SurvWide& U, BlockScratch& s, ScanLds& sc,
                                          WalkLds& WL) {
  const int row = blockIdx.x, t = threadIdx.x;
  double* stage = reinterpret_cast<double*>(U.wide);
  uint32_t key[ITEMS];
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) key[i] = tkey(x[i]);
  auto wv = [&](float v) { return tc_exp_d((double)(opaque(v) - maximum)); };
  uint32_t pos = 0, inexact = 0;  // survivors with a positive weight; one not exp(0)
#pragma unroll
  for (int i = 0; i < ITEMS; ++i)
    if (((surv >> i) & 1u) && wv(x[i]) > 0.0) {
      pos |= 1u << i;
      inexact |= x[i] != maximum ? 1u : 0u;
    }
  inexact = block_or_u(inexact, s);
  if (a.topk_count) {
    const uint32_t c = write_ids<ITEMS>(a.topk_ids, a.cap, row, pos, e0, s);
    if (t == 0) a.topk_count[row] = c;
  }
  uint32_t flags = 0;
  uint32_t kept = surv;
  if (a.do_topp) {
    uint32_t rk[ITEMS];
    block_rank_keys<ITEMS>(key, surv, n, true, U.wide, s, rk);
    const int p0 = ITEMS * t;
    auto wt = [&](int i) { return p0 + i < (int)n ? wv(untkey(~rk[i])) : 0.0; };
    double part = 0.0;
#pragma unroll
    for (int i = 0; i < ITEMS; ++i) part += wt(i);
    double S;
    const double W0 = block_excl_scan_d(part, sc, &S);
    uint32_t le = 0;
    double W = W0;
#pragma unroll
    for (int i = 0; i < ITEMS; ++i) {
      W += wt(i);
      le += (p0 + i < (int)n && !(W / S > a.top_p_d)) ? 1u : 0u;
    }
    uint32_t r_star = block_sum_u(le, s);  // the first rank past top_p (n: none)
    uint32_t near = 0;
    W = W0;
#pragma unroll
    for (int i = 0; i < ITEMS; ++i) {
      W += wt(i);
      const uint32_t p = (uint32_t)(p0 + i);
      if (p < n && (p + 1u == r_star || p == r_star) && !settled(W / S, a.top_p_d, n)) near = 1;
    }
    if (block_or_u(near, s)) {
      // the reference's loops: the total in vocabulary order, the running sum
      // in rank order
      const VocabPos<ITEMS> vp = vocab_pos<ITEMS>(surv, s);
      auto wx = [&](int i) { return wv(x[i]); };
      double tot = -0.0;
      staged_walk<ITEMS>(n, vp, wx, stage, WL, [&](uint32_t, double v) {
        tot += v;
        return true;
      });
      if (t == 0) WL.d[0] = tot;
      __syncthreads();
      tot = WL.d[0];
      double cum = 0.0, c_lo = -1.0, c_hi = 2.0;
      uint32_t r = 0;
      auto rpos = [&](int i) { return p0 + i < (int)n ? (uint32_t)(p0 + i) : 0xffffffffu; };
      staged_walk<ITEMS>(n, rpos, wt, stage, WL, [&](uint32_t, double v) {
        const double before = cum;
        cum += v / tot;
        if (cum > a.top_p_d) {
          c_hi = cum;
          c_lo = before;
          return false;
        }
        c_lo = cum;
        ++r;
        return true;
      });
      if (t == 0) {
        WL.u[0] = r;
        WL.u[1] = (inexact && ((r < n && !settled_exp(c_hi, a.top_p_d)) || (r > 0u && !settled_exp(c_lo, a.top_p_d))))
                      ? 1u : 0u;
      }
      __syncthreads();
      r_star = WL.u[0];
      if (WL.u[1]) flags |= TC_FLAG_NEAR_TIE;
      __syncthreads();
    }
    if (r_star < n) {
      uint32_t kc = 0;
#pragma unroll
      for (int i = 0; i < ITEMS; ++i)
        if ((uint32_t)(p0 + i) == r_star) WL.u[2] = ~rk[i];
      __syncthreads();
      kc = WL.u[2];
      __syncthreads();
      uint32_t gt = 0;
#pragma unroll
      for (int i = 0; i < ITEMS; ++i) gt += (((surv >> i) & 1u) && key[i] > kc) ? 1u : 0u;
      const uint32_t g0 = block_sum_u(gt, s);
      kept = select_above_and_ties<ITEMS>(key, surv, kc, 0u, r_star - g0 + 1u, s);
    }
  }
  kept &= pos;
  double part = 0.0;
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) part += ((kept >> i) & 1u) ? wv(x[i]) : 0.0;
  double SW;
  double P = block_excl_scan_d(part, sc, &SW);
  const double u = reinterpret_cast<const double*>(a.uniforms)[row];
  const double uS = u * SW;
  uint32_t first = 0xffffffffu, lastp = 0;
  double f_in = 0.0, f_ex = 0.0, p_last = 0.0;
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) {
    if (!((kept >> i) & 1u)) continue;
    const double prev = P;
    P += wv(x[i]);
    lastp = (uint32_t)(e0 + i) + 1u;
    p_last = P;
    if (first == 0xffffffffu && P >= uS) {
      first = (uint32_t)(e0 + i);
      f_in = P;
      f_ex = prev;
    }
  }
  uint32_t pick = block_min_u(first, s);
  const uint32_t last = block_max_u(lastp, s);
  uint32_t near = 0;
  if (first == pick && pick != 0xffffffffu && (!settled(f_in, uS, n) || (f_ex > 0.0 && !settled(f_ex, uS, n))))
    near = 1u;
  if (pick == 0xffffffffu && last != 0u && lastp == last && !settled(p_last, uS, n)) near = 1u;
  int32_t st = pick != 0xffffffffu ? TC_OK : TC_EDIST;
  if (block_or_u(near, s)) {
    // the reference's loops over the kept ids in vocabulary order: their sum,
    // then draw -= w until draw <= 0
    const uint32_t nk = block_sum_u((uint32_t)__builtin_popcount(kept), s);
    const VocabPos<ITEMS> vp = vocab_pos<ITEMS>(kept, s);
    auto wx = [&](int i) { return wv(x[i]); };
    double sw = -0.0;
    staged_walk<ITEMS>(nk, vp, wx, stage, WL, [&](uint32_t, double v) {
      sw += v;
      return true;
    });
    if (t == 0) WL.d[0] = sw;
    __syncthreads();
    sw = WL.d[0];
    double draw = u * sw, d_ex = draw, d_in = 0.0;
    uint32_t jp = 0xffffffffu;
    staged_walk<ITEMS>(nk, vp, wx, stage, WL, [&](uint32_t j, double v) {
      d_ex = draw;
      draw -= v;
      if (v > 0.0 && draw <= 0.0) {
        jp = j;
        d_in = draw;
        return false;
      }
      return true;
    });
    if (t == 0) {
      WL.u[0] = jp;
      // draw <= 0 at jp and > 0 before it, each clear of the exp's error
      WL.u[1] = (inexact && (jp == 0xffffffffu || !(__builtin_fabs(d_in) > exp_margin() * sw) ||
                             (jp != 0u && !(__builtin_fabs(d_ex) > exp_margin() * sw)))) ? 1u : 0u;
    }
    __syncthreads();
    jp = WL.u[0];
    if (WL.u[1]) flags |= TC_FLAG_NEAR_TIE;
    __syncthreads();
    uint32_t id = 0xffffffffu;
#pragma unroll
    for (int i = 0; i < ITEMS; ++i)
      if (vp(i) == jp) id = (uint32_t)(e0 + i);
    pick = block_min_u(id, s);
    st = pick != 0xffffffffu ? TC_OK : TC_EDIST;
  }
  finish_row(a, row, pick != 0xffffffffu ? pick : 0u, st, flags);
  if (a.keep_count) {
    uint32_t tot;
    uint32_t p = block_excl_scan((uint32_t)__builtin_popcount(kept), s, &tot);
#pragma unroll
    for (int i = 0; i < ITEMS; ++i)
      if ((kept >> i) & 1u) {
        if (p < a.cap) {
          a.keep_ids[(size_t)row * a.cap + p] = (uint32_t)(e0 + i);
          a.keep_probs[(size_t)row * a.cap + p] = (float)(wv(x[i]) / SW);
        }
        ++p;
      }
    if (t == 0) a.keep_count[row] = tot;
  }
}

template <typename InT, int ITEMS>
__global__ void __launch_bounds__(max_threads(ITEMS)) k_nano(RowArgs a) {
  __shared__ uint8_t s_seen[kMaxVocabReg];
  __shared__ SurvWide U;
  SurvLds& sv = U.sv;
  __shared__ ScanLds sc;
  __shared__ WalkLds wl;
  __shared__ uint32_t s_hist[256];
  __shared__ BlockScratch s;
  const int row = blockIdx.x, t = threadIdx.x, V = a.V;
  const InT* rp = reinterpret_cast<const InT*>(a.logits) + (size_t)row * (size_t)a.ld;
  float x[ITEMS];
  int shift;
  put_norm(a, row, __builtin_nanf(""));
  load_row<ITEMS>(rp, V, x, &shift);
  const uint32_t vm = valid_mask<ITEMS>(V, shift);
  const int e0 = t * ITEMS - shift;
  uint32_t bad = 0;
#pragma unroll
  for (int i = 0; i < ITEMS; ++i)
    if (((vm >> i) & 1u) && !__builtin_isfinite(x[i])) bad = 1u;
  bad = block_or_u(bad, s);
  if (bad) {  // nano/sampling.rs:24-27
    finish_row(a, row, 0u, TC_ENONFINITE, 0u);
    no_verify(a, row);
    return;
  }
  // every history id must be inside the vocabulary (nano/sampling.rs:28-31)
  const bool oob = build_seen(a, row, s_seen, s);
  if (oob) {
    finish_row(a, row, 0u, TC_EINVAL, 0u);
    no_verify(a, row);
    return;
  }
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) {
    if (!((vm >> i) & 1u)) continue;
    float v = x[i];
    if (s_seen[e0 + i]) v = v < 0.0f ? v * a.pen_f : v / a.pen_f;
    x[i] = v / a.t_f;
  }
  // stable rank order: value descending (total_cmp), id ascending
  const uint32_t K = (uint32_t)(a.top_k < V ? a.top_k : V);
  uint32_t key[ITEMS];
  uint32_t kmax = 0;
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) {
    key[i] = tkey(x[i]);
    if ((vm >> i) & 1u) kmax = key[i] > kmax ? key[i] : kmax;
  }
  uint32_t kk = 0;
  block_kth_largest<ITEMS>(key, vm, K, s_hist, s, &kk);
  const float threshold = untkey(kk);
  // max of the row under total order = ranked[0]
  {
    uint32_t v = kmax;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) { uint32_t w = __shfl_xor(v, o); v = w > v ? w : v; }
    if (lane_id() == 0) s.u[wave_id()] = v;
    __syncthreads();
    uint32_t r = 0;
    for (int w = 0; w < num_waves(); ++w) r = s.u[w] > r ? s.u[w] : r;
    __syncthreads();
    kmax = r;
  }
  const float maximum = untkey(kmax);
  uint32_t surv = 0;
#pragma unroll
  for (int i = 0; i < ITEMS; ++i)
    if (((vm >> i) & 1u) && !(x[i] < threshold)) surv |= 1u << i;
  const uint32_t n = compact<ITEMS>(x, surv, e0, sv, s);
  if (n > (uint32_t)kSurvCap) {
    nano_wide<ITEMS>(a, x, surv, e0, n, maximum, U, s, sc, wl);
    return;
  }
  for (uint32_t j = t; j < n; j += blockDim.x) {
    sv.w[j] = tc_exp_d((double)(sv.val[j] - maximum));
    sv.key[j] = ((uint64_t)(~tkey(sv.val[j])) << 32) | (uint64_t)j;
  }
  __syncthreads();
  if (a.topk_count) {
    if (t == 0) {
      uint32_t c = 0;
      for (uint32_t j = 0; j < n; ++j)
        if (sv.w[j] > 0.0) { if (c < a.cap) a.topk_ids[(size_t)row * a.cap + c] = sv.idx[j]; ++c; }
      a.topk_count[row] = c;
    }
  }
  if (a.do_topp) {
    sort_survivors(sv, n);
    if (t == 0) {
      double total = -0.0;
      for (uint32_t j = 0; j < n; ++j) total += sv.w[j];
      double cum = 0.0;
      for (uint32_t r = 0; r < n; ++r) {
        const uint32_t j = (uint32_t)sv.key[r];
        if (cum > a.top_p_d) sv.w[j] = 0.0;
        else cum += sv.w[j] / total;
      }
    }
    __syncthreads();
  }
  if (t == 0) {
    double sw = -0.0;
    for (uint32_t j = 0; j < n; ++j) sw += sv.w[j];
    double draw = reinterpret_cast<const double*>(a.uniforms)[row] * sw;
    uint32_t tok = 0;
    int32_t st = TC_EDIST;
    for (uint32_t j = 0; j < n; ++j) {
      draw -= sv.w[j];
      if (sv.w[j] > 0.0 && draw <= 0.0) { tok = sv.idx[j]; st = TC_OK; break; }
    }
    put_result(a, row, tok, st, 0u);
    if (a.keep_count) {
      uint32_t c = 0;
      for (uint32_t j = 0; j < n; ++j)
        if (sv.w[j] > 0.0) {
          if (c < a.cap) {
            a.keep_ids[(size_t)row * a.cap + c] = sv.idx[j];
            a.keep_probs[(size_t)row * a.cap + c] = (float)(sv.w[j] / sw);
          }
          ++c;
        }
      a.keep_count[row] = c;
    }
  }
}


TC_DEFINE_LAUNCH(k_moss)
TC_DEFINE_LAUNCH(k_nano)

}  // namespace tc
