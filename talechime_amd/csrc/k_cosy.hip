// k_cosy.hip -- cosyvoice3 repetition-aware sampling (crates/cosyvoice3/src/llm.rs:517-604).

#include "tc_row.h"

namespace tc {

// ================================================================ cosyvoice3
// The softmax denominator and the fallback CDF are the reference's sequential
// f32 sums, reproduced bit for bit by block_seqsum; the nucleus candidates are
// exactly the top_k largest under (probability descending, id ascending).
struct CosyGenLds {
  float stage[kMaxVocabReg / 4];  // staging for the one-lane fallback walks
  SurvLds sv;
  uint32_t hist[256];
  BlockScratch s;
  ScanLds sc;
  SeqLds sq;
  uint32_t out[4];
};

// random_sample_probs (llm.rs:594-604): acc in vocabulary order over every
// probability (pv, the thread's ITEMS elements from e0), the first index with
// pick < acc, else V - 1.  Every thread of the block calls it.
template <int ITEMS>
__device__ __forceinline__ uint32_t cosy_random(const RowArgs& a, int row, const float (&pv)[ITEMS], uint32_t vm,
                                                int e0, CosyGenLds& G) {
  const int t = threadIdx.x, V = a.V;
  const float pick = reinterpret_cast<const float*>(a.uniforms)[2 * row + 1];
  uint32_t found = 0xffffffffu;
  SeqThread<ITEMS> th;
  float p2[ITEMS];
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) p2[i] = ((vm >> i) & 1u) ? pv[i] : 0.0f;
  auto same = [](float v) { return v; };
  float Sp;
  if (block_seqsum<ITEMS>(p2, ~0u, p2, same, e0, 0, th, G.sq, G.sc, &Sp)) {
    float pre[ITEMS];
    seq_prefix<ITEMS>(th, G.sq, pre);
    uint32_t first = 0xffffffffu;
#pragma unroll
    for (int i = ITEMS - 1; i >= 0; --i)
      if (((vm >> i) & 1u) && pick < pre[i]) first = (uint32_t)(e0 + i);
    found = block_min_u(first, G.s);
  } else {
    constexpr int kChunk = kMaxVocabReg / 4;
    float acc = 0.0f;
    for (int c0 = 0; c0 < V; c0 += kChunk) {
#pragma unroll
      for (int i = 0; i < ITEMS; ++i) {
        const int e = e0 + i;
        if (((vm >> i) & 1u) && e >= c0 && e < c0 + kChunk) G.stage[e - c0] = p2[i];
      }
      __syncthreads();
      if (t == 0 && found == 0xffffffffu) {
        const int c1 = (c0 + kChunk < V) ? c0 + kChunk : V;
        for (int e = c0; e < c1; ++e) {
          acc += G.stage[e - c0];
          if (pick < acc) { found = (uint32_t)e; break; }
        }
        G.out[2] = found;
      }
      __syncthreads();
      found = G.out[2];
      if (found != 0xffffffffu) break;
    }
  }
  return found != 0xffffffffu ? found : (uint32_t)(V - 1);
}

// General path: any top_k, non-finite rows.
template <typename InT, int ITEMS>
__device__ __forceinline__ void cosy_general(const RowArgs& a, CosyGenLds& G) {
  float* s_stage = G.stage;
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
  // ignore_eos mask (llm.rs:525-529), then candle softmax_last_dim: max,
  // exp(x - max), sequential f32 sum, divide
  float m = -__builtin_inff();
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) {
    if (!((vm >> i) & 1u)) continue;
    if (a.eos_id >= 0) x[i] = x[i] + (e0 + i == a.eos_id ? -__builtin_inff() : 0.0f);
    m = rmaxf(m, x[i]);
  }
  const float mx = block_max(m, s);
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) x[i] = ((vm >> i) & 1u) ? expf_glibc(x[i] - mx) : 0.0f;
  auto same = [](float v) { return v; };
  float S;
  if (!__builtin_isfinite(mx)) {
    S = __builtin_nanf("");
  } else {
    SeqThread<ITEMS> th;
    if (!block_seqsum<ITEMS>(x, ~0u, x, same, e0, 0, th, sq, sc, &S))
      S = block_seqsum_slow<ITEMS>(x, e0, V, s_stage, kMaxVocabReg / 4, &sq.S);
  }
  put_norm(a, row, S);
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) x[i] = x[i] / S;  // probabilities
  // nucleus (llm.rs:556-592): candidates are the top_k first under the total
  // order (prob desc, id asc)
  const uint32_t nvalid = (uint32_t)V;
  const uint32_t K = (a.top_k > 0 && (uint32_t)a.top_k < nvalid) ? (uint32_t)a.top_k : nvalid;
  uint32_t surv = vm;
  if (K < nvalid) {
    uint32_t key[ITEMS];
#pragma unroll
    for (int i = 0; i < ITEMS; ++i) key[i] = tkey(x[i]);
    uint32_t kk;
    if (block_kth_largest<ITEMS>(key, vm, K, s_hist, s, &kk)) surv = block_first_k<ITEMS>(key, vm, kk, K, s);
  }
  const uint32_t n = compact<ITEMS>(x, surv, e0, sv, s);
  if (n > (uint32_t)kSurvCap) {
    finish_row(a, row, 0u, TC_EUNSUPPORTED, 0u);
    no_verify(a, row);
    return;
  }
  for (uint32_t j = t; j < n; j += blockDim.x) {
    sv.key[j] = ((uint64_t)(~tkey(sv.val[j])) << 32) | (uint64_t)j;
    sv.flag[j] = 0;
  }
  __syncthreads();
  sort_survivors(sv, n);
  if (t == 0) {
    float cum = 0.0f;
    uint32_t nc = 0;
    for (uint32_t r = 0; r < n; ++r) {
      if (cum < a.top_p_f && nc < (uint32_t)a.top_k) {
        cum += sv.val[(uint32_t)sv.key[r]];
        ++nc;
      } else {
        break;
      }
    }
    uint32_t top;
    if (nc == 0) {
      top = sv.idx[(uint32_t)sv.key[0]];
    } else {
      float total = -0.0f;
      for (uint32_t r = 0; r < nc; ++r) total += sv.val[(uint32_t)sv.key[r]];
      const float pick = reinterpret_cast<const float*>(a.uniforms)[2 * row] * total;
      float acc = 0.0f;
      top = sv.idx[(uint32_t)sv.key[nc - 1]];
      for (uint32_t r = 0; r < nc; ++r) {
        acc += sv.val[(uint32_t)sv.key[r]];
        if (pick < acc) { top = sv.idx[(uint32_t)sv.key[r]]; break; }
      }
    }
    for (uint32_t r = 0; r < nc; ++r) sv.flag[(uint32_t)sv.key[r]] = 1;
    s_out[0] = top;
    s_out[1] = nc;
  }
  __syncthreads();
  const uint32_t top = s_out[0];
  // repetition window (llm.rs:532-536)
  uint32_t h0, h1;
  hist_range(a, row, &h0, &h1);
  const uint32_t w0 = (h1 - h0) > (uint32_t)a.ras_win ? h1 - (uint32_t)a.ras_win : h0;
  uint32_t rep = 0;
  for (uint32_t j = w0 + t; j < h1; j += blockDim.x) rep += a.hist_ids[j] == top;
  rep = block_sum_u(rep, s);
  uint32_t tok = top, flags = 0;
  if ((float)rep >= a.ras_thresh) {
    flags = TC_FLAG_RAS;
    tok = cosy_random<ITEMS>(a, row, x, vm, e0, G);
  }
  finish_row(a, row, tok, TC_OK, flags);
  if (a.topk_count) {
    const uint32_t nc = s_out[1];
    __syncthreads();
    if (t == 0) {
      uint32_t c = 0;
      for (uint32_t j = 0; j < n; ++j)
        if (sv.flag[j]) {
          if (c < a.cap) {
            a.topk_ids[(size_t)row * a.cap + c] = sv.idx[j];
            a.keep_ids[(size_t)row * a.cap + c] = sv.idx[j];
            a.keep_probs[(size_t)row * a.cap + c] = sv.val[j];
          }
          ++c;
        }
      a.topk_count[row] = nc;
      a.keep_count[row] = nc;
    }
  }
}

struct CosyFastLds {
  static constexpr int kWalk = 1024;
  uint32_t bins[64];  // thread maxima of d per 0.25-wide bucket below the row max
  float wmax[kMaxWaves];
  float wfin[kMaxWaves];
  uint32_t wcand[kMaxWaves];
  uint32_t out[4];
  double wd[2][kMaxWaves];  // the repetition fallback's wave sums of p and of id * p
  SeqFastLds seq;
  FinLds fin;
  float walk[kWalk];  // the repetition fallback's probabilities around the crossing
};

// random_sample_probs (llm.rs:594-604) from the fast path's registers: d,
// the thread's ITEMS values of x - max from e0, vm their mask (outside the
// row and the EOS id clear: probability an exact zero), S the reference's
// softmax denominator.  The reference adds the probabilities p = expf(d) / S
// in f32 in index order; each add rounds by at most 2^-24 of the running sum
// after it, so its running sum acc_j lies within 2^-24 * 1.01 * Q_j of the
// exact one P_j, Q_j = sum_{k <= j} P_k = (j + 1) P_j - sum_{m <= j} m p_m
// (the 1.01 covers the errors carried from earlier adds, below V 2^-24 < 4e-4
// of Q).  The window search runs on approximate probabilities q =
// exp_approx(d) * (1 / S) in f32, within 2^-20 of p (2^-21 for exp_approx, a
// few 2^-24 for the roundings of glibc's expf, the division and the product;
// d < -87 counts as 0, p below 2^-125), summed per thread in f32 (ITEMS
// terms: relative error below 2^-19.4) and across threads in f64 scans.
// Together with the errors of the f32 partial sums inside a thread and of Q
// (at most 2^-16.7 V P), E = 2^-24 * 1.01 * Q + 2^-16 P + 2^-50 at a thread's
// last element bounds acc_j - P_j for each of its elements.  An element's
// tests compare its thread-local f32 partial sum with pick - base -/+ E,
// widened by 2^-23 of itself before rounding to f32: "acc_j may exceed pick"
// and "acc_j exceeds pick".  The token, the first index with pick < acc, lies
// in [lo, hi], lo the first element that may exceed, hi the first that
// exceeds; when the two agree that is the token.  Otherwise pv gets the exact
// probabilities (every lane active: the wave-cooperative expf), the exact
// sequential sum up to the window is SeqSum over those before it (elements
// from the window on count as zeros), and one lane walks the window.  Returns
// the token, or 0xffffffff when the window or the list does not fit (then
// the caller's general walk decides from pv).  Every thread of the block
// calls it.
template <int ITEMS>
__device__ __forceinline__ uint32_t cosy_random_fast(const RowArgs& a, int row, const float (&d)[ITEMS], uint32_t vm,
                                                     float S, int e0, CosyFastLds& F, float (&pv)[ITEMS]) {
  const int t = threadIdx.x, V = a.V, lane = lane_id(), wv = wave_id(), nw = num_waves();
  const float pick = reinterpret_cast<const float*>(a.uniforms)[2 * row + 1];
  const float rS = 1.0f / S;
  float q[ITEMS];
  float tpf = 0.0f, tmf = 0.0f;
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) {
    q[i] = ((vm >> i) & 1u) && d[i] >= -87.0f ? exp_approx(d[i]) * rS : 0.0f;
    tpf += q[i];
    tmf += (float)i * q[i];
  }
  const double tp = (double)tpf, tm = (double)e0 * tp + (double)tmf;
  const double ip = dpp_scan_f64(tp), im = dpp_scan_f64(tm);
  if (lane == kWave - 1) {
    F.wd[0][wv] = ip;
    F.wd[1][wv] = im;
  }
  lds_barrier();
  double pb = 0.0, mb = 0.0;
  {
    const double vp = lane < nw ? F.wd[0][lane] : 0.0, vq = lane < nw ? F.wd[1][lane] : 0.0;
    const double cp = dpp_scan_f64(vp), cm = dpp_scan_f64(vq);
    const int w = __builtin_amdgcn_readfirstlane(wv);
    if (w > 0) {
      pb = rl_f64(cp, w - 1);
      mb = rl_f64(cm, w - 1);
    }
  }
  const double base = pb + (ip - tp);
  const double A = base + tp, M = mb + im;  // at the thread's last element
  const double Q = (double)(e0 + ITEMS) * A - M;
  const double E = 0x1p-24 * 1.01 * Q + 0x1p-16 * A + 0x1p-50;
  const double r = (double)pick - base;
  const double tl = r - E, th = r + E;
  const float fl = (float)(tl - 0x1p-23 * __builtin_fabs(tl) - 0x1p-140);  // at most tl
  const float fh = (float)(th + 0x1p-23 * __builtin_fabs(th) + 0x1p-140);  // at least th
  uint32_t lo = 0xffffffffu, hi = 0xffffffffu;
  float pf = 0.0f;
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) {
    const int e = e0 + i;
    pf += q[i];
    const bool in = e >= 0 && e < V;
    if (lo == 0xffffffffu && in && pf > fl) lo = (uint32_t)e;
    if (hi == 0xffffffffu && in && pf > fh) hi = (uint32_t)e;
  }
  // elements are in lane order: the wave's first is its first lane's
  const uint64_t bl = __ballot(lo != 0xffffffffu), bh = __ballot(hi != 0xffffffffu);
  lo = bl ? rl_u32(lo, __builtin_ctzll(bl)) : 0xffffffffu;
  hi = bh ? rl_u32(hi, __builtin_ctzll(bh)) : 0xffffffffu;
  if (lane == 0) {
    F.wcand[wv] = lo;
    F.bins[wv] = hi;
  }
  lds_barrier();
  for (int w = 0; w < nw; ++w) {
    lo = F.wcand[w] < lo ? F.wcand[w] : lo;
    hi = F.bins[w] < hi ? F.bins[w] : hi;
  }
  // one element can be the first whose acc exceeds pick: it is the token
  // (acc is non-decreasing; before lo it is <= pick, at hi above it)
  if (lo != 0xffffffffu && lo == hi) return lo;
  if (lo == 0xffffffffu) return (uint32_t)(V - 1);  // no running sum can exceed pick
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) {
    const float e = expf_glibc_wave(((vm >> i) & 1u) ? d[i] : 0.0f);
    pv[i] = ((vm >> i) & 1u) ? e / S : 0.0f;
  }
  const uint32_t end = hi == 0xffffffffu ? (uint32_t)(V - 1) : hi;  // inclusive
  if (end - lo + 1u > (uint32_t)CosyFastLds::kWalk) return 0xffffffffu;
  // the exact sequential sum of the probabilities before the window
  float ap[ITEMS];
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) ap[i] = (e0 + i < (int)lo) ? pv[i] : 0.0f;
  SeqSum<ITEMS> sq;
  sq.predict(ap, F.seq);
  lds_barrier();
  sq.classify(ap, ~0u, 0u, e0, F.seq);
  lds_barrier();  // write_list reads every wave's classification totals
  const bool ok = sq.write_list(ap, ap, e0, F.seq, 0u, [](int) {});
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) {
    const int e = e0 + i;
    if (e >= (int)lo && e <= (int)end) F.walk[e - (int)lo] = pv[i];
  }
  lds_barrier();
  if (ok) sq.replay_terms([](float v) { return v; }, F.seq);
  lds_barrier();
  if (wv == 0 && ok) sq.replay_walk(F.seq);
  lds_barrier();
  if (!ok || F.seq.bad) return 0xffffffffu;
  if (t == 0) {
    float acc = F.seq.S;
    uint32_t found = (uint32_t)(V - 1);
    for (uint32_t e = lo; e <= end; ++e) {
      acc += F.walk[e - lo];
      if (pick < acc) {
        found = e;
        break;
      }
    }
    F.out[2] = found;
  }
  __syncthreads();
  return F.out[2];
}
// The fast path hands a row to the general path before the general path
// touches LDS, and uses the general path's arrays only after its own are done.
union CosyLds {
  CosyFastLds f;
  CosyGenLds g;
};

// One-wave finish of a cosyvoice3 row from its n (top_k <= n <= 128)
// candidates (F.cand: bits of d = x - max and the id, vocabulary order): the
// exact probabilities expf(d) / S, the rank order (probability descending, id
// ascending), the nucleus loop and draw (llm.rs:556-592) as the reference's
// sequential f32 sums over at most top_k ranks, and the repetition window
// (llm.rs:532-536).  C.out[0] = the nucleus token, C.out[1] = 1 when the
// window fired (the row then draws from random_sample_probs instead).
// wid: lane j's id of the repetition window (the last ras_win decoded ids),
// loaded at the start of the row when the window fits a wave; else unused.
template <int NS>
__device__ __forceinline__ void cosy_fast_finish_t(const RowArgs& a, int row, uint32_t n, float S, CosyFastLds& C,
                                                   uint32_t wid) {
  FinLds& F = C.fin;
  const int lane = lane_id();
  float p[2];
  uint32_t id[2];
  bool has[2];
  uint64_t key[2];
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const uint32_t c = (uint32_t)(q * kWave + lane);
    has[q] = q < NS && c < n;
    const uint64_t v = has[q] ? F.cand[c] : 0ull;
    id[q] = (uint32_t)v;
    float e = 0.0f;
    if (q < NS) e = expf_glibc_wave(has[q] ? u2f((uint32_t)(v >> 32)) : 0.0f);
    p[q] = has[q] ? e / S : 0.0f;
    key[q] = has[q] ? (((uint64_t)tkey(p[q]) << 32) | (uint64_t)(0xffffffffu - id[q])) : 0ull;
    if (q < NS) F.rkey[c] = key[q];
  }
  lds_wait();
  // rank = number of candidates with a larger key (zero keys pad the slots
  // past n up to a multiple of 4)
  uint32_t rk[2] = {0u, 0u};
  {
    const uint32_t nr = (n + 3u) & ~3u;
    uint32_t a0 = 0, a1 = 0, b0 = 0, b1 = 0;
    for (uint32_t j = 0; j < nr; j += 4) {
      const uint64_t k0 = F.rkey[j], k1 = F.rkey[j + 1], k2 = F.rkey[j + 2], k3 = F.rkey[j + 3];
      a0 += (k0 > key[0] ? 1u : 0u) + (k1 > key[0] ? 1u : 0u);
      a1 += (k2 > key[0] ? 1u : 0u) + (k3 > key[0] ? 1u : 0u);
      if (NS == 2) {
        b0 += (k0 > key[1] ? 1u : 0u) + (k1 > key[1] ? 1u : 0u);
        b1 += (k2 > key[1] ? 1u : 0u) + (k3 > key[1] ? 1u : 0u);
      }
    }
    rk[0] = has[0] ? a0 + a1 : 0xffffffffu;
    rk[1] = has[1] ? b0 + b1 : 0xffffffffu;
  }
  auto at_rank = [&](uint32_t r, float* pr, uint32_t* ir) {
    const uint64_t m0 = __ballot(rk[0] == r), m1 = __ballot(rk[1] == r);
    if (m0) {
      *pr = rl_f32(p[0], __builtin_ctzll(m0));
      *ir = rl_u32(id[0], __builtin_ctzll(m0));
    } else {
      *pr = rl_f32(p[1], __builtin_ctzll(m1));
      *ir = rl_u32(id[1], __builtin_ctzll(m1));
    }
  };
  // The nucleus loop, its total and the draw add the same terms in the same
  // (rank) order from zero, so one running sum cum_r decides all three: the
  // kept count nc (the first r <= kmax - 2 with cum_r >= top_p, plus one;
  // else kmax), total = cum_{nc-1}, and the token at the first r < nc with
  // u total < cum_r.  Without verification outputs they are first decided
  // from a wave scan of the probabilities by rank, which stays within
  // (n + 32) 2^-22 of the sequential sums; a decision inside that margin runs
  // the reference's loops below.
  const uint32_t kmax = (uint32_t)a.top_k < n ? (uint32_t)a.top_k : n;
  if (!a.topk_count && kmax >= 1u) {
#pragma unroll
    for (int q = 0; q < 2; ++q)
      if (has[q]) {
        F.wr32[rk[q]] = p[q];
        F.k32[rk[q]] = id[q];
      }
    lds_wait();
    float pr[2], c[2];
    float carry = 0.0f;
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const uint32_t r = (uint32_t)(q * kWave + lane);
      pr[q] = (q < NS && r < n) ? F.wr32[r] : 0.0f;
      c[q] = q < NS ? dpp_scan_f32(pr[q]) + carry : 0.0f;
      if (q < NS) carry = rl_f32(c[q], kWave - 1);
    }
    auto cum_at = [&](uint32_t r) { return rl_f32(r < 64u ? c[0] : c[1], (int)(r & 63u)); };
    const float mg = (float)(n + 32u) * 0x1p-22f;
    const float tp = a.top_p_f;
    // the crossing among ranks 0 .. kmax - 2
    const uint32_t lim = kmax - 1u;
    const uint64_t x0 = __ballot((uint32_t)lane < lim && c[0] >= tp);
    const uint64_t x1 = __ballot((uint32_t)(kWave + lane) < lim && c[1] >= tp);
    const uint32_t rx = x0 ? (uint32_t)__builtin_ctzll(x0) : (x1 ? 64u + (uint32_t)__builtin_ctzll(x1) : lim);
    bool ok = true;
    uint32_t nc2;
    if (rx < lim) {
      nc2 = rx + 1u;
      ok = cum_at(rx) - tp > mg && (rx == 0u || tp - cum_at(rx - 1u) > mg);
    } else {
      nc2 = kmax;
      ok = lim == 0u || tp - cum_at(lim - 1u) > mg;
    }
    if (ok) {
      const float total = cum_at(nc2 - 1u);
      const float pick = reinterpret_cast<const float*>(a.uniforms)[2 * row] * total;
      const uint64_t d0 = __ballot((uint32_t)lane < nc2 && c[0] > pick);
      const uint64_t d1 = __ballot((uint32_t)(kWave + lane) < nc2 && c[1] > pick);
      const uint32_t rd = d0 ? (uint32_t)__builtin_ctzll(d0) : (d1 ? 64u + (uint32_t)__builtin_ctzll(d1) : nc2);
      // pick carries the total's uncertainty (mg, scaled by u <= 1) and its
      // own rounding
      const float mgd = 2.0f * mg + pick * 0x1p-23f;
      ok = rd < nc2 && cum_at(rd) - pick > mgd && (rd == 0u || pick - cum_at(rd - 1u) > mgd);
      if (ok) {
        const uint32_t tk = F.k32[rd];
        uint32_t rep = 0;
        if (a.ras_win <= kWave) {
          rep = (uint32_t)__popcll(__ballot(wid == tk));
        } else {
          uint32_t h0, h1;
          hist_range(a, row, &h0, &h1);
          const uint32_t w0 = (h1 - h0) > (uint32_t)a.ras_win ? h1 - (uint32_t)a.ras_win : h0;
          for (uint32_t j = w0 + (uint32_t)lane; j < h1; j += (uint32_t)kWave) rep += a.hist_ids[j] == tk ? 1u : 0u;
          rep = rl_u32(dpp_scan_u32(rep), kWave - 1);
        }
        const bool ras = (float)rep >= a.ras_thresh;
        if (lane == 0) {
          if (!ras) put_result(a, row, tk, TC_OK, 0u);
          C.out[0] = tk;
          C.out[1] = ras ? 1u : 0u;
        }
        return;
      }
    }
  }
  // while cum < top_p and len < top_k: cum += p (the crossing token is kept)
  float cum = 0.0f;
  uint32_t nc = 0;
  while (nc < kmax && cum < a.top_p_f) {
    float pr;
    uint32_t ir;
    at_rank(nc, &pr, &ir);
    cum += pr;
    ++nc;
  }
  uint32_t top;
  {
    float p0;
    at_rank(nc ? nc - 1u : 0u, &p0, &top);  // fallback: the last candidate (idx[0] when none)
  }
  if (nc) {
    float total = -0.0f;
    for (uint32_t r = 0; r < nc; ++r) {
      float pr;
      uint32_t ir;
      at_rank(r, &pr, &ir);
      total += pr;
    }
    const float pick = reinterpret_cast<const float*>(a.uniforms)[2 * row] * total;
    float acc = 0.0f;
    for (uint32_t r = 0; r < nc; ++r) {
      float pr;
      uint32_t ir;
      at_rank(r, &pr, &ir);
      acc += pr;
      if (pick < acc) {
        top = ir;
        break;
      }
    }
  }
  // the repetition window: how often top occurs in the last ras_win decoded
  uint32_t rep = 0;
  if (a.ras_win <= kWave) {
    rep = (uint32_t)__popcll(__ballot(wid == top));
  } else {
    uint32_t h0, h1;
    hist_range(a, row, &h0, &h1);
    const uint32_t w0 = (h1 - h0) > (uint32_t)a.ras_win ? h1 - (uint32_t)a.ras_win : h0;
    for (uint32_t j = w0 + (uint32_t)lane; j < h1; j += (uint32_t)kWave) rep += a.hist_ids[j] == top ? 1u : 0u;
    rep = rl_u32(dpp_scan_u32(rep), kWave - 1);
  }
  const bool ras = (float)rep >= a.ras_thresh;
  if (lane == 0) {
    if (!ras) put_result(a, row, top, TC_OK, 0u);
    C.out[0] = top;
    C.out[1] = ras ? 1u : 0u;
  }
  if (a.topk_count) {
    // the nucleus candidates in vocabulary order, with their probabilities
    const uint64_t below = (1ull << lane) - 1ull;
    uint32_t base = 0;
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const bool in = has[q] && rk[q] < nc;
      const uint64_t m = __ballot(in);
      if (in) {
        const uint32_t j = base + (uint32_t)__popcll(m & below);
        if (j < a.cap) {
          a.topk_ids[(size_t)row * a.cap + j] = id[q];
          a.keep_ids[(size_t)row * a.cap + j] = id[q];
          a.keep_probs[(size_t)row * a.cap + j] = p[q];
        }
      }
      base += (uint32_t)__popcll(m);
    }
    if (lane == 0) {
      a.topk_count[row] = nc;
      a.keep_count[row] = nc;
    }
  }
}

// cosyvoice3 fast path for 1 <= top_k <= 64 < V on rows whose logits are
// finite (the ignore_eos id aside): the row streams once into registers;
// softmax's sequential f32 denominator is reproduced exactly (SeqSum, as in
// the indextts kernel: approximate terms, classification, a list of the
// undecided elements replayed with glibc's expf); candidates for the top_k
// are every element within 2^-9 of a lower bound on the top_k-th largest
// logit (from a histogram of per-thread maxima), far above the roundings that
// expf and the division by S can merge; one wave finishes.  A row whose
// repetition window fires draws from every probability (cosy_random).
// Returns false (nothing written, LDS untouched by the general path) when the
// row needs the general path.
template <typename InT, int ITEMS>
__device__ __forceinline__ bool cosy_fast(const RowArgs& a, CosyLds& U) {
  CosyFastLds& F = U.f;
  const int row = blockIdx.x, t = threadIdx.x, V = a.V;
  const InT* rp = reinterpret_cast<const InT*>(a.logits) + (size_t)row * (size_t)a.ld;
  float x[ITEMS];
  int shift;
  load_row<ITEMS>(rp, V, x, &shift);
  // the repetition window's ids (the last ras_win of the history), in flight
  // with the row for the finishing wave; 0xffffffff matches no token
  uint32_t wid = 0xffffffffu;
  if (wave_id() == 0 && a.ras_win <= kWave) {
    uint32_t h0, h1;
    hist_range(a, row, &h0, &h1);
    const uint32_t w0 = (h1 - h0) > (uint32_t)a.ras_win ? h1 - (uint32_t)a.ras_win : h0;
    if (w0 + (uint32_t)lane_id() < h1) wid = a.hist_ids[w0 + (uint32_t)lane_id()];
  }
  if (t < 64) F.bins[t] = 0u;
  const int e0 = t * ITEMS - shift;
  // the ignore_eos mask (llm.rs:525-529): the EOS term is an exact zero
  uint32_t zm = 0;
  if (a.eos_id >= 0) {
#pragma unroll
    for (int i = 0; i < ITEMS; ++i) zm |= (e0 + i == a.eos_id ? 1u : 0u) << i;
  }
  const uint32_t vm = valid_mask<ITEMS>(V, shift) & ~zm;
  float m = -__builtin_inff(), fsum = 0.0f;
#pragma unroll
  for (int i = 0; i < ITEMS; ++i)
    if ((vm >> i) & 1u) {
      m = m > x[i] ? m : x[i];
      fsum += x[i];
    }
  m = dpp_wave_max(m);
  fsum = dpp_wave_sum(fsum);
  if (lane_id() == 0) {
    F.wmax[wave_id()] = m;
    F.wfin[wave_id()] = fsum;
  }
  lds_barrier();
  float mx, fin;
  {
    const bool in = lane_id() < num_waves();
    mx = dpp_wave_max(in ? F.wmax[lane_id()] : -__builtin_inff());
    fin = dpp_wave_sum(in ? F.wfin[lane_id()] : 0.0f);
  }
  if (!(__builtin_isfinite(fin) && __builtin_isfinite(mx))) {
    __syncthreads();
    return false;
  }
  float d[ITEMS], ap[ITEMS];
  uint32_t exm = 0, force = 0;
  float mns = -__builtin_inff();
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) {
    const bool v = (vm >> i) & 1u;
    d[i] = x[i] - mx;
    if (v) mns = mns > d[i] ? mns : d[i];
    ap[i] = v ? exp_approx(d[i]) : 0.0f;
    exm |= (v ? 0u : 1u) << i;
    force |= (v && !(d[i] >= -87.0f) ? 1u : 0u) << i;  // below the approximation's range
  }
  if (mns > -16.0f) atomicAdd(&F.bins[(uint32_t)(-mns * 4.0f)], 1u);
  SeqSum<ITEMS> sq;
  sq.predict(ap, F.seq);
  lds_barrier();
  // the top_k-th largest d is above -(b0 + 1) / 4; probabilities are monotone
  // in d, and a d below it by more than 2^-9 has a strictly smaller one
  const uint32_t cum = dpp_scan_u32(F.bins[lane_id()]);
  const uint64_t reach = __ballot(cum >= (uint32_t)a.top_k);
  const float thr = reach ? -(float)(__builtin_ctzll(reach) + 1) * 0.25f - 0x1p-9f : __builtin_inff();
  sq.classify(ap, exm, force, e0, F.seq);
  uint32_t sel = 0;
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) sel |= (d[i] >= thr ? 1u : 0u) << i;
  sel &= vm;
  const uint32_t c = (uint32_t)__builtin_popcount(sel);
  const uint32_t ci = dpp_scan_u32(c);
  if (lane_id() == kWave - 1) F.wcand[wave_id()] = ci;
  lds_barrier();
  uint32_t off, n;
  wave_table_u32(F.wcand, &off, &n);
  off += ci - c;
  const bool stage = reach && n <= (uint32_t)FinLds::kCap;
  const bool listed_ok = sq.write_list(ap, d, e0, F.seq, stage ? sel : 0u, [&](int i) {
    F.fin.cand[off++] = ((uint64_t)f2u(d[i]) << 32) | (uint32_t)(e0 + i);
  });
  if (!stage) {
    __syncthreads();
    return false;
  }
  lds_barrier();
  if (listed_ok) sq.replay_terms([](float v) { return expf_glibc_wave(v); }, F.seq);
  lds_barrier();
  if (wave_id() == 0 && listed_ok) sq.replay_walk(F.seq);
  lds_barrier();
  float S = F.seq.S;
  if (!listed_ok || F.seq.bad) {
    float ex[ITEMS];
#pragma unroll
    for (int i = 0; i < ITEMS; ++i) ex[i] = ((vm >> i) & 1u) ? expf_glibc(d[i]) : 0.0f;
    __syncthreads();
    S = block_seqsum_slow<ITEMS>(ex, e0, V, &F.seq.e[0].x, SeqFastLds::kCap, &F.seq.S);
  }
  put_norm(a, row, S);
  if (wave_id() == 0) {
    if (n <= (uint32_t)kWave) cosy_fast_finish_t<1>(a, row, n, S, F, wid);
    else cosy_fast_finish_t<2>(a, row, n, S, F, wid);
  }
  __syncthreads();
  const bool ras = F.out[1] != 0u;  // the nucleus token (F.out[0]) is already written otherwise
  if (ras) {
    // random_sample_probs over every probability
    float pv[ITEMS];
    uint32_t tok = cosy_random_fast<ITEMS>(a, row, d, vm, S, e0, F, pv);
    if (tok == 0xffffffffu) {
      __syncthreads();  // the general path's arrays overlay the fast path's
      tok = cosy_random<ITEMS>(a, row, pv, valid_mask<ITEMS>(V, shift), e0, U.g);
    }
    finish_row(a, row, tok, TC_OK, TC_FLAG_RAS);
  }
  return true;
}

template <typename InT, int ITEMS>
__global__ void __launch_bounds__(max_threads(ITEMS)) k_cosy(RowArgs a) {
  __shared__ CosyLds U;
  if (a.fast && cosy_fast<InT, ITEMS>(a, U)) return;
  cosy_general<InT, ITEMS>(a, U.g);
}


TC_DEFINE_LAUNCH(k_cosy)

}  // namespace tc
