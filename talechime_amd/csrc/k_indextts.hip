// k_indextts.hip -- indextts mel-code sampling (crates/indextts/src/generation.rs:95-303,
// 643-676): the certified fast path; other rows take the general path.

#include "tc_idx_general.h"

namespace tc {

struct IdxFastLds {
  uint32_t bits[kMaxVocabReg / 32];  // history ids present (bit per id)
  uint32_t bins[64];                 // thread maxima of d per 0.25-wide bucket below the row max
  float wmax[kMaxWaves];
  float wfin[kMaxWaves];
  uint32_t wcand[kMaxWaves];
  double lnref, invref;  // log and reciprocal of fref, the refined prediction of the sum
  float fref;
  SeqFastLds seq;
  FinLds fin;
};
// The fast path hands a row to the general path before the general path
// touches LDS, so the two share it.
union IdxLds {
  IdxFastLds f;
  IdxGenLds g;
};

// indextts (generation.rs:643-676 with one draw, 280-303).  Fast path for
// 1 <= K <= 64 < V on rows whose logits are all finite: the row is streamed
// once into registers with the history ids in flight beside it;
// log_softmax's sequential f32 denominator is reproduced exactly
// (block_seqsum_fast); the K-th largest penalised log-prob x' is bounded from
// below by a histogram of the per-thread maxima of d = x - max over ids not
// in the history (x' = d - L is monotone in d for them), and every element
// whose x' lies within a quarter nat of that bound becomes a candidate -- a
// margin far wider than the few floats the later division by T can round
// together.  One wave finishes the row.  Everything else takes idx_general.
template <typename InT, int ITEMS>
__global__ void __launch_bounds__(max_threads(ITEMS)) k_indextts(RowArgs a) {
  __shared__ IdxLds U;
  IdxFastLds& F = U.f;
  const int row = blockIdx.x, t = threadIdx.x, V = a.V;
  if (a.fast) {
    const InT* rp = reinterpret_cast<const InT*>(a.logits) + (size_t)row * (size_t)a.ld;
    float x[ITEMS];
    int shift;
    load_row<ITEMS>(rp, V, x, &shift);
    // history ids: up to kHpt per thread in flight with the row
    constexpr int kHpt = 4;
    uint32_t h0 = 0, h1 = 0;
    if (a.do_pen) hist_range(a, row, &h0, &h1);
    uint32_t hid[kHpt];
#pragma unroll
    for (int j = 0; j < kHpt; ++j) {
      const uint32_t k = h0 + (uint32_t)t + (uint32_t)j * blockDim.x;
      hid[j] = k < h1 ? a.hist_ids[k] : 0xffffffffu;
    }
    const int nwords = (V + 31) >> 5;
    for (int w = t; w < nwords; w += blockDim.x) F.bits[w] = 0u;
    if (t < 64) F.bins[t] = 0u;
    lds_barrier();
    const uint32_t vm = valid_mask<ITEMS>(V, shift);
    const int e0 = t * ITEMS - shift;
    // row max; the sum of the row is finite iff every logit is (or overflows:
    // then the general path)
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
    if (__builtin_isfinite(fin) && __builtin_isfinite(mx)) {
      // the history bitmap, its ids' loads (two dependent rounds: offsets,
      // then ids) overlapping the max and the terms below; read after the
      // terms' barrier
#pragma unroll
      for (int j = 0; j < kHpt; ++j)
        if (hid[j] < (uint32_t)V) atomicOr(&F.bits[hid[j] >> 5], 1u << (hid[j] & 31u));
      for (uint32_t k = h0 + (uint32_t)t + (uint32_t)kHpt * blockDim.x; k < h1; k += blockDim.x) {
        const uint32_t id = a.hist_ids[k];
        if (id < (uint32_t)V) atomicOr(&F.bits[id >> 5], 1u << (id & 31u));
      }
      // log_softmax (generation.rs:95-105): d = x - max; S = sequential f32 sum of exp(d)
      float d[ITEMS], ap[ITEMS];
      uint32_t exm = 0, force = 0;
      float mns = -__builtin_inff(), tsum = 0.0f;
      // Without verification outputs the row is first decided from an
      // interval on L (below), which needs only the sum: v_exp_f32 terms here,
      // each within (2 |d| + 2) 2^-23 of exp(d) relative (the roundings of
      // d log2 e and the instruction's own error).  Weighted by the terms
      // (exp(d) |d| against a sum >= 1) that is below 2^-19 of the sum for any
      // row of up to 16384 logits; with the f32 thread and wave sums the
      // prediction is within 2^-16 more than seq_tau of the sequential sum.
      // The exact sum's terms are computed only when the interval does not
      // settle the row.
      const bool cert_mode = !a.topk_count;
#pragma unroll
      for (int i = 0; i < ITEMS; ++i) {
        const bool v = (vm >> i) & 1u;
        d[i] = x[i] - mx;
        if (cert_mode) tsum += v ? __builtin_amdgcn_exp2f(d[i] * 1.44269504088896341f) : 0.0f;
      }
      SeqSum<ITEMS> sq;
      // the exact sum's approximate terms and their prediction (SeqSum)
      auto exact_terms = [&]() {
#pragma unroll
        for (int i = 0; i < ITEMS; ++i) {
          const bool v = (vm >> i) & 1u;
          ap[i] = v ? exp_approx(d[i]) : 0.0f;
          exm |= (v ? 0u : 1u) << i;
          force |= (v && !(d[i] >= -87.0f) ? 1u : 0u) << i;  // below the approximation's range
        }
        sq.predict(ap, F.seq);
      };
      if (cert_mode) {
        const float tw = dpp_wave_sum(tsum);
        if (lane_id() == 0) F.seq.wsum[wave_id()] = tw;
      } else {
        exact_terms();
      }
      lds_barrier();
      // ids in the history, bit i = element e0 + i, and the histogram of the
      // per-thread maxima of d over the others
      uint64_t seen = 0;
      if (a.do_pen) {
        const int w0 = e0 >= 0 ? (e0 >> 5) : 0;
        const uint32_t lo = w0 < nwords ? F.bits[w0] : 0u;
        const uint32_t hi = w0 + 1 < nwords ? F.bits[w0 + 1] : 0u;
        seen = ((((uint64_t)hi << 32) | lo) >> (e0 >= 0 ? (e0 & 31) : 0));
        if (e0 < 0) seen <<= (uint32_t)(-e0);
      }
#pragma unroll
      for (int i = 0; i < ITEMS; ++i)
        if (((vm >> i) & 1u) && !((seen >> i) & 1ull)) mns = mns > d[i] ? mns : d[i];
      if (mns > -16.0f) atomicAdd(&F.bins[(uint32_t)(-mns * 4.0f)], 1u);
      lds_barrier();
      // Candidates, staged while the exact sum is finished.  The histogram of
      // per-thread maxima of d over ids not in the history puts the K-th largest
      // such d above -(b0 + 1) / 4; x' = d - L is monotone in d for those ids, so
      // every one whose x' can reach the K-th largest has d >= -(b0 + 1) / 4 less
      // a margin (2^-9, far above the roundings of d - L and the floats the
      // division by T can merge).  Ids in the history (x' * pen) are admitted
      // against the same bound for every L the prediction allows.  The
      // thresholds come first (cross-lane, every lane active), so their LDS
      // and DPP latency overlaps the classification.
      const float Sp = sq.total(F.seq);
      const uint32_t cum = dpp_scan_u32(F.bins[lane_id()]);
      const uint64_t reach = __ballot(cum >= (uint32_t)a.K);
      // An interval [Llo, Lhi] that holds log_sum: the reference's sequential
      // sum S lies within seq_tau(V) of the prediction Sp (2^-16 more for the
      // v_exp_f32 terms and their sums), and log_sum is glibc's logf(S),
      // within an ulp of log S; v_log_f32 is within a few ulps of log2, and
      // the slack covers both.
      const float tt = seq_tau(V) + (cert_mode ? 0x1p-16f : 0.0f);
      const float s_lo = Sp * (1.0f - tt), s_hi = Sp * (1.0f + tt);
      const float Llo = __logf(s_lo) * (1.0f - 0x1p-18f) - 0x1p-20f;
      const float Lhi = __logf(s_hi) * (1.0f + 0x1p-18f) + 0x1p-20f;
      float thr_d = __builtin_inff(), thr_s = __builtin_inff();
      if (reach) {
        const uint32_t b0 = (uint32_t)__builtin_ctzll(reach);
        thr_d = -(float)(b0 + 1u) * 0.25f - 0x1p-9f;
        // an id in the history reaches the bound for some L in [L_lo, L_hi]
        // when (d - L_lo) * pen >= thr_d - L_hi, i.e. (pen > 0) d >= thr_s,
        // taken a margin far above its roundings lower
        thr_s = -__builtin_inff();
        if (a.do_pen && a.pen_f > 0.0f) {
          const float L_lo = Llo - 1e-3f, L_hi = Lhi + 1e-3f;
          thr_s = L_lo + (thr_d - L_hi) / a.pen_f - 0x1p-9f;
        }
      }
      // one compare per element against the lower threshold; the few hits are
      // then held to their own
      uint32_t sel = 0;
      const float thr_lo = thr_s < thr_d ? thr_s : thr_d;
#pragma unroll
      for (int i = 0; i < ITEMS; ++i) sel |= (d[i] >= thr_lo ? 1u : 0u) << i;
      sel &= vm;
      if (sel) {
#pragma unroll
        for (int i = 0; i < ITEMS; ++i)
          sel &= ~((d[i] >= (((seen >> i) & 1ull) ? thr_s : thr_d) ? 0u : 1u) << i);
      }
      const uint32_t c = (uint32_t)__builtin_popcount(sel);
      const uint32_t ci = dpp_scan_u32(c);
      if (lane_id() == kWave - 1) F.wcand[wave_id()] = ci;
      lds_barrier();
      uint32_t off, n;
      wave_table_u32(F.wcand, &off, &n);
      off += ci - c;
      const bool stage = reach && n <= (uint32_t)FinLds::kCap;
      auto put_cand = [&](int i) {
        F.fin.cand[off++] = ((uint64_t)f2u(d[i]) << 32) | (((seen >> i) & 1ull) ? 0x80000000u : 0u) | (uint32_t)(e0 + i);
      };
      // idx_cert_finish writes the id when every L in [Llo, Lhi] gives it;
      // otherwise (and with verification outputs) the exact sum below.
      const bool cert = stage && cert_mode;
      if (cert) {
#pragma unroll
        for (int i = 0; i < ITEMS; ++i)
          if ((sel >> i) & 1u) put_cand(i);
        lds_barrier();
        if (wave_id() == 0) {
          bool done = false;
          if (s_lo > 1.0009765625f && s_hi < 1.0e30f) {
            const float La = __logf(Sp);
            done = idx_cert_finish(a, row, n, La < Llo ? Llo : (La > Lhi ? Lhi : La), Llo, Lhi, F.fin);
          }
          if (lane_id() == 0) F.fin.done = done ? 1u : 0u;
        }
        lds_barrier();
        if (F.fin.done) return;
      }
      if (cert_mode) {
        exact_terms();
        lds_barrier();
      }
      sq.classify(ap, exm, force, e0, F.seq);
      lds_barrier();
      // the list (and, when not staged above, the candidates) in one pass over
      // the elements
      const bool listed_ok = sq.write_list(ap, d, e0, F.seq, stage && !cert ? sel : 0u, put_cand);
      // the exception keys of glibc logf around the expected sum, in flight
      // while the sum is finished
      LogfKeys lk;
      if (wave_id() == 0) {
        const float tt = seq_tau((int)sq.u_tot) + 0x1p-22f;
        logf_keys_index(lk, sq.p2_tot * (1.0f - tt), sq.p2_tot * (1.0f + tt));
      }
      if (stage) {
        lds_barrier();
        if (listed_ok) sq.replay_terms([](float v) { return expf_glibc_wave(v); }, F.seq);
        lds_barrier();
        // wave 1, idle during the walk: log and reciprocal of the refined
        // prediction of the sum, from which wave 0 gets the log of the sum
        if (wave_id() == 1 && lane_id() == 0) {
          const float ref = (sq.p2_tot >= 1.0f && sq.p2_tot < 16777216.0f) ? sq.p2_tot : 1.0f;
          F.fref = ref;
          F.lnref = tc_log_d((double)ref);
          F.invref = 1.0 / (double)ref;
        }
        if (wave_id() == 0) {
          logf_keys_load(lk);
          if (listed_ok) sq.replay_walk(F.seq);
        }
        lds_barrier();
        float S = F.seq.S;
        if (!listed_ok || F.seq.bad) {
          float ex[ITEMS];
#pragma unroll
          for (int i = 0; i < ITEMS; ++i) ex[i] = ((vm >> i) & 1u) ? expf_glibc(d[i]) : 0.0f;
          __syncthreads();
          S = block_seqsum_slow<ITEMS>(ex, e0, V, &F.seq.e[0].x, SeqFastLds::kCap, &F.seq.S);
        }
        if (wave_id() == 0) {
          const float L = logf_glibc_near(S, F.fref, F.lnref, F.invref, lk);
          put_norm(a, row, L);
          idx_fast_finish(a, row, n, L, F.fin, cert ? (uint32_t)TC_FLAG_EXACT_SUM : 0u);
        }
        return;
      }
    }
    __syncthreads();
  }
  idx_general<InT, ITEMS>(a, U.g);
}


TC_DEFINE_LAUNCH(k_indextts)

}  // namespace tc
