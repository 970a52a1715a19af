// k_qwen.hip -- qwen3-tts sampling (crates/qwen3-tts/src/generation/sampling.rs:169-400)
// over register-resident rows: the fast path, the general path, top-p over
// many survivors.

#include "tc_row.h"

namespace tc {

// ================================================================ qwen, many survivors
// No top-p and more survivors than the LDS stage holds (top-k off or wide):
// softmax over the survivors and the multinomial draw (sampling.rs:302-328)
// over the register-resident row.  The denominator is the reference's
// sequential f32 sum in vocabulary order of the exact terms (non-survivors
// add +0), and the CDF its running sums of e / S2 (block_seqsum, seq_prefix);
// the first index whose running sum reaches u is the token (0 when u <= 0 or
// none does).  Verification outputs: the first `cap` survivors in vocabulary
// order with their probabilities.
// surv: the ids the draw runs over (n of them); tk: the top-k survivors for
// the verification outputs.
template <int ITEMS>
__device__ __forceinline__ void qwen_wide_cdf(const RowArgs& a, const float (&x)[ITEMS], uint32_t surv, uint32_t tk,
                                              uint32_t vm, int e0, uint32_t n, uint32_t flags, SurvLds& sv,
                                              BlockScratch& s, SeqLds& sq, ScanLds& sc) {
  const int row = blockIdx.x, t = threadIdx.x, V = a.V;
  float* stage = reinterpret_cast<float*>(&sv);  // the survivor stage is not in use here
  constexpr int kStage = (int)(sizeof(SurvLds) / sizeof(float));
  float m = -__builtin_inff();
#pragma unroll
  for (int i = 0; i < ITEMS; ++i)
    if ((surv >> i) & 1u) m = rmaxf(m, x[i]);
  const float vmax = block_max(m, s);
  float ev[ITEMS];
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) ev[i] = ((surv >> i) & 1u) ? expf_glibc(x[i] - vmax) : 0.0f;
  auto same = [](float v) { return v; };
  float S2;
  {
    SeqThread<ITEMS> th;
    if (!block_seqsum<ITEMS>(ev, ~0u, ev, same, e0, 0, th, sq, sc, &S2))
      S2 = block_seqsum_slow<ITEMS>(ev, e0, V, stage, kStage, &sq.S);
  }
  float pv[ITEMS];
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) pv[i] = ((surv >> i) & 1u) ? ev[i] / S2 : 0.0f;
  const float u = reinterpret_cast<const float*>(a.uniforms)[row];
  uint32_t tok = 0;
  if (u > 0.0f) {
    uint32_t found = 0xffffffffu;
    SeqThread<ITEMS> th;
    float Sp;
    if (block_seqsum<ITEMS>(pv, ~0u, pv, same, e0, 0, th, sq, sc, &Sp)) {
      float pre[ITEMS];
      seq_prefix<ITEMS>(th, sq, pre);
      uint32_t first = 0xffffffffu;
#pragma unroll
      for (int i = ITEMS - 1; i >= 0; --i)
        if (((vm >> i) & 1u) && pre[i] >= u) first = (uint32_t)(e0 + i);
      found = block_min_u(first, s);
    } else {
      // one lane walks the staged probabilities a chunk at a time
      __shared__ uint32_t s_found;
      float acc = 0.0f;
      for (int c0 = 0; c0 < V; c0 += kStage) {
#pragma unroll
        for (int i = 0; i < ITEMS; ++i) {
          const int e = e0 + i;
          if (((vm >> i) & 1u) && e >= c0 && e < c0 + kStage) stage[e - c0] = pv[i];
        }
        __syncthreads();
        if (t == 0) {
          const int c1 = (c0 + kStage < V) ? c0 + kStage : V;
          for (int e = c0; e < c1 && found == 0xffffffffu; ++e) {
            acc += stage[e - c0];
            if (acc >= u) found = (uint32_t)e;
          }
          s_found = found;
        }
        __syncthreads();
        found = s_found;
        __syncthreads();
        if (found != 0xffffffffu) break;
      }
    }
    tok = found != 0xffffffffu ? found : 0u;
  }
  finish_row(a, row, tok, TC_OK, flags);
  put_norm(a, row, S2);
  if (a.topk_count || a.keep_count) {
    uint32_t tot;
    uint32_t p = block_excl_scan((uint32_t)__builtin_popcount(tk), s, &tot);
#pragma unroll
    for (int i = 0; i < ITEMS; ++i)
      if ((tk >> i) & 1u) {
        if (p < a.cap && a.topk_count) a.topk_ids[(size_t)row * a.cap + p] = (uint32_t)(e0 + i);
        ++p;
      }
    p = block_excl_scan((uint32_t)__builtin_popcount(surv), s, &tot);
#pragma unroll
    for (int i = 0; i < ITEMS; ++i)
      if ((surv >> i) & 1u) {
        if (p < a.cap && a.keep_count) {
          a.keep_ids[(size_t)row * a.cap + p] = (uint32_t)(e0 + i);
          a.keep_probs[(size_t)row * a.cap + p] = pv[i];
        }
        ++p;
      }
    if (t == 0 && a.keep_count) a.keep_count[row] = n;
  }
}

// ================================================================ qwen, fast path
// qwen semantics (sampling.rs:169-328 with the caller's penalty, masks and
// EOS) for 1 <= K <= 64 < V on rows whose scores are finite or -inf:
//  * the row, its history map and the transform, then the row max;
//  * a 64-bucket histogram (quarter-unit wide) of the per-thread maxima below
//    the row max bounds the K-th largest score from below, since K threads
//    hold a score at or above the bucket where the count reaches K; every
//    score at or above that bound (less a margin above the roundings of the
//    bucket arithmetic) is a candidate, staged in vocabulary order (at most
//    kQCand);
//  * one wave finishes: ranks (value descending, id ascending: the general
//    path's order), the top-k cut (ties kept), exp terms, and the reference's
//    sequential f32 sums: the top-p denominator and running sum in rank order
//    (255-299), then the softmax denominator and the CDF in vocabulary order
//    (302-328), as readlane chains over at most kQCand lanes.
// Anything else takes the general path below.
constexpr int kQCand = 128;

struct QFastLds {
  uint32_t bits[kMaxVocabReg / 32];  // history ids present
  uint32_t bins[64];
  float wmax[kMaxWaves];
  uint32_t wbad[kMaxWaves];
  uint32_t wcand[kMaxWaves];
  uint64_t cand[kQCand];  // (bits of the score << 32) | id, vocabulary order
  uint64_t rkey[kQCand];
  float er[kQCand];       // survivors' terms by rank
  float vr[kQCand];       // and their scores
};

template <int NS>
__device__ __forceinline__ void qwen_fast_finish_t(const RowArgs& a, int row, uint32_t n, float vmax, QFastLds& F) {
  const int lane = lane_id();
  float v[2];
  uint32_t id[2];
  bool has[2];
  uint64_t key[2];
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const uint32_t c = (uint32_t)(q * kWave + lane);
    has[q] = q < NS && c < n;
    const uint64_t cv = has[q] ? F.cand[c] : 0ull;
    v[q] = u2f((uint32_t)(cv >> 32));
    id[q] = (uint32_t)cv;
    key[q] = has[q] ? (((uint64_t)ckey(v[q]) << 32) | (uint64_t)(~c)) : 0ull;
  }
  const uint32_t K = (uint32_t)a.K;
  uint32_t rk[2] = {0u, 0u};
  float kth;
  if (a.do_topp) {
    // ranks (value descending, id ascending) for the rank-order sums
#pragma unroll
    for (int q = 0; q < NS; ++q) F.rkey[q * kWave + lane] = key[q];
    lds_wait();
    const uint32_t nr = (n + 3u) & ~3u;
    for (uint32_t j = 0; j < nr; j += 4) {
      const uint64_t k0 = F.rkey[j], k1 = F.rkey[j + 1], k2 = F.rkey[j + 2], k3 = F.rkey[j + 3];
#pragma unroll
      for (int q = 0; q < NS; ++q)
        rk[q] += ((k0 > key[q] ? 1u : 0u) + (k1 > key[q] ? 1u : 0u)) + ((k2 > key[q] ? 1u : 0u) + (k3 > key[q] ? 1u : 0u));
    }
    // top-k (224-249): keep v >= the K-th largest, ties kept
    const uint64_t bk0 = __ballot(has[0] && rk[0] == K - 1u), bk1 = __ballot(has[1] && rk[1] == K - 1u);
    kth = bk0 ? rl_f32(v[0], __builtin_ctzll(bk0)) : rl_f32(v[1], __builtin_ctzll(bk1));
  } else {
    // without top-p only the K-th largest value is needed: the largest
    // 32-bit key T with at least K keys >= T, bit by bit over wave ballots
    // (at least K candidates are staged, so it exists)
    uint32_t k32[2];
#pragma unroll
    for (int q = 0; q < 2; ++q) k32[q] = has[q] ? (uint32_t)(key[q] >> 32) : 0u;
    uint32_t T = 0;
#pragma unroll
    for (int b = 31; b >= 0; --b) {
      const uint32_t c = T | (1u << b);
      uint32_t cnt = (uint32_t)__popcll(__ballot(k32[0] >= c));
      if (NS == 2) cnt += (uint32_t)__popcll(__ballot(k32[1] >= c));
      T = cnt >= K ? c : T;
    }
    const uint64_t e0 = __ballot(k32[0] == T), e1 = __ballot(k32[1] == T);
    kth = e0 ? rl_f32(v[0], __builtin_ctzll(e0)) : rl_f32(v[1], __builtin_ctzll(e1));
  }
  bool surv[2];
#pragma unroll
  for (int q = 0; q < 2; ++q) surv[q] = has[q] && v[q] >= kth;
  const uint64_t sm0 = __ballot(surv[0]), sm1 = __ballot(surv[1]);
  const uint32_t ns = (uint32_t)(__popcll(sm0) + __popcll(sm1));
  // softmax numerators over the survivors; the row max is the largest survivor
  float e[2];
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const float t = q < NS ? expf_glibc_wave(surv[q] ? v[q] - vmax : 0.0f) : 0.0f;
    e[q] = surv[q] ? t : 0.0f;
  }
  uint32_t flags = 0;
  // ---- decisions from tree-ordered f32 sums first (no verification outputs):
  // a prefix scan of at most 128 non-negative terms and its quotients stay
  // within (n + 32) * 2^-22 of the reference's sequential running sums (a
  // relative bound on values <= 1); a decision inside that margin goes to the
  // reference's loops below.
  if (!a.topk_count && !a.norm) {
    bool ok = true;
    uint32_t cut = ns;
    if (a.do_topp) {
#pragma unroll
      for (int q = 0; q < 2; ++q)
        if (surv[q]) {
          F.er[rk[q]] = e[q];
          F.vr[rk[q]] = v[q];
        }
      lds_wait();
      const float St = dpp_wave_sum(e[0] + e[1]);
      float c[2];
      float carry = 0.0f;
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const uint32_t r = (uint32_t)(q * kWave + lane);
        const float pr = (q < NS && r < ns) ? F.er[r] / St : 0.0f;
        c[q] = q < NS ? dpp_scan_f32(pr) + carry : 0.0f;
        if (q < NS) carry = rl_f32(c[q], kWave - 1);
      }
      const float mg = (float)(ns + 32u) * 0x1p-22f;
      const uint64_t over0 = __ballot((uint32_t)lane < ns && c[0] > a.top_p_f);
      const uint64_t over1 = __ballot((uint32_t)(kWave + lane) < ns && c[1] > a.top_p_f);
      const uint32_t r = over0 ? (uint32_t)__builtin_ctzll(over0) : (over1 ? 64u + (uint32_t)__builtin_ctzll(over1) : ns);
      // the running sums at the cut and just before it against p
      const float c_at = r < ns ? rl_f32(r < 64u ? c[0] : c[1], (int)(r & 63u)) : 0.0f;
      const uint32_t rp = r < ns ? r : ns;  // the last position below the cut is rp - 1
      const float c_prev = rp ? rl_f32(rp - 1u < 64u ? c[0] : c[1], (int)((rp - 1u) & 63u)) : 0.0f;
      ok = (r >= ns || c_at - a.top_p_f > mg) && (rp == 0u || a.top_p_f - c_prev > mg);
      cut = r < ns ? r + 1u : ns;
      if (ok && cut < ns && F.vr[cut - 1u] == F.vr[cut]) flags |= TC_FLAG_TIE_CUT;
    }
    if (ok) {
      bool kp[2];
#pragma unroll
      for (int q = 0; q < 2; ++q) kp[q] = surv[q] && (!a.do_topp || rk[q] < cut);
      const float S2t = dpp_wave_sum((kp[0] ? e[0] : 0.0f) + (kp[1] ? e[1] : 0.0f));
      const uint64_t km0 = __ballot(kp[0]), km1 = __ballot(kp[1]);
      const uint32_t nk = (uint32_t)(__popcll(km0) + __popcll(km1));
      const float c0 = dpp_scan_f32(kp[0] ? e[0] / S2t : 0.0f);
      const float c1 = NS == 2 ? dpp_scan_f32(kp[1] ? e[1] / S2t : 0.0f) + rl_f32(c0, kWave - 1) : 0.0f;
      const float u = reinterpret_cast<const float*>(a.uniforms)[row];
      const float mg = (float)(nk + 32u) * 0x1p-22f;
      uint32_t tok = 0;
      if (u > 0.0f) {
        // the first kept entry whose running sum reaches u, else 0
        const uint64_t h0 = __ballot(kp[0] && c0 >= u), h1 = __ballot(kp[1] && c1 >= u);
        uint32_t pk = 0xffffffffu;
        if (h0) pk = (uint32_t)__builtin_ctzll(h0);
        else if (h1) pk = 64u + (uint32_t)__builtin_ctzll(h1);
        // the kept entry before it (or the last kept one when none reaches u)
        uint64_t b0 = km0, b1 = km1;
        if (pk != 0xffffffffu) {
          b0 = pk < 64u ? (km0 & ((1ull << pk) - 1ull)) : km0;
          b1 = pk < 64u ? 0ull : (km1 & ((1ull << (pk - 64u)) - 1ull));
        }
        const uint32_t pv = b1 ? 64u + 63u - (uint32_t)__builtin_clzll(b1) : (b0 ? 63u - (uint32_t)__builtin_clzll(b0) : 0xffffffffu);
        const float c_pk = pk != 0xffffffffu ? rl_f32(pk < 64u ? c0 : c1, (int)(pk & 63u)) : 0.0f;
        const float c_pv = pv != 0xffffffffu ? rl_f32(pv < 64u ? c0 : c1, (int)(pv & 63u)) : 0.0f;
        ok = (pk == 0xffffffffu || c_pk - u > mg) && (pv == 0xffffffffu || u - c_pv > mg);
        if (pk != 0xffffffffu) tok = rl_u32(pk < 64u ? id[0] : id[1], (int)(pk & 63u));
      }
      if (ok) {
        if (lane == 0) put_result(a, row, tok, TC_OK, flags);
        return;
      }
    }
    flags = 0;
  }
  bool kept[2] = {surv[0], surv[1]};
  if (a.do_topp) {
    // top-p (255-299): survivors occupy ranks [0, ns)
#pragma unroll
    for (int q = 0; q < 2; ++q)
      if (surv[q]) {
        F.er[rk[q]] = e[q];
        F.vr[rk[q]] = v[q];
      }
    lds_wait();
    float er[2];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const uint32_t r = (uint32_t)(q * kWave + lane);
      er[q] = (q < NS && r < ns) ? F.er[r] : 0.0f;
    }
    float S = -0.0f;
    for (uint32_t r = 0; r < ns; ++r) S += rl_f32(r < (uint32_t)kWave ? er[0] : er[1], (int)(r & 63u));
    float pr[2];
#pragma unroll
    for (int q = 0; q < 2; ++q) pr[q] = er[q] / S;
    float cum = 0.0f;
    uint32_t cut = ns;
    for (uint32_t r = 0; r < ns; ++r) {
      cum += rl_f32(r < (uint32_t)kWave ? pr[0] : pr[1], (int)(r & 63u));
      if (cum > a.top_p_f) {
        cut = r + 1u;
        break;
      }
    }
    if (cut < ns && F.vr[cut - 1u] == F.vr[cut]) flags |= TC_FLAG_TIE_CUT;
#pragma unroll
    for (int q = 0; q < 2; ++q) kept[q] = surv[q] && rk[q] < cut;
  }
  // softmax + multinomial in vocabulary order (302-328): non-kept entries add +0
  const uint64_t km0 = __ballot(kept[0]), km1 = __ballot(kept[1]);
  float S2 = 0.0f;
  for (uint64_t m = km0; m; m &= m - 1ull) S2 += rl_f32(e[0], __builtin_ctzll(m));
  for (uint64_t m = km1; m; m &= m - 1ull) S2 += rl_f32(e[1], __builtin_ctzll(m));
  const float u = reinterpret_cast<const float*>(a.uniforms)[row];
  uint32_t tok = 0;
  float pk[2];
#pragma unroll
  for (int q = 0; q < 2; ++q) pk[q] = e[q] / S2;
  if (u > 0.0f) {
    float cum = 0.0f;
    bool done = false;
    for (uint64_t m = km0; m && !done; m &= m - 1ull) {
      const int l = __builtin_ctzll(m);
      cum += rl_f32(pk[0], l);
      if (cum >= u) {
        tok = rl_u32(id[0], l);
        done = true;
      }
    }
    for (uint64_t m = km1; m && !done; m &= m - 1ull) {
      const int l = __builtin_ctzll(m);
      cum += rl_f32(pk[1], l);
      if (cum >= u) {
        tok = rl_u32(id[1], l);
        done = true;
      }
    }
  }
  if (lane == 0) {
    put_result(a, row, tok, TC_OK, flags);
    if (a.norm) a.norm[row] = S2;
    if (a.topk_count) a.topk_count[row] = ns;
    if (a.keep_count) a.keep_count[row] = (uint32_t)(__popcll(km0) + __popcll(km1));
  }
  const uint64_t below = (1ull << lane) - 1ull;
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    if (a.topk_count && surv[q]) {
      const uint32_t j = (q == 0 ? 0u : (uint32_t)__popcll(sm0)) + (uint32_t)__popcll((q == 0 ? sm0 : sm1) & below);
      if (j < a.cap) a.topk_ids[(size_t)row * a.cap + j] = id[q];
    }
    if (a.keep_count && kept[q]) {
      const uint32_t j = (q == 0 ? 0u : (uint32_t)__popcll(km0)) + (uint32_t)__popcll((q == 0 ? km0 : km1) & below);
      if (j < a.cap) {
        a.keep_ids[(size_t)row * a.cap + j] = id[q];
        a.keep_probs[(size_t)row * a.cap + j] = pk[q];
      }
    }
  }
}

// true: the row is sampled; false: every thread goes on to the general path
// (the decision is the same in every thread).
template <typename InT, int ITEMS>
__device__ __forceinline__ bool qwen_fast(const RowArgs& a, QFastLds& F) {
  const int row = blockIdx.x, t = threadIdx.x, V = a.V;
  const InT* rp = reinterpret_cast<const InT*>(a.logits) + (size_t)row * (size_t)a.ld;
  float x[ITEMS];
  int shift;
  load_row<ITEMS>(rp, V, x, &shift);
  const bool use_seen = a.do_pen && a.hist_mode != TC_HIST_MASK;
  constexpr int kHpt = 4;
  uint32_t h0 = 0, h1 = 0;
  if (use_seen) hist_range(a, row, &h0, &h1);
  uint32_t hid[kHpt];
#pragma unroll
  for (int j = 0; j < kHpt; ++j) {
    const uint32_t k = h0 + (uint32_t)t + (uint32_t)j * blockDim.x;
    hid[j] = k < h1 ? a.hist_ids[k] : 0xffffffffu;
  }
  const int nwords = (V + 31) >> 5;
  if (use_seen)
    for (int w = t; w < nwords; w += blockDim.x) F.bits[w] = 0u;
  if (t < 64) F.bins[t] = 0u;
  lds_barrier();
  if (use_seen) {
#pragma unroll
    for (int j = 0; j < kHpt; ++j)
      if (hid[j] < (uint32_t)V) atomicOr(&F.bits[hid[j] >> 5], 1u << (hid[j] & 31u));
    for (uint32_t k = h0 + (uint32_t)t + (uint32_t)kHpt * blockDim.x; k < h1; k += blockDim.x) {
      const uint32_t hv = a.hist_ids[k];
      if (hv < (uint32_t)V) atomicOr(&F.bits[hv >> 5], 1u << (hv & 31u));
    }
  }
  lds_barrier();
  const uint32_t vm = valid_mask<ITEMS>(V, shift);
  const int e0 = t * ITEMS - shift;
  uint64_t seen = 0;
  if (use_seen) {
    const int w0 = e0 >= 0 ? (e0 >> 5) : 0;
    const uint32_t lo = w0 < nwords ? F.bits[w0] : 0u;
    const uint32_t hi = w0 + 1 < nwords ? F.bits[w0 + 1] : 0u;
    seen = ((((uint64_t)hi << 32) | lo) >> (e0 >= 0 ? (e0 & 31) : 0));
    if (e0 < 0) seen <<= (uint32_t)(-e0);
  }
  // the caller chain (synthesis.rs:1238-1276) then temperature (sampling.rs:175-184)
  float tmax = -__builtin_inff();
  uint32_t bad = 0;
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) {
    if (!((vm >> i) & 1u)) continue;
    const int e = e0 + i;
    float v = x[i];
    if (a.do_pen) {
      const bool pen = use_seen ? ((seen >> i) & 1ull) != 0ull : (a.pen_mask[e] > 0.0f);
      if (pen) v = v * (v > 0.0f ? a.inv_pen : a.pen_f);
    }
    if (a.add_mask) v = v + a.add_mask[e];
    if (e == a.eos_id) v = -__builtin_inff();
    if (a.do_temp) v = v * a.tmul + 0.0f;
    x[i] = v;
    bad |= (__builtin_isnan(v) || v == __builtin_inff()) ? 1u : 0u;
    tmax = v > tmax ? v : tmax;
  }
  {
    const float wm = dpp_wave_max(tmax);
    const uint32_t wb = dpp_wave_or(bad);
    if (lane_id() == 0) {
      F.wmax[wave_id()] = wm;
      F.wbad[wave_id()] = wb;
    }
  }
  lds_barrier();
  const bool inw = lane_id() < num_waves();
  const float vmax = dpp_wave_max(inw ? F.wmax[lane_id()] : -__builtin_inff());
  const uint32_t any_bad = dpp_wave_or(inw ? F.wbad[lane_id()] : 0u);
  if (any_bad || !(vmax > -__builtin_inff())) return false;
  if (tmax >= vmax - 16.0f) {
    const float db = (vmax - tmax) * 4.0f;
    if (db < 64.0f) atomicAdd(&F.bins[(uint32_t)db], 1u);
  }
  lds_barrier();
  const uint32_t cum = dpp_scan_u32(F.bins[lane_id()]);
  const uint64_t reach = __ballot(cum >= (uint32_t)a.K);
  if (!reach) return false;
  const uint32_t b0 = (uint32_t)__builtin_ctzll(reach);
  const float thr = vmax - ((float)(b0 + 1u) * 0.25f + (0x1p-16f + __builtin_fabsf(vmax) * 0x1p-20f));
  uint32_t sel = 0;
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) sel |= (x[i] >= thr ? 1u : 0u) << i;
  sel &= vm;
  const uint32_t c = (uint32_t)__builtin_popcount(sel);
  const uint32_t ci = dpp_scan_u32(c);
  if (lane_id() == kWave - 1) F.wcand[wave_id()] = ci;
  lds_barrier();
  uint32_t off, n;
  wave_table_u32(F.wcand, &off, &n);
  if (n > (uint32_t)kQCand) return false;
  off += ci - c;
#pragma unroll
  for (int i = 0; i < ITEMS; ++i)
    if ((sel >> i) & 1u) F.cand[off++] = ((uint64_t)f2u(x[i]) << 32) | (uint32_t)(e0 + i);
  lds_barrier();
  if (wave_id() == 0) {
    if (n <= (uint32_t)kWave) qwen_fast_finish_t<1>(a, row, n, vmax, F);
    else qwen_fast_finish_t<2>(a, row, n, vmax, F);
  }
  return true;
}

// ================================================================ qwen, top-p over many survivors
// The general path's LDS: the history map and the survivor stage, or, past
// them, the rank keys of every survivor of a register-resident row.
constexpr int kWideCap = kMaxVocabReg;
struct QGenLds {
  uint8_t seen[kMaxVocabReg];
  SurvLds sv;
};
// The fast path's LDS shares the union: it hands a row over only after its
// last access.  Kept under 80 KB, so two workgroups fit a CU.
union QGenU {
  QGenLds g;
  uint32_t wide[kWideCap];  // ~ckey of each survivor's value: ascending = value descending
  QFastLds f;
};

// top-p (sampling.rs:255-299) over more than kSurvCap survivors (top-k off or
// wide), then softmax and the draw (302-328) by qwen_wide_cdf over the kept
// ones.  The survivors' values are sorted into rank order (value descending;
// equal values are equal terms, so the sums need no ids); thread t then holds
// ranks ITEMS * t + i (n <= V <= ITEMS * blockDim), the sequential f32
// denominator in rank order and the running sum of e / S are block_seqsum
// and seq_prefix over those positions, and the cut follows the first running
// sum above p (the crossing rank kept).  The kept ids are the values above
// the cut's, and of the values equal to it the lowest ids, as many as the
// cut leaves (the reference's unstable sort leaves that order open:
// TC_FLAG_TIE_CUT where equal values straddle the cut).
template <int ITEMS>
__device__ __forceinline__ void qwen_wide_topp(const RowArgs& a, const float (&x)[ITEMS], uint32_t surv, uint32_t vm,
                                               int e0, uint32_t n, uint32_t flags, QGenU& U, BlockScratch& s,
                                               uint32_t* s_out, SeqLds& sq, ScanLds& sc) {
  const int t = threadIdx.x;
  // the survivors' rank keys, padded, sorted
  uint32_t tot;
  uint32_t pos = block_excl_scan((uint32_t)__builtin_popcount(surv), s, &tot);
#pragma unroll
  for (int i = 0; i < ITEMS; ++i)
    if ((surv >> i) & 1u) U.wide[pos++] = ~ckey(x[i]);
  const int n_pad = next_pow2((int)n < 2 ? 2 : (int)n);
  for (int j = (int)n + t; j < n_pad; j += blockDim.x) U.wide[j] = 0xffffffffu;
  __syncthreads();
  block_bitonic_sort(U.wide, n_pad);
  // ranks ITEMS * t + i in registers
  const int p0 = ITEMS * t;
  float v[ITEMS], e[ITEMS];
  const float vmax = untkey(~U.wide[0]);
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) {
    const bool in = p0 + i < (int)n;
    v[i] = in ? untkey(~U.wide[p0 + i]) : 0.0f;
    e[i] = in ? expf_glibc(v[i] - vmax) : 0.0f;
  }
  __syncthreads();  // the sort buffer is free from here
  float* stage = reinterpret_cast<float*>(U.wide);
  auto same = [](float y) { return y; };
  float S;
  {
    SeqThread<ITEMS> th;
    if (!block_seqsum<ITEMS>(e, ~0u, e, same, p0, 0, th, sq, sc, &S))
      S = block_seqsum_slow<ITEMS>(e, p0, (int)n, stage, kWideCap, &sq.S);
  }
  float q[ITEMS];
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) q[i] = p0 + i < (int)n ? e[i] / S : 0.0f;
  // the running sum of q in rank order: the first rank above p
  uint32_t first = 0xffffffffu;
  {
    SeqThread<ITEMS> th;
    float Sq;
    if (block_seqsum<ITEMS>(q, ~0u, q, same, p0, 0, th, sq, sc, &Sq)) {
      float pre[ITEMS];
      seq_prefix<ITEMS>(th, sq, pre);
#pragma unroll
      for (int i = ITEMS - 1; i >= 0; --i)
        if (p0 + i < (int)n && pre[i] > a.top_p_f) first = (uint32_t)(p0 + i);
      first = block_min_u(first, s);
    } else {
      // one lane walks the running sum
#pragma unroll
      for (int i = 0; i < ITEMS; ++i)
        if (p0 + i < (int)n) stage[p0 + i] = q[i];
      __syncthreads();
      if (t == 0) {
        float cum = 0.0f;
        uint32_t f = 0xffffffffu;
        for (uint32_t r = 0; r < n; ++r) {
          cum += stage[r];
          if (cum > a.top_p_f) {
            f = r;
            break;
          }
        }
        s_out[2] = f;
      }
      __syncthreads();
      first = s_out[2];
    }
  }
  const uint32_t cut = first != 0xffffffffu ? first + 1u : n;
  // the values at ranks cut - 1 and cut (equal: a tie straddles the cut)
  __syncthreads();
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) {
    if ((uint32_t)(p0 + i) + 1u == cut) s_out[2] = f2u(v[i]);
    if ((uint32_t)(p0 + i) == cut) s_out[3] = f2u(v[i]);
  }
  __syncthreads();
  const float vcut = u2f(s_out[2]);
  if (cut < n && s_out[2] == s_out[3]) flags |= TC_FLAG_TIE_CUT;
  // kept: values above vcut, and the first (cut - above) ids, in vocabulary
  // order, of those equal to it
  uint32_t above = 0, eq = 0;
#pragma unroll
  for (int i = 0; i < ITEMS; ++i)
    if ((surv >> i) & 1u) {
      above += x[i] > vcut ? 1u : 0u;
      eq += x[i] == vcut ? 1u : 0u;
    }
  const uint32_t n_above = block_sum_u(above, s);
  uint32_t eq_tot;
  uint32_t eq_rank = block_excl_scan(eq, s, &eq_tot);
  const uint32_t keep_eq = cut - n_above;
  uint32_t kept = 0;
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) {
    if (!((surv >> i) & 1u)) continue;
    if (x[i] > vcut) kept |= 1u << i;
    else if (x[i] == vcut) {
      if (eq_rank < keep_eq) kept |= 1u << i;
      ++eq_rank;
    }
  }
  __syncthreads();  // the sort buffer shares LDS with the CDF's staging
  qwen_wide_cdf<ITEMS>(a, x, kept, surv, vm, e0, cut, flags, U.g.sv, s, sq, sc);
}

// ================================================================ qwen
template <typename InT, int ITEMS>
__global__ void __launch_bounds__(max_threads(ITEMS)) k_qwen(RowArgs a) {
  __shared__ QGenU U;
  if (a.fast) {
    if (qwen_fast<InT, ITEMS>(a, U.f)) return;
    __syncthreads();
  }
  uint8_t* s_seen = U.g.seen;
  SurvLds& sv = U.g.sv;
  __shared__ uint32_t s_hist[256];
  __shared__ BlockScratch s;
  __shared__ uint32_t s_out[4];
  __shared__ SeqLds qsq;
  __shared__ ScanLds qsc;
  const int row = blockIdx.x, t = threadIdx.x, V = a.V;
  const InT* rp = reinterpret_cast<const InT*>(a.logits) + (size_t)row * (size_t)a.ld;
  float x[ITEMS];
  int shift;
  load_row<ITEMS>(rp, V, x, &shift);
  const uint32_t vm = valid_mask<ITEMS>(V, shift);
  const int e0 = t * ITEMS - shift;
  const bool use_seen = a.do_pen && a.hist_mode != TC_HIST_MASK;
  if (use_seen) build_seen(a, row, s_seen, s);

  // caller chain (synthesis.rs:1238-1276) then temperature (sampling.rs:175-184)
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) {
    if (!((vm >> i) & 1u)) continue;
    const int e = e0 + i;
    float v = x[i];
    if (a.do_pen) {
      bool pen = use_seen ? (s_seen[e] != 0) : (a.pen_mask[e] > 0.0f);
      if (pen) v = v * (v > 0.0f ? a.inv_pen : a.pen_f);
    }
    if (a.add_mask) v = v + a.add_mask[e];
    if (e == a.eos_id) v = -__builtin_inff();
    if (a.do_temp) v = v * a.tmul + 0.0f;
    x[i] = v;
  }

  if (a.greedy) {
    // candle argmax: first index whose value is strictly greater (NaN skipped)
    uint64_t best = 0;
#pragma unroll
    for (int i = 0; i < ITEMS; ++i) {
      if (!((vm >> i) & 1u) || __builtin_isnan(x[i])) continue;
      uint64_t k = ((uint64_t)ckey(x[i]) << 32) | (uint64_t)(~(uint32_t)(e0 + i));
      best = k > best ? k : best;
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      uint64_t other = __shfl_xor(best, o);
      best = other > best ? other : best;
    }
    uint64_t* wb = sv.key;
    if (lane_id() == 0) wb[wave_id()] = best;
    if (t == 0) s_out[0] = 0u;
    __syncthreads();
    // x[0] NaN: the reference never updates its accumulator and returns 0
#pragma unroll
    for (int i = 0; i < ITEMS; ++i)
      if (e0 + i == 0 && __builtin_isnan(x[i])) s_out[0] = 1u;
    __syncthreads();
    if (t == 0) {
      uint64_t b = 0;
      for (int w = 0; w < num_waves(); ++w) b = wb[w] > b ? wb[w] : b;
      uint32_t tok = (b == 0 || s_out[0]) ? 0u : ~(uint32_t)(b & 0xffffffffu);
      put_result(a, row, tok, TC_OK, TC_FLAG_GREEDY);
    }
    no_verify(a, row);
    return;
  }

  // top-k (sampling.rs:224-249): keep v >= k-th largest, ties kept
  uint32_t key[ITEMS];
  uint32_t sel = 0, nanm = 0;
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) {
    key[i] = 0u;
    if (!((vm >> i) & 1u)) continue;
    if (__builtin_isnan(x[i])) { nanm |= 1u << i; continue; }
    key[i] = ckey(x[i]);
    sel |= 1u << i;
  }
  uint32_t flags = block_or_u(nanm, s) ? (uint32_t)TC_FLAG_NAN_ROW : 0u;
  float thr = -__builtin_inff();
  if (a.K > 0) {
    uint32_t kk;
    if (block_kth_largest<ITEMS>(key, sel, (uint32_t)a.K, s_hist, s, &kk)) thr = untkey(kk);
  }
  uint32_t surv = 0;
#pragma unroll
  for (int i = 0; i < ITEMS; ++i)
    if (((sel >> i) & 1u) && x[i] >= thr && x[i] != -__builtin_inff()) surv |= 1u << i;
  const uint32_t n = compact<ITEMS>(x, surv, e0, sv, s);
  write_topk(a, row, sv, n);
  if (n > (uint32_t)kSurvCap) {
    if (!a.do_topp) {
      qwen_wide_cdf<ITEMS>(a, x, surv, surv, vm, e0, n, flags, sv, s, qsq, qsc);
      return;
    }
    if (n <= (uint32_t)kWideCap) {
      qwen_wide_topp<ITEMS>(a, x, surv, vm, e0, n, flags, U, s, s_out, qsq, qsc);
      return;
    }
    // top-p over more survivors than the rank sort holds: not handled
    finish_row(a, row, 0u, TC_EUNSUPPORTED, flags);
    if (t == 0 && a.keep_count) a.keep_count[row] = 0;
    put_norm(a, row, __builtin_nanf(""));
    return;
  }
  if (n == 0) {  // every entry -inf (or NaN): the reference's CDF is NaN -> index 0
    finish_row(a, row, 0u, TC_OK, flags);
    if (t == 0 && a.keep_count) a.keep_count[row] = 0;
    put_norm(a, row, __builtin_nanf(""));
    return;
  }
  // softmax numerators over the survivors; the row max is the largest survivor
  float m = -__builtin_inff();
  for (uint32_t j = t; j < n; j += blockDim.x) m = rmaxf(m, sv.val[j]);
  const float vmax = block_max(m, s);
  for (uint32_t j = t; j < n; j += blockDim.x) {
    sv.e[j] = expf_glibc(sv.val[j] - vmax);
    sv.flag[j] = a.do_topp ? 0 : 1;
    if (a.do_topp) sv.key[j] = ((uint64_t)(~ckey(sv.val[j])) << 32) | (uint64_t)j;
  }
  __syncthreads();
  if (a.do_topp) {
    // top-p (sampling.rs:255-299): rank order = value descending, id ascending
    sort_survivors(sv, n);
    if (t == 0) {
      float S = -0.0f;
      for (uint32_t r = 0; r < n; ++r) S += sv.e[(uint32_t)sv.key[r]];
      float cum = 0.0f;
      uint32_t cut = n;
      for (uint32_t r = 0; r < n; ++r) {
        cum += sv.e[(uint32_t)sv.key[r]] / S;
        if (cum > a.top_p_f) { cut = r + 1; break; }
      }
      if (cut < n && sv.val[(uint32_t)sv.key[cut - 1]] == sv.val[(uint32_t)sv.key[cut]])
        flags |= TC_FLAG_TIE_CUT;
      for (uint32_t r = 0; r < cut; ++r) sv.flag[(uint32_t)sv.key[r]] = 1;
      s_out[1] = flags;
    }
    __syncthreads();
    flags = s_out[1];
  }
  // softmax + multinomial in vocabulary order (sampling.rs:302-328)
  if (t == 0) {
    float S2 = 0.0f;
    for (uint32_t j = 0; j < n; ++j)
      if (sv.flag[j]) S2 += sv.e[j];
    const float u = reinterpret_cast<const float*>(a.uniforms)[row];
    uint32_t tok = 0;
    if (u > 0.0f) {
      float cum = 0.0f;
      for (uint32_t j = 0; j < n; ++j) {
        if (!sv.flag[j]) continue;
        cum += sv.e[j] / S2;
        if (cum >= u) { tok = sv.idx[j]; break; }
      }
    }
    put_result(a, row, tok, TC_OK, flags);
    s_out[2] = __float_as_uint(S2);
    if (a.norm) a.norm[row] = S2;
  }
  if (a.keep_count) {
    __syncthreads();
    const float S2 = __uint_as_float(s_out[2]);
    if (t == 0) {
      uint32_t c = 0;
      for (uint32_t j = 0; j < n; ++j)
        if (sv.flag[j]) {
          if (c < a.cap) {
            a.keep_ids[(size_t)row * a.cap + c] = sv.idx[j];
            a.keep_probs[(size_t)row * a.cap + c] = sv.e[j] / S2;
          }
          ++c;
        }
      a.keep_count[row] = c;
    }
  }
}


TC_DEFINE_LAUNCH(k_qwen)

}  // namespace tc
