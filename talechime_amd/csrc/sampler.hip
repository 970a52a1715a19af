// sampler.hip -- per-step token sampler kernels for gfx950 and the C ABI
// declared in include/talechime_hip.h.
//
// One workgroup samples one row.  The row is streamed from HBM once with
// 16-byte loads and stays in registers (ITEMS consecutive elements per
// thread); the history ids become a bit or byte map in LDS.
//  * Fast paths (indextts and qwen with 1 <= top_k <= 64): a histogram of the
//    per-thread maxima bounds the k-th score, the few candidates above it are
//    staged in LDS, and one wave finishes the row (ranks by counting, the
//    reference's order-dependent sums as wave scans or readlane chains).  The
//    indextts log_softmax denominator is the reference's sequential f32 sum,
//    reproduced exactly (tc_fast.h).
//  * General paths: the top-k threshold is a four-pass radix select over
//    32-bit order keys with LDS histograms; the survivors are compacted into
//    LDS in vocabulary order with a block scan; the order-dependent steps (the
//    reference's sequential f32/f64 sums, cumulative cut-offs and inverse-CDF
//    walks) run over the survivors in exactly the reference's order.
//
// Variants and the reference code each kernel follows (talechime repository):
//   k_qwen      crates/qwen3-tts/src/generation/sampling.rs:169-219, 224-328, 334-395,
//               tts.rs:44-51, synthesis.rs:1228-1279
//   k_indextts  crates/indextts/src/generation.rs:95-194, 280-303, 643-676
//   k_cosy      crates/cosyvoice3/src/llm.rs:517-604
//   k_moss      crates/moss-tts/src/sampling.rs:22-85
//   k_nano      crates/moss-tts/src/nano/sampling.rs:11-75

#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>

#include <mutex>
#include <type_traits>
#include <string>

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
    if (q < NS) F.rkey[c] = key[q];
  }
  lds_wait();
  uint32_t rk[2] = {0u, 0u};
  {
    const uint32_t nr = (n + 3u) & ~3u;
    for (uint32_t j = 0; j < nr; j += 4) {
      const uint64_t k0 = F.rkey[j], k1 = F.rkey[j + 1], k2 = F.rkey[j + 2], k3 = F.rkey[j + 3];
#pragma unroll
      for (int q = 0; q < NS; ++q)
        rk[q] += ((k0 > key[q] ? 1u : 0u) + (k1 > key[q] ? 1u : 0u)) + ((k2 > key[q] ? 1u : 0u) + (k3 > key[q] ? 1u : 0u));
    }
  }
  // top-k (224-249): keep v >= the K-th largest, ties kept
  const uint32_t K = (uint32_t)a.K;
  const uint64_t bk0 = __ballot(has[0] && rk[0] == K - 1u), bk1 = __ballot(has[1] && rk[1] == K - 1u);
  const float kth = bk0 ? rl_f32(v[0], __builtin_ctzll(bk0)) : rl_f32(v[1], __builtin_ctzll(bk1));
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
      for (int q = 0; q < 2; ++q) kp[q] = surv[q] && rk[q] < cut;
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
  SurvLds sv;
  uint32_t hist[256];
  BlockScratch s;
  ScanLds sc;
  SeqLds sq;
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

// General path: any K, non-finite scores, more candidates than the fast path
// stages, the typical warper (TYPICAL: k_idx_typical).  Survivors of the
// top-k cut are staged in LDS (at most kSurvCap).
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
    write_topk(a, row, sv, n);
    finish_row(a, row, 0u, TC_EUNSUPPORTED, row_flags);
    if (t == 0 && a.keep_count) a.keep_count[row] = 0;
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
constexpr int kLargeThreads = 1024;
constexpr int kLargeCand = 2048;
constexpr int kLargeU = 4;  // 16-byte chunks in flight per thread in the streaming passes
constexpr int kLargeR = 3;  // tiles of kLargeU * blockDim chunks kept in registers across the passes
constexpr int kLargePer = kLargeCand / kLargeThreads;  // candidate slots per thread
constexpr int kLargeVocab = 262144;
constexpr int kLargeWords = kLargeVocab / 32;
static_assert(kLargeCand == 2048 && kLargeThreads == 1024, "block_sort2048 sorts 2048 keys over 1024 threads");

struct QLargeLds {
  uint4 ltile[kLargeU * kLargeThreads];  // the row's tile kLargeR (chunk kLargeU * t + u at u * blockDim + t)
  uint32_t bits[kLargeWords];  // history ids and the EOS id
  uint32_t hist[256];
  uint64_t cand[kLargeCand];   // rank order after the sort
  uint64_t candv[kLargeCand];  // vocabulary order
  float stage[kLargeCand];
  uint32_t wtot[2][kMaxWaves];
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
  const uint32_t hb = bits_at_fn(bits, nwords, e0);
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
// The history bitmap (S.bits) must be built when the penalty reads it.
template <typename InT>
__device__ __forceinline__ uint32_t large_candidates(const RowArgs& a, QLargeLds& S, int row, int eos,
                                                     uint32_t* row_flags) {
  constexpr int E = LargeRow<InT>::kEpc;
  const LargeRow<InT> R(a, row);
  const int t = threadIdx.x, V = a.V, nwords = (V + 31) >> 5;
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
    const uint32_t hb = use_bits ? bits_at_fn(S.bits, nwords, c0) : 0u;
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
      if (l == 0) {
        const int w = m ? __builtin_ctzll(m) : 0;
        S.misc[0] = m ? rl_u32(b, w) : 0xffffffffu;
        S.misc[1] = m ? need - rl_u32(before, w) : 0u;
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
  const float u = reinterpret_cast<const float*>(a.uniforms)[row];
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

// indextts with the typical warper (generation.rs:649-651, off by default):
// the general path with idx_typical between the penalty and the temperature.
template <typename InT, int ITEMS>
__global__ void __launch_bounds__(max_threads(ITEMS)) k_idx_typical(RowArgs a) {
  __shared__ IdxGenLds G;
  idx_general<InT, ITEMS, true>(a, G);
}

__global__ void __launch_bounds__(kLargeThreads) k_qwen_large(RowArgs a) {
  __shared__ QLargeLds S;
  const int row = blockIdx.x, t = threadIdx.x, V = a.V;
  const uint16_t* rp = reinterpret_cast<const uint16_t*>(a.logits) + (size_t)row * (size_t)a.ld;
  const int shift = (int)((reinterpret_cast<uintptr_t>(rp) >> 1) & 7u);
  const uint4* base = reinterpret_cast<const uint4*>(rp - shift);
  const int nchunks = (V + shift + 7) >> 3;
  const int eos = (a.eos_id >= 0 && a.eos_id < V) ? a.eos_id : -1;
  // history bitmap
  const int nwords = (V + 31) >> 5;
  for (int w = t; w < nwords; w += blockDim.x) S.bits[w] = 0u;
  if (t < 256) S.hist[t] = 0u;
  __syncthreads();
  if (a.do_pen) {
    uint32_t h0, h1;
    hist_range(a, row, &h0, &h1);
    for (uint32_t k = h0 + (uint32_t)t; k < h1; k += blockDim.x) {
      const uint32_t id = a.hist_ids[k];
      if (id < (uint32_t)V) atomicOr(&S.bits[id >> 5], 1u << (id & 31u));
    }
  }
  __syncthreads();
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
  // only, so every thread runs every body (pass C's holds barriers).
  const int tile = kLargeU * bd;
  uint4 cache[kLargeR][kLargeU];
  auto tiles = [&](bool fill, auto&& body) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < kLargeR; ++i)
      if (i * tile < nchunks) body(cache[i], i * tile);
    int tb = kLargeR * tile;
    uint4 raw[kLargeU], nxt[kLargeU];
    if (tb < nchunks) {
#pragma unroll
      for (int u = 0; u < kLargeU; ++u) raw[u] = fill ? base[min(tb + kLargeU * t + u, nchunks - 1)] : S.ltile[u * bd + t];
#pragma unroll
      for (int u = 0; u < kLargeU; ++u) nxt[u] = base[min(tb + tile + kLargeU * t + u, nchunks - 1)];
      if (fill) {
#pragma unroll
        for (int u = 0; u < kLargeU; ++u) S.ltile[u * bd + t] = raw[u];
      }
      body(raw, tb);
      tb += tile;
#pragma unroll
      for (int u = 0; u < kLargeU; ++u) raw[u] = nxt[u];
    }
    for (; tb < nchunks; tb += tile) {
#pragma unroll
      for (int u = 0; u < kLargeU; ++u) nxt[u] = base[min(tb + tile + kLargeU * t + u, nchunks - 1)];
      body(raw, tb);
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
    tiles(true, [&](const uint4 (&raw)[kLargeU], int tb) __attribute__((always_inline)) {
#pragma unroll
      for (int u = 0; u < kLargeU; ++u) {
        const int q = tb + kLargeU * t + u;
        if (q >= nchunks) break;
        const int c0 = q * 8 - shift;  // in [-7, V)
        const uint32_t hb = bits_at_fn(S.bits, nwords, c0) & 0xffu;
        uint32_t inm = 0xffu;
        if (c0 < 0) inm &= 0xffu << (uint32_t)(-c0);
        if (c0 + 8 > V) inm &= (1u << (uint32_t)(V - c0)) - 1u;
        const uint32_t em = (eos >= c0 && eos < c0 + 8) ? 1u << (uint32_t)(eos - c0) : 0u;
        const uint32_t live = inm & ~hb & ~em;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint32_t w = u4_word(raw[u], j);
          const uint32_t k2 = bkey16x2(w) & half_mask(live, j);
          km2 = __builtin_elementwise_max(km2, __builtin_bit_cast(u16x2, k2));
          bad2 |= nonfinite16x2(w) & half_mask(inm, j);
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
    tiles(false, [&](const uint4 (&raw)[kLargeU], int tb) __attribute__((always_inline)) {
  #pragma unroll
      for (int u = 0; u < kLargeU; ++u) {
        const int q = tb + kLargeU * t + u;
        if (q >= nchunks) break;
        const int c0 = q * 8 - shift;  // in [-7, V)
        const uint32_t hb = bits_at_fn(S.bits, nwords, c0) & 0xffu;
        uint32_t inm = 0xffu;
        if (c0 < 0) inm &= 0xffu << (uint32_t)(-c0);
        if (c0 + 8 > V) inm &= (1u << (uint32_t)(V - c0)) - 1u;
        const uint32_t em = (eos >= c0 && eos < c0 + 8) ? 1u << (uint32_t)(eos - c0) : 0u;
        const uint32_t live = inm & ~hb & ~em;
  #pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint32_t d2 = __builtin_bit_cast(uint32_t, kmax2 - __builtin_bit_cast(u16x2, bkey16x2(u4_word(raw[u], j))));
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
      if (l == 0) S.misc[0] = m ? rl_u32(b, __builtin_ctzll(m)) : 0xffffffffu;
    }
    __syncthreads();
    bK = S.misc[0];
  }
  const uint32_t keyK = kmax - bK;
  const float xK = untkey(keyK << 16 | ((keyK & 0x8000u) ? 0u : 0xffffu));
  const float thr = a.do_temp ? xK * a.tmul + 0.0f : xK;  // its logit (not in the history)
  if (bad || bK == 0xffffffffu || (a.do_pen && a.pen_f < 0.0f) || thr == -__builtin_inff()) {
    n_c = large_candidates<uint16_t>(a, S, row, eos, &row_flags);
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
    tiles(false, [&](const uint4 (&raw)[kLargeU], int tb) __attribute__((always_inline)) {
      uint64_t sel = 0, pens = 0;  // bit 8u + h
  #pragma unroll
      for (int u = 0; u < kLargeU; ++u) {
        const int q = tb + kLargeU * t + u;
        if (q < nchunks) {
          const int c0 = q * 8 - shift;  // in [-7, V)
          const uint32_t hb = bits_at_fn(S.bits, nwords, c0) & 0xffu;
          uint32_t inm = 0xffu;
          if (c0 < 0) inm &= 0xffu << (uint32_t)(-c0);
          if (c0 + 8 > V) inm &= (1u << (uint32_t)(V - c0)) - 1u;
          const uint32_t em = (eos >= c0 && eos < c0 + 8) ? 1u << (uint32_t)(eos - c0) : 0u;
          const uint32_t live = inm & ~hb & ~em, pen = inm & hb & ~em;
          uint32_t ge = 0;  // bit h: key >= keyK (live ids) or keyP (the others)
  #pragma unroll
          for (int j = 0; j < 4; ++j) {
            const uint32_t k2 = bkey16x2(u4_word(raw[u], j));
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
            const uint32_t b = (h & 1) ? (wv & 0xffff0000u) : (wv << 16);
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
  const uint32_t n_c = large_candidates<InT>(a, S, row, eos, &row_flags);
  if (n_c == 0xffffffffu) {  // a +inf logit: the reference's CDF is NaN -> index 0
    finish_row(a, row, 0u, TC_OK, row_flags);
    no_verify(a, row);
    return;
  }
  large_finish(a, S, row, n_c, row_flags);
}

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
  SeqFastLds seq;
  FinLds fin;
  float walk[kWalk];  // the repetition fallback's probabilities around the crossing
};

// random_sample_probs (llm.rs:594-604) from the fast path's registers: pv,
// the exact probabilities of the thread's ITEMS elements from e0 (0 outside
// the row and at the EOS id).  An approximate running sum A (thread, wave and
// block scans) is within E = (V + 64) * 2^-24 * 1.01 * total of the
// reference's sequential one, so the first index with pick < acc lies in
// [first i with A + E > pick, first i with A - E > pick].  The exact
// sequential sum up to the window is SeqSum over the probabilities before it
// (exact terms; elements from the window on count as zeros), and one lane
// walks the window.  Returns the token, or 0xffffffff when the window or the
// list does not fit (then the caller's general walk decides).  Every thread
// of the block calls it.
template <int ITEMS>
__device__ __forceinline__ uint32_t cosy_random_fast(const RowArgs& a, int row, const float (&pv)[ITEMS], int e0,
                                                     CosyFastLds& F) {
  const int t = threadIdx.x, V = a.V, lane = lane_id(), wv = wave_id(), nw = num_waves();
  const float pick = reinterpret_cast<const float*>(a.uniforms)[2 * row + 1];
  float pre[ITEMS];
  float tp = 0.0f;
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) {
    tp += pv[i];
    pre[i] = tp;
  }
  const float tinc = dpp_scan_f32(tp);
  if (lane == kWave - 1) F.wmax[wv] = tinc;
  lds_barrier();
  float woff, wall;
  wave_table_f32(F.wmax, &woff, &wall);
  const float base = woff + (tinc - tp);
  const float E = ((float)V + 64.0f) * 0x1p-24f * 1.01f * wall + 0x1p-60f;
  uint32_t lo = 0xffffffffu, hi = 0xffffffffu;
#pragma unroll
  for (int i = ITEMS - 1; i >= 0; --i) {
    const int e = e0 + i;
    const float A = base + pre[i];
    if (e >= 0 && e < V && A + E > pick) lo = (uint32_t)e;
    if (e >= 0 && e < V && A - E > pick) hi = (uint32_t)e;
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const uint32_t l2 = __shfl_xor(lo, o), h2 = __shfl_xor(hi, o);
    lo = l2 < lo ? l2 : lo;
    hi = h2 < hi ? h2 : hi;
  }
  if (lane == 0) {
    F.wcand[wv] = lo;
    F.bins[wv] = hi;
  }
  lds_barrier();
  for (int w = 0; w < nw; ++w) {
    lo = F.wcand[w] < lo ? F.wcand[w] : lo;
    hi = F.bins[w] < hi ? F.bins[w] : hi;
  }
  if (lo == 0xffffffffu) return (uint32_t)(V - 1);  // no running sum can exceed pick
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
template <int NS>
__device__ __forceinline__ void cosy_fast_finish_t(const RowArgs& a, int row, uint32_t n, float S, CosyFastLds& C) {
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
  // rank = number of candidates with a larger key
  uint32_t rk[2] = {0u, 0u};
  {
    const uint32_t nr = (n + 3u) & ~3u;
    uint32_t a0 = 0, a1 = 0, b0 = 0, b1 = 0;
    for (uint32_t j = 0; j < nr; j += 2) {
      const uint64_t k0 = F.rkey[j], k1 = F.rkey[j + 1];
      a0 += k0 > key[0] ? 1u : 0u;
      a1 += k1 > key[0] ? 1u : 0u;
      if (NS == 2) {
        b0 += k0 > key[1] ? 1u : 0u;
        b1 += k1 > key[1] ? 1u : 0u;
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
  // while cum < top_p and len < top_k: cum += p (the crossing token is kept)
  float cum = 0.0f;
  uint32_t nc = 0;
  const uint32_t kmax = (uint32_t)a.top_k < n ? (uint32_t)a.top_k : n;
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
  uint32_t h0, h1;
  hist_range(a, row, &h0, &h1);
  const uint32_t w0 = (h1 - h0) > (uint32_t)a.ras_win ? h1 - (uint32_t)a.ras_win : h0;
  uint32_t rep = 0;
  for (uint32_t j = w0 + (uint32_t)lane; j < h1; j += (uint32_t)kWave) rep += a.hist_ids[j] == top ? 1u : 0u;
  rep = rl_u32(dpp_scan_u32(rep), kWave - 1);
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
    if (n <= (uint32_t)kWave) cosy_fast_finish_t<1>(a, row, n, S, F);
    else cosy_fast_finish_t<2>(a, row, n, S, F);
  }
  __syncthreads();
  const bool ras = F.out[1] != 0u;  // the nucleus token (F.out[0]) is already written otherwise
  if (ras) {
    // random_sample_probs over every probability: exact terms for all (every
    // lane active: the wave-cooperative expf)
    float pv[ITEMS];
#pragma unroll
    for (int i = 0; i < ITEMS; ++i) {
      const float e = expf_glibc_wave(((vm >> i) & 1u) ? d[i] : 0.0f);
      pv[i] = ((vm >> i) & 1u) ? e / S : 0.0f;
    }
    uint32_t tok = cosy_random_fast<ITEMS>(a, row, pv, e0, F);
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

// ================================================================ moss
template <typename InT, int ITEMS>
__global__ void __launch_bounds__(max_threads(ITEMS)) k_moss(RowArgs a) {
  __shared__ uint8_t s_seen[kMaxVocabReg];
  __shared__ SurvLds sv;
  __shared__ uint32_t s_hist[256];
  __shared__ BlockScratch s;
  __shared__ uint32_t s_out[4];
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
    finish_row(a, row, 0u, TC_EUNSUPPORTED, 0u);
    no_verify(a, row);
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
template <typename InT, int ITEMS>
__global__ void __launch_bounds__(max_threads(ITEMS)) k_nano(RowArgs a) {
  __shared__ uint8_t s_seen[kMaxVocabReg];
  __shared__ SurvLds sv;
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
    finish_row(a, row, 0u, TC_EUNSUPPORTED, 0u);
    no_verify(a, row);
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

// ================================================================ qwen building blocks
__global__ void k_fill_u8(uint8_t* p, size_t n) {
  for (size_t j = blockIdx.x * (size_t)blockDim.x + threadIdx.x; j < n; j += (size_t)gridDim.x * blockDim.x) p[j] = 0;
}

__global__ void k_penalty_ids_mask(const uint32_t* ids, size_t n, uint8_t* mask, int V) {
  for (size_t j = blockIdx.x * (size_t)blockDim.x + threadIdx.x; j < n; j += (size_t)gridDim.x * blockDim.x) {
    uint32_t id = ids[j];
    if (id < (uint32_t)V) mask[id] = 1;
  }
}

__global__ void k_apply_penalty(const float* in, float* out, int rows, int V, long long ld, const uint8_t* bmask,
                                const float* fmask, float pen_f, float inv_pen) {
  const size_t total = (size_t)rows * (size_t)V;
  for (size_t k = blockIdx.x * (size_t)blockDim.x + threadIdx.x; k < total; k += (size_t)gridDim.x * blockDim.x) {
    const size_t r = k / (size_t)V, c = k % (size_t)V;
    const size_t o = r * (size_t)ld + c;
    float v = in[o];
    const bool pen = bmask ? (bmask[c] != 0) : (fmask[c] > 0.0f);
    out[o] = pen ? v * (v > 0.0f ? inv_pen : pen_f) : v;
  }
}

__global__ void k_add_mask(const float* in, float* out, int rows, int V, long long ld, const float* mask) {
  const size_t total = (size_t)rows * (size_t)V;
  for (size_t k = blockIdx.x * (size_t)blockDim.x + threadIdx.x; k < total; k += (size_t)gridDim.x * blockDim.x) {
    const size_t r = k / (size_t)V, c = k % (size_t)V;
    const size_t o = r * (size_t)ld + c;
    out[o] = in[o] + mask[c];
  }
}

__global__ void k_build_suppression(float* mask, int V, uint32_t eos) {
  const int start = V >= 1024 ? V - 1024 : 0;
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < V; i += gridDim.x * blockDim.x)
    mask[i] = (i >= start && (uint32_t)i != eos) ? -__builtin_inff() : 0.0f;
}

__global__ void k_update_penalty_mask(float* mask, int V, const uint32_t* token) {
  if (threadIdx.x == 0 && blockIdx.x == 0) {
    const uint32_t id = *token;
    if (id < (uint32_t)V) mask[id] = 1.0f;
  }
}

template <typename InT, int ITEMS>
__global__ void __launch_bounds__(max_threads(ITEMS)) k_greedy(const InT* logits, long long ld, int V, uint32_t* out) {
  __shared__ uint64_t s_best[kMaxWaves];
  __shared__ uint32_t s_nan0;
  const int row = blockIdx.x, t = threadIdx.x;
  const InT* rp = logits + (size_t)row * (size_t)ld;
  float x[ITEMS];
  int shift;
  load_row<ITEMS>(rp, V, x, &shift);
  const uint32_t vm = valid_mask<ITEMS>(V, shift);
  const int e0 = t * ITEMS - shift;
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
  if (t == 0) s_nan0 = 0u;
  if (lane_id() == 0) s_best[wave_id()] = best;
  __syncthreads();
#pragma unroll
  for (int i = 0; i < ITEMS; ++i)
    if (e0 + i == 0 && __builtin_isnan(x[i])) s_nan0 = 1u;
  __syncthreads();
  if (t == 0) {
    uint64_t b = 0;
    for (int w = 0; w < num_waves(); ++w) b = s_best[w] > b ? s_best[w] : b;
    out[row] = (b == 0 || s_nan0) ? 0u : ~(uint32_t)(b & 0xffffffffu);
  }
}

// ---------------------------------------------------------------- indextts beam-sample step
// generation.rs:640-701 after the processors: per batch element, the kept
// (finite) scores of its num_beams rows joined beam-major (flat index
// beam * V + id) with each row's running beam score added in f64, then
// sample_without_replacement with n_draws draws (280-303) and the candidates
// sorted by score descending, stable (690).  The row pass (k_indextts with
// keep_scores set) leaves each row's kept ids, ascending, and their scores.
constexpr int kBeamCap = 1024;    // kept ids per beam row (the row pass stages at most kSurvCap)
constexpr int kJointCap = 4096;   // kept entries per batch element
constexpr int kBeamMaxDraws = 64;
constexpr int kBeamMaxBeams = 64;

struct BeamArgs {
  int nb, V, n_draws;
  const int32_t* row_status;
  const uint32_t* row_flags;
  const uint32_t* keep_count;
  const uint32_t* keep_ids;   // [rows, kBeamCap]
  const float* keep_scores;   // [rows, kBeamCap]
  const double* beam_scores;  // [rows]
  const double* uniforms;     // [batch, n_draws]
  uint32_t* cand_flat;        // [batch, n_draws]
  double* cand_scores;        // [batch, n_draws]
  int32_t* out_status;        // [batch]
  uint32_t* out_flags;        // [batch]
};

struct BeamLds {
  double s[kJointCap];     // joint scores
  double e[kJointCap];     // exp(s - max), then the normalised weights
  uint32_t flat[kJointCap];
  uint8_t gone[kJointCap];  // drawn already, or not finite
  uint32_t off[kBeamMaxBeams + 1];
  double ps[kBeamMaxDraws];
  uint32_t pf[kBeamMaxDraws];
  double bcast;
  uint32_t flags;
};

__device__ __forceinline__ uint64_t tkey64(double v) {  // f64::total_cmp as an unsigned key
  const uint64_t b = (uint64_t)__double_as_longlong(v);
  return (b >> 63) ? ~b : (b | 0x8000000000000000ull);
}

// The n_draws draws of one element with its L <= 64 * NS joint entries in
// registers (entry k at slot k / 64 of lane k % 64).  A draw compares the
// prefix scan of e = exp(s - max) (tree order) against u * (its total): in
// exact arithmetic the reference's acc > u * total over w = e / sum.
// order_margin bounds what separates the two (the sequential sums, the
// divisions, exp's difference from libm); a draw whose decision falls inside
// it runs the reference's sequential loops.  e is recomputed only when the
// maximum changes: exp(s - max) of an unchanged maximum is the same value.
// Call with every lane active.
template <int NS>
__device__ __forceinline__ bool beam_draws_reg(const BeamArgs& b, BeamLds& B, uint32_t L, int bi, uint32_t off,
                                               double bonus, double ud, uint32_t* flags_io) {
  const int lane = lane_id(), nd = b.n_draws, nb = b.nb;
  double s[NS], e[NS];
  uint32_t f[NS];
  bool live[NS];
  uint32_t nlive = 0;
#pragma unroll
  for (int q = 0; q < NS; ++q) {
    // entry k belongs to the last beam whose offset is <= k (beams without
    // kept ids share their offset with the next one)
    const uint32_t k = (uint32_t)(q * kWave + lane);
    uint32_t jj = 0, oj = 0;
    double bj = 0.0;
    for (int j = 0; j < nb; ++j) {
      const uint32_t o = rl_u32(off, j);
      const double bo = rl_f64(bonus, j);
      if (k >= o) {
        jj = (uint32_t)j;
        oj = o;
        bj = bo;
      }
    }
    s[q] = 0.0;
    f[q] = 0u;
    if (k < L) {
      const size_t at = (size_t)(bi * nb + (int)jj) * kBeamCap + (k - oj);
      s[q] = (double)b.keep_scores[at] + bj;
      f[q] = jj * (uint32_t)b.V + b.keep_ids[at];
    }
    live[q] = k < L && __builtin_isfinite(s[q]);
    e[q] = 0.0;
    nlive += (uint32_t)__popcll(__ballot(live[q]));
  }
  if (nlive < (uint32_t)nd) return false;
  const double mg_rel = order_margin(L);
  double m_prev = __builtin_nan("");
  uint32_t flags = 0;
  for (int d = 0; d < nd; ++d) {
    double m = -__builtin_inf();
#pragma unroll
    for (int q = 0; q < NS; ++q) m = live[q] ? rmaxd(m, s[q]) : m;
    m = dpp_wave_max_d(m);
    if (!(m == m_prev)) {
#pragma unroll
      for (int q = 0; q < NS; ++q) e[q] = live[q] ? tc_exp_d(s[q] - m) : 0.0;
      m_prev = m;
    }
    bool tiny = false;
#pragma unroll
    for (int q = 0; q < NS; ++q) tiny = tiny || (e[q] > 0.0 && e[q] < 0x1p-1000);  // e / sum may round to 0
    double carry = 0.0, c[NS];
    uint64_t pos[NS], hit[NS];
#pragma unroll
    for (int q = 0; q < NS; ++q) {
      c[q] = dpp_scan_f64(e[q]) + carry;
      carry = rl_f64(c[q], kWave - 1);
    }
    const double u = rl_f64(ud, d);
    const double total = carry, target = u * total;
    uint32_t pick = 0xffffffffu, lastp = 0xffffffffu;
#pragma unroll
    for (int q = 0; q < NS; ++q) {
      pos[q] = __ballot(e[q] > 0.0);  // removed entries hold e = 0
      hit[q] = __ballot(e[q] > 0.0 && c[q] > target);
      if (pick == 0xffffffffu && hit[q]) pick = (uint32_t)(q * kWave + __builtin_ctzll(hit[q]));
      if (pos[q]) lastp = (uint32_t)(q * kWave + 63 - __builtin_clzll(pos[q]));
    }
    const bool found = pick != 0xffffffffu;
    if (!found) pick = lastp;
    // the running sums at the pick and at the positive entry before it
    uint32_t prev = 0xffffffffu;
#pragma unroll
    for (int q = 0; q < NS; ++q) {
      const int qp = (int)(pick >> 6);
      uint64_t below = 0ull;
      if (q < qp) below = pos[q];
      else if (q == qp) below = pos[q] & ((1ull << (pick & 63u)) - 1ull);
      if (below) prev = (uint32_t)(q * kWave + 63 - __builtin_clzll(below));
    }
    double a_pick = 0.0, a_prev = 0.0;
#pragma unroll
    for (int q = 0; q < NS; ++q) {
      if (pick != 0xffffffffu && (int)(pick >> 6) == q) a_pick = rl_f64(c[q], (int)(pick & 63u));
      if (prev != 0xffffffffu && (int)(prev >> 6) == q) a_prev = rl_f64(c[q], (int)(prev & 63u));
    }
    const double mg = mg_rel * total;
    bool close = __ballot(tiny) != 0ull || lastp == 0xffffffffu || __builtin_fabs(a_pick - target) <= mg;
    if (found && prev != 0xffffffffu) close = close || __builtin_fabs(a_prev - target) <= mg;
    if (close) {
      // the reference's order: sequential sums over live entries in flat order
      uint64_t lm[NS];
#pragma unroll
      for (int q = 0; q < NS; ++q) lm[q] = __ballot(live[q]);
      double S = -0.0;
#pragma unroll
      for (int q = 0; q < NS; ++q)
        for (uint64_t mm = lm[q]; mm; mm &= mm - 1) S += rl_f64(e[q], __builtin_ctzll(mm));
      double wv[NS];
#pragma unroll
      for (int q = 0; q < NS; ++q) wv[q] = live[q] ? e[q] / S : 0.0;
      double tot = -0.0;
#pragma unroll
      for (int q = 0; q < NS; ++q)
        for (uint64_t mm = lm[q]; mm; mm &= mm - 1) tot += rl_f64(wv[q], __builtin_ctzll(mm));
      const double ue = u * tot;
      double acc = 0.0;
      uint32_t last = 0xffffffffu, pk = 0xffffffffu;
      bool near = false;
#pragma unroll
      for (int q = 0; q < NS; ++q) {
        for (uint64_t mm = lm[q]; mm && pk == 0xffffffffu; mm &= mm - 1) {
          const uint32_t k = (uint32_t)(q * kWave + __builtin_ctzll(mm));
          if (last == 0xffffffffu) last = k;  // last_positive starts at live[0]
          const double wc = rl_f64(wv[q], __builtin_ctzll(mm));
          if (wc <= 0.0) continue;
          last = k;
          acc += wc;
          near = near || __builtin_fabs(acc - ue) <= exp_margin() * tot;
          if (acc > ue) pk = k;
        }
      }
      pick = pk != 0xffffffffu ? pk : last;
      if (near) flags |= TC_FLAG_NEAR_TIE;
    }
    double ps = 0.0;
    uint32_t pf = 0u;
#pragma unroll
    for (int q = 0; q < NS; ++q) {
      if ((int)(pick >> 6) == q) {
        ps = rl_f64(s[q], (int)(pick & 63u));
        pf = rl_u32(f[q], (int)(pick & 63u));
        if (lane == (int)(pick & 63u)) {
          live[q] = false;
          e[q] = 0.0;
        }
      }
    }
    if (lane == 0) {
      B.ps[d] = ps;
      B.pf[d] = pf;
    }
  }
  *flags_io |= flags;
  return true;
}

__global__ void __launch_bounds__(64) k_beam_joint(BeamArgs b) {
  __shared__ BeamLds B;
  const int bi = blockIdx.x, lane = threadIdx.x, nb = b.nb, nd = b.n_draws;
  // one round of loads: the beam rows (lane j) and the element's uniforms (lane d)
  int32_t rs = TC_OK;
  uint32_t rf = 0u, cnt = 0u;
  double bonus = 0.0, ud = 0.0;
  if (lane < nb) {
    const int r = bi * nb + lane;
    rs = b.row_status[r];
    rf = b.row_flags[r] & TC_FLAG_NEAR_TIE;
    cnt = b.keep_count[r];
    bonus = b.beam_scores[r];
  }
  if (lane < nd) ud = b.uniforms[(size_t)bi * nd + lane];
  // a row without a finite score (TC_ETOOFEW) adds nothing to the joint row;
  // the first other failing row gives the element its status
  const uint64_t fm = __ballot(lane < nb && rs != TC_OK && rs != TC_ETOOFEW);
  int32_t st = fm ? (int32_t)rl_u32((uint32_t)rs, __builtin_ctzll(fm)) : TC_OK;
  uint32_t c = (lane < nb && rs == TC_OK) ? cnt : 0u;
  if (__ballot(c > (uint32_t)kBeamCap) && st == TC_OK) st = TC_EUNSUPPORTED;
  c = c > (uint32_t)kBeamCap ? 0u : c;
  const uint32_t incl = dpp_scan_u32(c);
  const uint32_t off = incl - c;
  const uint32_t Lall = rl_u32(incl, kWave - 1);
  if (Lall > (uint32_t)kJointCap && st == TC_OK) st = TC_EUNSUPPORTED;
  uint32_t flags = dpp_wave_or(rf);
  // every loop below stays inside the element's entries (L <= kJointCap when OK)
  const uint32_t L = st == TC_OK ? Lall : 0u;
  bool run = false;
  if (st == TC_OK && L <= 64u) {
    run = beam_draws_reg<1>(b, B, L, bi, off, bonus, ud, &flags);
  } else if (st == TC_OK && L <= 128u) {
    run = beam_draws_reg<2>(b, B, L, bi, off, bonus, ud, &flags);
  } else if (st == TC_OK && L <= 256u) {
    run = beam_draws_reg<4>(b, B, L, bi, off, bonus, ud, &flags);
  } else if (st == TC_OK) {
    // more entries than registers hold: staged in LDS, the reference's loops on one lane
    if (lane < nb) B.off[lane] = off;
    if (lane == 0) {
      B.off[nb] = L;
      B.flags = flags;
    }
    __syncthreads();
    for (int j = 0; j < nb; ++j) {
      const int r = bi * nb + j;
      const uint32_t o = B.off[j], cj = B.off[j + 1] - o;
      const double bo = rl_f64(bonus, j);
      for (uint32_t k = (uint32_t)lane; k < cj; k += 64u) {
        const double js = (double)b.keep_scores[(size_t)r * kBeamCap + k] + bo;
        B.s[o + k] = js;
        B.flat[o + k] = (uint32_t)j * (uint32_t)b.V + b.keep_ids[(size_t)r * kBeamCap + k];
        B.gone[o + k] = __builtin_isfinite(js) ? 0 : 1;
      }
    }
    __syncthreads();
    uint32_t nlive = 0;
    for (uint32_t k = (uint32_t)lane; k < L; k += 64u) nlive += B.gone[k] ? 0u : 1u;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) nlive += __shfl_xor(nlive, o);
    run = nlive >= (uint32_t)nd;
  }
  if (run && L > 256u) {
    // more entries than registers hold: the reference's loops on one lane
    for (int d = 0; d < nd; ++d) {
      double m = -__builtin_inf();
      for (uint32_t k = (uint32_t)lane; k < L; k += 64u)
        if (!B.gone[k]) m = rmaxd(m, B.s[k]);
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) m = rmaxd(m, __shfl_xor(m, o));
      for (uint32_t k = (uint32_t)lane; k < L; k += 64u)
        if (!B.gone[k]) B.e[k] = tc_exp_d(B.s[k] - m);
      __syncthreads();
      if (lane == 0) {
        double sum = -0.0;
        for (uint32_t k = 0; k < L; ++k)
          if (!B.gone[k]) sum += B.e[k];
        B.bcast = sum;
      }
      __syncthreads();
      const double sum = B.bcast;
      for (uint32_t k = (uint32_t)lane; k < L; k += 64u)
        if (!B.gone[k]) B.e[k] = B.e[k] / sum;
      __syncthreads();
      if (lane == 0) {
        double total = -0.0;
        for (uint32_t k = 0; k < L; ++k)
          if (!B.gone[k]) total += B.e[k];
        const double u = b.uniforms[(size_t)bi * nd + d] * total;
        // inverse_cdf (251-265): the first positive weight whose running sum
        // exceeds u, else the last positive one (index 0 of live when none is)
        double acc = 0.0;
        uint32_t last = 0xffffffffu, pick = 0xffffffffu;
        bool near = false;
        for (uint32_t k = 0; k < L; ++k) {
          if (B.gone[k]) continue;
          if (last == 0xffffffffu) last = k;
          const double w = B.e[k];
          if (w <= 0.0) continue;
          last = k;
          acc += w;
          near = near || __builtin_fabs(acc - u) <= exp_margin() * total;
          if (acc > u) {
            pick = k;
            break;
          }
        }
        if (pick == 0xffffffffu) pick = last;
        if (near) B.flags |= TC_FLAG_NEAR_TIE;
        B.gone[pick] = 1;
        B.ps[d] = B.s[pick];
        B.pf[d] = B.flat[pick];
      }
      __syncthreads();
    }
    flags = B.flags;
  }
  if (lane == 0) {
    double* cs = b.cand_scores + (size_t)bi * nd;
    uint32_t* cf = b.cand_flat + (size_t)bi * nd;
    if (run) {
      // candidates.sort_by(|a, x| x.0.total_cmp(&a.0)): stable, descending
      for (int d = 1; d < nd; ++d) {
        const double v = B.ps[d];
        const uint32_t f = B.pf[d];
        int k = d;
        while (k > 0 && tkey64(B.ps[k - 1]) < tkey64(v)) {
          B.ps[k] = B.ps[k - 1];
          B.pf[k] = B.pf[k - 1];
          --k;
        }
        B.ps[k] = v;
        B.pf[k] = f;
      }
      for (int d = 0; d < nd; ++d) {
        cs[d] = B.ps[d];
        cf[d] = B.pf[d];
      }
    } else {
      for (int d = 0; d < nd; ++d) {
        cs[d] = 0.0;
        cf[d] = 0u;
      }
    }
    b.out_status[bi] = st != TC_OK ? st : (run ? TC_OK : TC_ETOOFEW);
    if (b.out_flags) b.out_flags[bi] = flags;
  }
}

// The beam-search branch (do_sample = false, generation.rs:671-679): the
// n_keep best joint scores of each element over its beams' kept lists (the
// row pass keeps every id at or above its row's n_keep-th score, ties
// included, so they hold the element's best n_keep), descending, equal
// scores in ascending flat order (the reference's stable sort of the flat
// indices).  One wave per element, n_keep rounds of a wave arg-max.
__global__ void __launch_bounds__(64) k_beam_topn(BeamArgs b) {
  __shared__ BeamLds B;
  const int bi = blockIdx.x, lane = threadIdx.x, nb = b.nb, nk = b.n_draws;
  int32_t rs = TC_OK;
  uint32_t cnt = 0u;
  double bonus = 0.0;
  if (lane < nb) {
    const int r = bi * nb + lane;
    rs = b.row_status[r];
    cnt = b.keep_count[r];
    bonus = b.beam_scores[r];
  }
  // a row without a finite score (TC_ETOOFEW) adds nothing; the first other
  // failing row gives the element its status
  const uint64_t fm = __ballot(lane < nb && rs != TC_OK && rs != TC_ETOOFEW);
  int32_t st = fm ? (int32_t)rl_u32((uint32_t)rs, __builtin_ctzll(fm)) : TC_OK;
  uint32_t c = (lane < nb && rs == TC_OK) ? cnt : 0u;
  if (__ballot(c > (uint32_t)kBeamCap) && st == TC_OK) st = TC_EUNSUPPORTED;
  c = c > (uint32_t)kBeamCap ? 0u : c;
  const uint32_t incl = dpp_scan_u32(c);
  const uint32_t Lall = rl_u32(incl, kWave - 1);
  if (Lall > (uint32_t)kJointCap && st == TC_OK) st = TC_EUNSUPPORTED;
  const uint32_t L = st == TC_OK ? Lall : 0u;
  if (lane < nb) B.off[lane] = incl - c;
  __syncthreads();
  for (int j = 0; j < nb && L; ++j) {
    const int r = bi * nb + j;
    const uint32_t o = B.off[j], cj = (j + 1 < nb ? B.off[j + 1] : L) - o;
    const double bo = rl_f64(bonus, j);
    for (uint32_t k = (uint32_t)lane; k < cj; k += 64u) {
      B.s[o + k] = (double)b.keep_scores[(size_t)r * kBeamCap + k] + bo;
      B.flat[o + k] = (uint32_t)j * (uint32_t)b.V + b.keep_ids[(size_t)r * kBeamCap + k];
      B.gone[o + k] = 0;
    }
  }
  __syncthreads();
  const bool enough = L >= (uint32_t)nk;
  for (int d = 0; d < nk && enough; ++d) {
    // the best remaining entry: total order descending, then flat ascending
    uint64_t bk = 0;
    uint32_t bf = 0xffffffffu, bidx = 0xffffffffu;
    for (uint32_t k = (uint32_t)lane; k < L; k += 64u) {
      if (B.gone[k]) continue;
      const uint64_t kk = tkey64(B.s[k]);
      if (bidx == 0xffffffffu || kk > bk || (kk == bk && B.flat[k] < bf)) {
        bk = kk;
        bf = B.flat[k];
        bidx = k;
      }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      const uint64_t ok = __shfl_xor(bk, o);
      const uint32_t of = __shfl_xor(bf, o), oi = __shfl_xor(bidx, o);
      if (oi != 0xffffffffu && (bidx == 0xffffffffu || ok > bk || (ok == bk && of < bf))) {
        bk = ok;
        bf = of;
        bidx = oi;
      }
    }
    if (lane == 0) {
      B.gone[bidx] = 1;
      B.ps[d] = B.s[bidx];
      B.pf[d] = bf;
    }
    __syncthreads();
  }
  if (lane == 0) {
    double* cs = b.cand_scores + (size_t)bi * nk;
    uint32_t* cf = b.cand_flat + (size_t)bi * nk;
    for (int d = 0; d < nk; ++d) {
      cs[d] = (st == TC_OK && enough) ? B.ps[d] : 0.0;
      cf[d] = (st == TC_OK && enough) ? B.pf[d] : 0u;
    }
    b.out_status[bi] = st != TC_OK ? st : (enough ? TC_OK : TC_ETOOFEW);
    if (b.out_flags) b.out_flags[bi] = 0u;
  }
}

}  // namespace tc

// ====================================================================== C ABI
struct tc_ctx {
  int device;
  size_t max_rows;
  size_t max_vocab;
  uint8_t* d_mask;  // [max_vocab] byte mask for tc_apply_repetition_penalty
  void* d_beam;     // the beam step's row-pass workspace (first beam step), or NULL
};

namespace {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

int hip_fail(hipError_t e, const char* what) {
  return fail(TC_EHIP, "%s: %s", what, hipGetErrorString(e));
}
}  // namespace

namespace tc {
// The error slot of tc_last_error, for the library's other source files.
int set_error(int code, const char* msg) { return fail(code, "%s", msg); }
}  // namespace tc

namespace {

struct DeviceGuard {
  int prev = -1;
  bool changed = false;
  explicit DeviceGuard(int dev) {
    if (hipGetDevice(&prev) == hipSuccess && prev != dev && hipSetDevice(dev) == hipSuccess) changed = true;
  }
  ~DeviceGuard() {
    if (changed) (void)hipSetDevice(prev);
  }
};

// Block shape for a register-resident row: ITEMS consecutive elements per
// thread (a multiple of the 16-byte load width), threads a multiple of 64 in
// [256, 1024]; rounded up to a multiple of 256 (four waves, one per SIMD) when
// that still fits, so the SIMDs share the row evenly.
bool pick_shape(int V, int dtype, int* items, int* threads) {
  const int pad = dtype == TC_BF16 ? 7 : 3;
  static const int f32_items[] = {8, 12, 16, 24}, bf16_items[] = {8, 16, 24};
  const int* its = dtype == TC_BF16 ? bf16_items : f32_items;
  const int n_its = dtype == TC_BF16 ? 3 : 4;
  for (int k = 0; k < n_its; ++k) {
    const int it = its[k];
    int nt = (V + pad + it - 1) / it;
    nt = (nt + 63) / 64 * 64;
    if (nt < 256) nt = 256;
    if (nt > tc::max_threads(it)) continue;
    const int bal = (nt + 255) / 256 * 256;
    *items = it;
    *threads = bal <= tc::max_threads(it) ? bal : nt;
    return true;
  }
  return false;
}

#define TC_DEFINE_LAUNCH(NAME)                                                                   \
  hipError_t launch_##NAME(int dtype, int items, int threads, int rows, hipStream_t st,          \
                           const tc::RowArgs& a) {                                               \
    dim3 g(rows), b(threads);                                                                    \
    if (dtype == TC_F32) {                                                                       \
      if (items == 8) hipLaunchKernelGGL((tc::NAME<float, 8>), g, b, 0, st, a);                  \
      else if (items == 12) hipLaunchKernelGGL((tc::NAME<float, 12>), g, b, 0, st, a);           \
      else if (items == 16) hipLaunchKernelGGL((tc::NAME<float, 16>), g, b, 0, st, a);           \
      else hipLaunchKernelGGL((tc::NAME<float, 24>), g, b, 0, st, a);                            \
    } else {                                                                                     \
      if (items == 8) hipLaunchKernelGGL((tc::NAME<uint16_t, 8>), g, b, 0, st, a);               \
      else if (items == 16) hipLaunchKernelGGL((tc::NAME<uint16_t, 16>), g, b, 0, st, a);        \
      else hipLaunchKernelGGL((tc::NAME<uint16_t, 24>), g, b, 0, st, a);                         \
    }                                                                                            \
    return hipGetLastError();                                                                    \
  }

TC_DEFINE_LAUNCH(k_qwen)
TC_DEFINE_LAUNCH(k_indextts)
TC_DEFINE_LAUNCH(k_idx_typical)
TC_DEFINE_LAUNCH(k_cosy)
TC_DEFINE_LAUNCH(k_moss)
TC_DEFINE_LAUNCH(k_nano)

}  // namespace

// The beam step's row-pass workspace: per row kBeamCap kept ids, scores,
// probabilities and top-k ids, then the counts, statuses and flags.  The
// context's copy is allocated on its first beam step, behind R zero uniforms
// (the row pass's own draw is not used); the allocation-free entry point keeps
// it in the file-scope `scratch` array below.
struct BeamWs {
  uint32_t* keep_ids;
  float* keep_scores;
  float* keep_probs;
  uint32_t* topk_ids;
  uint32_t* topk_count;
  uint32_t* keep_count;
  uint32_t* ids;
  int32_t* status;
  uint32_t* flags;
};

static constexpr size_t beam_ws_bytes(size_t R) { return R * (size_t)tc::kBeamCap * 16 + R * 20; }

static BeamWs beam_ws(void* base, size_t R) {
  const size_t C = (size_t)tc::kBeamCap;
  char* p = static_cast<char*>(base);
  BeamWs w;
  w.keep_ids = reinterpret_cast<uint32_t*>(p);
  p += R * C * 4;
  w.keep_scores = reinterpret_cast<float*>(p);
  p += R * C * 4;
  w.keep_probs = reinterpret_cast<float*>(p);
  p += R * C * 4;
  w.topk_ids = reinterpret_cast<uint32_t*>(p);
  p += R * C * 4;
  w.topk_count = reinterpret_cast<uint32_t*>(p);
  p += R * 4;
  w.keep_count = reinterpret_cast<uint32_t*>(p);
  p += R * 4;
  w.ids = reinterpret_cast<uint32_t*>(p);
  p += R * 4;
  w.status = reinterpret_cast<int32_t*>(p);
  p += R * 4;
  w.flags = reinterpret_cast<uint32_t*>(p);
  return w;
}

// Allocation-free beam step: its row-pass workspace for up to kStaticBeamRows
// beam rows (4.2 MB) in a file-scope device array, and the zero uniforms in a
// second one that nothing ever writes.  Each GPU holds its own copy of both
// for the life of the process; host code reaches them only through the
// addresses hipGetSymbolAddress returns for the current device.
namespace tc {
constexpr int kStaticBeamRows = 256;
constexpr int kMaxDevices = 64;
}  // namespace tc
static_assert(tc::kStaticBeamRows == TC_NOALLOC_BEAM_ROWS, "header and library agree on the static workspace");
static __device__ __align__(256) unsigned char scratch[beam_ws_bytes(tc::kStaticBeamRows)];
static __device__ __align__(256) double static_zero_uniforms[tc::kStaticBeamRows];

namespace {
struct StaticWs {
  bool ready = false;
  void* scratch = nullptr;
  const double* zeros = nullptr;
};
StaticWs g_static[tc::kMaxDevices];
std::mutex g_static_mu;

// Resolves the two arrays' addresses on `device` (made current by the
// caller), once per device.
int static_ws_setup(int device, StaticWs* out) {
  if (device < 0 || device >= tc::kMaxDevices) return fail(TC_EINVAL, "device %d out of range", device);
  std::lock_guard<std::mutex> lk(g_static_mu);
  StaticWs& w = g_static[device];
  if (!w.ready) {
    void* sp = nullptr;
    void* zp = nullptr;
    hipError_t e = hipGetSymbolAddress(&sp, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)");
    e = hipGetSymbolAddress(&zp, HIP_SYMBOL(static_zero_uniforms));
    if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(static_zero_uniforms)");
    w.scratch = sp;
    w.zeros = static_cast<const double*>(zp);
    w.ready = true;
  }
  *out = w;
  return TC_OK;
}
}  // namespace

extern "C" {

const char* tc_last_error(void) { return g_err.c_str(); }

int tc_abi_version(void) { return TC_ABI_VERSION; }

int tc_create(int device, size_t max_rows, size_t max_vocab, tc_ctx** out) {
  if (!out) return fail(TC_EINVAL, "tc_create: out is NULL");
  *out = nullptr;
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess) return hip_fail(e, "hipGetDeviceCount");
  if (device < 0 || device >= n) return fail(TC_EINVAL, "tc_create: device %d of %d", device, n);
  if (max_vocab == 0 || max_vocab > (size_t)INT32_MAX) return fail(TC_EINVAL, "tc_create: bad max_vocab");
  DeviceGuard g(device);
  StaticWs sw;  // the allocation-free beam step's arrays on this device
  int rc = static_ws_setup(device, &sw);
  if (rc != TC_OK) return rc;
  tc_ctx* c = new tc_ctx{device, max_rows, max_vocab, nullptr, nullptr};
  e = hipMalloc(&c->d_mask, max_vocab);
  if (e != hipSuccess) {
    delete c;
    return fail(TC_ENOMEM, "hipMalloc(%zu): %s", max_vocab, hipGetErrorString(e));
  }
  *out = c;
  return TC_OK;
}

void tc_destroy(tc_ctx* ctx) {
  if (!ctx) return;
  DeviceGuard g(ctx->device);
  if (ctx->d_mask) (void)hipFree(ctx->d_mask);
  if (ctx->d_beam) (void)hipFree(ctx->d_beam);
  delete ctx;
}

// tc_sample; keep_scores (indextts only, with verify outputs) also receives
// the final score of each kept id.
static int sample_impl(int device, size_t max_vocab, const tc_sample_params* p, const void* d_logits, int dtype,
                       size_t rows, size_t vocab, size_t ld, const uint32_t* d_hist_off, const uint32_t* d_hist_ids,
                       const void* d_uniforms, uint32_t* d_out_ids, int32_t* d_out_status, uint32_t* d_out_flags,
                       const tc_verify_out* verify, float* keep_scores, tc_stream stream) {
  if (!p) return fail(TC_EINVAL, "tc_sample: params is NULL");
  if (rows == 0) return TC_OK;
  if (!d_logits || !d_out_ids || !d_uniforms) return fail(TC_EINVAL, "tc_sample: NULL device pointer");
  if (dtype != TC_F32 && dtype != TC_BF16) return fail(TC_EINVAL, "tc_sample: dtype %d", dtype);
  if (vocab == 0) return fail(TC_EINVAL, "tc_sample: vocab is 0");
  if (ld < vocab) return fail(TC_EINVAL, "tc_sample: ld %zu < vocab %zu", ld, vocab);
  if (rows > (size_t)INT32_MAX || vocab > (size_t)INT32_MAX) return fail(TC_EINVAL, "tc_sample: shape too large");
  const int V = (int)vocab;
  tc::RowArgs a{};
  a.logits = d_logits;
  a.ld = (long long)ld;
  a.V = V;
  a.rows = (int)rows;
  a.hist_off = d_hist_off;
  a.hist_ids = d_hist_ids;
  a.hist_mode = p->hist_mode;
  a.pen_mask = p->d_pen_mask;
  a.add_mask = p->d_add_mask;
  a.mark = p->d_mark_mask;
  if (a.mark && rows > 1 && a.mark == p->d_pen_mask)
    return fail(TC_EINVAL, "tc_sample: d_mark_mask equals d_pen_mask with %zu rows (the rows would race)", rows);
  a.uniforms = d_uniforms;
  a.out_ids = d_out_ids;
  a.out_status = d_out_status;
  a.out_flags = d_out_flags;
  if (verify && verify->cap) {
    if (!verify->d_topk_count || !verify->d_topk_ids || !verify->d_keep_count || !verify->d_keep_ids ||
        !verify->d_keep_probs)
      return fail(TC_EINVAL, "tc_sample: incomplete verify outputs");
    a.cap = verify->cap;
    a.topk_count = verify->d_topk_count;
    a.topk_ids = verify->d_topk_ids;
    a.keep_count = verify->d_keep_count;
    a.keep_ids = verify->d_keep_ids;
    a.keep_probs = verify->d_keep_probs;
    a.norm = verify->d_norm;
    a.keep_scores = keep_scores;
  }
  a.eos_id = p->eos_id;
  a.exclude_id = p->exclude_id;
  a.min_keep = (int)p->min_keep;
  const bool need_hist = p->hist_mode != TC_HIST_MASK;
  if (p->hist_mode < 0 || p->hist_mode > TC_HIST_MASK) return fail(TC_EINVAL, "tc_sample: hist_mode");
  switch (p->variant) {
    case TC_QWEN: {
      a.do_pen = fabs(p->repetition_penalty - 1.0) >= 1e-9;
      if (a.do_pen && need_hist && (!d_hist_off || !d_hist_ids))
        return fail(TC_EINVAL, "tc_sample: penalty needs a history");
      if (a.do_pen && !need_hist && !p->d_pen_mask) return fail(TC_EINVAL, "tc_sample: penalty mask is NULL");
      a.pen_f = (float)p->repetition_penalty;
      a.inv_pen = 1.0f / a.pen_f;
      a.do_temp = (p->temperature != 1.0 && p->temperature > 0.0);
      a.tmul = (float)(1.0 / p->temperature);
      a.greedy = p->temperature < 0.01;
      a.K = p->top_k > 0 ? (int)(p->top_k < vocab ? p->top_k : vocab) : 0;
      a.do_topp = p->top_p < 1.0 && p->top_p > 0.0;
      a.top_p_f = (float)p->top_p;
      a.fast = !a.greedy && a.K >= 1 && a.K <= 64 && a.K < V;
      break;
    }
    case TC_COSY_RAS: {  // llm.rs:436-445
      const float tp = (float)p->top_p, tau = p->ras_tau;
      if (!isfinite(tp) || tp <= 0.0f || tp > 1.0f || p->top_k == 0 || p->ras_win == 0 || !isfinite(tau) ||
          !(tau >= 0.0f && tau <= 1.0f))
        return fail(TC_EINVAL, "invalid RAS sampling parameters");
      if (!d_hist_off || !d_hist_ids) return fail(TC_EINVAL, "tc_sample: cosyvoice3 needs the decoded history");
      a.top_k = (int)(p->top_k < (uint32_t)INT32_MAX ? p->top_k : (uint32_t)INT32_MAX);
      a.top_p_f = tp;
      a.ras_win = (int)p->ras_win;
      a.ras_thresh = (float)p->ras_win * tau;
      a.fast = a.top_k >= 1 && a.top_k <= 64 && a.top_k < V;
      break;
    }
    case TC_INDEXTTS: {  // generation.rs:559-571
      if (p->repetition_penalty <= 0.0) return fail(TC_EINVAL, "repetition_penalty must be > 0");
      if (p->temperature <= 0.0) return fail(TC_EINVAL, "temperature must be > 0 when sampling");
      a.do_pen = p->repetition_penalty != 1.0;
      if (a.do_pen && (!d_hist_off || !d_hist_ids)) return fail(TC_EINVAL, "tc_sample: penalty needs a history");
      a.pen_f = (float)p->repetition_penalty;
      a.do_temp = p->temperature != 1.0;
      a.t_f = (float)p->temperature;
      if (p->top_k != 0) {
        size_t k = p->top_k > p->min_keep ? p->top_k : p->min_keep;
        if (k > vocab) k = vocab;
        a.K = (int)k;
      }
      a.do_topp = p->top_p < 1.0;
      a.top_p_d = p->top_p;
      if (p->typical) {  // GenerateConfig.typical_mass, checked as typical_sampling's mass
        if (!(p->typical_mass > 0.0 && p->typical_mass < 1.0)) return fail(TC_EINVAL, "typical_mass must be in (0, 1)");
        a.typical_mass = p->typical_mass;
      }
      a.fast = a.K >= 1 && a.K <= 64 && a.K < V && a.min_keep <= a.K && !p->typical;
      break;
    }
    case TC_MOSS: {
      if (p->top_k == 0 && (float)p->temperature != 0.0f) return fail(TC_EINVAL, "moss: top_k must be >= 1");
      if (p->exclude_id >= 0 && (size_t)p->exclude_id >= vocab) return fail(TC_EINVAL, "moss: exclude id out of range");
      a.do_pen = d_hist_off && d_hist_ids;
      a.pen_f = (float)p->repetition_penalty;
      a.t_f = (float)p->temperature;
      a.greedy = a.t_f == 0.0f;
      a.top_k = (int)(p->top_k < vocab ? p->top_k : vocab);
      a.top_p_d = p->top_p;
      break;
    }
    case TC_MOSS_NANO: {
      if (p->top_k == 0) return fail(TC_EINVAL, "nano: top_k must be >= 1");
      a.pen_f = (float)p->repetition_penalty;
      a.t_f = (float)p->temperature;
      a.top_k = (int)(p->top_k < vocab ? p->top_k : vocab);
      a.do_topp = p->top_p < 1.0;
      a.top_p_d = p->top_p;
      break;
    }
    default:
      return fail(TC_EINVAL, "tc_sample: variant %d", p->variant);
  }
  if ((size_t)V > max_vocab) return fail(TC_EINVAL, "tc_sample: vocab %d > context max %zu", V, max_vocab);
  int items = 0, threads = 0;
  if (!pick_shape(V, dtype, &items, &threads) || V > tc::kMaxVocabReg) {
    // qwen over bf16 rows up to kLargeVocab: the large-vocabulary kernel
    if (p->variant == TC_QWEN && a.do_pen && (a.pen_f == 0.0f || !isfinite(a.pen_f)))
      return fail(TC_EUNSUPPORTED, "tc_sample: repetition penalty %g above %d logits", p->repetition_penalty,
                  tc::kMaxVocabReg);
    if (p->variant == TC_QWEN && V <= tc::kLargeVocab && (a.K >= 1 || a.greedy) && a.K <= tc::kLargeCand) {
      // bf16 rows without masks: the packed passes; f32 rows and the masks:
      // candidates selected on the final logits
      DeviceGuard g(device);
      hipStream_t st = reinterpret_cast<hipStream_t>(stream);
      const dim3 gr((unsigned)rows), bl(tc::kLargeThreads);
      if (dtype == TC_BF16 && p->hist_mode != TC_HIST_MASK && !p->d_add_mask)
        hipLaunchKernelGGL(tc::k_qwen_large, gr, bl, 0, st, a);
      else if (dtype == TC_BF16)
        hipLaunchKernelGGL(tc::k_qwen_large_gen<uint16_t>, gr, bl, 0, st, a);
      else
        hipLaunchKernelGGL(tc::k_qwen_large_gen<float>, gr, bl, 0, st, a);
      hipError_t e = hipGetLastError();
      return e == hipSuccess ? TC_OK : hip_fail(e, "tc_sample launch");
    }
    return fail(TC_EUNSUPPORTED, "tc_sample: vocab %d exceeds the register-resident kernel", V);
  }
  DeviceGuard g(device);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  hipError_t e;
  switch (p->variant) {
    case TC_QWEN: e = launch_k_qwen(dtype, items, threads, (int)rows, st, a); break;
    case TC_COSY_RAS: e = launch_k_cosy(dtype, items, threads, (int)rows, st, a); break;
    case TC_INDEXTTS:
      e = a.typical_mass > 0.0 ? launch_k_idx_typical(dtype, items, threads, (int)rows, st, a)
                               : launch_k_indextts(dtype, items, threads, (int)rows, st, a);
      break;
    case TC_MOSS: e = launch_k_moss(dtype, items, threads, (int)rows, st, a); break;
    default: e = launch_k_nano(dtype, items, threads, (int)rows, st, a); break;
  }
  if (e != hipSuccess) return hip_fail(e, "tc_sample launch");
  return TC_OK;
}

int tc_sample(tc_ctx* ctx, const tc_sample_params* p, const void* d_logits, int dtype, size_t rows,
              size_t vocab, size_t ld, const uint32_t* d_hist_off, const uint32_t* d_hist_ids,
              const void* d_uniforms, uint32_t* d_out_ids, int32_t* d_out_status, uint32_t* d_out_flags,
              const tc_verify_out* verify, tc_stream stream) {
  if (!ctx) return fail(TC_EINVAL, "tc_sample: ctx is NULL");
  return sample_impl(ctx->device, ctx->max_vocab, p, d_logits, dtype, rows, vocab, ld, d_hist_off, d_hist_ids,
                     d_uniforms, d_out_ids, d_out_status, d_out_flags, verify, nullptr, stream);
}

// The beam step over a workspace `ws` of `ws_rows` rows and `zero_u` (>= rows
// zero f64 uniforms); `device` is current.
static int beam_step_impl(int device, size_t max_vocab, void* ws, size_t ws_rows, const double* zero_u,
                          const tc_sample_params* p, const void* d_logits, int dtype, size_t batch,
                          size_t num_beams, size_t vocab, size_t ld, const uint32_t* d_hist_off,
                          const uint32_t* d_hist_ids, const double* d_beam_scores, const double* d_uniforms,
                          size_t n_draws, uint32_t* d_cand_flat, double* d_cand_scores, int32_t* d_out_status,
                          uint32_t* d_out_flags, tc_stream stream, bool search = false) {
  const size_t rows = batch * num_beams;
  const BeamWs w = beam_ws(ws, ws_rows);
  tc_verify_out v{};
  v.cap = (uint32_t)tc::kBeamCap;
  v.d_topk_count = w.topk_count;
  v.d_topk_ids = w.topk_ids;
  v.d_keep_count = w.keep_count;
  v.d_keep_ids = w.keep_ids;
  v.d_keep_probs = w.keep_probs;
  v.d_norm = nullptr;
  tc_sample_params rp = *p;
  rp.d_mark_mask = nullptr;
  if (search) {
    // without sampling the row keeps log_softmax and the penalty only
    // (generation.rs:653-662), and its n_keep best scores, ties included
    rp.temperature = 1.0;
    rp.top_p = 1.0;
    rp.top_k = (uint32_t)n_draws;
    rp.min_keep = 0;
  }
  int rc = sample_impl(device, max_vocab, &rp, d_logits, dtype, rows, vocab, ld, d_hist_off, d_hist_ids, zero_u,
                       w.ids, w.status, w.flags, &v, w.keep_scores, stream);
  if (rc != TC_OK) return rc;
  tc::BeamArgs b{};
  b.nb = (int)num_beams;
  b.V = (int)vocab;
  b.n_draws = (int)n_draws;
  b.row_status = w.status;
  b.row_flags = w.flags;
  b.keep_count = w.keep_count;
  b.keep_ids = w.keep_ids;
  b.keep_scores = w.keep_scores;
  b.beam_scores = d_beam_scores;
  b.uniforms = d_uniforms;
  b.cand_flat = d_cand_flat;
  b.cand_scores = d_cand_scores;
  b.out_status = d_out_status;
  b.out_flags = d_out_flags;
  if (search)
    hipLaunchKernelGGL(tc::k_beam_topn, dim3((unsigned)batch), dim3(64), 0, reinterpret_cast<hipStream_t>(stream), b);
  else
    hipLaunchKernelGGL(tc::k_beam_joint, dim3((unsigned)batch), dim3(64), 0, reinterpret_cast<hipStream_t>(stream), b);
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? TC_OK : hip_fail(e, "tc_indextts_beam_step launch");
}

// Argument checks shared by both beam entry points.
static int beam_check(const char* fn, const tc_sample_params* p, const void* d_logits, size_t batch,
                      size_t num_beams, size_t vocab, const double* d_beam_scores, const double* d_uniforms,
                      size_t n_draws, const uint32_t* d_cand_flat, const double* d_cand_scores,
                      const int32_t* d_out_status) {
  if (!p) return fail(TC_EINVAL, "%s: params is NULL", fn);
  if (p->variant != TC_INDEXTTS) return fail(TC_EINVAL, "%s: variant must be TC_INDEXTTS", fn);
  if (batch == 0) return TC_OK;
  if (!d_logits || !d_beam_scores || !d_uniforms || !d_cand_flat || !d_cand_scores || !d_out_status)
    return fail(TC_EINVAL, "%s: NULL device pointer", fn);
  if (num_beams == 0 || num_beams > (size_t)tc::kBeamMaxBeams)
    return fail(TC_EINVAL, "%s: num_beams %zu (1..%d)", fn, num_beams, tc::kBeamMaxBeams);
  if (n_draws == 0 || n_draws > (size_t)tc::kBeamMaxDraws)
    return fail(TC_EINVAL, "%s: n_draws %zu (1..%d)", fn, n_draws, tc::kBeamMaxDraws);
  if (vocab == 0 || vocab > (size_t)INT32_MAX || num_beams * vocab > (size_t)UINT32_MAX)
    return fail(TC_EINVAL, "%s: num_beams * vocab must fit 32 bits", fn);
  if (batch > (size_t)INT32_MAX / num_beams) return fail(TC_EINVAL, "%s: batch too large", fn);
  return TC_OK;
}

// The context's beam workspace (allocated on its first beam step): R zero
// uniforms, then the row-pass workspace of R rows.  The caller made the
// context's device current.
static int ctx_beam_ws(tc_ctx* ctx) {
  if (ctx->d_beam) return TC_OK;
  const size_t R = ctx->max_rows;
  const size_t bytes = R * 8 + beam_ws_bytes(R);
  hipError_t e = hipMalloc(&ctx->d_beam, bytes);
  if (e != hipSuccess) {
    ctx->d_beam = nullptr;
    return fail(TC_ENOMEM, "hipMalloc(%zu): %s", bytes, hipGetErrorString(e));
  }
  e = hipMemset(ctx->d_beam, 0, bytes);
  if (e != hipSuccess) return hip_fail(e, "hipMemset");
  return TC_OK;
}

int tc_indextts_beam_step(tc_ctx* ctx, const tc_sample_params* p, const void* d_logits, int dtype, size_t batch,
                          size_t num_beams, size_t vocab, size_t ld, const uint32_t* d_hist_off,
                          const uint32_t* d_hist_ids, const double* d_beam_scores, const double* d_uniforms,
                          size_t n_draws, uint32_t* d_cand_flat, double* d_cand_scores, int32_t* d_out_status,
                          uint32_t* d_out_flags, tc_stream stream) {
  if (!ctx) return fail(TC_EINVAL, "tc_indextts_beam_step: ctx is NULL");
  int rc = beam_check("tc_indextts_beam_step", p, d_logits, batch, num_beams, vocab, d_beam_scores, d_uniforms,
                      n_draws, d_cand_flat, d_cand_scores, d_out_status);
  if (rc != TC_OK || batch == 0) return rc;
  const size_t rows = batch * num_beams;
  if (rows > ctx->max_rows) return fail(TC_EINVAL, "tc_indextts_beam_step: %zu rows > context max %zu", rows, ctx->max_rows);
  DeviceGuard g(ctx->device);
  rc = ctx_beam_ws(ctx);
  if (rc != TC_OK) return rc;
  const size_t R = ctx->max_rows;
  const double* zero_u = static_cast<const double*>(ctx->d_beam);
  void* ws = static_cast<char*>(ctx->d_beam) + R * 8;
  return beam_step_impl(ctx->device, ctx->max_vocab, ws, R, zero_u, p, d_logits, dtype, batch, num_beams, vocab, ld,
                        d_hist_off, d_hist_ids, d_beam_scores, d_uniforms, n_draws, d_cand_flat, d_cand_scores,
                        d_out_status, d_out_flags, stream);
}

int tc_indextts_beam_search_step(tc_ctx* ctx, const tc_sample_params* p, const void* d_logits, int dtype,
                                 size_t batch, size_t num_beams, size_t vocab, size_t ld, const uint32_t* d_hist_off,
                                 const uint32_t* d_hist_ids, const double* d_beam_scores, size_t n_keep,
                                 uint32_t* d_cand_flat, double* d_cand_scores, int32_t* d_out_status,
                                 tc_stream stream) {
  if (!ctx) return fail(TC_EINVAL, "tc_indextts_beam_search_step: ctx is NULL");
  // the uniforms argument is not read in this mode: d_beam_scores stands in
  int rc = beam_check("tc_indextts_beam_search_step", p, d_logits, batch, num_beams, vocab, d_beam_scores,
                      d_beam_scores, n_keep, d_cand_flat, d_cand_scores, d_out_status);
  if (rc != TC_OK || batch == 0) return rc;
  const size_t rows = batch * num_beams;
  if (rows > ctx->max_rows)
    return fail(TC_EINVAL, "tc_indextts_beam_search_step: %zu rows > context max %zu", rows, ctx->max_rows);
  DeviceGuard g(ctx->device);
  rc = ctx_beam_ws(ctx);
  if (rc != TC_OK) return rc;
  const size_t R = ctx->max_rows;
  const double* zero_u = static_cast<const double*>(ctx->d_beam);
  void* ws = static_cast<char*>(ctx->d_beam) + R * 8;
  return beam_step_impl(ctx->device, ctx->max_vocab, ws, R, zero_u, p, d_logits, dtype, batch, num_beams, vocab, ld,
                        d_hist_off, d_hist_ids, d_beam_scores, nullptr, n_keep, d_cand_flat, d_cand_scores,
                        d_out_status, nullptr, stream, true);
}

int tc_indextts_beam_step_noalloc(const tc_sample_params* p, const void* d_logits, int dtype, size_t batch,
                                  size_t num_beams, size_t vocab, size_t ld, const uint32_t* d_hist_off,
                                  const uint32_t* d_hist_ids, const double* d_beam_scores, const double* d_uniforms,
                                  size_t n_draws, uint32_t* d_cand_flat, double* d_cand_scores,
                                  int32_t* d_out_status, uint32_t* d_out_flags, tc_stream stream) {
  int rc = beam_check("tc_indextts_beam_step_noalloc", p, d_logits, batch, num_beams, vocab, d_beam_scores,
                      d_uniforms, n_draws, d_cand_flat, d_cand_scores, d_out_status);
  if (rc != TC_OK || batch == 0) return rc;
  const size_t rows = batch * num_beams;
  if (rows > (size_t)tc::kStaticBeamRows)
    return fail(TC_EINVAL, "tc_indextts_beam_step_noalloc: %zu beam rows > the static workspace's %d", rows,
                tc::kStaticBeamRows);
  if (vocab > (size_t)tc::kMaxVocabReg)
    return fail(TC_EUNSUPPORTED, "tc_indextts_beam_step_noalloc: vocab %zu > %d", vocab, tc::kMaxVocabReg);
  int device = 0;
  hipError_t e = hipGetDevice(&device);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  StaticWs w;
  rc = static_ws_setup(device, &w);
  if (rc != TC_OK) return rc;
  return beam_step_impl(device, (size_t)tc::kMaxVocabReg, w.scratch, (size_t)tc::kStaticBeamRows, w.zeros, p,
                        d_logits, dtype, batch, num_beams, vocab, ld, d_hist_off, d_hist_ids, d_beam_scores,
                        d_uniforms, n_draws, d_cand_flat, d_cand_scores, d_out_status, d_out_flags, stream);
}

static int grid_for(size_t n) {
  size_t g = (n + 255) / 256;
  if (g > 4096) g = 4096;
  return (int)(g ? g : 1);
}

int tc_apply_repetition_penalty(tc_ctx* ctx, const float* d_in, float* d_out, size_t rows, size_t vocab, size_t ld,
                                const uint32_t* d_ids, size_t n_ids, double penalty, tc_stream stream) {
  // the [V] byte mask lives in the context's workspace (one context per stream)
  if (!ctx || !d_in || !d_out || (n_ids && !d_ids)) return fail(TC_EINVAL, "tc_apply_repetition_penalty: NULL pointer");
  if (ld < vocab || vocab > (size_t)INT32_MAX) return fail(TC_EINVAL, "tc_apply_repetition_penalty: shape");
  if (vocab > ctx->max_vocab) return fail(TC_EINVAL, "tc_apply_repetition_penalty: vocab %zu > context max %zu", vocab, ctx->max_vocab);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (fabs(penalty - 1.0) < 1e-9) {
    if (d_in != d_out) {
      hipError_t e = hipMemcpy2DAsync(d_out, ld * 4, d_in, ld * 4, vocab * 4, rows, hipMemcpyDeviceToDevice, st);
      if (e != hipSuccess) return hip_fail(e, "hipMemcpy2DAsync");
    }
    return TC_OK;
  }
  DeviceGuard g(ctx->device);
  uint8_t* mask = ctx->d_mask;
  hipLaunchKernelGGL(tc::k_fill_u8, dim3(grid_for(vocab)), dim3(256), 0, st, mask, vocab);
  if (n_ids)
    hipLaunchKernelGGL(tc::k_penalty_ids_mask, dim3(grid_for(n_ids)), dim3(256), 0, st, d_ids, n_ids, mask, (int)vocab);
  const float pf = (float)penalty;
  hipLaunchKernelGGL(tc::k_apply_penalty, dim3(grid_for(rows * vocab)), dim3(256), 0, st, d_in, d_out, (int)rows,
                     (int)vocab, (long long)ld, (const uint8_t*)mask, (const float*)nullptr, pf, 1.0f / pf);
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? TC_OK : hip_fail(e, "tc_apply_repetition_penalty");
}

int tc_apply_repetition_penalty_with_mask(const float* d_in, float* d_out, size_t rows, size_t vocab, size_t ld,
                                          const float* d_mask, double penalty, tc_stream stream) {
  if (!d_in || !d_out || !d_mask) return fail(TC_EINVAL, "tc_apply_repetition_penalty_with_mask: NULL pointer");
  if (ld < vocab || vocab > (size_t)INT32_MAX) return fail(TC_EINVAL, "tc_apply_repetition_penalty_with_mask: shape");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (fabs(penalty - 1.0) < 1e-9) {
    if (d_in != d_out) {
      hipError_t e = hipMemcpy2DAsync(d_out, ld * 4, d_in, ld * 4, vocab * 4, rows, hipMemcpyDeviceToDevice, st);
      if (e != hipSuccess) return hip_fail(e, "hipMemcpy2DAsync");
    }
    return TC_OK;
  }
  const float pf = (float)penalty;
  hipLaunchKernelGGL(tc::k_apply_penalty, dim3(grid_for(rows * vocab)), dim3(256), 0, st, d_in, d_out, (int)rows,
                     (int)vocab, (long long)ld, (const uint8_t*)nullptr, d_mask, pf, 1.0f / pf);
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? TC_OK : hip_fail(e, "tc_apply_repetition_penalty_with_mask");
}

int tc_build_suppression_mask(float* d_mask, size_t vocab, uint32_t eos_id, tc_stream stream) {
  if (!d_mask || vocab == 0 || vocab > (size_t)INT32_MAX) return fail(TC_EINVAL, "tc_build_suppression_mask: args");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(tc::k_build_suppression, dim3(grid_for(vocab)), dim3(256), 0, st, d_mask, (int)vocab, eos_id);
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? TC_OK : hip_fail(e, "tc_build_suppression_mask");
}

int tc_apply_token_suppression_with_mask(const float* d_in, float* d_out, size_t rows, size_t vocab, size_t ld,
                                         const float* d_mask, tc_stream stream) {
  if (!d_in || !d_out || !d_mask) return fail(TC_EINVAL, "tc_apply_token_suppression_with_mask: NULL pointer");
  if (ld < vocab || vocab > (size_t)INT32_MAX) return fail(TC_EINVAL, "tc_apply_token_suppression_with_mask: shape");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(tc::k_add_mask, dim3(grid_for(rows * vocab)), dim3(256), 0, st, d_in, d_out, (int)rows,
                     (int)vocab, (long long)ld, d_mask);
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? TC_OK : hip_fail(e, "tc_apply_token_suppression_with_mask");
}

int tc_update_penalty_mask(float* d_mask, size_t vocab, const uint32_t* d_token, tc_stream stream) {
  if (!d_mask || !d_token || vocab > (size_t)INT32_MAX) return fail(TC_EINVAL, "tc_update_penalty_mask: args");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(tc::k_update_penalty_mask, dim3(1), dim3(64), 0, st, d_mask, (int)vocab, d_token);
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? TC_OK : hip_fail(e, "tc_update_penalty_mask");
}

int tc_greedy_sample(const void* d_logits, int dtype, size_t rows, size_t vocab, size_t ld, uint32_t* d_out_ids,
                     tc_stream stream) {
  if (!d_logits || !d_out_ids) return fail(TC_EINVAL, "tc_greedy_sample: NULL pointer");
  if (rows == 0) return TC_OK;
  if (vocab == 0 || ld < vocab || vocab > (size_t)INT32_MAX || rows > (size_t)INT32_MAX)
    return fail(TC_EINVAL, "tc_greedy_sample: shape");
  if (dtype != TC_F32 && dtype != TC_BF16) return fail(TC_EINVAL, "tc_greedy_sample: dtype");
  int items, threads;
  if (!pick_shape((int)vocab, dtype, &items, &threads))
    return fail(TC_EUNSUPPORTED, "tc_greedy_sample: vocab %zu too large", vocab);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  dim3 g((unsigned)rows), b(threads);
  if (dtype == TC_F32) {
    if (items == 8) hipLaunchKernelGGL((tc::k_greedy<float, 8>), g, b, 0, st, (const float*)d_logits, (long long)ld, (int)vocab, d_out_ids);
    else if (items == 12) hipLaunchKernelGGL((tc::k_greedy<float, 12>), g, b, 0, st, (const float*)d_logits, (long long)ld, (int)vocab, d_out_ids);
    else if (items == 16) hipLaunchKernelGGL((tc::k_greedy<float, 16>), g, b, 0, st, (const float*)d_logits, (long long)ld, (int)vocab, d_out_ids);
    else hipLaunchKernelGGL((tc::k_greedy<float, 24>), g, b, 0, st, (const float*)d_logits, (long long)ld, (int)vocab, d_out_ids);
  } else {
    if (items == 8) hipLaunchKernelGGL((tc::k_greedy<uint16_t, 8>), g, b, 0, st, (const uint16_t*)d_logits, (long long)ld, (int)vocab, d_out_ids);
    else if (items == 16) hipLaunchKernelGGL((tc::k_greedy<uint16_t, 16>), g, b, 0, st, (const uint16_t*)d_logits, (long long)ld, (int)vocab, d_out_ids);
    else hipLaunchKernelGGL((tc::k_greedy<uint16_t, 24>), g, b, 0, st, (const uint16_t*)d_logits, (long long)ld, (int)vocab, d_out_ids);
  }
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? TC_OK : hip_fail(e, "tc_greedy_sample");
}

}  // extern "C"
