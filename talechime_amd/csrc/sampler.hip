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

#include "tc_row.h"

namespace tc {

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
// that still fits, so the SIMDs share the row evenly.  The row may start up
// to 3 (f32) or 7 (bf16) elements past a 16-byte boundary, unless every row
// is aligned (`aligned`: the base and the row pitch are multiples of 16
// bytes).
bool pick_shape(int V, int dtype, bool aligned, int* items, int* threads) {
  const int pad = aligned ? 0 : (dtype == TC_BF16 ? 7 : 3);
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
  const size_t esize = dtype == TC_BF16 ? 2 : 4;
  const bool aligned = (reinterpret_cast<uintptr_t>(d_logits) & 15u) == 0 && (ld * esize) % 16 == 0;
  if (!pick_shape(V, dtype, aligned, &items, &threads) || V > tc::kMaxVocabReg) {
    // qwen over bf16 rows up to kLargeVocab: the large-vocabulary kernel
    if (p->variant == TC_QWEN && a.do_pen && (a.pen_f == 0.0f || !isfinite(a.pen_f)))
      return fail(TC_EUNSUPPORTED, "tc_sample: repetition penalty %g above %d logits", p->repetition_penalty,
                  tc::kMaxVocabReg);
    if (p->variant == TC_QWEN && V <= tc::kLargeVocab && (a.K >= 1 || a.greedy) && a.K <= tc::kLargeCand) {
      // bf16 rows without masks: the packed passes; f32 rows and the masks:
      // candidates selected on the final logits
      DeviceGuard g(device);
      hipStream_t st = reinterpret_cast<hipStream_t>(stream);
      const bool packed = dtype == TC_BF16 && p->hist_mode != TC_HIST_MASK && !p->d_add_mask;
      hipError_t e = tc::launch_k_large(packed, dtype, (int)rows, st, a);
      return e == hipSuccess ? TC_OK : hip_fail(e, "tc_sample launch");
    }
    return fail(TC_EUNSUPPORTED, "tc_sample: vocab %d exceeds the register-resident kernel", V);
  }
  DeviceGuard g(device);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  hipError_t e;
  switch (p->variant) {
    case TC_QWEN: e = tc::launch_k_qwen(dtype, items, threads, (int)rows, st, a); break;
    case TC_COSY_RAS: e = tc::launch_k_cosy(dtype, items, threads, (int)rows, st, a); break;
    case TC_INDEXTTS:
      e = a.typical_mass > 0.0 ? tc::launch_k_idx_typical(dtype, items, threads, (int)rows, st, a)
                               : tc::launch_k_indextts(dtype, items, threads, (int)rows, st, a);
      break;
    case TC_MOSS: e = tc::launch_k_moss(dtype, items, threads, (int)rows, st, a); break;
    default: e = tc::launch_k_nano(dtype, items, threads, (int)rows, st, a); break;
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
  const size_t esize = dtype == TC_BF16 ? 2 : 4;
  const bool aligned = (reinterpret_cast<uintptr_t>(d_logits) & 15u) == 0 && (ld * esize) % 16 == 0;
  if (!pick_shape((int)vocab, dtype, aligned, &items, &threads))
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
