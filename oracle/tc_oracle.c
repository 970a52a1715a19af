/*
 * tc_oracle.c -- CPU restatement of talechime's per-step token samplers.
 *
 * TEST INFRASTRUCTURE ONLY (the oracle).  The product path never calls this.
 *
 * Each function follows the Rust code cited next to it, keeping its element
 * types, its operation order and its summation order.  Where the reference
 * relies on a third-party routine the restatement follows the routine's
 * algorithm as used by the cited call site:
 *   - candle_nn::ops::softmax_last_dim (CPU): max via f32::max from x[0],
 *     e = exp(x - max), sequential f32 sum from 0, then divide;
 *   - candle `Tensor / f64`: affine(1/t, 0), i.e. x * (f32)(1/t) + 0.0f;
 *   - candle argmax: first index with a strictly greater value, from x[0];
 *   - Rust `Iterator::sum` of floats: sequential, starting from -0.0;
 *   - Rust f32::exp / f32::ln / f64::exp: the platform libm (glibc).
 * Rust's unstable sorts leave the order of equal keys unspecified; this file
 * breaks such ties by ascending vocabulary id and raises TCO_FLAG_TIE_CUT on
 * every row where the tie order could change the result.
 *
 * Pinning (tests/test_oracle_kats.py, tests/test_oracle_moss.py,
 * tests/test_oracle_crosscheck.py): the RNGs by their integer closed forms and
 * the reference's constants; qwen, indextts, cosyvoice3 and moss-nano by every
 * vector of the reference's own unit tests for these functions; row_moss
 * (moss-tts/src/sampling.rs:22-85), which has reference vectors only for its
 * errors and greedy path, by what the mathematics fixes (rows of equal logits
 * with exact weights and shares, rank-order CDFs, a brute force over a grid of
 * uniforms against inverse-CDF intervals computed in double); the beam-search
 * step by a stable argsort of the joint scores.  Parity unpinned:
 *   - the candle softmax summation order and the `Tensor / f64` lowering
 *     listed above (no reference test fixes them beyond dyadic rows).
 */
#define _GNU_SOURCE
#include "tc_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* small helpers                                                             */
/* ------------------------------------------------------------------------ */

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint64_t d2u(double d) { uint64_t u; memcpy(&u, &d, 8); return u; }

/* Unsigned key whose order is Rust's f32::total_cmp. */
static inline uint32_t tkey32(float f) {
  uint32_t b = f2u(f);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
static inline float untkey32(uint32_t k) {
  return u2f((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}
static inline uint64_t tkey64(double d) {
  uint64_t b = d2u(d);
  return (b & 0x8000000000000000ull) ? ~b : (b | 0x8000000000000000ull);
}

/* Rust f32::max / f64::max: NaN operands are ignored. */
static inline float rmaxf(float a, float b) { return isnan(a) ? b : (isnan(b) ? a : (a > b ? a : b)); }
static inline double rmax(double a, double b) { return isnan(a) ? b : (isnan(b) ? a : (a > b ? a : b)); }

static int cmp_u64(const void* a, const void* b) {
  uint64_t x = *(const uint64_t*)a, y = *(const uint64_t*)b;
  return (x > y) - (x < y);
}

/* k-th smallest (0-based) of a[0..n) in place (three-way quickselect). */
static void nth_u64(uint64_t* a, size_t n, size_t k) {
  size_t lo = 0, hi = n;
  uint64_t seed = 0x9E3779B97F4A7C15ull ^ n;
  while (hi - lo > 1) {
    seed = seed * 6364136223846793005ull + 1442695040888963407ull;
    uint64_t piv = a[lo + (size_t)((seed >> 33) % (hi - lo))];
    size_t lt = lo, i = lo, gt = hi;
    while (i < gt) {
      if (a[i] < piv) { uint64_t t = a[lt]; a[lt] = a[i]; a[i] = t; lt++; i++; }
      else if (a[i] > piv) { gt--; uint64_t t = a[gt]; a[gt] = a[i]; a[i] = t; }
      else i++;
    }
    if (k < lt) hi = lt;
    else if (k >= gt) lo = gt;
    else return;
  }
}

/* ------------------------------------------------------------------------ */
/* RNGs                                                                      */
/* ------------------------------------------------------------------------ */

/* crates/qwen3-tts/src/generation/sampling.rs:90-93 */
uint64_t tco_qwen_initial_state(uint64_t seed) {
  return seed * 2685821657736338717ull + 1442695040888963407ull;
}

/* crates/qwen3-tts/src/generation/sampling.rs:75-85 (seeded PCG XSH RR 64/32) */
float tco_qwen_rand_f32(uint64_t* state) {
  uint64_t old = *state;
  *state = old * 6364136223846793005ull + 1442695040888963407ull;
  uint32_t xs = (uint32_t)(((old >> 18) ^ old) >> 27);
  uint32_t rot = (uint32_t)(old >> 59);
  uint32_t out = (xs >> rot) | (xs << ((32u - rot) & 31u));
  return (float)out / (float)UINT32_MAX;
}

/* crates/cosyvoice3/src/rng.rs:169-175 */
uint32_t tco_steprng_next_u32(uint64_t* state, uint64_t inc) {
  uint64_t old = *state;
  *state = old * 6364136223846793005ull + inc;
  uint32_t xs = (uint32_t)(((old >> 18) ^ old) >> 27);
  uint32_t rot = (uint32_t)(old >> 59);
  return (xs >> rot) | (xs << ((32u - rot) & 31u));
}

/* crates/cosyvoice3/src/rng.rs:158-167 */
void tco_steprng_new(uint64_t seed, uint64_t* state, uint64_t* inc) {
  *state = 0;
  *inc = (seed << 1) | 1ull;
  (void)tco_steprng_next_u32(state, *inc);
  *state += 0x853C49E6748FEA9Dull;
  (void)tco_steprng_next_u32(state, *inc);
}

/* crates/cosyvoice3/src/rng.rs:178-180 */
float tco_steprng_next_f32(uint64_t* state, uint64_t inc) {
  return (float)(tco_steprng_next_u32(state, inc) >> 8) * (1.0f / (float)(1u << 24));
}

/* crates/moss-tts/src/nano/sampling.rs:66-67: the LCG draw as a unit f64 */
double tco_nano_next_unit(uint32_t* state) {
  *state = *state * 1664525u + 1013904223u;
  return (double)(*state >> 8) / 16777216.0;
}

/* ------------------------------------------------------------------------ */
/* qwen (crates/qwen3-tts/src/generation/sampling.rs, tts.rs)                */
/* ------------------------------------------------------------------------ */

/* sampling.rs:388-395 applied where the mask is set (sampling.rs:377-385). */
static inline float qwen_pen_one(float x, float pen_f32, float inv_pen) {
  return x * (x > 0.0f ? inv_pen : pen_f32);
}

/* sampling.rs:334-360: ids (flattened, ids >= V ignored) -> [1,V] mask,
 * broadcast over every row. */
void tco_qwen_penalty_ids(float* x, size_t rows, size_t V, const uint32_t* ids, size_t n_ids,
                          double penalty) {
  if (fabs(penalty - 1.0) < 1e-9) return;
  unsigned char* mask = (unsigned char*)calloc(V ? V : 1, 1);
  for (size_t i = 0; i < n_ids; i++)
    if ((size_t)ids[i] < V) mask[ids[i]] = 1;
  float pf = (float)penalty, inv = 1.0f / pf;
  for (size_t r = 0; r < rows; r++)
    for (size_t v = 0; v < V; v++)
      if (mask[v]) x[r * V + v] = qwen_pen_one(x[r * V + v], pf, inv);
  free(mask);
}

/* sampling.rs:368-395: penalised where mask > 0. */
void tco_qwen_penalty_mask(float* x, size_t rows, size_t V, const float* mask, double penalty) {
  if (fabs(penalty - 1.0) < 1e-9) return;
  float pf = (float)penalty, inv = 1.0f / pf;
  for (size_t r = 0; r < rows; r++)
    for (size_t v = 0; v < V; v++)
      if (mask[v] > 0.0f) x[r * V + v] = qwen_pen_one(x[r * V + v], pf, inv);
}

/* tts.rs:22-41 */
void tco_qwen_suppression_mask(float* mask, size_t V, uint32_t eos) {
  size_t start = V >= 1024 ? V - 1024 : 0;
  for (size_t v = 0; v < V; v++) mask[v] = (v >= start && v != eos) ? -INFINITY : 0.0f;
}

/* tts.rs:44-51 (broadcast add) */
void tco_qwen_add_mask(float* x, size_t rows, size_t V, const float* add) {
  for (size_t r = 0; r < rows; r++)
    for (size_t v = 0; v < V; v++) x[r * V + v] = x[r * V + v] + add[v];
}

/* sampling.rs:175-184 with candle's `Tensor / f64` = affine(1/t, 0). */
void tco_qwen_temperature(float* x, size_t n, double t) {
  if (!(t != 1.0 && t > 0.0)) return;
  float mul = (float)(1.0 / t), add = (float)0.0;
  for (size_t i = 0; i < n; i++) x[i] = x[i] * mul + add;
}

/* candle argmax over the last dim: first strictly greater value wins. */
uint32_t tco_argmax_f32(const float* row, size_t V) {
  float acc = row[0];
  uint32_t best = 0;
  for (size_t i = 0; i < V; i++)
    if (acc < row[i]) { acc = row[i]; best = (uint32_t)i; }
  return best;
}

/* partial_cmp descending with NaN treated as Equal (sampling.rs:235). */
static int qwen_desc_partial(float a, float b) {
  if (b > a) return 1;
  if (b < a) return -1;
  return 0;
}

/* sampling.rs:224-249 */
void tco_qwen_top_k(float* row, size_t V, size_t k, uint32_t* flags) {
  if (V == 0) return;
  if (k > V) k = V;
  if (k == 0) return; /* the reference indexes sorted[k - 1]: k == 0 never reaches here */
  int has_nan = 0;
  for (size_t i = 0; i < V; i++) has_nan |= isnan(row[i]);
  float thr;
  if (has_nan) {
    /* Reference: sort_unstable_by with an inconsistent comparator; the order
     * is unspecified.  A stable insertion sort is used here. */
    if (flags) *flags |= TCO_FLAG_NAN_ROW;
    float* s = (float*)malloc(V * sizeof(float));
    memcpy(s, row, V * sizeof(float));
    for (size_t i = 1; i < V; i++) {
      float v = s[i];
      size_t j = i;
      while (j > 0 && qwen_desc_partial(s[j - 1], v) > 0) { s[j] = s[j - 1]; j--; }
      s[j] = v;
    }
    thr = s[k - 1];
    free(s);
  } else {
    /* select_nth_unstable_by(k-1, desc): the k-th largest value. */
    uint64_t* keys = (uint64_t*)malloc(V * sizeof(uint64_t));
    for (size_t i = 0; i < V; i++) keys[i] = (uint64_t)(~tkey32(row[i]));
    nth_u64(keys, V, k - 1);
    thr = untkey32(~(uint32_t)keys[k - 1]);
    free(keys);
  }
  for (size_t i = 0; i < V; i++)
    if (!(row[i] >= thr)) row[i] = -INFINITY;
}

static __thread const float* t_sort_row;
static int qwen_idx_desc_cmp(const void* pa, const void* pb) {
  uint32_t a = *(const uint32_t*)pa, b = *(const uint32_t*)pb;
  int c = qwen_desc_partial(t_sort_row[a], t_sort_row[b]);
  if (c) return c;
  return (a > b) - (a < b); /* tie order: ascending id */
}

/* sampling.rs:255-299 */
void tco_qwen_top_p(float* row, size_t V, double p, uint32_t* flags) {
  if (V == 0) return;
  uint32_t* idx = (uint32_t*)malloc(V * sizeof(uint32_t));
  float* e = (float*)malloc(V * sizeof(float));
  for (size_t i = 0; i < V; i++) idx[i] = (uint32_t)i;
  t_sort_row = row;
  qsort(idx, V, sizeof(uint32_t), qwen_idx_desc_cmp);
  float max_val = row[idx[0]];
  for (size_t i = 0; i < V; i++) e[i] = expf(row[idx[i]] - max_val);
  float sum = -0.0f;
  for (size_t i = 0; i < V; i++) sum += e[i];
  for (size_t i = 0; i < V; i++) e[i] /= sum;
  float cum = 0.0f, pf = (float)p;
  size_t cutoff = V;
  for (size_t i = 0; i < V; i++) {
    cum += e[i];
    if (cum > pf) { cutoff = i + 1; break; }
  }
  if (flags && cutoff < V && row[idx[cutoff - 1]] == row[idx[cutoff]])
    *flags |= TCO_FLAG_TIE_CUT;
  unsigned char* keep = (unsigned char*)calloc(V, 1);
  for (size_t i = 0; i < cutoff; i++) keep[idx[i]] = 1;
  for (size_t i = 0; i < V; i++)
    if (!keep[i]) row[i] = -INFINITY;
  free(keep);
  free(e);
  free(idx);
}

/* candle_nn::ops::softmax_last_dim on CPU (one row). */
static float softmax_last_dim_sum(float* row, size_t V) {
  if (V == 0) return NAN;
  float max = row[0];
  for (size_t i = 1; i < V; i++) max = rmaxf(max, row[i]);
  for (size_t i = 0; i < V; i++) row[i] = expf(row[i] - max);
  float sum = 0.0f;
  for (size_t i = 0; i < V; i++) sum += row[i];
  for (size_t i = 0; i < V; i++) row[i] /= sum;
  return sum;
}

void tco_softmax_last_dim(float* row, size_t V) { (void)softmax_last_dim_sum(row, V); }

/* sampling.rs:319-328; -1 = None */
int64_t tco_qwen_first_cdf_index(const float* row, size_t V, float thr) {
  float cum = 0.0f;
  for (size_t i = 0; i < V; i++) {
    cum += row[i];
    if (cum >= thr) return (int64_t)i;
  }
  return -1;
}

/* ------------------------------------------------------------------------ */
/* indextts (crates/indextts/src/generation.rs)                              */
/* ------------------------------------------------------------------------ */

/* :95-105 */
/* returns log_sum, NaN when the row max is not finite (row left as is) */
static float idx_log_softmax_ls(float* row, size_t V) {
  float max = -INFINITY;
  for (size_t i = 0; i < V; i++) max = rmaxf(max, row[i]);
  if (!isfinite(max)) return NAN;
  float sum = -0.0f;
  for (size_t i = 0; i < V; i++) sum += expf(row[i] - max);
  float log_sum = logf(sum);
  for (size_t i = 0; i < V; i++) row[i] = (row[i] - max) - log_sum;
  return log_sum;
}

void tco_idx_log_softmax(float* row, size_t V) { (void)idx_log_softmax_ls(row, V); }

/* :108-116 */
static void idx_softmax_f64(const double* row, size_t V, double* out) {
  double max = -INFINITY;
  for (size_t i = 0; i < V; i++) max = rmax(max, row[i]);
  if (!isfinite(max)) { for (size_t i = 0; i < V; i++) out[i] = 0.0; return; }
  for (size_t i = 0; i < V; i++) out[i] = exp(row[i] - max);
  double sum = -0.0;
  for (size_t i = 0; i < V; i++) sum += out[i];
  for (size_t i = 0; i < V; i++) out[i] = out[i] / sum;
}

/* :122-134 */
void tco_idx_penalty(float* row, size_t V, const uint32_t* ids, size_t n, double pen) {
  float* orig = (float*)malloc((V ? V : 1) * sizeof(float));
  memcpy(orig, row, V * sizeof(float));
  float pf = (float)pen;
  for (size_t i = 0; i < n; i++) {
    size_t id = ids[i];
    if (id < V) {
      float s = orig[id];
      row[id] = s < 0.0f ? s * pf : s / pf;
    }
  }
  free(orig);
}

/* :137-142 */
void tco_idx_temperature(float* row, size_t V, double t) {
  float tf = (float)t;
  for (size_t i = 0; i < V; i++) row[i] /= tf;
}

/* :148-161 */
void tco_idx_top_k(float* row, size_t V, size_t top_k, size_t min_keep) {
  size_t k = top_k > min_keep ? top_k : min_keep;
  if (k > V) k = V;
  if (k == 0 || k >= V) return;
  uint64_t* keys = (uint64_t*)malloc(V * sizeof(uint64_t));
  for (size_t i = 0; i < V; i++) keys[i] = (uint64_t)(~tkey32(row[i]));
  nth_u64(keys, V, k - 1);
  float kth = untkey32(~(uint32_t)keys[k - 1]);
  free(keys);
  for (size_t i = 0; i < V; i++)
    if (row[i] < kth) row[i] = -INFINITY;
}

/* :169-194 */
void tco_idx_top_p(float* row, size_t V, double top_p, size_t min_keep) {
  double* s64 = (double*)malloc((V ? V : 1) * sizeof(double));
  double* probs = (double*)malloc((V ? V : 1) * sizeof(double));
  for (size_t i = 0; i < V; i++) s64[i] = (double)row[i];
  idx_softmax_f64(s64, V, probs);
  uint64_t* order = (uint64_t*)malloc((V ? V : 1) * sizeof(uint64_t));
  size_t n = 0;
  for (size_t i = 0; i < V; i++)
    if (row[i] != -INFINITY) order[n++] = ((uint64_t)tkey32(row[i]) << 32) | (uint64_t)i;
  if (n > 0) {
    /* stable sort ascending by total_cmp: equal keys keep ascending id */
    qsort(order, n, sizeof(uint64_t), cmp_u64);
    unsigned char* remove = (unsigned char*)calloc(V, 1);
    double cum = 0.0;
    for (size_t j = 0; j < n; j++) {
      uint32_t i = (uint32_t)order[j];
      cum += probs[i];
      if (cum <= 1.0 - top_p) remove[i] = 1;
    }
    for (size_t j = 0; j < n && j < min_keep; j++) remove[(uint32_t)order[n - 1 - j]] = 0;
    for (size_t i = 0; i < V; i++)
      if (remove[i]) row[i] = -INFINITY;
    free(remove);
  }
  free(order);
  free(probs);
  free(s64);
}

/* :201-248 */
void tco_idx_typical(float* row, size_t V, double mass, size_t min_keep) {
  if (V == 0) return;
  float* nz = (float*)malloc(V * sizeof(float));
  memcpy(nz, row, V * sizeof(float));
  tco_idx_log_softmax(nz, V);
  double ent = 0.0;
  for (size_t i = 0; i < V; i++) {
    double term = -(double)nz[i] * (double)expf(nz[i]);
    if (!isnan(term)) ent += term;
  }
  double* shifted = (double*)malloc(V * sizeof(double));
  for (size_t i = 0; i < V; i++) shifted[i] = fabs(-(double)nz[i] - ent);
  /* stable sort ascending by shifted (total_cmp): equal keys keep ascending id */
  size_t* order = (size_t*)malloc(V * sizeof(size_t));
  typedef struct { uint64_t k; uint32_t i; } kv;
  kv* tmp = (kv*)malloc(V * sizeof(kv));
  kv* buf = (kv*)malloc(V * sizeof(kv));
  for (size_t i = 0; i < V; i++) { tmp[i].k = tkey64(shifted[i]); tmp[i].i = (uint32_t)i; }
  for (size_t w = 1; w < V; w <<= 1) { /* bottom-up merge sort, left wins ties */
    for (size_t lo = 0; lo < V; lo += 2 * w) {
      size_t mid = lo + w < V ? lo + w : V, hi = lo + 2 * w < V ? lo + 2 * w : V;
      size_t a = lo, b = mid, o = lo;
      while (a < mid && b < hi) buf[o++] = (tmp[b].k < tmp[a].k) ? tmp[b++] : tmp[a++];
      while (a < mid) buf[o++] = tmp[a++];
      while (b < hi) buf[o++] = tmp[b++];
    }
    kv* t = tmp; tmp = buf; buf = t;
  }
  for (size_t i = 0; i < V; i++) order[i] = tmp[i].i;
  free(buf);
  double* sorted = (double*)malloc(V * sizeof(double));
  double* probs = (double*)malloc(V * sizeof(double));
  for (size_t k = 0; k < V; k++) sorted[k] = (double)row[order[k]];
  idx_softmax_f64(sorted, V, probs);
  double cum = 0.0;
  size_t last_ind = V - 1;
  for (size_t k = 0; k < V; k++) {
    cum += probs[k];
    if (cum >= mass) { last_ind = k; break; }
  }
  unsigned char* remove = (unsigned char*)calloc(V, 1);
  for (size_t k = 0; k < V; k++)
    if (shifted[order[k]] > shifted[order[last_ind]]) remove[order[k]] = 1;
  size_t keep_first = min_keep > 0 ? min_keep - 1 : 0;
  for (size_t k = 0; k < V && k < keep_first; k++) remove[order[k]] = 0;
  for (size_t i = 0; i < V; i++)
    if (remove[i]) row[i] = -INFINITY;
  free(remove); free(probs); free(sorted); free(tmp); free(order); free(shifted); free(nz);
}

/* :251-265 */
size_t tco_idx_inverse_cdf(const double* w, size_t n, double u) {
  double acc = 0.0;
  size_t last_positive = 0;
  for (size_t i = 0; i < n; i++) {
    if (w[i] <= 0.0) continue;
    last_positive = i;
    acc += w[i];
    if (acc > u) return i;
  }
  return last_positive;
}

/* :280-303, with the uniforms supplied by the caller (one per draw). */
int tco_idx_sample_wo_replacement(const double* scores, size_t n_scores, size_t n,
                                  const double* uniforms, size_t* out) {
  size_t* live = (size_t*)malloc((n_scores ? n_scores : 1) * sizeof(size_t));
  size_t nl = 0;
  for (size_t i = 0; i < n_scores; i++)
    if (isfinite(scores[i])) live[nl++] = i;
  if (nl < n) { free(live); return TCO_ETOOFEW; }
  double* ex = (double*)malloc((nl ? nl : 1) * sizeof(double));
  for (size_t d = 0; d < n; d++) {
    double max = -INFINITY;
    for (size_t j = 0; j < nl; j++) max = rmax(max, scores[live[j]]);
    for (size_t j = 0; j < nl; j++) ex[j] = exp(scores[live[j]] - max);
    double sum = -0.0;
    for (size_t j = 0; j < nl; j++) sum += ex[j];
    for (size_t j = 0; j < nl; j++) ex[j] = ex[j] / sum;
    double total = -0.0;
    for (size_t j = 0; j < nl; j++) total += ex[j];
    double u = uniforms[d] * total;
    size_t pick = tco_idx_inverse_cdf(ex, nl, u);
    out[d] = live[pick];
    memmove(live + pick, live + pick + 1, (nl - pick - 1) * sizeof(size_t));
    nl--;
  }
  free(ex);
  free(live);
  return TCO_OK;
}

/* ------------------------------------------------------------------------ */
/* cosyvoice3 (crates/cosyvoice3/src/llm.rs)                                 */
/* ------------------------------------------------------------------------ */

/* :556-592.  Candidates are reported in rank order. */
uint32_t tco_cosy_nucleus(const float* probs, size_t V, float top_p, size_t top_k, float u0,
                          int* used_u0, uint32_t* cand_ids, float* cand_p, uint32_t* n_cands) {
  /* rank key: prob descending by total_cmp, then id ascending -- a total order */
  uint64_t* idx = (uint64_t*)malloc((V ? V : 1) * sizeof(uint64_t));
  for (size_t i = 0; i < V; i++) idx[i] = ((uint64_t)(~tkey32(probs[i])) << 32) | (uint64_t)i;
  size_t n;
  if (top_k > 0 && top_k < V) {
    nth_u64(idx, V, top_k);               /* select_nth_unstable_by(top_k) */
    qsort(idx, top_k, sizeof(uint64_t), cmp_u64); /* head.sort_unstable_by */
    n = top_k + 1;                        /* idx.truncate(top_k + 1) */
  } else {
    qsort(idx, V, sizeof(uint64_t), cmp_u64);
    n = V;
  }
  float cum = 0.0f;
  size_t nc = 0;
  for (size_t j = 0; j < n; j++) {
    uint32_t i = (uint32_t)idx[j];
    if (cum < top_p && nc < top_k) {
      cum += probs[i];
      if (cand_ids) cand_ids[nc] = i;
      if (cand_p) cand_p[nc] = probs[i];
      nc++;
    } else {
      break;
    }
  }
  if (n_cands) *n_cands = (uint32_t)nc;
  uint32_t result;
  if (nc == 0) {
    *used_u0 = 0;
    result = (uint32_t)idx[0];
  } else {
    *used_u0 = 1;
    /* candidates are the first nc entries of idx in rank order */
    float total = -0.0f;
    for (size_t j = 0; j < nc; j++) total += probs[(uint32_t)idx[j]];
    float pick = u0 * total;
    float acc = 0.0f;
    result = (uint32_t)idx[nc - 1];
    for (size_t j = 0; j < nc; j++) {
      acc += probs[(uint32_t)idx[j]];
      if (pick < acc) { result = (uint32_t)idx[j]; break; }
    }
  }
  free(idx);
  return result;
}

/* :594-604 */
uint32_t tco_cosy_random(const float* probs, size_t V, float u1) {
  float acc = 0.0f;
  for (size_t i = 0; i < V; i++) {
    acc += probs[i];
    if (u1 < acc) return (uint32_t)i;
  }
  return (uint32_t)(V - 1);
}

/* ------------------------------------------------------------------------ */
/* per-row pipelines                                                         */
/* ------------------------------------------------------------------------ */

typedef struct {
  uint32_t n_topk;
  uint32_t* topk;     /* ascending ids (cap entries) */
  uint32_t n_keep;
  uint32_t* keep;
  float* keep_p;
  uint32_t cap;
  float norm;         /* indextts log_sum; qwen / cosyvoice3 softmax denominator */
} row_verify;

static void rv_set_topk_from_row(row_verify* rv, const float* row, size_t V) {
  if (!rv) return;
  uint32_t n = 0;
  for (size_t i = 0; i < V; i++)
    if (row[i] != -INFINITY) { if (n < rv->cap) rv->topk[n] = (uint32_t)i; n++; }
  rv->n_topk = n;
}

/* Reports a candidate set given in any order as the verify contract wants it:
 * the first `cap` ids of the whole set in ascending order (with their
 * probabilities when pr is given). */
static void rv_put_set(uint32_t* dst, float* dst_p, uint32_t cap, const uint32_t* ids, const float* pr,
                       size_t n) {
  uint64_t* t = (uint64_t*)malloc((n ? n : 1) * sizeof(uint64_t));
  for (size_t j = 0; j < n; j++) {
    float q = pr ? pr[j] : 0.0f;
    uint32_t qb;
    memcpy(&qb, &q, 4);
    t[j] = ((uint64_t)ids[j] << 32) | qb;
  }
  qsort(t, n, sizeof(uint64_t), cmp_u64);
  for (size_t j = 0; j < n && j < cap; j++) {
    dst[j] = (uint32_t)(t[j] >> 32);
    if (dst_p) dst_p[j] = u2f((uint32_t)t[j]);
  }
  free(t);
}

/* qwen: caller penalty chain (synthesis.rs:1228-1279) + sample_cpu (sampling.rs:169-219). */
static int row_qwen(const tco_params* p, float* x, size_t V, const uint32_t* ids, size_t n_ids,
                    float u, uint32_t* tok, uint32_t* flags, row_verify* rv) {
  if (fabs(p->penalty - 1.0) >= 1e-9) {
    if (p->hist_mode == TCO_HIST_MASK) tco_qwen_penalty_mask(x, 1, V, p->pen_mask, p->penalty);
    else tco_qwen_penalty_ids(x, 1, V, ids, n_ids, p->penalty);
  }
  if (p->add_mask) tco_qwen_add_mask(x, 1, V, p->add_mask);
  if (p->eos_id >= 0 && (size_t)p->eos_id < V) x[p->eos_id] = -INFINITY;
  tco_qwen_temperature(x, V, p->temperature);
  if (p->temperature < 0.01) {
    *tok = tco_argmax_f32(x, V);
    *flags |= TCO_FLAG_GREEDY;
    if (rv) { rv->n_topk = 0; rv->n_keep = 0; }
    return TCO_OK;
  }
  if (p->top_k > 0) tco_qwen_top_k(x, V, p->top_k, flags);
  rv_set_topk_from_row(rv, x, V);
  if (p->top_p < 1.0 && p->top_p > 0.0) tco_qwen_top_p(x, V, p->top_p, flags);
  unsigned char* alive = rv ? (unsigned char*)malloc(V) : NULL;
  if (rv) for (size_t i = 0; i < V; i++) alive[i] = x[i] != -INFINITY;
  float norm = softmax_last_dim_sum(x, V);
  if (rv) rv->norm = norm;
  int64_t i = tco_qwen_first_cdf_index(x, V, u);
  *tok = i < 0 ? 0u : (uint32_t)i;
  if (rv) {
    uint32_t n = 0;
    for (size_t v = 0; v < V; v++)
      if (alive[v]) { if (n < rv->cap) { rv->keep[n] = (uint32_t)v; rv->keep_p[n] = x[v]; } n++; }
    rv->n_keep = n;
    free(alive);
  }
  return TCO_OK;
}

/* cosyvoice3: llm.rs:517-538 */
static int row_cosy(const tco_params* p, float* x, size_t V, size_t row, const uint32_t* hist,
                    size_t n_hist, float u0, float u1, uint32_t* tok, uint32_t* flags, row_verify* rv) {
  if (p->eos_id >= 0) {
    for (size_t i = 0; i < V; i++) x[i] = x[i] + ((size_t)p->eos_id == i ? -INFINITY : 0.0f);
  }
  {
    float sum = softmax_last_dim_sum(x, V);
    if (rv) rv->norm = sum;
  }
  int used = 0;
  uint32_t nc = 0;
  uint32_t* cids = (uint32_t*)malloc((p->top_k + 1) * sizeof(uint32_t) + 4);
  float* cp = (float*)malloc((p->top_k + 1) * sizeof(float) + 4);
  size_t tk = p->top_k;
  uint32_t* cids_full = NULL;
  float* cp_full = NULL;
  if (tk >= V) {
    cids_full = (uint32_t*)malloc(V * sizeof(uint32_t));
    cp_full = (float*)malloc(V * sizeof(float));
  }
  uint32_t top = tco_cosy_nucleus(x, V, (float)p->top_p, tk, u0, &used,
                                  cids_full ? cids_full : cids, cp_full ? cp_full : cp, &nc);
  uint32_t* ci = cids_full ? cids_full : cids;
  float* cpp = cp_full ? cp_full : cp;
  size_t w = p->ras_win;
  size_t start = n_hist > w ? n_hist - w : 0;
  size_t rep = 0;
  for (size_t i = start; i < n_hist; i++) rep += hist[i] == top;
  if ((float)rep >= (float)w * p->ras_tau) {
    top = tco_cosy_random(x, V, u1);
    *flags |= TCO_FLAG_RAS;
  }
  *tok = top;
  if (rv) {
    rv_put_set(rv->topk, NULL, rv->cap, ci, NULL, nc);
    rv_put_set(rv->keep, rv->keep_p, rv->cap, ci, cpp, nc);
    rv->n_topk = nc;
    rv->n_keep = nc;
  }
  free(cids); free(cp); free(cids_full); free(cp_full);
  return TCO_OK;
}

/* indextts: generation.rs:643-666 for one row with beam score 0, then
 * sample_without_replacement with n = 1 (generation.rs:280-303). */
/* The processors of one row, in place (generation.rs:643-662, sampling on). */
static void idx_process_row(const tco_params* p, float* x, size_t V, const uint32_t* ids, size_t n_ids,
                            row_verify* rv) {
  {
    float ls = idx_log_softmax_ls(x, V);
    if (rv) rv->norm = ls;
  }
  if (p->penalty != 1.0) tco_idx_penalty(x, V, ids, n_ids, p->penalty);
  if (p->typical) tco_idx_typical(x, V, p->typical_mass, 2);
  if (p->temperature != 1.0) tco_idx_temperature(x, V, p->temperature);
  if (p->top_k != 0) tco_idx_top_k(x, V, p->top_k, p->min_keep);
  rv_set_topk_from_row(rv, x, V);
  if (p->top_p < 1.0) tco_idx_top_p(x, V, p->top_p, p->min_keep);
}

static int row_indextts(const tco_params* p, float* x, size_t V, size_t row, const uint32_t* ids,
                        size_t n_ids, double u, uint32_t* tok, uint32_t* flags, row_verify* rv) {
  (void)flags;
  (void)row;
  idx_process_row(p, x, V, ids, n_ids, rv);
  double* joint = (double*)malloc((V ? V : 1) * sizeof(double));
  for (size_t i = 0; i < V; i++) joint[i] = (double)x[i] + 0.0;
  size_t pick = 0;
  int st = tco_idx_sample_wo_replacement(joint, V, 1, &u, &pick);
  *tok = (uint32_t)pick;
  if (rv) {
    /* weights of the single draw: softmax over the live (finite) entries */
    double max = -INFINITY;
    for (size_t i = 0; i < V; i++) if (isfinite(joint[i])) max = rmax(max, joint[i]);
    double sum = -0.0;
    for (size_t i = 0; i < V; i++) if (isfinite(joint[i])) sum += exp(joint[i] - max);
    uint32_t n = 0;
    for (size_t i = 0; i < V; i++)
      if (isfinite(joint[i])) {
        if (n < rv->cap) { rv->keep[n] = (uint32_t)i; rv->keep_p[n] = (float)(exp(joint[i] - max) / sum); }
        n++;
      }
    rv->n_keep = n;
  }
  free(joint);
  return st;
}

/* moss: moss-tts/src/sampling.rs:22-85 */
static int row_moss(const tco_params* p, float* x, size_t V, const uint32_t* hist, size_t n_hist,
                    double u, uint32_t* tok, uint32_t* flags, row_verify* rv) {
  float pen = (float)p->penalty, temp = (float)p->temperature;
  unsigned char* seen = (unsigned char*)calloc(V ? V : 1, 1);
  for (size_t i = 0; i < n_hist; i++) {
    size_t id = hist[i];
    if (id < V && !seen[id]) {
      seen[id] = 1;
      x[id] = x[id] < 0.0f ? x[id] * pen : x[id] / pen;
    }
  }
  free(seen);
  if (p->exclude_id >= 0) {
    if ((size_t)p->exclude_id >= V) return TCO_EINVAL; /* values[id] would panic */
    x[p->exclude_id] = -INFINITY;
  }
  int any_finite = 0, any_nan = 0;
  for (size_t i = 0; i < V; i++) { any_finite |= isfinite(x[i]) != 0; any_nan |= isnan(x[i]) != 0; }
  if (!any_finite || any_nan) return TCO_ENONFINITE;
  uint64_t* ranked = (uint64_t*)malloc(V * sizeof(uint64_t));
  for (size_t i = 0; i < V; i++) ranked[i] = ((uint64_t)(~tkey32(x[i])) << 32) | (uint64_t)i;
  qsort(ranked, V, sizeof(uint64_t), cmp_u64);
  if (temp == 0.0f) {
    *tok = (uint32_t)ranked[0];
    if (V > 1 && ranked[0] >> 32 == ranked[1] >> 32) *flags |= TCO_FLAG_TIE_CUT;
    free(ranked);
    return TCO_OK;
  }
  size_t k = p->top_k < V ? p->top_k : V;
  if (k == 0) { free(ranked); return TCO_EINVAL; } /* ranked[0] would panic */
  if (k < V && ranked[k - 1] >> 32 == ranked[k] >> 32) *flags |= TCO_FLAG_TIE_CUT;
  float maximum = x[(uint32_t)ranked[0]];
  double* w = (double*)malloc(k * sizeof(double));
  for (size_t i = 0; i < k; i++) w[i] = (double)expf((x[(uint32_t)ranked[i]] - maximum) / temp);
  double total = -0.0;
  for (size_t i = 0; i < k; i++) total += w[i];
  double cumulative = 0.0;
  size_t keep = k;
  for (size_t i = 0; i < k; i++) {
    cumulative += w[i] / total;
    if (cumulative > p->top_p) { keep = i + 1; break; }
  }
  if (keep < k && ranked[keep - 1] >> 32 == ranked[keep] >> 32) *flags |= TCO_FLAG_TIE_CUT;
  double s = -0.0;
  for (size_t i = 0; i < keep; i++) s += w[i];
  double draw = u * s;
  uint32_t result = (uint32_t)ranked[keep - 1];
  for (size_t i = 0; i < keep; i++) {
    draw -= w[i];
    if (draw <= 0.0) { result = (uint32_t)ranked[i]; break; }
  }
  *tok = result;
  if (rv) {
    uint32_t* ids = (uint32_t*)malloc(k * sizeof(uint32_t));
    float* pk = (float*)malloc(k * sizeof(float));
    for (size_t j = 0; j < k; j++) { ids[j] = (uint32_t)ranked[j]; pk[j] = (float)(w[j] / s); }
    rv_put_set(rv->topk, NULL, rv->cap, ids, NULL, k);
    rv_put_set(rv->keep, rv->keep_p, rv->cap, ids, pk, keep);
    rv->n_topk = (uint32_t)k;
    rv->n_keep = (uint32_t)keep;
    free(ids);
    free(pk);
  }
  free(w);
  free(ranked);
  return TCO_OK;
}

/* moss-nano: moss-tts/src/nano/sampling.rs:96-160 (u = the LCG draw / 2^24). */
static int row_nano(const tco_params* p, float* x, size_t V, const uint32_t* hist, size_t n_hist,
                    double u, uint32_t* tok, uint32_t* flags, row_verify* rv) {
  (void)flags;
  float pen = (float)p->penalty, temp = (float)p->temperature;
  if (V == 0) return TCO_ENONFINITE;
  for (size_t i = 0; i < V; i++) if (!isfinite(x[i])) return TCO_ENONFINITE;
  unsigned char* seen = (unsigned char*)calloc(V, 1);
  for (size_t i = 0; i < n_hist; i++) {
    size_t id = hist[i];
    if (id >= V) { free(seen); return TCO_EINVAL; }
    if (!seen[id]) { seen[id] = 1; x[id] = x[id] < 0.0f ? x[id] * pen : x[id] / pen; }
  }
  free(seen);
  for (size_t i = 0; i < V; i++) x[i] /= temp;
  uint64_t* ranked = (uint64_t*)malloc(V * sizeof(uint64_t));
  for (size_t i = 0; i < V; i++) ranked[i] = ((uint64_t)(~tkey32(x[i])) << 32) | (uint64_t)i;
  qsort(ranked, V, sizeof(uint64_t), cmp_u64); /* stable by construction (id tie-break) */
  size_t k = p->top_k < V ? p->top_k : V;
  if (k == 0) { free(ranked); return TCO_EINVAL; }
  float threshold = x[(uint32_t)ranked[k - 1]];
  float maximum = x[(uint32_t)ranked[0]];
  double* w = (double*)malloc(V * sizeof(double));
  for (size_t i = 0; i < V; i++) w[i] = x[i] < threshold ? 0.0 : exp((double)(x[i] - maximum));
  if (rv) {
    uint32_t n = 0;
    for (size_t i = 0; i < V; i++) if (w[i] > 0.0) { if (n < rv->cap) rv->topk[n] = (uint32_t)i; n++; }
    rv->n_topk = n;
  }
  if (p->top_p < 1.0) {
    double total = -0.0;
    for (size_t i = 0; i < V; i++) total += w[i];
    double cumulative = 0.0;
    for (size_t j = 0; j < V; j++) {
      uint32_t id = (uint32_t)ranked[j];
      if (cumulative > p->top_p) w[id] = 0.0;
      else cumulative += w[id] / total;
    }
  }
  double s = -0.0;
  for (size_t i = 0; i < V; i++) s += w[i];
  double draw = u * s;
  int st = TCO_EDIST;
  for (size_t i = 0; i < V; i++) {
    draw -= w[i];
    if (w[i] > 0.0 && draw <= 0.0) { *tok = (uint32_t)i; st = TCO_OK; break; }
  }
  if (rv) {
    uint32_t n = 0;
    for (size_t i = 0; i < V; i++)
      if (w[i] > 0.0) { if (n < rv->cap) { rv->keep[n] = (uint32_t)i; rv->keep_p[n] = (float)(w[i] / s); } n++; }
    rv->n_keep = n;
  }
  free(w);
  free(ranked);
  return st;
}

/* Parameter checks the reference makes before sampling. */
static int check_params(const tco_params* p) {
  switch (p->variant) {
    case TCO_QWEN: return TCO_OK;
    case TCO_COSY_RAS: { /* llm.rs:436-445 */
      float tp = (float)p->top_p, tau = p->ras_tau;
      if (!isfinite(tp) || tp <= 0.0f || tp > 1.0f || p->top_k == 0 || p->ras_win == 0 ||
          !isfinite(tau) || !(tau >= 0.0f && tau <= 1.0f))
        return TCO_EINVAL;
      return TCO_OK;
    }
    case TCO_INDEXTTS: /* generation.rs:559-571 (sampling enabled) */
      if (p->penalty <= 0.0 || p->temperature <= 0.0) return TCO_EINVAL;
      if (p->typical && !(0.0 < p->typical_mass && p->typical_mass < 1.0)) return TCO_EINVAL;
      return TCO_OK;
    case TCO_MOSS:
    case TCO_MOSS_NANO:
      return p->top_k == 0 ? TCO_EINVAL : TCO_OK;
    default:
      return TCO_EINVAL;
  }
}

static void sample_one_row(const tco_params* p, const float* logits, size_t r, size_t V,
                           const uint32_t* hist_off, const uint32_t* hist_ids,
                           const void* uniforms, uint32_t* out_ids, int32_t* out_status,
                           uint32_t* out_flags, const tco_verify* ver) {
  float* x = (float*)malloc((V ? V : 1) * sizeof(float));
  memcpy(x, logits + r * V, V * sizeof(float));
  const uint32_t* ids = NULL;
  size_t n_ids = 0;
  if (hist_off && hist_ids) {
    if (p->hist_mode == TCO_HIST_BROADCAST) { ids = hist_ids + hist_off[0]; n_ids = hist_off[1] - hist_off[0]; }
    else if (p->hist_mode == TCO_HIST_PER_ROW) { ids = hist_ids + hist_off[r]; n_ids = hist_off[r + 1] - hist_off[r]; }
  }
  row_verify rvs, *rv = NULL;
  if (ver && ver->cap) {
    rv = &rvs;
    rv->cap = ver->cap;
    rv->topk = ver->topk_ids ? ver->topk_ids + r * ver->cap : (uint32_t*)calloc(ver->cap, 4);
    rv->keep = ver->keep_ids ? ver->keep_ids + r * ver->cap : (uint32_t*)calloc(ver->cap, 4);
    rv->keep_p = ver->keep_probs ? ver->keep_probs + r * ver->cap : (float*)calloc(ver->cap, 4);
    rv->n_topk = rv->n_keep = 0;
    rv->norm = NAN;
  }
  uint32_t tok = 0, flags = 0;
  int st;
  switch (p->variant) {
    case TCO_QWEN: st = row_qwen(p, x, V, ids, n_ids, ((const float*)uniforms)[r], &tok, &flags, rv); break;
    case TCO_COSY_RAS:
      st = row_cosy(p, x, V, r, ids, n_ids, ((const float*)uniforms)[2 * r],
                    ((const float*)uniforms)[2 * r + 1], &tok, &flags, rv);
      break;
    case TCO_INDEXTTS:
      st = row_indextts(p, x, V, r, ids, n_ids, ((const double*)uniforms)[r], &tok, &flags, rv);
      break;
    case TCO_MOSS: st = row_moss(p, x, V, ids, n_ids, ((const double*)uniforms)[r], &tok, &flags, rv); break;
    case TCO_MOSS_NANO: st = row_nano(p, x, V, ids, n_ids, ((const double*)uniforms)[r], &tok, &flags, rv); break;
    default: st = TCO_EINVAL;
  }
  out_ids[r] = tok;
  if (out_status) out_status[r] = st;
  if (out_flags) out_flags[r] = flags;
  if (rv) {
    if (ver->topk_count) ver->topk_count[r] = rv->n_topk;
    if (ver->keep_count) ver->keep_count[r] = rv->n_keep;
    if (ver->norm) ver->norm[r] = rv->norm;
    if (!ver->topk_ids) free(rv->topk);
    if (!ver->keep_ids) free(rv->keep);
    if (!ver->keep_probs) free(rv->keep_p);
  }
  free(x);
}

/* One beam-sample step of indextts (generation.rs:640-701) for `batch`
 * elements of `nb` beam rows each (row bi * nb + j is beam j of element bi):
 * each row's processors (643-662), the joint beam-major scores with the row's
 * running beam score added, score as f64 + bonus (663-664), then per element
 * sample_without_replacement with n_draws draws (680; the uniforms of element
 * bi are uniforms[bi * n_draws ..]) and the candidates (joint score, flat
 * index j * V + id) sorted by score descending, stable (690).  status[bi] is
 * TCO_ETOOFEW when the element has fewer than n_draws finite joint scores. */
int tco_idx_beam_step(const tco_params* p, const float* logits, size_t batch, size_t nb, size_t V,
                      const uint32_t* hist_off, const uint32_t* hist_ids, const double* beam_scores,
                      const double* uniforms, size_t n_draws, uint32_t* cand_flat, double* cand_scores,
                      int32_t* status) {
  if (p->variant != TCO_INDEXTTS) return TCO_EINVAL;
  int st = check_params(p);
  if (st != TCO_OK) return st;
  float* x = (float*)malloc((V ? V : 1) * sizeof(float));
  double* joint = (double*)malloc((nb * V > 0 ? nb * V : 1) * sizeof(double));
  size_t* picks = (size_t*)malloc((n_draws ? n_draws : 1) * sizeof(size_t));
  for (size_t bi = 0; bi < batch; bi++) {
    for (size_t j = 0; j < nb; j++) {
      const size_t r = bi * nb + j;
      memcpy(x, logits + r * V, V * sizeof(float));
      const uint32_t* ids = NULL;
      size_t n_ids = 0;
      if (hist_off && hist_ids) { ids = hist_ids + hist_off[r]; n_ids = hist_off[r + 1] - hist_off[r]; }
      idx_process_row(p, x, V, ids, n_ids, NULL);
      for (size_t i = 0; i < V; i++) joint[j * V + i] = (double)x[i] + beam_scores[r];
    }
    status[bi] = tco_idx_sample_wo_replacement(joint, nb * V, n_draws, uniforms + bi * n_draws, picks);
    uint32_t* cf = cand_flat + bi * n_draws;
    double* cs = cand_scores + bi * n_draws;
    if (status[bi] != TCO_OK) {
      for (size_t d = 0; d < n_draws; d++) { cf[d] = 0; cs[d] = 0.0; }
      continue;
    }
    /* candidates.sort_by(|a, x| x.0.total_cmp(&a.0)): stable, descending */
    for (size_t d = 0; d < n_draws; d++) {
      size_t k = d;
      const double v = joint[picks[d]];
      while (k > 0 && tkey64(cs[k - 1]) < tkey64(v)) {
        cs[k] = cs[k - 1];
        cf[k] = cf[k - 1];
        k--;
      }
      cs[k] = v;
      cf[k] = (uint32_t)picks[d];
    }
  }
  free(picks); free(joint); free(x);
  return TCO_OK;
}

/* The beam-search branch of the same loop, do_sample = false
 * (generation.rs:643-664 and 671-679): each row's log_softmax, penalty and
 * typical warper only (the do_sample warpers are skipped), the joint
 * beam-major scores, every flat index sorted by joint score descending
 * (stable, so equal scores keep ascending flat order), truncated to n_keep,
 * then sorted by score descending again (stable: the same order). */
int tco_idx_beam_search_step(const tco_params* p, const float* logits, size_t batch, size_t nb, size_t V,
                             const uint32_t* hist_off, const uint32_t* hist_ids, const double* beam_scores,
                             size_t n_keep, uint32_t* cand_flat, double* cand_scores) {
  if (p->variant != TCO_INDEXTTS) return TCO_EINVAL;
  int st = check_params(p);
  if (st != TCO_OK) return st;
  tco_params q = *p;
  q.temperature = 1.0;
  q.top_k = 0;
  q.top_p = 1.0;
  const size_t n = nb * V;
  float* x = (float*)malloc((V ? V : 1) * sizeof(float));
  double* joint = (double*)malloc((n ? n : 1) * sizeof(double));
  for (size_t bi = 0; bi < batch; bi++) {
    for (size_t j = 0; j < nb; j++) {
      const size_t r = bi * nb + j;
      memcpy(x, logits + r * V, V * sizeof(float));
      const uint32_t* ids = NULL;
      size_t n_ids = 0;
      if (hist_off && hist_ids) { ids = hist_ids + hist_off[r]; n_ids = hist_off[r + 1] - hist_off[r]; }
      idx_process_row(&q, x, V, ids, n_ids, NULL);
      for (size_t i = 0; i < V; i++) joint[j * V + i] = (double)x[i] + beam_scores[r];
    }
    /* order.sort_by(|&a, &x| joint[x].total_cmp(&joint[a])) is stable: the
     * first n_keep of it are the n_keep best under (total order descending,
     * flat ascending), taken here by repeated scans (n_keep is small) */
    {
      unsigned char* used = (unsigned char*)calloc(n ? n : 1, 1);
      for (size_t d = 0; d < n_keep; d++) {
        size_t best = (size_t)-1;
        for (size_t f = 0; f < n; f++) {
          if (used[f]) continue;
          if (best == (size_t)-1 || tkey64(joint[f]) > tkey64(joint[best])) best = f;
        }
        if (best == (size_t)-1) { cand_flat[bi * n_keep + d] = 0; cand_scores[bi * n_keep + d] = 0.0; continue; }
        used[best] = 1;
        cand_flat[bi * n_keep + d] = (uint32_t)best;
        cand_scores[bi * n_keep + d] = joint[best];
      }
      free(used);
    }
  }
  free(joint); free(x);
  return TCO_OK;
}

int tco_sample(const tco_params* p, const float* logits, size_t rows, size_t V,
               const uint32_t* hist_off, const uint32_t* hist_ids, const void* uniforms,
               uint32_t* out_ids, int32_t* out_status, uint32_t* out_flags,
               const tco_verify* verify, int nthreads) {
  int st = check_params(p);
  if (st != TCO_OK) return st;
#ifdef _OPENMP
#pragma omp parallel for schedule(dynamic, 1) num_threads(nthreads > 0 ? nthreads : 1)
#endif
  for (long r = 0; r < (long)rows; r++)
    sample_one_row(p, logits, (size_t)r, V, hist_off, hist_ids, uniforms, out_ids, out_status,
                   out_flags, verify);
  (void)nthreads;
  return TCO_OK;
}
