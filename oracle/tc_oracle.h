/*
 * tc_oracle.h -- CPU restatement of talechime's five per-step token samplers.
 *
 * TEST INFRASTRUCTURE ONLY.  This is the oracle for the HIP sampler: only the
 * test suite, the smoke check and the CPU-baseline leg of the benchmark may
 * load it.  The product library never links or calls it.
 *
 * Every function restates the reference Rust code it cites (paths are relative
 * to the talechime repository).  Arithmetic is kept in the reference's types
 * and order: f32 where the reference uses f32, f64 where it uses f64, glibc
 * expf/logf/exp where Rust's f32::exp / f32::ln / f64::exp call the platform
 * libm.  Build with -O2 -fno-fast-math -ffp-contract=off.
 */
#ifndef TC_ORACLE_H
#define TC_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Variants: same numbering as the device library. */
enum {
  TCO_QWEN = 0,      /* crates/qwen3-tts/src/generation/sampling.rs            */
  TCO_COSY_RAS = 1,  /* crates/cosyvoice3/src/llm.rs:517-604                   */
  TCO_INDEXTTS = 2,  /* crates/indextts/src/generation.rs:95-303,640-666       */
  TCO_MOSS = 3,      /* crates/moss-tts/src/sampling.rs:22-85                  */
  TCO_MOSS_NANO = 4  /* crates/moss-tts/src/nano/sampling.rs:96-160            */
};

/* Row status codes (same values as the device library). */
enum {
  TCO_OK = 0,
  TCO_EINVAL = 1,
  TCO_ENONFINITE = 2,
  TCO_ETOOFEW = 3,
  TCO_EDIST = 6
};

/* Per-row flags. */
enum {
  TCO_FLAG_TIE_CUT = 1u,     /* equal values straddle a cut made by an unstable sort */
  TCO_FLAG_RAS = 2u,         /* cosyvoice3: repetition window fired, second uniform used */
  TCO_FLAG_GREEDY = 4u,      /* qwen: temperature < 0.01 took the argmax path */
  TCO_FLAG_NAN_ROW = 8u      /* qwen top-k met a NaN (reference order unspecified) */
};

/* History handling for the penalty stage. */
enum {
  TCO_HIST_PER_ROW = 0,   /* CSR: ids[off[r]..off[r+1]) belong to row r */
  TCO_HIST_BROADCAST = 1, /* qwen apply_repetition_penalty: all ids, flattened, one [1,V] mask */
  TCO_HIST_MASK = 2       /* qwen apply_repetition_penalty_with_mask: f32 [V] mask, >0 = seen */
};

typedef struct tco_params {
  int32_t variant;
  int32_t hist_mode;
  double temperature;      /* qwen: GenerationConfig.temperature (f64); others cast to f32 */
  double top_p;            /* qwen/indextts/moss/nano: f64; cosyvoice3: cast to f32 */
  double penalty;          /* repetition penalty (1.0 = off) */
  uint32_t top_k;          /* 0 = off (qwen, indextts) */
  uint32_t min_keep;       /* indextts min_tokens_to_keep (2 in the reference loop) */
  uint32_t ras_win;        /* cosyvoice3 win_size */
  float ras_tau;           /* cosyvoice3 tau_r */
  int32_t eos_id;          /* qwen: EOS forced to -inf (min_new_tokens); cosyvoice3: ignore_eos id; -1 = none */
  int32_t exclude_id;      /* moss: id forced to -inf; -1 = none */
  int32_t typical;         /* indextts typical warper on/off */
  double typical_mass;
  const float* add_mask;   /* qwen additive suppression mask [V] or NULL */
  const float* pen_mask;   /* qwen penalty mask [V] (hist_mode == MASK) */
} tco_params;

/* Per-row verification outputs (any pointer may be NULL). */
typedef struct tco_verify {
  uint32_t cap;            /* capacity of the id/prob arrays per row */
  uint32_t* topk_count;    /* [rows] size of the top-k survivor set */
  uint32_t* topk_ids;      /* [rows*cap] ascending vocab ids */
  uint32_t* keep_count;    /* [rows] size of the final candidate set */
  uint32_t* keep_ids;      /* [rows*cap] ascending vocab ids */
  float* keep_probs;       /* [rows*cap] probability used by the draw, per kept id */
  float* norm;             /* [rows] indextts log_sum, qwen / cosyvoice3 softmax denominator
                              (NaN where the row has none) */
} tco_verify;

/* ---- RNGs (integer-exact restatements) ---- */
uint64_t tco_qwen_initial_state(uint64_t seed);                 /* sampling.rs:90-93 */
float tco_qwen_rand_f32(uint64_t* state);                        /* sampling.rs:75-85 */
void tco_steprng_new(uint64_t seed, uint64_t* state, uint64_t* inc); /* rng.rs:158-167 */
uint32_t tco_steprng_next_u32(uint64_t* state, uint64_t inc);    /* rng.rs:169-175 */
float tco_steprng_next_f32(uint64_t* state, uint64_t inc);       /* rng.rs:178-180 */
double tco_nano_next_unit(uint32_t* state);                       /* nano/sampling.rs:66-67 */

/* ---- qwen building blocks (crates/qwen3-tts/src/generation) ---- */
void tco_qwen_penalty_ids(float* x, size_t rows, size_t V, const uint32_t* ids, size_t n_ids,
                          double penalty);                          /* sampling.rs:334-360 */
void tco_qwen_penalty_mask(float* x, size_t rows, size_t V, const float* mask,
                           double penalty);                         /* sampling.rs:368-395 */
void tco_qwen_suppression_mask(float* mask, size_t V, uint32_t eos); /* tts.rs:22-41 */
void tco_qwen_add_mask(float* x, size_t rows, size_t V, const float* add); /* tts.rs:44-51 */
void tco_qwen_temperature(float* x, size_t n, double t);           /* sampling.rs:175-184 */
void tco_qwen_top_k(float* row, size_t V, size_t k, uint32_t* flags); /* sampling.rs:224-249 */
void tco_qwen_top_p(float* row, size_t V, double p, uint32_t* flags);  /* sampling.rs:255-299 */
void tco_softmax_last_dim(float* row, size_t V);                   /* candle softmax_last_dim */
int64_t tco_qwen_first_cdf_index(const float* row, size_t V, float thr); /* sampling.rs:319-328 */
uint32_t tco_argmax_f32(const float* row, size_t V);               /* candle argmax */

/* ---- indextts processors (crates/indextts/src/generation.rs) ---- */
void tco_idx_log_softmax(float* row, size_t V);                    /* :95-105 */
void tco_idx_penalty(float* row, size_t V, const uint32_t* ids, size_t n, double pen); /* :122-134 */
void tco_idx_temperature(float* row, size_t V, double t);          /* :137-142 */
void tco_idx_top_k(float* row, size_t V, size_t k, size_t min_keep);  /* :148-161 */
void tco_idx_top_p(float* row, size_t V, double p, size_t min_keep);  /* :169-194 */
void tco_idx_typical(float* row, size_t V, double mass, size_t min_keep); /* :201-248 */
size_t tco_idx_inverse_cdf(const double* w, size_t n, double u);   /* :251-265 */
int tco_idx_sample_wo_replacement(const double* scores, size_t n_scores, size_t n,
                                  const double* uniforms, size_t* out); /* :280-303 */
/* one beam-sample step (:640-701): per element of nb beam rows, the joint
 * scores, n_draws draws without replacement, candidates sorted descending */
int tco_idx_beam_step(const tco_params* p, const float* logits, size_t batch, size_t nb, size_t V,
                      const uint32_t* hist_off, const uint32_t* hist_ids, const double* beam_scores,
                      const double* uniforms, size_t n_draws, uint32_t* cand_flat, double* cand_scores,
                      int32_t* status);
/* generation.rs:671-679 (do_sample = false): the n_keep best joint scores per
 * element, descending, equal scores in ascending flat order. */
int tco_idx_beam_search_step(const tco_params* p, const float* logits, size_t batch, size_t nb, size_t V,
                             const uint32_t* hist_off, const uint32_t* hist_ids, const double* beam_scores,
                             size_t n_keep, uint32_t* cand_flat, double* cand_scores);

/* ---- cosyvoice3 (crates/cosyvoice3/src/llm.rs) ---- */
uint32_t tco_cosy_nucleus(const float* probs, size_t V, float top_p, size_t top_k, float u0,
                          int* used_u0, uint32_t* cand_ids, float* cand_p, uint32_t* n_cands); /* :556-592 */
uint32_t tco_cosy_random(const float* probs, size_t V, float u1);  /* :594-604 */

/* ---- full per-row pipelines ----
 * logits: [rows, V] f32 (a bf16 input is upcast exactly by the caller).
 * hist_off/hist_ids: CSR per-row histories (hist_mode PER_ROW), or hist_ids with
 *   n = hist_off[1] for BROADCAST.
 * uniforms: qwen/cosyvoice3 f32 (1 resp. 2 per row); indextts/moss/nano f64 (1 per row).
 * out_ids[rows], out_status[rows], out_flags[rows].
 * nthreads: >1 samples rows in parallel (rows are independent given their uniforms).
 * Returns 0, or TCO_EINVAL for parameters the reference rejects up front.
 */
int tco_sample(const tco_params* p, const float* logits, size_t rows, size_t V,
               const uint32_t* hist_off, const uint32_t* hist_ids, const void* uniforms,
               uint32_t* out_ids, int32_t* out_status, uint32_t* out_flags,
               const tco_verify* verify, int nthreads);

#ifdef __cplusplus
}
#endif
#endif
