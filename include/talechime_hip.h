/*
 * talechime_hip.h -- C ABI of the MI355X (gfx950) per-step token sampler.
 *
 * Drop-in device implementation of talechime's logits-processing stage that
 * follows the LM head in its autoregressive TTS crates: repetition penalty,
 * temperature, top-k, top-p and an inverse-CDF draw over caller-supplied
 * uniforms, with the arithmetic of each crate's own sampler (see
 * tc_variant).  Plain pointers and sizes only; every pointer named d_* is
 * device memory owned by the caller and never freed by the library.  All
 * calls are asynchronous on the given HIP stream (NULL = default stream)
 * unless stated otherwise.
 *
 * Reference interfaces replaced (paths relative to the talechime repository):
 *   tc_sample (TC_QWEN)      crates/qwen3-tts/src/generation/sampling.rs:137 `sample`
 *                            (with the caller chain of synthesis.rs:1228-1279 folded in:
 *                            penalty mask, additive suppression mask, min-new-token EOS)
 *   tc_sample (TC_COSY_RAS)  crates/cosyvoice3/src/llm.rs:517 `CosyVoice3Lm::sample`
 *   tc_sample (TC_INDEXTTS)  crates/indextts/src/generation.rs:643-676, the processors
 *                            (log_softmax, apply_repetition_penalty, apply_temperature,
 *                            apply_top_k, apply_top_p) then sample_without_replacement
 *                            (generation.rs:280) with one draw per row
 *   tc_indextts_beam_step    crates/indextts/src/generation.rs:640-701, the joint scores
 *                            and sample_without_replacement of the beam-sample loop
 *   tc_indextts_beam_search_step  generation.rs:671-679, the same loop with do_sample false
 *   tc_lm_head / tc_head_sample    the Linear before the sampler (generation.rs:632,
 *                            code_predictor.rs:208-216), alone and with the sampler
 *   tc_sample (TC_MOSS)      crates/moss-tts/src/sampling.rs:22 `sample`
 *   tc_sample (TC_MOSS_NANO) crates/moss-tts/src/nano/sampling.rs:11 `Sampler::sample`
 *   tc_apply_repetition_penalty            sampling.rs:334
 *   tc_apply_repetition_penalty_with_mask  sampling.rs:368
 *   tc_greedy_sample                       sampling.rs:398
 *   tc_build_suppression_mask              crates/qwen3-tts/src/generation/tts.rs:22
 *   tc_apply_token_suppression_with_mask   tts.rs:44
 *   tc_update_penalty_mask                 crates/qwen3-tts/src/synthesis.rs:568
 *                                          (also fused into tc_sample: d_mark_mask)
 */
#ifndef TALECHIME_HIP_H
#define TALECHIME_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TC_ABI_VERSION 3

typedef struct tc_ctx tc_ctx;
typedef void* tc_stream; /* a hipStream_t */

/* Status codes.  Row-level outcomes are written per row to d_out_status. */
enum tc_status {
  TC_OK = 0,
  TC_EINVAL = 1,       /* bad argument; mirrors llm.rs:436-445, generation.rs:559-571,
                          nano "invalid repetition token" */
  TC_ENONFINITE = 2,   /* moss / nano: non-finite logits (sampling.rs:51-54, nano:24-27) */
  TC_ETOOFEW = 3,      /* indextts: fewer finite candidates than draws (generation.rs:284-286) */
  TC_EHIP = 4,         /* a HIP runtime call failed */
  TC_ENOMEM = 5,       /* device allocation failed */
  TC_EDIST = 6,        /* nano: no token reached by the draw (nano:74) */
  TC_EUNSUPPORTED = 7  /* this library does not implement the requested shape/option */
};

/* Sampler arithmetic to reproduce. */
enum tc_variant {
  TC_QWEN = 0,
  TC_COSY_RAS = 1,
  TC_INDEXTTS = 2,
  TC_MOSS = 3,
  TC_MOSS_NANO = 4
};

enum tc_dtype { TC_F32 = 0, TC_BF16 = 1 };

/* How d_hist_off / d_hist_ids are read. */
enum tc_hist_mode {
  TC_HIST_PER_ROW = 0,   /* CSR: row r owns ids[off[r] .. off[r+1]) */
  TC_HIST_BROADCAST = 1, /* qwen apply_repetition_penalty: ids[off[0] .. off[1]) mark one
                            [1,V] mask applied to every row */
  TC_HIST_MASK = 2       /* qwen apply_repetition_penalty_with_mask: params.d_pen_mask [V],
                            entries > 0 are penalised */
};

/* Per-row flag bits written to d_out_flags. */
enum tc_flag {
  TC_FLAG_TIE_CUT = 1u,  /* equal values straddle a cut the reference makes with an
                            unstable sort (qwen top-p, moss top-k/top-p); ties are broken
                            by ascending id here */
  TC_FLAG_RAS = 2u,      /* cosyvoice3: the repetition window fired and the second
                            uniform was used (the reference's StepRng advanced twice) */
  TC_FLAG_GREEDY = 4u,   /* qwen: temperature < 0.01, argmax, no uniform used */
  TC_FLAG_NAN_ROW = 8u,  /* qwen: NaN met at top-k (reference order unspecified) */
  TC_FLAG_NEAR_TIE = 16u, /* indextts: a top-p, draw or typical-warper decision lay
                            within the error of this library's f64 exp and sums
                            against the reference's (about 2^-46 relative); the id
                            follows this library's arithmetic */
  TC_FLAG_EXACT_SUM = 32u /* indextts without verification outputs: the row's decisions
                             were not settled by the interval on the log-sum and took the
                             exact sequential sum (informational; the id is the same) */
};

typedef struct tc_sample_params {
  int32_t variant;          /* tc_variant */
  int32_t hist_mode;        /* tc_hist_mode */
  double temperature;       /* qwen: GenerationConfig.temperature; others use (float) */
  double top_p;             /* cosyvoice3 uses (float) */
  double repetition_penalty;/* 1.0 = off */
  uint32_t top_k;           /* qwen / indextts: 0 = off; cosyvoice3 / moss / nano: >= 1 */
  uint32_t min_keep;        /* indextts min_tokens_to_keep (the reference loop passes 2) */
  uint32_t ras_win;         /* cosyvoice3 win_size */
  float ras_tau;            /* cosyvoice3 tau_r */
  int32_t eos_id;           /* qwen: forced to -inf (token_count < min_new_tokens);
                               cosyvoice3: the ignore_eos mask id; -1 = none */
  int32_t exclude_id;       /* moss: forced to -inf; -1 = none */
  const float* d_add_mask;  /* qwen: additive [V] mask (suppression), or NULL */
  const float* d_pen_mask;  /* qwen: [V] penalty mask for TC_HIST_MASK */
  float* d_mark_mask;       /* optional [V] f32: each row sampled with TC_OK sets
                               d_mark_mask[id] = 1.0 (synthesis.rs:568-579
                               update_penalty_mask fused into the step; ids >= V are
                               ignored).  May equal d_pen_mask only when rows == 1:
                               the row reads the mask before it marks it.  NULL = off */
  int32_t typical;          /* indextts: GenerateConfig.typical_sampling (generation.rs:649-651,
                               apply_typical :196-248); 0 = off.  ABI version 3 */
  double typical_mass;      /* indextts: GenerateConfig.typical_mass, in (0, 1) when typical */
} tc_sample_params;

/* Optional verification outputs (device pointers; pass NULL to skip).  Ids are
 * ascending; keep_probs holds the probability the draw used for each kept id
 * (f64 variants are rounded to float).  Counts are exact even when > cap.
 * d_norm (may be NULL) receives the row's normaliser: the log-sum of the
 * indextts log_softmax, the softmax denominator for qwen and cosyvoice3, NaN
 * where the row has none. */
typedef struct tc_verify_out {
  uint32_t cap;
  uint32_t* d_topk_count;  /* [rows] */
  uint32_t* d_topk_ids;    /* [rows * cap] survivors of the top-k stage */
  uint32_t* d_keep_count;  /* [rows] */
  uint32_t* d_keep_ids;    /* [rows * cap] final candidates */
  float* d_keep_probs;     /* [rows * cap] */
  float* d_norm;           /* [rows] */
} tc_verify_out;

/* Create a context on `device` for batches up to max_rows x max_vocab.  The
 * context owns the library's device workspace (its only allocation). */
int tc_create(int device, size_t max_rows, size_t max_vocab, tc_ctx** out);
void tc_destroy(tc_ctx* ctx);

/*
 * One sampler step over `rows` independent rows.
 *   d_logits   [rows, ld] f32 or bf16 (bf16 is widened exactly, like to_dtype(F32))
 *   d_hist_off [rows + 1] u32, d_hist_ids u32 (see tc_hist_mode; may be NULL when the
 *              variant needs no history)
 *   d_uniforms per row: qwen 1 f32; cosyvoice3 2 f32 (u0 nucleus, u1 fallback);
 *              indextts, moss, nano 1 f64 (nano: (state >> 8) / 2^24 of its LCG)
 *   d_out_ids [rows] u32; d_out_status [rows] i32 (tc_status); d_out_flags [rows] u32
 * Returns TC_OK once the work is enqueued, or an error for arguments the reference
 * rejects before sampling (row-level errors go to d_out_status).
 */
int tc_sample(tc_ctx* ctx, const tc_sample_params* params, const void* d_logits, int dtype,
              size_t rows, size_t vocab, size_t ld, const uint32_t* d_hist_off,
              const uint32_t* d_hist_ids, const void* d_uniforms, uint32_t* d_out_ids,
              int32_t* d_out_status, uint32_t* d_out_flags, const tc_verify_out* verify,
              tc_stream stream);

/*
 * One indextts beam-sample step (crates/indextts/src/generation.rs:640-701 after the
 * logits: the processors of each beam row (643-662), the joint beam-major scores
 * score + beam score in f64 (663-664), sample_without_replacement with n_draws
 * draws per batch element (680, 280-303), candidates sorted by score descending,
 * stable (690)).  Replaces the `joint` / `candidates` computation of that loop;
 * BeamSearchScorer::process (generation.rs:386-440) consumes the candidates.
 *   d_logits      [batch * num_beams, ld]; row bi * num_beams + j is beam j of element bi
 *   d_hist_off/ids CSR histories per row (the beam's input ids), as tc_sample
 *   d_beam_scores [batch * num_beams] f64 running beam scores
 *   d_uniforms    [batch * n_draws] f64, element bi's draws at bi * n_draws (the
 *                 reference's rng.random::<f64>() calls in order); n_draws is
 *                 2 * num_beams in the reference (generation.rs:620), at most 64
 *   d_cand_flat   [batch * n_draws] u32 flat index beam * vocab + id
 *   d_cand_scores [batch * n_draws] f64 joint scores, descending
 *   d_out_status  [batch] i32: TC_ETOOFEW when fewer than n_draws joint scores are
 *                 finite (generation.rs:284-286); d_out_flags [batch] (may be NULL):
 *                 TC_FLAG_NEAR_TIE when a top-p or draw decision lay within the f64
 *                 exp error of the reference's libm
 * num_beams <= 64, num_beams * vocab < 2^32, batch * num_beams <= the context's
 * max_rows; at most 1024 kept ids per row and 4096 per element (else
 * TC_EUNSUPPORTED in d_out_status).  The context's first beam step allocates its
 * row-pass workspace (16 KiB per max_rows row): make one call before capturing
 * a graph.  params->variant must be TC_INDEXTTS; d_mark_mask is ignored.
 */
int tc_indextts_beam_step(tc_ctx* ctx, const tc_sample_params* params, const void* d_logits, int dtype,
                          size_t batch, size_t num_beams, size_t vocab, size_t ld,
                          const uint32_t* d_hist_off, const uint32_t* d_hist_ids,
                          const double* d_beam_scores, const double* d_uniforms, size_t n_draws,
                          uint32_t* d_cand_flat, double* d_cand_scores, int32_t* d_out_status,
                          uint32_t* d_out_flags, tc_stream stream);

/*
 * The same loop without sampling (GenerateConfig.do_sample = false): the beam-search
 * branch of crates/indextts/src/generation.rs:671-679.  Each beam row keeps
 * log_softmax and the repetition penalty only (the temperature, top-k and top-p of
 * params are not applied, generation.rs:653-662); the candidates are the n_keep best
 * joint scores score + beam score of each element over all num_beams * vocab flat
 * indices, by score descending, equal scores in ascending flat order (the
 * reference's stable sorts).  n_keep is 2 * num_beams in the reference, at most 64.
 * d_cand_flat / d_cand_scores [batch * n_keep]; d_out_status [batch].  Shares the
 * context's beam workspace with tc_indextts_beam_step.
 */
int tc_indextts_beam_search_step(tc_ctx* ctx, const tc_sample_params* params, const void* d_logits, int dtype,
                                 size_t batch, size_t num_beams, size_t vocab, size_t ld,
                                 const uint32_t* d_hist_off, const uint32_t* d_hist_ids,
                                 const double* d_beam_scores, size_t n_keep, uint32_t* d_cand_flat,
                                 double* d_cand_scores, int32_t* d_out_status, tc_stream stream);

/*
 * tc_indextts_beam_step without any allocation.  No counterpart in the reference:
 * this entry point is for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * Same arguments, results and row-level statuses as tc_indextts_beam_step, on the
 * current device and without a context.  The row-pass workspace is a file-scope
 * device array sized for batch * num_beams <= TC_NOALLOC_BEAM_ROWS (4.2 MB per GPU,
 * held until the process ends); larger calls return TC_EINVAL, vocabularies above
 * 16384 TC_EUNSUPPORTED.  Every call on one GPU shares that array: calls that
 * overlap on one GPU (different streams, or threads without ordering) race.  The
 * first call on a device (or tc_create on it) resolves the array's address.
 */
#define TC_NOALLOC_BEAM_ROWS 256
int tc_indextts_beam_step_noalloc(const tc_sample_params* params, const void* d_logits, int dtype,
                                  size_t batch, size_t num_beams, size_t vocab, size_t ld,
                                  const uint32_t* d_hist_off, const uint32_t* d_hist_ids,
                                  const double* d_beam_scores, const double* d_uniforms,
                                  size_t n_draws, uint32_t* d_cand_flat, double* d_cand_scores,
                                  int32_t* d_out_status, uint32_t* d_out_flags, tc_stream stream);

/*
 * The LM head that feeds the sampler: logits[r] = weight . hidden[r] + bias, the
 * candle Linear of crates/indextts/src/generation.rs:632 (mel_head, 1280 -> 8194,
 * with a bias, :981) and of the qwen3-tts code predictor's lm_heads
 * (crates/qwen3-tts/src/models/code_predictor.rs:208-216, no bias).
 *   d_hidden [rows, hidden_ld] f32; d_weight [vocab, dim] f32 or bf16 (tc_dtype),
 *   16-byte aligned, rows of dim elements; d_bias [vocab] f32 or NULL;
 *   d_logits [rows, logits_ld] f32.  dim a multiple of 8 (bf16) or 4 (f32), at most
 *   4096 (bf16) or 2048 (f32).  f32 accumulation; the summation order is this
 *   library's (the reference's matmul has its own), so the logits agree with an
 *   exact product to within rounding, not bit for bit.
 */
int tc_lm_head(const float* d_hidden, size_t hidden_ld, const void* d_weight, int w_dtype, const float* d_bias,
               size_t rows, size_t dim, size_t vocab, float* d_logits, size_t logits_ld, tc_stream stream);

/*
 * tc_lm_head then tc_sample on its logits, in one call on one stream: the head's
 * output stays on the device (d_logits, [rows, vocab] f32, caller-owned) and the
 * sampler reads it back from the cache.  Replaces the head + sample pair of one AR
 * step (generation.rs:628-662; code_predictor.rs with sampling.rs:137).
 * Arguments as tc_lm_head and tc_sample (no verification outputs).
 */
int tc_head_sample(tc_ctx* ctx, const tc_sample_params* params, const float* d_hidden, size_t hidden_ld,
                   const void* d_weight, int w_dtype, const float* d_bias, size_t rows, size_t dim, size_t vocab,
                   float* d_logits, const uint32_t* d_hist_off, const uint32_t* d_hist_ids,
                   const void* d_uniforms, uint32_t* d_out_ids, int32_t* d_out_status, uint32_t* d_out_flags,
                   tc_stream stream);

/* qwen building blocks on f32 [rows, ld] (d_in may equal d_out).
 * tc_apply_repetition_penalty builds its [V] mask in the context's workspace. */
int tc_apply_repetition_penalty(tc_ctx* ctx, const float* d_in, float* d_out, size_t rows, size_t vocab,
                                size_t ld, const uint32_t* d_ids, size_t n_ids, double penalty,
                                tc_stream stream);
int tc_apply_repetition_penalty_with_mask(const float* d_in, float* d_out, size_t rows,
                                          size_t vocab, size_t ld, const float* d_mask,
                                          double penalty, tc_stream stream);
int tc_build_suppression_mask(float* d_mask, size_t vocab, uint32_t eos_id, tc_stream stream);
int tc_apply_token_suppression_with_mask(const float* d_in, float* d_out, size_t rows,
                                         size_t vocab, size_t ld, const float* d_mask,
                                         tc_stream stream);
/* mask[token] = 1 when token < vocab; the token is read on the device. */
int tc_update_penalty_mask(float* d_mask, size_t vocab, const uint32_t* d_token,
                           tc_stream stream);
int tc_greedy_sample(const void* d_logits, int dtype, size_t rows, size_t vocab, size_t ld,
                     uint32_t* d_out_ids, tc_stream stream);

/* Thread-local description of the last error returned on this thread. */
const char* tc_last_error(void);
int tc_abi_version(void);

#ifdef __cplusplus
}
#endif
#endif /* TALECHIME_HIP_H */
