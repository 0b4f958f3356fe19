/*
 * ax_oracle.h — CPU restatement of AX Engine's per-step sampling law.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker for the HIP
 * sampler: only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg load it, and never as the thing measured or shipped.
 *
 * It restates, line by line, the reference's Rust CPU sampler
 * (crates/ax-engine-mlx/src/sampling.rs), its MTP acceptance law
 * (crates/ax-engine-mlx/src/runner/mod.rs:12333-12462) and the core
 * DeterministicSampler (crates/ax-engine-core/src/sampling.rs:94-191).
 * Built with gcc -ffp-contract=off and no fast-math: every f32 operation is
 * one IEEE single-precision operation in the reference's order, and expf /
 * logf are glibc's, which is what Rust's f32::exp / f32::ln call on Linux.
 * The reference itself (Rust) cannot be built in this image.
 */
#ifndef AX_ORACLE_H
#define AX_ORACLE_H

#include <stdint.h>
#include "../include/ax_hip_sampler.h"

#ifdef __cplusplus
extern "C" {
#endif

/* path taken by axo_sample_row */
#define AXO_PATH_EMPTY     0  /* V == 0 → token 0 (sampling.rs:213-215)          */
#define AXO_PATH_GREEDY    1  /* temperature <= 0 → argmax (sampling.rs:236-238)  */
#define AXO_PATH_FALLBACK  2  /* zero mass / empty min-p set → argmax             */
#define AXO_PATH_FAST      3  /* index-order draw over all V (sampling.rs:246-270) */
#define AXO_PATH_FILTERED  4  /* candidates path (sampling.rs:273-316)            */

typedef struct axo_explain {
    uint32_t token;
    uint32_t path;
    uint32_t drew;        /* a uniform was consumed                         */
    uint32_t sorted;      /* draw order is (p desc, id asc)                 */
    uint32_t n_cand;      /* candidates after min-p                         */
    uint32_t n_nucleus;   /* keep count after top-p (before top-k)          */
    uint32_t n_kept;      /* kept set size                                  */
    uint32_t boundary;    /* AXS_FLAG_NEAR_* bits                           */
    float    m;           /* max logit after processors                     */
    float    total;       /* sorted total mass used by top-p                */
    float    cutoff;      /* top_p * total                                  */
    float    F;           /* filtered sum (S on the fast path)              */
    float    u;
    float    thr;
    float    logprob;     /* max(ln(p/F), -30) of the drawn token           */
    float    pad0;
    double   margin_draw;     /* min distance of u*F to the bracketing cums / F  */
    double   margin_nucleus;  /* same for top_p*total, / total                   */
    double   margin_minp;     /* min |p - cutoff| / cutoff                       */
    double   margin_tie;      /* |p_a - p_b| / ulp across the kept cut           */
} axo_explain;

/* ---- RNGs --------------------------------------------------------------- */
/* Xorshift64 (crates/ax-engine-mlx/src/sampling.rs:15-37) */
uint64_t axo_xorshift64_new(uint64_t seed);
uint64_t axo_xorshift64_next_u64(uint64_t* state);
float    axo_xorshift64_next_f32(uint64_t* state);

/* Philox4x32-10 (Salmon, Moraes, Dror, Shaw, SC'11) */
void  axo_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]);
/* uniform = (word >> 8) * 2^-24 of Philox(ctr = (row, step_lo, step_hi, purpose),
 * key = (seed_lo, seed_hi)), word index `word` in 0..3 */
float axo_philox_uniform(uint64_t seed, uint32_t row, uint64_t step,
                         uint32_t purpose, uint32_t word);

/* ---- single-row law ----------------------------------------------------- */
/* argmax_index_f32 / argmax_f32 (sampling.rs:954-970) */
uint32_t axo_argmax_f32(const float* logits, uint32_t n);

/* Applies the processors to `row` in place (repetition sampling.rs:875-894,
 * n-gram :896-920, the build extensions, in the documented order).  Returns 1
 * if anything was applied. */
int axo_apply_processors(float* row, uint32_t V, const axs_sampling_params* p,
                         const uint32_t* hist, uint32_t nhist,
                         const uint32_t* mask_words,
                         const uint32_t* bias_ids, const float* bias_vals,
                         uint32_t nbias);

/* sample_categorical_into (sampling.rs:204-316).  The uniform comes from
 * `u_supplied` if non-NULL, else from the Xorshift64 `rng` (which must then be
 * non-NULL); it is consumed only when the row draws.  `explain`, `kept_ids`
 * are optional.  Returns the token id. */
uint32_t axo_sample_row(const float* logits, uint32_t V,
                        const axs_sampling_params* p,
                        const uint32_t* hist, uint32_t nhist,
                        const uint32_t* mask_words,
                        const uint32_t* bias_ids, const float* bias_vals,
                        uint32_t nbias,
                        const float* u_supplied, uint64_t* rng,
                        axo_explain* explain,
                        uint32_t* kept_ids, uint32_t kept_cap);

/* Batched wrapper (sample_batched_host, batched_sampling.rs:123-149) over a
 * [B, stride] host array of dtype AXS_DTYPE_*; rows split over `nthreads`
 * POSIX threads (1 = the reference's serial loop).  uniforms == NULL →
 * Philox(seed, row, step, purpose 0, word 0). */
int axo_sample_batch(const void* logits, int dtype, uint32_t B, uint32_t V,
                     uint64_t stride, const axs_sampling_params* params,
                     const uint32_t* hist, const int64_t* hist_off,
                     const uint32_t* mask_words, uint64_t mask_stride,
                     const uint32_t* bias_ids, const float* bias_vals,
                     const int64_t* bias_off, const float* uniforms,
                     uint32_t* out_ids, axo_explain* explain,
                     uint32_t* kept_ids, uint32_t kept_cap, int nthreads);

/* token_distribution (sampling.rs:647-707): writes up to `cap` entries,
 * returns the entry count (-1 = None, -2 = more than cap). */
int axo_token_distribution(const float* logits, uint32_t V,
                           const axs_sampling_params* p,
                           uint32_t* ids, float* probs, uint32_t cap);

/* TokenDistribution::new (sampling.rs:128-144) in place; returns the entry
 * count, -1 for None. */
int axo_distribution_new(uint32_t* ids, float* probs, uint32_t n);

/* sample_from_token_distribution (sampling.rs:709-731); returns AXS_NONE_U32
 * for None. */
uint32_t axo_sample_from_distribution(const uint32_t* ids, const float* probs,
                                      uint32_t n, float u);

/* sample_residual_token_distribution (sampling.rs:733-752) */
uint32_t axo_sample_residual(const uint32_t* t_ids, const float* t_probs, uint32_t tn,
                             const uint32_t* d_ids, const float* d_probs, uint32_t dn,
                             float u);

/* TokenDistribution::probability + sample_with_logprob's log (sampling.rs:147-160) */
float axo_distribution_prob(const uint32_t* ids, const float* probs, uint32_t n,
                            uint32_t token);
float axo_logprob_of(float prob);

/* full_vocab_token_logprob (sampling.rs:761-787) */
float axo_full_vocab_token_logprob(const float* logits, uint32_t n, uint32_t token,
                                   float temperature);

/* mtp_accept_count (crates/ax-engine-mlx/src/runner/mod.rs:12333-12462).
 * Distributions in CSR form (ids/probs/offsets, `ndist` entries, NULL = none).
 * sources: 0 None, 1 Mtp, 2 Gemma4Assistant, 3 Ngram, 4 HybridMtp
 * (runner/mtp_routing.rs:15-31); model_mode: 0 Greedy, 1 RejectionSampling;
 * ngram_mode: 0 Confidence, 1 Delta, 2 Greedy.  Uniforms come from `rng`
 * (Xorshift64) if non-NULL else from `uniforms` in consumption order.
 * Returns accept_count; *all_accepted, *correction (AXS_NONE_U32 = None). */
uint32_t axo_mtp_accept_count(uint32_t n, const uint32_t* pending,
                              const float* pending_log_probs, uint32_t n_log_probs,
                              const uint32_t* d_ids, const float* d_probs,
                              const int64_t* d_off, uint32_t n_draft_dists,
                              const uint32_t* sources, uint32_t n_sources,
                              const float* target_probs,
                              const uint32_t* t_ids, const float* t_probs,
                              const int64_t* t_off, uint32_t n_target_dists,
                              const uint32_t* predicted,
                              uint64_t* rng, const float* uniforms, uint32_t n_uniforms,
                              float draft_temperature, float target_temperature,
                              int model_mode, int ngram_mode,
                              uint32_t* all_accepted, uint32_t* correction);

/* One MTP verify step for one sequence (the composite law of axs_mtp_verify):
 * target rows [depth+1][V], draft rows [depth][V] (f32), uniforms[depth+1].
 * Writes out_ids[depth+1]; returns out_count; *accept_count, *flags. */
uint32_t axo_mtp_verify_seq(const float* target, const float* draft, uint32_t V,
                            uint32_t depth, const uint32_t* draft_ids,
                            const axs_sampling_params* tparams,
                            const axs_sampling_params* dparams,
                            const float* uniforms, uint32_t* out_ids,
                            uint32_t* accept_count, uint32_t* flags);

/* Batched MTP verify over [B, depth+1, stride] / [B, depth, stride] host logits
 * (dtype AXS_DTYPE_*); uniforms [B, depth+1] or NULL → Philox. */
int axo_mtp_verify_batch(const void* target, const void* draft, int dtype,
                         uint32_t B, uint32_t depth, uint32_t V, uint64_t stride,
                         const uint32_t* draft_ids,
                         const axs_sampling_params* tparams,
                         const axs_sampling_params* dparams,
                         const float* uniforms, uint32_t* out_ids,
                         uint32_t* out_count, uint32_t* accept_count,
                         uint32_t* flags, int nthreads);

/* DeterministicSampler row (crates/ax-engine-core/src/sampling.rs:97-191):
 * returns 1 and (token, logprob) for valid logits, 0 for invalid (None). */
int axo_core_argmax_logprob(const float* logits, uint32_t n,
                            const axs_sampling_params* p,
                            const uint32_t* recent, uint32_t nrecent,
                            uint32_t* token, float* logprob);

/* bf16 → f32 widening (exact) */
void axo_bf16_to_f32(const uint16_t* in, float* out, uint64_t n);

#ifdef __cplusplus
}
#endif

#endif /* AX_ORACLE_H */
