/*
 * ax_hip_sampler.h — C ABI of the MI355X (gfx950) per-step token sampler.
 *
 * This is the boundary a `hip-sys` crate binds, as a sibling of the
 * reference's `crates/mlx-sys` (plain C header, opaque context handle,
 * `int` status codes, thread-local last-error string:
 * crates/mlx-sys/native/ax_shim.h:24-40,106-110 and
 * crates/mlx-sys/native/ax_shim.cpp:47-57 in the reference).
 *
 * Conventions
 *   - Every entry point returns AXS_OK (0) or a nonzero AXS_E_* code; the
 *     message of the last failure on the calling thread is returned by
 *     axs_last_error().  A caller that gets a nonzero status falls back to
 *     its CPU sampler, as the reference's GPU helpers decline with `None`
 *     (crates/ax-engine-mlx/src/generate.rs:221-238).
 *   - Every array pointer in the *_desc / *_outputs structs is a DEVICE
 *     pointer (HBM), borrowed for the duration of the call.  Outputs are
 *     caller-allocated.  `stream` is a hipStream_t passed as void* (NULL =
 *     the null stream); all work is enqueued on it and the call returns
 *     without synchronising.
 *   - No torch or HIP types appear in the signatures.
 *   - A context may be shared by threads: its calls are serialised (a lock
 *     around each call's enqueue), and a call on another stream than the
 *     previous call's first waits for the work enqueued on that stream (an
 *     event recorded there), so the context's workspace is never used by two
 *     streams at once; that previous stream must still exist.  Consecutive
 *     calls on one stream add no event.  One context per thread avoids the
 *     waiting.
 */
#ifndef AX_HIP_SAMPLER_H
#define AX_HIP_SAMPLER_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define AXS_ABI_VERSION 2

/* status codes */
#define AXS_OK            0
#define AXS_E_INVALID     1   /* bad argument (shape, pointer, size) */
#define AXS_E_HIP         2   /* HIP runtime error */
#define AXS_E_CAPACITY    3   /* larger than the context was created for */
#define AXS_E_UNSUPPORTED 4

/* logits element types; bf16 is widened exactly to f32 before any arithmetic,
 * as production casts the lm_head output to f32 before sampling
 * (crates/ax-engine-mlx/src/model/mod.rs:1771-1774). */
#define AXS_DTYPE_F32  0
#define AXS_DTYPE_BF16 1

#define AXS_NONE_U32 0xFFFFFFFFu

/*
 * Per-row sampling parameters.  Mirrors MlxSamplingParams
 * (crates/ax-engine-mlx/src/sampling.rs:39-114) and the core SamplingParams
 * (crates/ax-engine-core/src/sampling.rs:7-41); the activity predicates are
 * the reference's:
 *   repetition penalty active iff finite, > 0 and != 1      (sampling.rs:91-95)
 *   min-p active iff has_min_p and min_p finite and > 0     (sampling.rs:86-89)
 *   no-repeat n-gram active iff no_repeat_ngram_size > 0    (sampling.rs:107-109)
 * presence_penalty, frequency_penalty, and the logit bias / allowed-token mask
 * of axs_batch_desc do not exist in the reference (its OpenAI route rejects
 * them: crates/ax-engine-server/src/openai/requests.rs:1240-1281); their
 * semantics here are build-defined (OpenAI convention):
 *   for each id t < V with count c > 0 in the repetition window:
 *       l = l - frequency_penalty * (float)c;  l = l - presence_penalty;
 *   then l += bias (each listed entry, in list order), then masked ids -> -inf.
 * Processor order: repetition -> presence/frequency -> bias -> mask -> n-gram
 * ban -> temperature.  Sizeof = 64 bytes.
 */
typedef struct axs_sampling_params {
    float    temperature;             /* <= 0: greedy argmax                  */
    float    top_p;                   /* >= 1: no nucleus truncation          */
    uint32_t top_k;                   /* 0: no top-k truncation               */
    float    min_p;                   /* read only when has_min_p != 0        */
    uint32_t has_min_p;               /* Option<f32> discriminant             */
    float    repetition_penalty;      /* 1.0: off                             */
    uint32_t repetition_context_size; /* AXS_NONE_U32: whole history          */
    uint32_t no_repeat_ngram_size;    /* 0: off                               */
    uint32_t ngram_window;            /* reference default 128                */
    float    presence_penalty;        /* build extension, 0: off              */
    float    frequency_penalty;       /* build extension, 0: off              */
    uint32_t reserved0;
    uint64_t seed;                    /* Philox key when no uniforms supplied */
    uint64_t step;                    /* Philox counter (decode step)         */
} axs_sampling_params;

/*
 * One batched sampling step.  Replaces, for a [B, V] logits tensor already in
 * HBM, the host readback + serial per-row loop of sample_batched_host
 * (crates/ax-engine-mlx/src/batched_sampling.rs:123-149) and
 * resolve_batched_group_tokens (crates/ax-engine-mlx/src/runner/mod.rs:3132-3210),
 * each row following sample_categorical_into
 * (crates/ax-engine-mlx/src/sampling.rs:204-316).
 */
typedef struct axs_batch_desc {
    const void*     logits;          /* [batch, row_stride] of dtype            */
    int32_t         dtype;           /* AXS_DTYPE_*                             */
    int32_t         batch;
    int32_t         vocab;
    int32_t         reserved0;
    int64_t         row_stride;      /* elements between rows (>= vocab)        */
    const axs_sampling_params* params;   /* [batch]                             */
    /* Token history (prompt + generated tail, oldest first) in CSR form, the
     * `repetition_tokens` slice of sample_categorical_into.  NULL = none. */
    const uint32_t* history;         /* [history_len]                           */
    const int64_t*  history_offsets; /* [batch + 1]                             */
    int64_t         history_len;
    /* Allowed-token bitmask (build extension): bit (t & 31) of word t >> 5,
     * LSB = lowest id; 0 = disallowed.  NULL = all allowed. */
    const uint32_t* mask_words;      /* [batch, mask_stride]                    */
    int64_t         mask_stride;     /* u32 words per row, >= ceil(vocab / 32)  */
    /* Sparse logit bias (build extension) in CSR form.  NULL = none. */
    const uint32_t* bias_ids;        /* [bias_len]                              */
    const float*    bias_values;     /* [bias_len], finite                      */
    const int64_t*  bias_offsets;    /* [batch + 1]                             */
    int64_t         bias_len;
    /* Supplied uniforms in [0, 1], one per row, consumed only when the row
     * draws.  NULL = Philox4x32-10 with key = params.seed, counter =
     * (row, step_lo, step_hi, 0), uniform = (word0 >> 8) * 2^-24. */
    const float*    uniforms;        /* [batch]                                 */
} axs_batch_desc;

/* per-row flag bits written to axs_outputs.flags */
#define AXS_FLAG_GREEDY          (1u << 0)  /* temperature <= 0: argmax          */
#define AXS_FLAG_ARGMAX_FALLBACK (1u << 1)  /* zero / non-finite mass or empty
                                               min-p set: argmax (sampling.rs:265,281,292,299) */
#define AXS_FLAG_DREW            (1u << 2)  /* a uniform was consumed            */
#define AXS_FLAG_EXACT_PATH      (1u << 3)  /* row resolved by the exact
                                               ordered-sum path (second pass)     */
#define AXS_FLAG_NEAR_DRAW       (1u << 4)  /* |cum - u*F| < 1e-6 F at the draw  */
#define AXS_FLAG_NEAR_NUCLEUS    (1u << 5)  /* |cum - top_p*total| < 1e-6 total  */
#define AXS_FLAG_NEAR_MINP       (1u << 6)  /* |p - min_p| < 1e-6 min_p          */
#define AXS_FLAG_NEAR_TIE        (1u << 7)  /* p within 2 ulp across the top-k cut */
#define AXS_FLAG_CAPACITY        (1u << 8)  /* with AXS_FLAG_ERROR: the row has more
                                               bias entries than the kernel holds
                                               (AXS_BIAS_ROW_MAX / AXS_BIAS_SEG_MAX) */
#define AXS_FLAG_ERROR           (1u << 31) /* invalid row input, or a capacity
                                               refusal (AXS_FLAG_CAPACITY): token 0 */

/* Logit-bias capacity.  Batches of 2 rows or more: up to AXS_BIAS_ROW_MAX
 * entries per row.  A batch of one row is cut into segments of at most
 * 65,536 ids, each holding up to AXS_BIAS_SEG_MAX entries: any row of up to
 * AXS_BIAS_SEG_MAX entries is accepted, a longer one when its entries spread
 * over the segments.  A row beyond these gets token 0 with AXS_FLAG_ERROR |
 * AXS_FLAG_CAPACITY (AXS_OK is still returned: the other rows are valid);
 * axs_sample_batch_host, which sees the offsets, returns AXS_E_CAPACITY for a
 * batch of 2 rows or more with a row above AXS_BIAS_ROW_MAX. */
#define AXS_BIAS_ROW_MAX 1024
#define AXS_BIAS_SEG_MAX 256

typedef struct axs_outputs {
    uint32_t* token_ids;   /* [batch], required                                   */
    float*    logprobs;    /* [batch] or NULL: greedy rows -ln sum exp(l - max),
                              the sum taken as the core sampler takes it (f32,
                              index order, reproduced bit for bit by the exact
                              path: crates/ax-engine-core/src/sampling.rs:177-190);
                              sampled rows max(ln(p/F), -30)
                              (crates/ax-engine-mlx/src/sampling.rs:156-160)      */
    uint32_t* flags;       /* [batch] or NULL, AXS_FLAG_* bits                    */
    uint32_t* kept_ids;    /* [batch, kept_cap] or NULL: the kept set in draw order
                              (diagnostics, e.g. top-k set parity).  Rows of the
                              exact path list kept entries whose probability is
                              below 2^-24 of the maximum's (never drawn) as
                              0xFFFFFFFF after the ordered prefix                 */
    uint32_t* kept_count;  /* [batch] or NULL: size of the kept set               */
    int32_t   kept_cap;
    int32_t   reserved0;
} axs_outputs;

/*
 * MTP speculative verify for `batch` sequences of draft depth `depth` (<= 7):
 * target logits [batch, depth + 1, row_stride], draft logits
 * [batch, depth, row_stride].  Per sequence and position i the law is the
 * reference's function-level one:
 *   P_i = token_distribution(target_i), Q_i = token_distribution(draft_i)
 *        (crates/ax-engine-mlx/src/sampling.rs:647-707)
 *   ln q = max(ln(max(Q_i(d_i), 1e-37)), -30)        (sampling.rs:156-160)
 *   accept iff u_i < min(1, P_i(d_i) / max(exp(ln q'), 1e-37)), with
 *   ln q' = ln q * (T_d / T_t) when both > 0 and differ by > 1e-6
 *        (crates/ax-engine-mlx/src/runner/mod.rs:12388-12419)
 *   on reject: residual max(P_i - Q_i, 0) in ascending id order
 *        (sampling.rs:733-752) drawn with the tail uniform;
 *   all accepted: bonus = sample_categorical_into(target_depth) with the tail
 *        uniform (crates/ax-engine-mlx/src/runner/mod.rs:9732-9775).
 * Uniforms: [batch, depth + 1]; slot i < depth is position i's accept uniform,
 * slot depth the residual/bonus uniform.  NULL = Philox counter
 * (row, step_lo, step_hi, 1), words 0..3 then (row, step_lo, step_hi, 2) ...
 * Distributions of any size are verified on the device (a kept list of more
 * than 2048 ids is read from its row's buffers).  A sequence whose row input
 * is invalid is declined (AXS_MTP_FLAG_ERROR, out_count 0): the caller uses
 * the CPU law for it, as the reference's GPU helpers decline with None
 * (crates/ax-engine-mlx/src/generate.rs:221-238).
 */
typedef struct axs_mtp_desc {
    const void*     target_logits;   /* [batch, depth + 1, row_stride]          */
    const void*     draft_logits;    /* [batch, depth, row_stride]              */
    int32_t         dtype;
    int32_t         batch;
    int32_t         depth;
    int32_t         vocab;
    int64_t         row_stride;
    const uint32_t* draft_ids;       /* [batch, depth]                          */
    const axs_sampling_params* target_params; /* [batch]                        */
    const axs_sampling_params* draft_params;  /* [batch]                        */
    const float*    uniforms;        /* [batch, depth + 1] or NULL              */
} axs_mtp_desc;

#define AXS_MTP_FLAG_RESIDUAL    (1u << 0)  /* tail token came from the residual */
#define AXS_MTP_FLAG_BONUS       (1u << 1)  /* all drafts accepted, bonus drawn  */
#define AXS_MTP_FLAG_NEAR_ACCEPT (1u << 2)  /* |u - p/q| < 1e-6 at a decision   */
#define AXS_MTP_FLAG_NEAR        (1u << 3)  /* a distribution had a near flag   */
#define AXS_MTP_FLAG_CORRECTION  (1u << 4)  /* tail = the target's prediction
                                               after a greedy comparison failed */
#define AXS_MTP_FLAG_TAIL_ROW    (1u << 5)  /* tail = the draw of the target row
                                               at the rejected position (no
                                               correction: an n-gram draft)   */
#define AXS_MTP_FLAG_ERROR       (1u << 31)

typedef struct axs_mtp_outputs {
    uint32_t* out_ids;       /* [batch, depth + 1]: accepted prefix then tail   */
    uint32_t* out_count;     /* [batch]: accept_count + 1                        */
    uint32_t* accept_count;  /* [batch] or NULL                                  */
    uint32_t* flags;         /* [batch] or NULL                                  */
} axs_mtp_outputs;

/*
 * Options of axs_mtp_verify_ex: the rest of mtp_accept_count's contract
 * (crates/ax-engine-mlx/src/runner/mod.rs:12333-12462) — per-position draft
 * sources, the model and n-gram acceptance modes, caller-supplied draft
 * log-probs and target predictions — and the full-softmax draft log-prob.
 */
#define AXS_MTP_SRC_DEFAULT 0  /* as AXS_MTP_SRC_MTP (the reference's None)   */
#define AXS_MTP_SRC_MTP     1  /* MtpDraftSource (crates/ax-engine-mlx/src/   */
#define AXS_MTP_SRC_GEMMA   2  /* runner/mtp_routing.rs:15-33): MTP head,     */
#define AXS_MTP_SRC_NGRAM   3  /* Gemma4 assistant, n-gram, hybrid MTP tail;  */
#define AXS_MTP_SRC_HYBRID  4  /* all but n-gram carry a draft distribution   */
#define AXS_MTP_MODEL_GREEDY     0  /* MtpModelAcceptanceMode (:79-83)         */
#define AXS_MTP_MODEL_REJECTION  1
#define AXS_MTP_NGRAM_CONFIDENCE 0  /* MtpNgramAcceptanceMode (:61-66)         */
#define AXS_MTP_NGRAM_DELTA      1
#define AXS_MTP_NGRAM_GREEDY     2
#define AXS_MTP_LNQ_DISTRIBUTION 0  /* ln q = ln Q_i(d), Q_i = token_distribution
                                       of draft row i (the filtered law)      */
#define AXS_MTP_TARGET_DISTRIBUTION 0  /* p(d) = P_i(d), P_i = token_distribution
                                          of target row i (the sampler's law) */
#define AXS_MTP_TARGET_FILTERED 1  /* p(d) as the runner forms it for the
                                      acceptance test: compute_mtp_target_probs
                                      + extract_cpu_into +
                                      filtered_target_token_probability
                                      (crates/ax-engine-mlx/src/runner/mod.rs:
                                      11836-12159): the softmax of target row i
                                      (full_vocab_token_logprob's terms and
                                      sum), its top_k (or target_topk) largest,
                                      min_p, then top_p cut on the running sum,
                                      renormalised; the residual still uses P_i */
#define AXS_MTP_LNQ_FULL_SOFTMAX 1  /* ln q = ln softmax(draft row i / T_d)[d],
                                       the full-vocabulary law of
                                       gpu_draft_log_prob_lazy
                                       (crates/ax-engine-mlx/src/mtp.rs:203-220),
                                       as axs_token_logprob_batch computes it */
typedef struct axs_mtp_options {
    const uint32_t* sources;            /* [batch, depth] AXS_MTP_SRC_*, or NULL:
                                           every position a model draft          */
    const float*    pending_log_probs;  /* [batch, depth] ln q per position, or
                                           NULL: computed for model drafts
                                           (lnq_mode); for n-gram drafts 0.0
                                           under AXS_MTP_NGRAM_DELTA, else NaN
                                           (no log-prob: greedy comparison)      */
    const uint32_t* predicted;          /* [batch, depth] the target's token per
                                           position for the greedy comparisons,
                                           or NULL: target row i's first argmax  */
    int32_t model_mode;                 /* AXS_MTP_MODEL_*                        */
    int32_t ngram_mode;                 /* AXS_MTP_NGRAM_*                        */
    int32_t lnq_mode;                   /* AXS_MTP_LNQ_*                          */
    int32_t delta_correction;           /* nonzero: a rejected draft without a
                                           draft distribution (n-gram) is
                                           corrected by the residual of the
                                           target against delta(draft)
                                           (sample_exact_mtp_delta_rejection_
                                           correction, runner/mod.rs:12161-12184);
                                           zero: no correction, the tail is the
                                           target row's own draw                 */
    int32_t target_law;                 /* AXS_MTP_TARGET_*: the target probability
                                           of the acceptance test                 */
    uint32_t target_topk;               /* AXS_MTP_TARGET_FILTERED only: the
                                           runner's mtp_target_softmax_topk,
                                           0 = none                              */
} axs_mtp_options;

typedef struct axs_context axs_context;

/* ABI version of the loaded library (AXS_ABI_VERSION). */
int axs_abi_version(void);

/* Thread-local message of the last failed call on this thread ("" if none). */
const char* axs_last_error(void);

/* Registers `handler`, called with the message of every failed call on the
 * failing call's own thread, after axs_last_error() is set; NULL unregisters.
 * The handler must not unwind into the library.  Mirrors the error-handler
 * hook of crates/mlx-sys/native/ax_shim.h:106-110, which the reference
 * records per thread on the Rust side (crates/mlx-sys/src/error.rs:21-99). */
typedef void (*axs_error_handler_func)(const char* msg, void* data);
void axs_set_error_handler(axs_error_handler_func handler, void* data);

/* Creates a sampler context on `device` with device workspace sized for up to
 * max_batch rows of up to max_vocab entries (MTP counts depth*2+1 rows per
 * sequence).  Replaces the reference's per-request sampler buffers
 * (probs_buf / logits_buf / candidates_buf of sample_categorical_into,
 * crates/ax-engine-mlx/src/sampling.rs:204-212). */
int axs_context_create(int device, int max_batch, int max_vocab, axs_context** out);
int axs_context_destroy(axs_context* ctx);

/* Batched sampling step (see axs_batch_desc). */
int axs_sample_batch(axs_context* ctx, const axs_batch_desc* desc,
                     const axs_outputs* out, void* stream);

/* Batched sampling step over HOST arrays: the engine-level TokenSampler
 * boundary (crates/ax-engine-core/src/sampling.rs:90-92), whose requests
 * carry their logits as host vectors (SamplerRequest.logits, :78).  Same
 * descriptor and outputs as axs_sample_batch, but EVERY pointer in `desc` and
 * `out` is a host pointer: the library copies the inputs into device staging
 * of the context (grown on demand) on the context's own stream, samples
 * there, copies the outputs back and waits for them before returning.  Used
 * by a HipTokenSampler implementation of the trait. */
int axs_sample_batch_host(axs_context* ctx, const axs_batch_desc* desc, const axs_outputs* out);

/* Greedy batched argmax + logprob over [batch, row_stride] logits: first
 * maximum (lowest id) wins, NaN skipped, all-NaN row -> 0
 * (crates/ax-engine-mlx/src/sampling.rs:954-966); replaces argmax_batched
 * (crates/ax-engine-mlx/src/batched_sampling.rs:102-111) and the Metal
 * sample_argmax_logprob_batched_f32 kernel
 * (metal/kernels/phase1_dense_path.metal:1273-1341).  out_logprob may be NULL;
 * it receives -ln sum_{finite l} exp(l - max) (NaN when the max is not finite),
 * summed in a fixed order per row (bit-reproducible), within 1e-5 of the
 * exact value; the core sampler's own f32 running sum, which drifts from it by
 * up to ~1e-4 relative over 1e5 terms, is what axs_sample_batch returns for
 * greedy rows. */
int axs_argmax_batch(axs_context* ctx, const void* logits, int dtype, int batch,
                     int vocab, int64_t row_stride, uint32_t* out_ids,
                     float* out_logprob, void* stream);

/* Greedy batched argmax + logprob with the result of axs_argmax_batch, but no
 * context and no device allocation.  No counterpart in the reference: it is
 * for callers that cannot allocate (code under HIP graph capture, serving
 * loops or harnesses that forbid hipMalloc).  Its scratch (per-segment
 * results of the one-row shape, ~260 KB) is a static device array of the
 * library, one per GPU for the life of the process, looked up on the first
 * call on `device`; each call clears what must start at zero with a fill
 * kernel on `stream`.  Limits: vocab <= 262144 and at most 128 scratch
 * segments (a one-row call up to 262,144 ids uses at most 128; batches of 2
 * rows or more use none); beyond them AXS_E_CAPACITY.  Calls that overlap on
 * one GPU (on different streams or threads) race on the shared scratch:
 * serialise them. */
int axs_argmax_batch_noalloc(int device, const void* logits, int dtype, int batch, int vocab,
                             int64_t row_stride, uint32_t* out_ids, float* out_logprob,
                             void* stream);

/* Full-vocabulary log-probability of one token per row:
 *   max(ln(max(softmax(l / T)[t], 1e-37)), -30)
 * over [batch, row_stride] logits, the softmax's normaliser summed as the
 * reference sums it (f32, index order, non-finite terms 0); T <= 0 gives 0
 * for the first maximum and -inf otherwise, t >= vocab gives -30.
 * full_vocab_token_logprob (crates/ax-engine-mlx/src/sampling.rs:761-787) per
 * row, e.g. the draft log-prob of MTP rejection sampling in the
 * full-softmax domain (crates/ax-engine-mlx/src/mtp.rs:203-220).  tokens
 * [batch], temperatures [batch] and out_logprob [batch] are device arrays. */
int axs_token_logprob_batch(axs_context* ctx, const void* logits, int dtype, int batch, int vocab,
                            int64_t row_stride, const uint32_t* tokens, const float* temperatures,
                            float* out_logprob, void* stream);

/* Top-N log-probabilities per row: the n (1..AXS_TOP_LOGPROBS_MAX) ids with
 * the largest full-softmax probability exp((l - max) / T) (non-finite as
 * 0; ties to the lower id), in that order, each with
 * full_vocab_token_logprob (crates/ax-engine-mlx/src/sampling.rs:761-787;
 * the same value axs_token_logprob_batch returns for the id).  The
 * reference's server rejects top_logprobs
 * (crates/ax-engine-server/src/openai/requests.rs:1283-1298): this is a
 * build extension over its sampled-token logprob.  T <= 0 lists the first
 * maximum (0) only; slots past it or past vocab hold AXS_NONE_U32 / -inf.
 * temperatures [batch], out_ids and out_logprob [batch, n]: device arrays. */
#define AXS_TOP_LOGPROBS_MAX 64
int axs_top_logprobs(axs_context* ctx, const void* logits, int dtype, int batch, int vocab,
                     int64_t row_stride, const float* temperatures, int n, uint32_t* out_ids, float* out_logprob,
                     void* stream);

/* Think soft-close rank probe, per row: out_hit[r] = 1 when think_ids[r]
 * sits within the top ranks[r] raw logits of row r (no processors, no
 * temperature), else 0 — think_soft_close_in_top_k
 * (crates/ax-engine-mlx/src/ngram_accel.rs:1609-1640), whose caller emits
 * the think-close token on a hit and samples the row otherwise
 * (ngram_accel.rs:1691-1713; a hit consumes no uniform).  rank 0 or an id
 * >= vocab is a miss.  Ties go to the lower id, as the reference's running
 * set keeps them; a row holding a NaN, or both -0 and +0, is replayed
 * exactly as the reference's loop runs (ranks up to 1024; above that
 * out_hit[r] = AXS_NONE_U32 and the caller runs the host probe).
 * think_ids, ranks and out_hit are device arrays of batch entries. */
int axs_soft_close_probe(axs_context* ctx, const void* logits, int dtype, int batch, int vocab,
                         int64_t row_stride, const uint32_t* think_ids, const uint32_t* ranks,
                         uint32_t* out_hit, void* stream);

/* MTP draft side, one depth over batch draft rows [batch, row_stride]:
 * per row the draft token and its full-softmax log-prob ln q, which
 * axs_mtp_verify_ex consumes as pending_log_probs.
 *   AXS_MTP_DRAFT_SAMPLED (mtp_draft_tokens_sampled,
 *     crates/ax-engine-mlx/src/mtp.rs:1454-1552): the argmax
 *     (lazy_argmax_logits, mtp.rs:192-196), ln q at the row's temperature;
 *   AXS_MTP_DRAFT_STOCHASTIC (mtp_draft_tokens_stochastic, mtp.rs:1554-1640):
 *     T > 0 a categorical draw from softmax(l / T) (lazy_random_sample,
 *     mtp.rs:228-233), ln q at T; T <= 0 the argmax, ln q at T = 1.
 * ln q = full_vocab_token_logprob(row, token, T)
 * (crates/ax-engine-mlx/src/sampling.rs:761-787), the CPU statement of
 * gpu_draft_log_prob_lazy (mtp.rs:203-220), as axs_token_logprob_batch
 * computes it.  The reference draws with MLX's own generator (its comment:
 * not reproducible); here the draw is sample_categorical_into with no
 * filters (sampling.rs:204-271) on uniforms[r] (device [batch], in [0, 1])
 * or, when uniforms is NULL, Philox(params[r].seed, r, params[r].step).
 * params [batch] (device): only temperature, seed and step are read; the
 * draft law applies no processors or filters.  out_ids and out_lnq [batch]:
 * device arrays. */
#define AXS_MTP_DRAFT_SAMPLED    0
#define AXS_MTP_DRAFT_STOCHASTIC 1
int axs_mtp_draft(axs_context* ctx, const void* logits, int dtype, int batch, int vocab, int64_t row_stride,
                  const axs_sampling_params* params, int mode, const float* uniforms, uint32_t* out_ids,
                  float* out_lnq, void* stream);

/* LM-head projection with the greedy decision in its epilogue (producer
 * fusion): for every batch row b and vocabulary id v,
 *   logits[b, v] = softcap(scale * f32(bf16(sum_k hidden[b, k] * weight[v, k])))
 * the reference's final projection (crates/ax-engine-mlx/src/model/mod.rs:1771-1775:
 * the bf16 product widened to f32) followed by apply_final_logit_softcap
 * (crates/ax-engine-mlx/src/model/shared/utils.rs:1826-1845: x * scale, then
 * tanh(x * (1 / cap)) * cap, in f32; scale 1 and softcap <= 0 turn them
 * off).  The products accumulate in f32 on the matrix cores and are rounded
 * to bf16 (nearest even) once, as a bf16 matmul's output is; only the
 * accumulation order differs from the reference's backend.
 * hidden [batch, hidden_stride] and weight [vocab, weight_stride] are bf16
 * device arrays (the final-norm output and the LM-head weight in its
 * [out, in] layout; quantised weights are not taken).  out_logits
 * [batch, out_stride] f32 receives the logits when non-NULL; out_argmax
 * [batch] receives each row's argmax under argmax_f32
 * (crates/ax-engine-mlx/src/sampling.rs:954-970: first maximum, NaN skipped,
 * an all-NaN row gives 0) when non-NULL, formed in the same kernel, so a
 * greedy row's logits need never be written.  Rows to be sampled go on to
 * axs_sample_batch over out_logits.  Requires hidden_size % 32 == 0, both
 * input strides multiples of 8 elements and 16-byte aligned inputs;
 * batch <= the context's max_batch (argmax keys live in its workspace).
 * The weight is read from HBM once per 128 batch rows. */
int axs_lm_head(axs_context* ctx, const void* hidden, int64_t hidden_stride, const void* weight,
                int64_t weight_stride, int batch, int hidden_size, int vocab, float scale, float softcap,
                float* out_logits, int64_t out_stride, uint32_t* out_argmax, void* stream);

/* MTP speculative verify (see axs_mtp_desc). */
/* MTP verify with options: per sequence, mtp_accept_count
 * (crates/ax-engine-mlx/src/runner/mod.rs:12333-12462) over the draft ids,
 * with target probabilities P_i(d) = token_distribution(target row i)(d)
 * when the target temperature is > 0 (none otherwise: greedy comparisons),
 * target distributions P_i and draft distributions Q_i (model drafts), then
 * the tail (runner/mod.rs:9732-9775, ngram_accel.rs:1543-1590): the
 * correction when there is one, the draw of target row depth when every
 * draft was accepted (bonus), else the draw of the target row at the
 * rejected position.  Uniforms follow the reference's stream: uniforms[b, k]
 * is the k-th uniform sequence b consumes (each rejection test, then the
 * residual or the tail draw), NULL = Philox (b, step, 1 + k/4, word k%4).
 * opts NULL: every position a model draft under rejection sampling, ln q
 * from the draft distributions (axs_mtp_verify's law, with the stream order
 * of uniforms). */
int axs_mtp_verify_ex(axs_context* ctx, const axs_mtp_desc* desc, const axs_mtp_options* opts,
                      const axs_mtp_outputs* out, void* stream);

int axs_mtp_verify(axs_context* ctx, const axs_mtp_desc* desc,
                   const axs_mtp_outputs* out, void* stream);

/* Per-kernel timing, for benchmarks (no counterpart in the reference).  While
 * enabled, every kernel the context launches is bracketed by hipEvents
 * recorded on its launch stream.  Enabling clears earlier records. */
#define AXS_KERNEL_STREAM    0  /* the single pass over the logits, with
                                   the per-row decisions                */
#define AXS_KERNEL_EXACT_MAT 1  /* exact path: second pass            */
#define AXS_KERNEL_EXACT_ROW 2  /* exact path: sort + exact sums      */
#define AXS_KERNEL_MTP       3  /* MTP accept / residual / bonus      */
#define AXS_KERNEL_LM_HEAD   4  /* LM-head projection + argmax        */
#define AXS_KERNEL_COUNT     5
int axs_timing_enable(axs_context* ctx, int enable);
/* Waits for the recorded events of one kernel class and returns their summed
 * duration in milliseconds and the number of launches since enabling. */
int axs_timing_read(axs_context* ctx, int kernel, double* total_ms, int* launches);

#ifdef __cplusplus
}
#endif

#endif /* AX_HIP_SAMPLER_H */
