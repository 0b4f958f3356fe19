// axs_sampler.hip — MI355X (gfx950) per-step token sampler behind the C ABI
// of include/ax_hip_sampler.h.
//
// One sampling step over [rows, V] logits in HBM runs on the caller's stream
// as one kernel for batches of 64 rows or more:
//
//   k_row       one 1024-thread workgroup per row: the single pass over the
//               logits (the HBM-bound kernel), the row's decision, and, for a
//               row that needs it, the exact path (second read, sort, exact
//               running sums, decisions) in the same workgroup;
//
// and as three kernels for smaller batches:
//
//   k_stream    the single pass over the logits (the HBM-bound kernel).  Work
//               item = (row, segment of <= 65536 ids); the segments of a row
//               are placed on one XCD.  Each workgroup builds the logits
//               processors' LDS tables for its segment (repetition,
//               presence/frequency, bias, mask, n-gram ban) while its first
//               tiles load, then streams the segment in double-buffered
//               register tiles: max/argmax, and for min-p rows every id within
//               the min-p window of the running maximum.  The last workgroup
//               of a row to finish decides the row in place (greedy, fallback,
//               min-p rows whose survivors were gathered) or lists it for
//               the exact path.
//   k_exact_mat exact path, pass 2 over the listed rows: exact probabilities
//               with the global max, written dense (index-order laws) or
//               compacted (sorted laws).
//   k_exact_row exact path, one workgroup per listed row: bucket sort by
//               (p desc, id asc), then the exact parallel reproduction of the
//               reference's sequential f32 running sums (axs_exact_sum.h), then
//               the nucleus / top-k / draw decisions by binary search.
//
// k_mtp_verify adds the MTP accept / residual / bonus step on top of the same
// pipeline run over the target and draft rows.
//
// Arithmetic follows sample_categorical_into
// (crates/ax-engine-mlx/src/sampling.rs:204-316) operation by operation:
// f32 round-to-nearest, no contraction (the file is built with
// -ffp-contract=off), correctly rounded division, and the host libm's expf
// restated bit for bit (axs_expf.h).

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdlib>
#include <mutex>
#include <type_traits>
#include <new>
#include <string>
#include <vector>

#include "axs_device.h"
#include "axs_lm_head.h"

namespace axs {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int NT_CHUNK = 256;
constexpr uint32_t SEG_MAX = 65536;   // ids per k_stream segment, 256-thread workgroups
constexpr uint32_t ROW_MAX = 262144;  // ids per row, one 1024-thread workgroup per row
constexpr uint32_t EX_SEGMAX = 32768; // ids per exact-path segment
constexpr uint32_t MAX_SEGS = 1024;   // segments per row (upper bound)
constexpr int NT_FIN = 256;
constexpr uint32_t FIN_CAP = 2048;    // min-p candidates merged per row (1024-thread rows)
constexpr uint32_t CAPS = 256;        // published candidates per segment (power of 2)
constexpr int NT_EX = 1024;
constexpr uint32_t NBUCKET = 13312;   // 13 per thread; covers p in [2^-24, 1]
constexpr uint32_t BIAS_LDS = 256;    // bias entries per chunk
constexpr uint32_t KEPT_CAP = 2048;   // kept entries per MTP distribution row
constexpr uint32_t BIG_LDS_SORT = 4096;
constexpr float P_FLOOR = 0x1p-24f;   // smaller terms never change a sum >= 1
// RowState.flags of an MTP pipeline row whose kept list stays in the row's
// buffers (sorted keys, or the dense row's p > 0 entries): too long for the
// KEPT_CAP lists.  Internal: never an output flag.
constexpr uint32_t RSF_LIST_IN_ROW = 1u << 30;

// chunk-stat flags
constexpr uint32_t CS_OVERFLOW = 1u;
constexpr uint32_t CS_ERROR = 2u;
constexpr uint32_t CS_CAPACITY = 4u;  // with CS_ERROR: more bias entries than the kernel holds

// A segment's result, published as two 64-bit words (see pub_u64)
struct ChunkStat {
    float m;        // max processed logit (-inf if the segment has no non-NaN)
    uint32_t amax;  // lowest id attaining m, NONE if none
    float gsum;     // sum of exp(l - m) over finite l (greedy logprob)
    uint32_t flags;  // CS_* in bits 0-7, published candidates in bits 8-31
};

struct Cand {
    uint32_t id;
    float l;
};

// Cross-workgroup publication inside one kernel.  Segment results and
// candidates are written with device-scope stores (write-through to the
// device coherence point) and read back with device-scope loads, and every
// writer waits for its stores to complete before the row's arrival counter
// is bumped; the last arriver therefore reads complete data without a
// device-wide cache write-back per workgroup.
__device__ __forceinline__ void pub_u64(void* p, uint64_t v) {
    __hip_atomic_store((uint64_t*)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t sub_u64(const void* p) {
    return __hip_atomic_load((uint64_t*)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t sub_u32(const uint32_t* p) {
    return __hip_atomic_load((uint32_t*)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void pub_u32(uint32_t* p, uint32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void pub_cand(Cand* p, Cand c) {
    pub_u64(p, (uint64_t)c.id | ((uint64_t)__float_as_uint(c.l) << 32));
}
__device__ __forceinline__ Cand sub_cand(const Cand* p) {
    const uint64_t v = sub_u64(p);
    Cand c;
    c.id = (uint32_t)v;
    c.l = __uint_as_float((uint32_t)(v >> 32));
    return c;
}
__device__ __forceinline__ void pub_stat(ChunkStat* p, const ChunkStat& st) {
    pub_u64(p, (uint64_t)__float_as_uint(st.m) | ((uint64_t)st.amax << 32));
    pub_u64((char*)p + 8, (uint64_t)__float_as_uint(st.gsum) | ((uint64_t)st.flags << 32));
}
__device__ __forceinline__ ChunkStat sub_stat(const ChunkStat* p) {
    const uint64_t v0 = sub_u64(p), v1 = sub_u64((const char*)p + 8);
    ChunkStat st;
    st.m = __uint_as_float((uint32_t)v0);
    st.amax = (uint32_t)(v0 >> 32);
    st.gsum = __uint_as_float((uint32_t)v1);
    st.flags = (uint32_t)(v1 >> 32);
    return st;
}
// waits until every memory operation this thread issued has completed
__device__ __forceinline__ void wait_mem() { __builtin_amdgcn_s_waitcnt(0); }

// Workgroup barrier for data exchanged through LDS only: waits for this
// wave's LDS (and scalar) operations, not for its outstanding global loads,
// which stay in flight across it (__syncthreads would drain them).
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

struct RowState {
    float m;
    float inv;
    uint32_t mode;
    uint32_t sorted;     // draw order is (p desc, id asc)
    uint32_t ncompact;   // compacted entries (atomic)
    uint32_t minp_mg;    // min |p - min_p| / min_p as f32 bits (atomicMin)
    uint32_t amax;
    uint32_t flags;
    float pmin;          // compaction floor
    float u;
    uint32_t kept;       // kept-set size (MTP distributions)
    float F;             // filtered sum (MTP distributions)
    uint32_t nlist;      // entries written to the kept list
    uint32_t pad[3];
};

struct KArgs {
    // inputs
    const void* logits;   // rows [0, n_first) (all rows outside MTP)
    const void* logits2;  // MTP draft rows
    int32_t dtype;
    int32_t nrows;
    int32_t vocab;
    int32_t nch;          // exact-path segments per row ...
    int32_t chunk;        // ... of this many ids
    int32_t snch;         // k_stream segments per row ...
    int32_t schunk;       // ... of this many ids
    int32_t mtp_depth;    // > 0: MTP layout
    int32_t mtp_batch;
    int32_t want_logprob;
    int32_t vec;          // rows are 16-byte aligned: vector loads
    int32_t inplace;      // k_row: a row's exact path in its own workgroup (else listed)
    int32_t exact_lp;     // greedy rows' logprob: the core sampler's sequential sum (exact path)
    int32_t pad0;
    // full-vocabulary token logprob rows (axs_token_logprob_batch): the token
    // and temperature of each row; the row's law is the untruncated softmax
    const uint32_t* lp_tokens;
    const float* lp_temps;
    // top-N rows (axs_top_logprobs): topn > 0 lists each row's n largest
    // full-softmax probabilities instead of one token's
    uint32_t topn;
    uint32_t* topn_ids;  // [rows, topn]
    float* topn_lp;      // [rows, topn]
    // MTP verify options (axs_mtp_verify_ex); mtp_stream: uniforms in the
    // reference's stream order (else the slot layout of axs_mtp_verify)
    const uint32_t* mtp_sources;  // [batch, depth] or NULL
    const float* mtp_lnq_in;      // [batch, depth] or NULL
    const uint32_t* mtp_pred;     // [batch, depth] or NULL
    const float* mtp_lnq_full;    // [batch, depth] full-softmax ln q, or NULL
    uint32_t* mtp_amax;           // [rows] each pipeline row's first argmax, or NULL
    int32_t mtp_model_mode, mtp_ngram_mode, mtp_delta, mtp_stream;
    int64_t stride;
    const axs_sampling_params* params;
    const axs_sampling_params* params2;
    const uint32_t* hist;
    const int64_t* hist_off;
    int64_t hist_len;
    const uint32_t* mask;
    int64_t mask_stride;
    const uint32_t* bias_ids;
    const float* bias_vals;
    const int64_t* bias_off;
    int64_t bias_len;
    const float* uniforms;
    // workspace
    ChunkStat* cstat;
    Cand* pool;             // published candidates [rows, segments, CAPS]
    RowState* rstate;
    uint32_t* exact_rows;
    uint32_t* exact_count;
    uint32_t* row_done;     // per-row segment counters (atomicInc, wrap to 0)
    uint32_t* ex_done;      // k_exact_row workgroup counter (atomicInc, wrap to 0)
    float* dense;
    uint64_t* ckey;
    uint64_t* ckey2;
    uint64_t* tmp64;
    float* sbuf;
    uint32_t* bend;
    uint32_t* ws_kept_id;   // MTP kept lists [rows, KEPT_CAP] (NULL outside MTP)
    float* ws_kept_p;
    int64_t tmp_stride;     // next_pow2(vocab)
    // outputs
    uint32_t* out_ids;
    float* out_lp;
    uint32_t* out_flags;
    uint32_t* out_kept;
    uint32_t* out_kept_count;
    int32_t out_kept_cap;
};

// --------------------------------------------------------------------------
// row addressing
// --------------------------------------------------------------------------
__device__ __forceinline__ size_t esize_of(int dt) { return dt == AXS_DTYPE_BF16 ? 2 : 4; }

__device__ __forceinline__ const char* row_ptr(const KArgs& a, int r) {
    size_t es = esize_of(a.dtype);
    if (a.mtp_depth > 0) {
        int nt = a.mtp_batch * (a.mtp_depth + 1);
        if (r >= nt) return (const char*)a.logits2 + (size_t)(r - nt) * a.stride * es;
    }
    return (const char*)a.logits + (size_t)r * a.stride * es;
}

__device__ __forceinline__ axs_sampling_params row_params(const KArgs& a, int r) {
    if (a.params == nullptr) {  // plain argmax entry point, or a token-logprob row
        axs_sampling_params p;
        p.temperature = a.lp_temps ? a.lp_temps[r] : 0.0f;
        p.top_p = 1.0f;
        p.top_k = 0;
        p.min_p = 0.0f;
        p.has_min_p = 0;
        p.repetition_penalty = 1.0f;
        p.repetition_context_size = NONE;
        p.no_repeat_ngram_size = 0;
        p.ngram_window = 128;
        p.presence_penalty = 0.0f;
        p.frequency_penalty = 0.0f;
        p.reserved0 = 0;
        p.seed = 0;
        p.step = 0;
        return p;
    }
    if (a.mtp_depth > 0) {
        int nt = a.mtp_batch * (a.mtp_depth + 1);
        if (r >= nt) return a.params2[(r - nt) / a.mtp_depth];
        return a.params[r / (a.mtp_depth + 1)];
    }
    return a.params[r];
}

// The draft source of position i of sequence b (AXS_MTP_SRC_DEFAULT and
// unknown codes read as a model draft) and whether it carries a draft
// distribution (MtpDraftSource::is_model_draft,
// crates/ax-engine-mlx/src/runner/mtp_routing.rs:24-30).
__device__ __forceinline__ uint32_t mtp_source(const KArgs& a, int b, int i) {
    const uint32_t s = a.mtp_sources ? a.mtp_sources[(size_t)b * a.mtp_depth + i] : AXS_MTP_SRC_MTP;
    return (s == AXS_MTP_SRC_GEMMA || s == AXS_MTP_SRC_NGRAM || s == AXS_MTP_SRC_HYBRID) ? s : AXS_MTP_SRC_MTP;
}
// Whether position i of sequence b is decided by a rejection test (and so
// consumes a uniform) rather than a greedy comparison: not a greedy-mode
// position, a finite draft log-prob, and target probabilities (target
// temperature > 0) (runner/mod.rs:12355-12392).  Known before any
// outcome: a model draft's ln q is always finite (floored at -30).
__device__ __forceinline__ bool mtp_is_test(const KArgs& a, int b, int i, float target_temp) {
    const uint32_t src = mtp_source(a, b, i);
    const bool has_dd = src != AXS_MTP_SRC_NGRAM;
    if (src == AXS_MTP_SRC_NGRAM && a.mtp_ngram_mode == AXS_MTP_NGRAM_GREEDY) return false;
    if (has_dd && a.mtp_model_mode == AXS_MTP_MODEL_GREEDY) return false;
    if (!(target_temp > 0.0f)) return false;
    if (a.mtp_lnq_in) return isfinite(a.mtp_lnq_in[(size_t)b * a.mtp_depth + i]);
    return has_dd || a.mtp_ngram_mode == AXS_MTP_NGRAM_DELTA;
}
// The k-th uniform of MTP sequence b: supplied [batch, depth + 1], or
// Philox counter (b, step, 1 + k/4), word k % 4.
__device__ __forceinline__ float mtp_uniform(const KArgs& a, int b, const axs_sampling_params& tp, uint32_t k) {
    const int D = a.mtp_depth;
    if (a.uniforms) return a.uniforms[(size_t)b * (D + 1) + k];
    return philox_uniform(tp.seed, (uint32_t)b, tp.step, 1u + k / 4u, k & 3u);
}

// the uniform a row's draw consumes: supplied, or Philox(seed, row, step)
__device__ __forceinline__ float row_uniform(const KArgs& a, int r, const axs_sampling_params& p) {
    if (a.mtp_depth > 0) {
        int D = a.mtp_depth;
        int nt = a.mtp_batch * (D + 1);
        if (a.mtp_stream) {
            // every target row j draws: it is the tail when the verify stops
            // at position j (or j = D, the bonus), after the rejection tests
            // of positions 0..min(j, D-1), which consume the first uniforms
            if (r >= nt) return 0.5f;
            const int b = r / (D + 1), j = r % (D + 1);
            uint32_t k = 0;
            for (int i = 0; i <= j && i < D; ++i) k += mtp_is_test(a, b, i, p.temperature) ? 1u : 0u;
            return mtp_uniform(a, b, p, k);
        }
        if (r >= nt || (r % (D + 1)) != D) return 0.5f;  // only the bonus row draws
        int b = r / (D + 1);
        if (a.uniforms) return a.uniforms[(size_t)b * (D + 1) + D];
        return philox_uniform(p.seed, (uint32_t)b, p.step, 1u + (uint32_t)D / 4u, (uint32_t)D & 3u);
    }
    if (a.uniforms) return a.uniforms[r];
    return philox_uniform(p.seed, (uint32_t)r, p.step, 0u, 0u);
}

// --------------------------------------------------------------------------
// logits processors: per-segment LDS tables
//   spec  bit per id of the segment: the id occurs in the repetition window,
//         has a bias entry or is banned.  These "special" ids are processed
//         one by one; the streaming passes read them as NaN.
//   pre   number of special ids before each bitmap word: with a popcount
//         inside the word, the rank of a special id
//   sid   the id of each rank
//   cnt   occurrences in the repetition window, by rank (CNT_BAN: banned by
//         the no-repeat n-gram rule)
// --------------------------------------------------------------------------
constexpr uint32_t CNT_BAN = 0x80000000u;

template <int NT, uint32_t SEGMAX>
struct ProcLds {
    static constexpr uint32_t NW = SEGMAX / 32;      // bitmap words
    static constexpr uint32_t PW = NW / NT;          // bitmap words per thread
    static constexpr uint32_t RCAP = NT >= 1024 ? SEGMAX / 32 : SEGMAX / 64;  // ranked special ids
    // bias entries per segment: the exact-path segments hold as many as a
    // k_row row (RBCAP), so no row that k_row accepted overflows them
    static constexpr uint32_t BCAP = (NT >= 1024 || SEGMAX == EX_SEGMAX) ? 1024u : BIAS_LDS;
    uint32_t spec[NW];
    uint16_t pre[NW];
    uint32_t sid[RCAP];
    uint32_t cnt[RCAP];
    uint32_t bias_id[BCAP];
    float bias_v[BCAP];
    uint32_t scan[NT / 64];
    uint32_t nspec;  // special ids in the segment
    uint32_t nbias;
    uint32_t err;    // bias entries beyond BCAP in one segment
};

struct RowCtx {
    axs_sampling_params p;
    uint32_t mode;
    bool rep_on, pf_on, cnt_on, bias_on, mask_on, ban_on, any_proc;
    int64_t w0, w1;     // repetition window [w0, w1) in the history array
    int64_t h0;         // history start
    int64_t b0, b1;     // bias entries
    bool err;
};

__device__ __forceinline__ RowCtx make_ctx(const KArgs& a, int r) {
    RowCtx c;
    c.p = row_params(a, r);
    c.mode = row_mode(c.p);
    c.err = false;
    c.h0 = c.w0 = c.w1 = 0;
    c.b0 = c.b1 = 0;
    int64_t nhist = 0;
    if (a.hist && a.hist_off && a.mtp_depth == 0) {
        int64_t h0 = a.hist_off[r], h1 = a.hist_off[r + 1];
        if (h0 < 0 || h1 < h0 || h1 > a.hist_len) {
            c.err = true;
        } else {
            c.h0 = h0;
            c.w1 = h1;
            nhist = h1 - h0;
        }
    }
    uint32_t ctxs = c.p.repetition_context_size;
    int64_t keep = ctxs == NONE ? nhist : (int64_t)ctxs;
    if (keep > nhist) keep = nhist;
    c.w0 = c.w1 - keep;
    bool ref_proc = (uses_rep(c.p) || c.p.no_repeat_ngram_size > 0) && nhist > 0;
    c.rep_on = ref_proc && uses_rep(c.p) && keep > 0;
    c.pf_on = (c.p.presence_penalty != 0.0f || c.p.frequency_penalty != 0.0f) && keep > 0;
    c.cnt_on = c.rep_on || c.pf_on;
    c.ban_on = ref_proc && c.p.no_repeat_ngram_size > 0 && nhist >= (int64_t)c.p.no_repeat_ngram_size;
    c.bias_on = false;
    if (a.bias_ids && a.bias_off && a.mtp_depth == 0) {
        int64_t b0 = a.bias_off[r], b1 = a.bias_off[r + 1];
        if (b0 < 0 || b1 < b0 || b1 > a.bias_len) c.err = true;
        else if (b1 > b0) {
            c.bias_on = true;
            c.b0 = b0;
            c.b1 = b1;
        }
    }
    c.mask_on = a.mask != nullptr && a.mtp_depth == 0;
    c.any_proc = c.cnt_on || c.bias_on || c.mask_on || c.ban_on;
    if (c.err) {
        c.cnt_on = c.bias_on = c.mask_on = c.ban_on = c.any_proc = false;
        c.rep_on = c.pf_on = false;
    }
    return c;
}

// The first 2048 tokens of the repetition window, loaded before the segment's
// logits are waited for so the tables can be built while those stream.
template <int NT>
struct HistPre {
    static constexpr int K = 2048 / NT;
    uint32_t t[K];
};

template <int NT>
__device__ __forceinline__ void hist_prefetch(const KArgs& a, const RowCtx& c, HistPre<NT>& hp) {
    const int tid = threadIdx.x;
#pragma unroll
    for (int k = 0; k < HistPre<NT>::K; ++k) {
        const int64_t i = c.w0 + tid + (int64_t)k * NT;
        hp.t[k] = (c.cnt_on && i < c.w1) ? a.hist[i] : NONE;
    }
}

// f(token) for every token of the repetition window, spread over the block
// (the first round from the prefetched registers)
template <int NT, typename F>
__device__ __forceinline__ void hist_each(const KArgs& a, const RowCtx& c, const HistPre<NT>& hp, F&& f) {
    constexpr int K = HistPre<NT>::K;
    const int tid = threadIdx.x;
    for (int64_t base = c.w0; base < c.w1; base += (int64_t)K * NT) {
        uint32_t t[K];
#pragma unroll
        for (int k = 0; k < K; ++k) {
            const int64_t i = base + tid + (int64_t)k * NT;
            t[k] = base == c.w0 ? hp.t[k] : (i < c.w1 ? a.hist[i] : NONE);
        }
#pragma unroll
        for (int k = 0; k < K; ++k) f(t[k]);
    }
}

// f(t) for every token t in [lo, hi) that the no-repeat n-gram rule bans
// (logits_with_no_repeat_ngram_in_place, sampling.rs:896-920), spread over
// the block
template <typename F>
__device__ __forceinline__ void ngram_each_g(const KArgs& a, const RowCtx& c, uint32_t lo, uint32_t hi, int64_t first,
                                             int64_t stride, F&& f) {
    const int64_t nhist = c.w1 - c.h0;
    const uint32_t ng = c.p.no_repeat_ngram_size;
    int64_t keep = (int64_t)(c.p.ngram_window > ng ? c.p.ngram_window : ng);
    if (keep > nhist) keep = nhist;
    const int64_t hs = c.w1 - keep;
    const int64_t plen = (int64_t)ng - 1;
    for (int64_t s = first; s + (int64_t)ng <= keep; s += stride) {
        bool match = true;
        for (int64_t j = 0; j < plen; ++j)
            if (a.hist[hs + s + j] != a.hist[c.w1 - plen + j]) {
                match = false;
                break;
            }
        if (match) {
            const uint32_t t = a.hist[hs + s + plen];
            if (t >= lo && t < hi) f(t);
        }
    }
}
template <int NT, typename F>
__device__ __forceinline__ void ngram_each(const KArgs& a, const RowCtx& c, uint32_t lo, uint32_t hi, F&& f) {
    ngram_each_g(a, c, lo, hi, (int64_t)threadIdx.x, (int64_t)NT, f);
}

// Marks the segment's special ids (ids in [lo, hi)) and lists its bias
// entries.  Block-uniform control.
template <int NT, uint32_t SEGMAX>
__device__ __forceinline__ void proc_build(const KArgs& a, const RowCtx& c, uint32_t lo, uint32_t hi,
                                           ProcLds<NT, SEGMAX>& L, const HistPre<NT>& hp) {
    const int tid = threadIdx.x;
    const uint32_t nw = (hi - lo + 31u) / 32u;
    if (tid == 0) {
        L.nbias = 0;
        L.err = 0;
        L.nspec = 0;
    }
    for (uint32_t i = tid; i < nw; i += NT) L.spec[i] = 0u;
    __syncthreads();
    auto mark = [&](uint32_t t) { atomicOr(&L.spec[(t - lo) >> 5], 1u << ((t - lo) & 31u)); };
    if (c.cnt_on)
        hist_each<NT>(a, c, hp, [&](uint32_t t) {
            if (t >= lo && t < hi) mark(t);
        });
    if (c.bias_on && tid < 64) {
        // ordered compaction of the in-range entries (list order is the order
        // the additions are applied in)
        const int lane = tid;
        uint32_t base = 0;
        for (int64_t s = c.b0; s < c.b1; s += 64) {
            int64_t i = s + lane;
            bool in = false;
            uint32_t t = 0;
            float v = 0.0f;
            if (i < c.b1) {
                t = a.bias_ids[i];
                v = a.bias_vals[i];
                in = t >= lo && t < hi;
            }
            uint64_t m = __ballot(in);
            uint32_t pre = __popcll(m & ((1ull << lane) - 1ull));
            if (in) {
                uint32_t slot = base + pre;
                if (slot < ProcLds<NT, SEGMAX>::BCAP) {
                    L.bias_id[slot] = t;
                    L.bias_v[slot] = v;
                    mark(t);
                } else {
                    L.err = 1;
                }
            }
            base += __popcll(m);
        }
        if (lane == 0) L.nbias = base < ProcLds<NT, SEGMAX>::BCAP ? base : ProcLds<NT, SEGMAX>::BCAP;
    }
    if (c.ban_on) ngram_each<NT>(a, c, lo, hi, mark);
    __syncthreads();
}

// rank of special id e (offset off in the segment)
template <int NT, uint32_t SEGMAX>
__device__ __forceinline__ uint32_t rank_of(const ProcLds<NT, SEGMAX>& L, uint32_t off) {
    const uint32_t w = off >> 5;
    return L.pre[w] + (uint32_t)__popc(L.spec[w] & ((1u << (off & 31u)) - 1u));
}

// Ranks the special ids, lists them by rank, counts the repetition window by
// rank and flags the banned ones.  Returns false when the segment has more
// special ids than ranks (they are then resolved one by one from HBM).
// Block-uniform control.
template <int NT, uint32_t SEGMAX>
__device__ __forceinline__ bool proc_rank(const KArgs& a, const RowCtx& c, uint32_t lo, uint32_t hi,
                                          ProcLds<NT, SEGMAX>& L, const HistPre<NT>& hp) {
    using PL = ProcLds<NT, SEGMAX>;
    const int tid = threadIdx.x;
    const uint32_t nw = (hi - lo + 31u) / 32u;
    static_assert(PL::PW % 4 == 0, "bitmap words per thread");
    // thread t owns words [t*PW, t*PW + PW), read four at a time as 16-byte
    // vectors (no bank conflicts); counted first, ranked after the scan
    const uint32_t w0 = (uint32_t)tid * PL::PW;
    uint32_t cnt = 0;
#pragma unroll
    for (uint32_t k = 0; k < PL::PW; k += 4) {
        const u32x4 x = *(const u32x4*)&L.spec[w0 + k];
#pragma unroll
        for (uint32_t q = 0; q < 4; ++q) cnt += w0 + k + q < nw ? (uint32_t)__popc(x[q]) : 0u;
    }
    uint32_t n;
    uint32_t pre = block_excl_scan_u32<NT>(cnt, L.scan, &n);
    const bool ranked = n <= PL::RCAP;
    uint32_t* pre32 = (uint32_t*)L.pre + w0 / 2;
#pragma unroll
    for (uint32_t k = 0; k < PL::PW; k += 4) {
        const u32x4 x = *(const u32x4*)&L.spec[w0 + k];
        uint32_t pk[2];
#pragma unroll
        for (uint32_t q = 0; q < 4; ++q) {
            const uint32_t wi = w0 + k + q;
            const uint32_t bits0 = wi < nw ? x[q] : 0u;
            const uint32_t p16 = pre < 65535u ? pre : 65535u;
            if (q & 1u) pk[q / 2] |= p16 << 16;
            else pk[q / 2] = p16;
            if (ranked) {
                uint32_t bits = bits0;
                uint32_t rk = pre;
                while (bits) {
                    const uint32_t b = (uint32_t)__ffs((int)bits) - 1u;
                    bits &= bits - 1u;
                    L.sid[rk] = lo + wi * 32u + b;
                    L.cnt[rk] = 0u;
                    ++rk;
                }
            }
            pre += (uint32_t)__popc(bits0);
        }
        *(uint2*)&pre32[k / 2] = make_uint2(pk[0], pk[1]);
    }
    if (tid == 0) L.nspec = n;
    __syncthreads();
    if (ranked) {
        if (c.cnt_on)
            hist_each<NT>(a, c, hp, [&](uint32_t t) {
                if (t >= lo && t < hi) atomicAdd(&L.cnt[rank_of(L, t - lo)], 1u);
            });
        if (c.ban_on) ngram_each<NT>(a, c, lo, hi, [&](uint32_t t) { atomicOr(&L.cnt[rank_of(L, t - lo)], CNT_BAN); });
        __syncthreads();
    }
    return ranked;
}

// Every processor in order for one special id e with raw logit l, window count
// cnt (CNT_BAN if banned) and mask word mw: repetition → presence/frequency →
// bias → mask → n-gram ban (sampling.rs:857-920 for the first and last; the
// others are this build's extensions).
template <int NT, uint32_t SEGMAX>
__device__ __forceinline__ float special_value(const RowCtx& c, const ProcLds<NT, SEGMAX>& L, uint32_t e,
                                               float l, uint32_t cw, uint32_t mw) {
    const uint32_t cnt = cw & ~CNT_BAN;
    if (c.cnt_on && cnt) {
        if (c.rep_on) {
            const float rep = c.p.repetition_penalty;
            l = l < 0.0f ? __fmul_rn(l, rep) : __fdiv_rn(l, rep);
        }
        if (c.pf_on) {
            l = __fsub_rn(l, __fmul_rn(c.p.frequency_penalty, (float)cnt));
            l = __fsub_rn(l, c.p.presence_penalty);
        }
    }
    if (c.bias_on)
        for (uint32_t j = 0; j < L.nbias; ++j)
            if (L.bias_id[j] == e) l = __fadd_rn(l, L.bias_v[j]);
    if (c.mask_on && !((mw >> (e & 31u)) & 1u)) l = -INFINITY;
    if (cw & CNT_BAN) l = -INFINITY;
    return l;
}

template <int DT>
__device__ __forceinline__ float raw_at(const char* rp, uint32_t e) {
    return DT == AXS_DTYPE_BF16 ? __uint_as_float((uint32_t)((const uint16_t*)rp)[e] << 16)
                                : ((const float*)rp)[e];
}

// count word of an unranked special id, from HBM: window occurrences and the
// n-gram ban (one scan each)
__device__ __forceinline__ uint32_t count_word_hbm(const KArgs& a, const RowCtx& c, uint32_t e) {
    uint32_t cnt = 0;
    if (c.cnt_on)
        for (int64_t i = c.w0; i < c.w1; ++i) cnt += a.hist[i] == e ? 1u : 0u;
    if (c.ban_on) {
        const int64_t nhist = c.w1 - c.h0;
        const uint32_t ng = c.p.no_repeat_ngram_size;
        int64_t keep = (int64_t)(c.p.ngram_window > ng ? c.p.ngram_window : ng);
        if (keep > nhist) keep = nhist;
        const int64_t hs = c.w1 - keep;
        const int64_t plen = (int64_t)ng - 1;
        for (int64_t s = 0; s + (int64_t)ng <= keep; ++s) {
            if (a.hist[hs + s + plen] != e) continue;
            bool match = true;
            for (int64_t j = 0; j < plen; ++j)
                if (a.hist[hs + s + j] != a.hist[c.w1 - plen + j]) {
                    match = false;
                    break;
                }
            if (match) {
                cnt |= CNT_BAN;
                break;
            }
        }
    }
    return cnt;
}

// f(e, processed logit) for the special ids of ranks rk0, rk0 + 1, ... (thread
// t takes ranks rk0 + t + k*NT, eight at a time with every load issued before
// any is used), or, for an unranked segment, for every special id by walking
// the bitmap.
template <int DT, int NT, uint32_t SEGMAX, typename F>
__device__ __forceinline__ void visit_specials(const KArgs& a, const RowCtx& c, const ProcLds<NT, SEGMAX>& L,
                                               bool ranked, uint32_t rk0, int r, const char* rp, uint32_t lo,
                                               uint32_t hi, F&& f) {
    using PL = ProcLds<NT, SEGMAX>;
    const int tid = threadIdx.x;
    if (ranked) {
        const uint32_t n = L.nspec;
        for (uint32_t b = rk0 + (uint32_t)tid; b < n; b += 8u * NT) {
            float raw[8];
            uint32_t mw[8];
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                const uint32_t rk = b + (uint32_t)q * NT;
                raw[q] = 0.0f;
                mw[q] = 0xFFFFFFFFu;
                if (rk < n) {
                    const uint32_t e = L.sid[rk];
                    raw[q] = raw_at<DT>(rp, e);
                    if (c.mask_on) mw[q] = a.mask[(size_t)r * a.mask_stride + (e >> 5)];
                }
            }
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                const uint32_t rk = b + (uint32_t)q * NT;
                if (rk < n) {
                    const uint32_t e = L.sid[rk];
                    f(e, special_value(c, L, e, raw[q], L.cnt[rk], mw[q]));
                }
            }
        }
        return;
    }
    const uint32_t nw = (hi - lo + 31u) / 32u;
    for (uint32_t wi = tid; wi < nw; wi += NT) {
        uint32_t bits = L.spec[wi];
        while (bits) {
            const uint32_t b = (uint32_t)__ffs((int)bits) - 1u;
            bits &= bits - 1u;
            const uint32_t e = lo + wi * 32u + b;
            const uint32_t mw = c.mask_on ? a.mask[(size_t)r * a.mask_stride + (e >> 5)] : 0xFFFFFFFFu;
            f(e, special_value(c, L, e, raw_at<DT>(rp, e), count_word_hbm(a, c, e), mw));
        }
    }
}

// Segment geometry: thread t holds NV vectors of EPV consecutive ids; vector j
// covers ids lo + (j*256 + t)*EPV + [0, EPV).
template <int DT>
struct Ev {
    static constexpr int EPV = DT == AXS_DTYPE_BF16 ? 8 : 4;
};

template <int DT, int NV>
struct Seg {
    static constexpr int EPV = Ev<DT>::EPV;
    u32x4 raw[NV];     // the logits as loaded (bf16 pairs or f32 bits)
    uint32_t mw[NV];   // mask word of each vector (when masked)
};

// Issues every load of the segment (16-byte nontemporal vectors when the rows
// are 16-byte aligned; element loads at the tail or otherwise).  ids >= hi read
// as NaN: never a maximum, never a candidate.
template <int DT, int NV>
__device__ __forceinline__ void seg_load(const KArgs& a, int r, uint32_t lo, uint32_t hi,
                                         bool vec, bool masked, Seg<DT, NV>& S) {
    constexpr int EPV = Ev<DT>::EPV;
    const int tid = threadIdx.x;
    const char* rp = row_ptr(a, r);
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        uint32_t e0 = lo + ((uint32_t)j * NT_CHUNK + tid) * EPV;
        if (vec && e0 + EPV <= hi) {
            S.raw[j] = __builtin_nontemporal_load((const u32x4*)(rp + (size_t)e0 * (EPV == 8 ? 2 : 4)));
        } else {
            uint32_t w[4];
            if (DT == AXS_DTYPE_BF16) {
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    uint32_t ea = e0 + 2 * q, eb = ea + 1;
                    uint32_t lo16 = ea < hi ? ((const uint16_t*)rp)[ea] : 0x7FC0u;
                    uint32_t hi16 = eb < hi ? ((const uint16_t*)rp)[eb] : 0x7FC0u;
                    w[q] = lo16 | (hi16 << 16);
                }
            } else {
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    uint32_t ea = e0 + q;
                    w[q] = ea < hi ? ((const uint32_t*)rp)[ea] : 0x7FC00000u;
                }
            }
            S.raw[j] = u32x4{w[0], w[1], w[2], w[3]};
        }
        S.mw[j] = (masked && e0 < hi) ? a.mask[(size_t)r * a.mask_stride + (e0 >> 5)] : 0xFFFFFFFFu;
    }
}

template <int DT>
__device__ __forceinline__ float unpack(const u32x4& w, int q) {
    if (DT == AXS_DTYPE_BF16) {
        uint32_t x = w[q >> 1];
        return __uint_as_float((q & 1) ? (x & 0xFFFF0000u) : (x << 16));
    }
    return __uint_as_float(w[q]);
}

// Register part of a pass: f(id, l) for every id the thread holds.  Special
// ids are skipped; they are visited by visit_specials.
template <int DT, int NV, int NT, uint32_t SEGMAX, typename F>
__device__ __forceinline__ void regs_visit(const RowCtx& c, const ProcLds<NT, SEGMAX>& L, uint32_t lo,
                                           Seg<DT, NV>& S, bool special, F&& f) {
    constexpr int EPV = Ev<DT>::EPV;
    const int tid = threadIdx.x;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        // recompute from the raw registers in every pass (keeps the unpacked
        // values out of the register budget)
        asm volatile("" : "+v"(S.raw[j]));
        const uint32_t e0 = lo + ((uint32_t)j * NT + tid) * EPV;
        const uint32_t off0 = e0 - lo;
        uint32_t sk = 0;
        if (special) sk = (L.spec[off0 >> 5] >> (off0 & 31u)) & ((1u << EPV) - 1u);
#pragma unroll
        for (int q = 0; q < EPV; ++q) {
            float l = unpack<DT>(S.raw[j], q);
            if (c.mask_on && !((S.mw[j] >> ((e0 + q) & 31u)) & 1u)) l = -INFINITY;
            if ((sk >> q) & 1u) continue;
            f(e0 + q, l);
        }
    }
}

// XCD-aware work-item mapping: the hardware hands workgroup b to XCD b % 8;
// give each XCD a contiguous range of (row, segment) items so the segments of
// a row share one L2.
__device__ __forceinline__ int64_t xcd_item(int64_t total) {
    int64_t per = (total + 7) / 8;
    int64_t b = blockIdx.x;
    return (b % 8) * per + b / 8;
}

// --------------------------------------------------------------------------
// outputs
// --------------------------------------------------------------------------
__device__ __forceinline__ void write_row(const KArgs& a, int r, uint32_t tok, float lp, uint32_t flags) {
    a.out_ids[r] = tok;
    if (a.out_lp) a.out_lp[r] = lp;
    if (a.out_flags) a.out_flags[r] = flags;
}

// A single-entry kept set (greedy / argmax fallback): token_distribution's
// (argmax, 1.0) (sampling.rs:655-657,672-674,688-690,697-699).
__device__ __forceinline__ void write_single_kept(const KArgs& a, int r, uint32_t tok) {
    if (a.out_kept && a.out_kept_cap > 0) a.out_kept[(size_t)r * a.out_kept_cap] = tok;
    if (a.out_kept_count) a.out_kept_count[r] = 1;
    if (a.ws_kept_id) {
        a.ws_kept_id[(size_t)r * KEPT_CAP] = tok;
        a.ws_kept_p[(size_t)r * KEPT_CAP] = 1.0f;
        a.rstate[r].kept = 1;
        a.rstate[r].nlist = 1;
        a.rstate[r].F = 1.0f;
    }
}

__device__ __forceinline__ double ulp_f(float x) {
    float ax = fabsf(x);
    return (double)nextafterf(ax, INFINITY) - (double)ax;
}

// lane k's value of v (k uniform)
__device__ __forceinline__ float lane_f(float v, int k) {
    return __uint_as_float((uint32_t)__builtin_amdgcn_readlane((int)__float_as_uint(v), k));
}

// --------------------------------------------------------------------------
// Row finish
// --------------------------------------------------------------------------
// first index i in [lo, hi) with S[i] >= t for non-decreasing S (hi if none)
__device__ __forceinline__ uint32_t first_ge(const float* S, uint32_t lo, uint32_t hi, float t) {
    uint32_t a = lo, b = hi;
    while (a < b) {
        uint32_t mid = a + (b - a) / 2;
        if (S[mid] >= t) b = mid;
        else a = mid + 1;
    }
    return a;
}

template <int NT>
struct FinLds {
    static constexpr uint32_t CAP = NT >= 1024 ? FIN_CAP : FIN_CAP / 2;
    uint64_t key[CAP];
    float S[CAP];            // running sums over the sorted candidates
    uint32_t cnt[MAX_SEGS];  // candidates published by each segment
    float rf[NT / 64];
    uint32_t ru[NT / 64];
    double rd[NT / 64];
    uint32_t n;
};

// first index i in [lo, hi) with S[i] >= t for non-decreasing S (hi if
// none), by the whole wave: one read per lane when the range fits in a wave,
// else a binary search (every lane the same, so the reads are broadcasts)
__device__ __forceinline__ uint32_t first_ge_wave(const float* S, uint32_t lo, uint32_t hi, float t) {
    const int lane = threadIdx.x & 63;
    if (hi - lo <= 64u) {
        const uint32_t i = lo + (uint32_t)lane;
        const uint64_t m = __ballot(i < hi && S[i] >= t);
        return m ? lo + (uint32_t)__builtin_ctzll(m) : hi;
    }
    return first_ge(S, lo, hi, t);
}

// Decisions over n sorted candidates (F.key), run by one wave with the
// row's uniform u.  The reference walks the candidates with f32 running sums
// (sampling.rs:283-316, 922-952): the top-p total, the nucleus cut, the
// filtered sum and the draw all read the same running sums
// S[i] = fl(S[i-1] + p_i) in the same order, so one sequential pass computes
// them (lane 0) and the cuts are searches.
template <int NT>
__device__ __forceinline__ void decide_sorted(const KArgs& a, int r, const axs_sampling_params& p, uint32_t mode,
                                              bool sorted, FinLds<NT>& F, uint32_t n, uint32_t flags0, float u) {
    const int lane = threadIdx.x & 63;
    auto P = [&](uint64_t k) { return sorted ? pdesc_p(k) : idasc_p(k); };
    auto ID = [&](uint64_t k) { return sorted ? pdesc_id(k) : idasc_id(k); };
    const uint32_t L = n;
    if (lane == 0) {
        float acc = 0.0f;
        uint32_t i = 0;
        for (; i + 8 <= L; i += 8) {
            float pv[8];
#pragma unroll
            for (int q = 0; q < 8; ++q) pv[q] = P(F.key[i + q]);
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                acc = __fadd_rn(acc, pv[q]);
                F.S[i + q] = acc;
            }
        }
        for (; i < L; ++i) {
            acc = __fadd_rn(acc, P(F.key[i]));
            F.S[i] = acc;
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const float* S = F.S;
    uint32_t flags = flags0 | AXS_FLAG_DREW;
    uint32_t nk = L;
    if (sorted && topp_active(p)) {
        // top-p over the full candidate mass (sampling.rs:931-945)
        const float total = S[L - 1];
        const float cutoff = __fmul_rn(p.top_p, total);
        const uint32_t j = first_ge_wave(S, 0, L, cutoff);
        nk = j < L ? j + 1 : L;
        const double up = (double)S[nk - 1] - (double)cutoff;
        const double lo = nk >= 2 ? (double)cutoff - (double)S[nk - 2] : INFINITY;
        if (fmin(up, lo) / (double)total < 1e-6 && (p.top_k == 0 || nk <= p.top_k)) flags |= AXS_FLAG_NEAR_NUCLEUS;
    }
    uint32_t kept = nk;
    if (sorted && p.top_k > 0 && kept > p.top_k) kept = p.top_k;
    if (sorted && kept < L) {
        const float pa = P(F.key[kept - 1]);
        const float pb = P(F.key[kept]);
        // near but not identical probabilities across the cut (identical
        // ones come from equal logits and are ordered by id everywhere)
        if (pa != pb && (double)pa - (double)pb <= 2.0 * ulp_f(pa)) flags |= AXS_FLAG_NEAR_TIE;
    }
    const float Fs = S[kept - 1];
    const float thr = __fmul_rn(u, Fs);
    uint32_t j = first_ge_wave(S, 0, kept, thr);
    if (j == kept) {
        // last maximum (sampling.rs:310-315); unreachable for u <= 1
        float bp = -1.0f;
        for (uint32_t i2 = 0; i2 < kept; ++i2)
            if (P(F.key[i2]) >= bp) {
                bp = P(F.key[i2]);
                j = i2;
            }
    } else {
        const double up = (double)S[j] - (double)thr;
        const double lo = j > 0 ? (double)thr - (double)S[j - 1] : INFINITY;
        if (fmin(up, lo) / (double)Fs < 1e-6) flags |= AXS_FLAG_NEAR_DRAW;
    }
    if (lane == 0) {
        const float pj = P(F.key[j]);
        write_row(a, r, ID(F.key[j]), logprob_of(__fdiv_rn(pj, Fs)), flags);
        if (a.out_kept_count) a.out_kept_count[r] = kept;
        if (a.ws_kept_id) {
            a.rstate[r].kept = kept;
            a.rstate[r].nlist = kept < KEPT_CAP ? kept : KEPT_CAP;
            a.rstate[r].F = Fs;
            a.rstate[r].flags = flags;
        }
    }
    if (a.out_kept && a.out_kept_cap > 0) {
        const uint32_t nw = kept < (uint32_t)a.out_kept_cap ? kept : (uint32_t)a.out_kept_cap;
        for (uint32_t i = lane; i < nw; i += 64) a.out_kept[(size_t)r * a.out_kept_cap + i] = ID(F.key[i]);
    }
    if (a.ws_kept_id) {
        const uint32_t nw = kept < KEPT_CAP ? kept : KEPT_CAP;
        for (uint32_t i = lane; i < nw; i += 64) {
            a.ws_kept_id[(size_t)r * KEPT_CAP + i] = ID(F.key[i]);
            a.ws_kept_p[(size_t)r * KEPT_CAP + i] = P(F.key[i]);
        }
    }
}

// A min-p row with no survivor (min_p > 1): argmax (sampling.rs:290-293).
// One thread.
__device__ __forceinline__ void empty_minp(const KArgs& a, int r, uint32_t am) {
    const uint32_t flags = AXS_FLAG_ARGMAX_FALLBACK | AXS_FLAG_EXACT_PATH;
    write_row(a, r, am, NAN, flags);
    write_single_kept(a, r, am);
    if (a.ws_kept_id) a.rstate[r].flags = flags;
}

// Row r's exact-path state from its maximum m (lowest id am).
__device__ __forceinline__ RowState exact_state(const KArgs& a, int r, const axs_sampling_params& p, float m, float inv,
                                                uint32_t mode, bool sorted, uint32_t am) {
    const bool minp = mode == M_MINP;
    RowState rs;
    rs.m = m;
    rs.inv = inv;
    rs.mode = mode;
    rs.sorted = sorted ? 1u : 0u;
    rs.ncompact = 0;
    rs.minp_mg = __float_as_uint(INFINITY);
    rs.amax = am;
    rs.flags = 0;
    rs.pmin = minp ? fmaxf(p.min_p, P_FLOOR) : P_FLOOR;
    rs.u = row_uniform(a, r, p);
    rs.kept = 0;
    rs.F = 0.0f;
    rs.nlist = 0;
    rs.pad[0] = rs.pad[1] = rs.pad[2] = 0;
    return rs;
}

// Lists row r for the exact path (second pass over its logits) with its
// maximum m.  One thread.
__device__ __forceinline__ void list_exact(const KArgs& a, int r, const axs_sampling_params& p, float m, float inv,
                                           uint32_t mode, bool sorted, uint32_t am) {
    a.rstate[r] = exact_state(a, r, p, m, inv, mode, sorted, am);
    const uint32_t idx = atomicAdd(a.exact_count, 1u);
    a.exact_rows[idx] = (uint32_t)r;
}

// The row's decision from its merged statistics: the maximum m and its lowest
// id am (NONE for an all-NaN row), the CS_* flags, gs = the sum of exp(l - m)
// over finite l (greedy logprob), and cands(f), which calls f(id, l) for this
// thread's share of the ncand gathered candidates (a superset of the ids that
// survive min-p).  Rows it cannot decide are listed for the exact path, or,
// with INPLACE, returned: true and their state in *xs, for the caller's
// workgroup to take the exact path itself.
// Called by all threads of the workgroup (uniform control flow).
template <int NT, bool INPLACE = false, typename CF>
__device__ __forceinline__ bool finish_decide(const KArgs& a, int r, const axs_sampling_params& p, float m,
                                              uint32_t am, uint32_t fl, double gs, uint32_t ncand,
                                              FinLds<NT>& F, CF&& cands, RowState* xs = nullptr) {
    const int tid = threadIdx.x;
    const uint32_t mode = row_mode(p);
    if (am == NONE) {  // all-NaN row: argmax_f32 → 0 (sampling.rs:966)
        am = 0;
        m = -INFINITY;
    }
    if (fl & CS_ERROR) {
        if (tid == 0) {
            write_row(a, r, 0u, NAN, AXS_FLAG_ERROR | ((fl & CS_CAPACITY) ? AXS_FLAG_CAPACITY : 0u));
            if (a.out_kept_count) a.out_kept_count[r] = 0;
            if (a.ws_kept_id) {
                a.rstate[r].kept = 0;
                a.rstate[r].nlist = 0;
                a.rstate[r].flags = AXS_FLAG_ERROR;
            }
        }
        return false;
    }
    if (a.lp_tokens) {
        // full_vocab_token_logprob (crates/ax-engine-mlx/src/sampling.rs:761-787):
        // t >= V -> -30; T <= 0 -> 0 for the first maximum, else -inf; no
        // finite maximum -> every term NaN -> zero sum -> -30; otherwise the
        // exact path's index-order normaliser at T
        const uint32_t t = a.lp_tokens[r];
        const bool direct = t >= (uint32_t)a.vocab || mode == M_GREEDY || !isfinite(m) ||
                            !isfinite(__fdiv_rn(1.0f, p.temperature));
        if (a.topn) {
            // top-N rows: T <= 0 lists the first maximum (0); no finite
            // maximum or temperature makes every p 0 (ids in order, -30)
            if (mode == M_GREEDY || !isfinite(m) || !isfinite(__fdiv_rn(1.0f, p.temperature))) {
                for (uint32_t k = (uint32_t)tid; k < a.topn; k += (uint32_t)NT) {
                    uint32_t id = NONE;
                    float lp = -INFINITY;
                    if (mode == M_GREEDY) {
                        if (k == 0) {
                            id = am;
                            lp = 0.0f;
                        }
                    } else if (k < (uint32_t)a.vocab) {
                        id = k;
                        lp = -30.0f;
                    }
                    a.topn_ids[(size_t)r * a.topn + k] = id;
                    a.topn_lp[(size_t)r * a.topn + k] = lp;
                }
                if (tid == 0) write_row(a, r, 0u, 0.0f, AXS_FLAG_EXACT_PATH);
                return false;
            }
        } else if (direct) {
            if (tid == 0) {
                float lp = -30.0f;
                if (t < (uint32_t)a.vocab && mode == M_GREEDY) lp = am == t ? 0.0f : -INFINITY;
                write_row(a, r, t, lp, AXS_FLAG_EXACT_PATH);
            }
            return false;
        }
        const float inv = __fdiv_rn(1.0f, p.temperature);
        if (INPLACE) {
            *xs = exact_state(a, r, p, m, inv, M_FAST, false, am);
            return true;
        }
        if (tid == 0) list_exact(a, r, p, m, inv, M_FAST, false, am);
        return false;
    }
    if (mode == M_GREEDY) {
        if (a.exact_lp && a.want_logprob && isfinite(m)) {
            // the core sampler's logprob -ln(sum exp(l - max)), its f32 sum
            // taken in index order over finite l
            // (crates/ax-engine-core/src/sampling.rs:177-190): the exact path's
            // index-order running sum of an untruncated law at T = 1
            if (INPLACE) {
                *xs = exact_state(a, r, p, m, 1.0f, M_GREEDY, false, am);
                return true;
            }
            if (tid == 0) list_exact(a, r, p, m, 1.0f, M_GREEDY, false, am);
            return false;
        }
        if (tid == 0) {
            const float lp = (a.want_logprob && isfinite(m) && gs > 0.0) ? (float)(-log(gs)) : NAN;
            write_row(a, r, am, lp, AXS_FLAG_GREEDY);
            write_single_kept(a, r, am);
            if (a.ws_kept_id) a.rstate[r].flags = AXS_FLAG_GREEDY;
        }
        return false;
    }
    const float inv = __fdiv_rn(1.0f, p.temperature);
    if (!(isfinite(m) && isfinite(inv))) {
        // every probability is zero or NaN → argmax (sampling.rs:264-266,279-281)
        if (tid == 0) {
            write_row(a, r, am, NAN, AXS_FLAG_ARGMAX_FALLBACK);
            write_single_kept(a, r, am);
            if (a.ws_kept_id) a.rstate[r].flags = AXS_FLAG_ARGMAX_FALLBACK;
        }
        return false;
    }
    const bool minp = mode == M_MINP;
    const bool sorted = minp ? filters_enabled(p) : (mode != M_FAST);
    bool exact = !minp || (fl & CS_OVERFLOW) || ncand > FinLds<NT>::CAP;
    if (!exact) {
        // min-p survivors: p = exp((l - m) / T) >= min_p (cutoff = min_p *
        // max_prob, max_prob = 1)
        if (tid == 0) F.n = 0;
        __syncthreads();
        float mg = INFINITY;
        cands([&](uint32_t id, float l) {
            const float pr = prob_of(l, m, inv);
            mg = fminf(mg, fabsf(pr - p.min_p) / p.min_p);
            if (!(pr >= p.min_p)) return;
            const uint32_t slot = atomicAdd(&F.n, 1u);
            F.key[slot] = sorted ? key_pdesc(pr, id) : key_idasc(pr, id);
        });
        mg = -block_max<NT>(-mg, F.rf);
        const uint32_t n = F.n;
        if (n == 0) {
            // min_p > 1: no survivor (sampling.rs:292)
            if (tid == 0) empty_minp(a, r, am);
            return false;
        }
        {
            const uint32_t flags0 = mg < 1e-6f ? AXS_FLAG_NEAR_MINP : 0u;
            constexpr uint32_t RS_MAX = 512;  // rank sort up to this many keys
            if (n <= RS_MAX) {
                // rank sort: each key's rank is the number of larger keys
                // (keys are distinct), read from LDS by every thread at once
                constexpr int KPT = (int)((RS_MAX + NT - 1) / NT);
                uint64_t mk[KPT];
                uint32_t rk[KPT];
#pragma unroll
                for (int k = 0; k < KPT; ++k) {
                    const uint32_t i = (uint32_t)tid + (uint32_t)k * NT;
                    mk[k] = i < n ? F.key[i] : 0ull;
                    rk[k] = 0;
                }
                for (uint32_t j = 0; j < n; ++j) {
                    const uint64_t kj = F.key[j];
#pragma unroll
                    for (int k = 0; k < KPT; ++k) rk[k] += kj > mk[k] ? 1u : 0u;
                }
                __syncthreads();
#pragma unroll
                for (int k = 0; k < KPT; ++k)
                    if ((uint32_t)tid + (uint32_t)k * NT < n) F.key[rk[k]] = mk[k];
            } else {
                const uint32_t np2 = next_pow2(n);
                for (uint32_t i = n + tid; i < np2; i += NT) F.key[i] = 0ull;
                __syncthreads();
                block_sort_desc<NT>(F.key, np2);
            }
            __syncthreads();
            if (tid < 64) decide_sorted<NT>(a, r, p, mode, sorted, F, n, flags0, row_uniform(a, r, p));
        }
    }
    if (exact) {
        if (INPLACE) {
            *xs = exact_state(a, r, p, m, inv, mode, sorted, am);
            return true;
        }
        if (tid == 0) list_exact(a, r, p, m, inv, mode, sorted, am);
    }
    return false;
}

// A min-p row decided by one wave from n <= 256 gathered candidates (a
// superset of its min-p survivors, sampling.rs:283-294): survivors p =
// exp((l - m) / T) >= min_p, ordered by (p desc, id asc) — or by id for an
// index-order draw — then decide_sorted.  x = (l - m) / T survives iff
// x >= xstar, the smallest f32 whose exp reaches min_p (the libm expf is
// monotone on x <= 0, checked exhaustively), so only survivors need their exp: after the ballot
// compaction into kbuf (LDS scratch of 256 keys, free once the candidates are
// read) each lane computes its survivors' in parallel.  Candidates within
// 1e-5 of ln(min_p) also get theirs, for the boundary flag.  The keys are then
// ranked (each key's rank = the keys above it, read as LDS broadcasts).
// cand_at(k) is the k-th candidate; lnmin = ln(min_p) and u the row's
// uniform.  Called by the 64 lanes of one wave; no block barriers.
template <int NT, typename CA>
__device__ __forceinline__ void wave_decide_minp(const KArgs& a, int r, const axs_sampling_params& p, float m, float inv,
                                                 uint32_t am, uint32_t n, CA&& cand_at, uint64_t* kbuf,
                                                 FinLds<NT>& F, double lnmin, float xstar, float u) {
    const int lane = threadIdx.x & 63;
    const bool sorted = filters_enabled(p);
    Cand mine[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t i = (uint32_t)lane + 64u * (uint32_t)j;
        mine[j] = i < n ? cand_at(i) : Cand{NONE, -INFINITY};
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    bool near = false;
    uint32_t ns = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        bool keep = false;
        uint64_t xk = 0;
        if (mine[j].id != NONE) {
            const float x = __fmul_rn(__fsub_rn(mine[j].l, m), inv);
            keep = x >= xstar;
            const double dx = (double)x - lnmin;
            if (dx >= -1e-5 && dx <= 1e-5) near |= fabsf(prob_of(mine[j].l, m, inv) - p.min_p) / p.min_p < 1e-6f;
            xk = ((uint64_t)__float_as_uint(x) << 32) | mine[j].id;
        }
        const uint64_t bk = __ballot(keep);
        if (keep) kbuf[ns + mbcnt64(bk)] = xk;
        ns += (uint32_t)__popcll(bk);
    }
    const bool anynear = __ballot(near) != 0ull;
    if (ns == 0) {  // min_p > 1: no survivor
        if (lane == 0) empty_minp(a, r, am);
        return;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // the survivors' keys: their probabilities, every lane at once
    const uint32_t nq = (ns + 63u) >> 6;  // keys per lane (uniform)
    uint64_t my[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const uint32_t i = (uint32_t)lane + 64u * (uint32_t)q;
        my[q] = 0ull;
        if (i < ns) {
            const uint64_t xk = kbuf[i];
            const float pr = prob_of(__uint_as_float((uint32_t)(xk >> 32)), 0.0f, 1.0f);  // exp_ref(x): x - 0, * 1 exact
            my[q] = sorted ? key_pdesc(pr, (uint32_t)xk) : key_idasc(pr, (uint32_t)xk);
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int q = 0; q < 4; ++q)
        if ((uint32_t)lane + 64u * (uint32_t)q < ns) kbuf[lane + 64 * q] = my[q];
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // rank = the keys above (keys are distinct), read as LDS broadcasts
    uint32_t rk[4] = {0u, 0u, 0u, 0u};
    for (uint32_t j = 0; j < ns; ++j) {
        const uint64_t kj = kbuf[j];
#pragma unroll
        for (int q = 0; q < 4; ++q)
            if ((uint32_t)q < nq) rk[q] += kj > my[q] ? 1u : 0u;
    }
#pragma unroll
    for (int q = 0; q < 4; ++q)
        if ((uint32_t)lane + 64u * (uint32_t)q < ns) F.key[rk[q]] = my[q];
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    decide_sorted<NT>(a, r, p, M_MINP, sorted, F, ns, anynear ? AXS_FLAG_NEAR_MINP : 0u, u);
}

// Merges the published results of the nseg segments of row r and decides it.
template <int NT>
__device__ __forceinline__ void finish_row(const KArgs& a, int r, int nseg, FinLds<NT>& F) {
    const int tid = threadIdx.x;
    float m = -INFINITY;
    uint32_t am = NONE;
    uint32_t fl = 0, ntot = 0;
    for (int c = tid; c < nseg; c += NT) {
        const ChunkStat st = sub_stat(&a.cstat[(size_t)r * nseg + c]);
        am_merge(m, am, st.m, st.amax);
        fl |= st.flags & 0xFFu;
        F.cnt[c] = st.flags >> 8;
        ntot += st.flags >> 8;
    }
    block_argmax<NT>(m, am, F.rf, F.ru);
    fl = block_or_u32<NT>(fl, F.ru);
    ntot = block_sum_u32<NT>(ntot, F.ru);
    double gs = 0.0;
    if (a.want_logprob) {
        for (int c = tid; c < nseg; c += NT) {
            const ChunkStat st = sub_stat(&a.cstat[(size_t)r * nseg + c]);
            if (isfinite(st.m) && st.amax != NONE) gs += (double)st.gsum * exp((double)st.m - (double)m);
        }
        gs = block_sum_d<NT>(gs, F.rd);
    }
    const Cand* pool = a.pool + (size_t)r * nseg * CAPS;
    if (a.mtp_amax && tid == 0) a.mtp_amax[r] = am == NONE ? 0u : am;  // argmax_f32 (all-NaN: 0)
    finish_decide<NT>(a, r, row_params(a, r), m, am, fl, gs, ntot, F, [&](auto&& f) {
        for (uint32_t i = tid; i < (uint32_t)nseg * CAPS; i += NT) {
            if (i % CAPS >= F.cnt[i / CAPS]) continue;
            const Cand cd = sub_cand(&pool[i]);
            f(cd.id, cd.l);
        }
    });
}

// --------------------------------------------------------------------------
// k_stream: the single pass over the logits.  One workgroup of NT threads per
// (row, segment); with one segment per row (large batches) the workgroup owns
// the whole row.  It builds the special-id bitmap of its segment from the
// history while its first tiles load, then streams the segment in
// double-buffered register tiles and keeps
//   - the argmax of the processed logits (special ids resolved one by one),
//   - min-p rows: every id within the min-p window of a lower bound of the
//     row maximum (so nothing that survives min-p is missed),
//   - greedy rows that want a logprob: the online sum of exp(l - max).
// A one-segment row is decided in place.  Otherwise each workgroup publishes
// its segment's result and the last one of the row to arrive (atomic arrival
// counter, no waiting) merges and decides.
// --------------------------------------------------------------------------
template <int DT, int TV, bool MASK>
struct Tile {
    u32x4 raw[TV];
    uint32_t mw[MASK ? TV : 1];
};

// The loads of one wave's chunk of a tile: `slot` is the thread's position in
// the tile (chunk's wave slot * 64 + lane); vector j covers ids
// t0 + (j*NT + slot)*EPV + [0, EPV).  Ids >= hi read as NaN.
template <int DT, int TV, bool MASK, int NT>
__device__ __forceinline__ void tile_load(const KArgs& a, int r, const char* rp, uint32_t t0, uint32_t hi,
                                          uint32_t slot, Tile<DT, TV, MASK>& T) {
    constexpr int EPV = Ev<DT>::EPV;
    constexpr uint32_t TILE = (uint32_t)NT * TV * EPV;
    const uint32_t tid = slot;
    if (a.vec && t0 + TILE <= hi) {
        // whole tile in range (uniform): 16-byte nontemporal loads only
#pragma unroll
        for (int j = 0; j < TV; ++j) {
            const uint32_t e0 = t0 + ((uint32_t)j * NT + tid) * EPV;
            T.raw[j] = __builtin_nontemporal_load((const u32x4*)(rp + (size_t)e0 * (EPV == 8 ? 2 : 4)));
            if (MASK) T.mw[j] = a.mask[(size_t)r * a.mask_stride + (e0 >> 5)];
        }
        return;
    }
#pragma unroll
    for (int j = 0; j < TV; ++j) {
        const uint32_t e0 = t0 + ((uint32_t)j * NT + tid) * EPV;
        if (a.vec && e0 + EPV <= hi) {
            T.raw[j] = __builtin_nontemporal_load((const u32x4*)(rp + (size_t)e0 * (EPV == 8 ? 2 : 4)));
        } else {
            uint32_t w[4];
            if (DT == AXS_DTYPE_BF16) {
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const uint32_t ea = e0 + 2 * q, eb = ea + 1;
                    const uint32_t lo16 = ea < hi ? ((const uint16_t*)rp)[ea] : 0x7FC0u;
                    const uint32_t hi16 = eb < hi ? ((const uint16_t*)rp)[eb] : 0x7FC0u;
                    w[q] = lo16 | (hi16 << 16);
                }
            } else {
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const uint32_t ea = e0 + q;
                    w[q] = ea < hi ? ((const uint32_t*)rp)[ea] : 0x7FC00000u;
                }
            }
            T.raw[j] = u32x4{w[0], w[1], w[2], w[3]};
        }
        if (MASK) T.mw[j] = e0 < hi ? a.mask[(size_t)r * a.mask_stride + (e0 >> 5)] : 0u;
    }
}

// Whole-vector tiles (16-byte aligned rows, segment end a multiple of EPV):
// every lane loads, the lanes past the end re-read the tile's first vector
// (their values are discarded by index), so the loads are the same on every
// path and the compiler can keep the next tile in flight.
// (valid = false: a chunk past the end of the work; every lane reads the
// row's first vector, one cache line, so the loads still issue)
template <int DT, int TV, bool MASK, int NT>
__device__ __forceinline__ void tile_load_fast(const KArgs& a, int r, const char* rp, uint32_t t0, uint32_t hi,
                                               uint32_t slot, bool valid, Tile<DT, TV, MASK>& T) {
    constexpr int EPV = Ev<DT>::EPV;
#pragma unroll
    for (int j = 0; j < TV; ++j) {
        uint32_t e0 = t0 + ((uint32_t)j * NT + slot) * EPV;
        e0 = e0 < hi ? e0 : t0;
        if (!valid) e0 = 0u;
        T.raw[j] = __builtin_nontemporal_load((const u32x4*)(rp + (size_t)e0 * (EPV == 8 ? 2 : 4)));
        if (MASK) T.mw[j] = a.mask[(size_t)r * a.mask_stride + (e0 >> 5)];
    }
}

template <int NT, uint32_t SEGMAX>
struct StreamLds {
    static constexpr uint32_t CAPC = NT >= 1024 ? 2048u : 1024u;  // gathered candidates
    union {
        ProcLds<NT, SEGMAX> P;
        FinLds<NT> F;
    } u;
    Cand cand[CAPC];
    u32x4 xt[256];  // bit pattern of a vector → per-word mask of its marked elements
    float red[NT / 64];
    float redf[NT / 64];
    uint32_t redu[NT / 64];
    uint32_t ncand;
    uint32_t next;  // next unclaimed chunk
    uint32_t last;
};

template <int DT, int TV, bool MASK, int NT, uint32_t SEGMAX, bool FAST>
__global__ __launch_bounds__(NT) void k_stream(KArgs a) {
    using SLT = StreamLds<NT, SEGMAX>;
    constexpr int EPV = Ev<DT>::EPV;
    constexpr uint32_t TILE = (uint32_t)NT * TV * EPV;
    constexpr uint32_t CAPC = SLT::CAPC;
    constexpr int CPT = (int)(CAPC / NT);  // candidates per thread
    __shared__ SLT SL;
    ProcLds<NT, SEGMAX>& L = SL.u.P;
    const int tid = threadIdx.x;
    const int wv = tid >> 6, lane = tid & 63;
    const int nseg = a.snch;
    const int64_t total = (int64_t)a.nrows * nseg;
    const int64_t w = xcd_item(total);
    if (w >= total) return;
    const int r = (int)(w / nseg);
    const int si = (int)(w % nseg);
    const uint32_t lo = (uint32_t)si * (uint32_t)a.schunk;
    const uint32_t hi = min(lo + (uint32_t)a.schunk, (uint32_t)a.vocab);
    const uint32_t ntile = (hi - lo + TILE - 1) / TILE;
    const char* rp = row_ptr(a, r);
    // The workgroups start their segments at different tiles (the order of
    // visits does not matter: ties are broken by id), so that they do not
    // all read the same HBM channels at the same time.
    const uint32_t rot = (uint32_t)(((uint64_t)w * 5u) % ntile);
    auto tbase = [&](uint32_t k) {
        uint32_t t = k + rot;
        if (t >= ntile) t -= ntile;
        return lo + t * TILE;
    };

    // loads in flight before anything waits: the segment's first two tiles,
    // then the first round of the repetition window
    // The segment is cut into chunks, one wave's share of a tile (64 lanes x
    // TV vectors): chunk c is slot c % NW of tile c / NW.  Each wave starts
    // with chunks wv and NW + wv and then takes the next unclaimed chunk from
    // an LDS counter, so waves that get their data sooner do more of the work.
    constexpr uint32_t NW = NT / 64;
    const uint32_t nchunk = ntile * NW;
    auto chunk_t0 = [&](uint32_t ch) { return tbase(ch / NW); };
    auto chunk_slot = [&](uint32_t ch) { return (ch % NW) * 64u + (uint32_t)lane; };
    auto load = [&](Tile<DT, TV, MASK>& T, uint32_t ch) __attribute__((always_inline)) {
        const bool valid = ch < nchunk;  // wave-uniform
        if (FAST) {
            tile_load_fast<DT, TV, MASK, NT>(a, r, rp, valid ? chunk_t0(ch) : lo, hi, valid ? chunk_slot(ch) : 0u,
                                             valid, T);
        } else {
            const uint32_t t0 = valid ? chunk_t0(ch) : lo;
            tile_load<DT, TV, MASK, NT>(a, r, rp, t0, valid ? hi : t0, valid ? chunk_slot(ch) : 0u, T);
        }
    };
    // FAST: 16-byte aligned rows whose length is a multiple of EPV
    uint32_t c0 = (uint32_t)wv, c1 = NW + (uint32_t)wv;
    Tile<DT, TV, MASK> b0, b1;
    load(b0, c0);
    load(b1, c1);
    if (tid == 0) SL.next = 2u * NW;
    const RowCtx c = make_ctx(a, r);
    HistPre<NT> hp;
    hist_prefetch<NT>(a, c, hp);
    const bool special = c.cnt_on || c.bias_on || c.ban_on;
    if (special || MASK) {
        // expansion table: bit q of an index marks element q of a vector; the
        // entry holds, per 32-bit word of the vector, all ones over the
        // marked elements (the barriers of proc_build publish it)
        for (uint32_t i = tid; i < 256u; i += NT) {
            u32x4 m;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                if (DT == AXS_DTYPE_BF16)
                    m[k] = (((i >> (2 * k)) & 1u) ? 0x0000FFFFu : 0u) | (((i >> (2 * k + 1)) & 1u) ? 0xFFFF0000u : 0u);
                else
                    m[k] = ((i >> k) & 1u) ? 0xFFFFFFFFu : 0u;
            }
            SL.xt[i] = m;
        }
    }
    if (c.any_proc) proc_build<NT, SEGMAX>(a, c, lo, hi, L, hp);
    bool ranked = true;
    if (special) ranked = proc_rank<NT, SEGMAX>(a, c, lo, hi, L, hp);
    // the first SPK*NT special ids' raw logits and mask words: loaded now,
    // used after the stream, so the loads never hold up a tile
    constexpr int SPK = 4;
    // (kept as the loaded bits: converting them here would wait for the loads)
    const uint32_t nspec = (special && ranked) ? L.nspec : 0u;
    uint32_t sraw[SPK];
    uint32_t smw[SPK];
#pragma unroll
    for (int k = 0; k < SPK; ++k) {
        // unconditional loads (rank 0's id stands in past the end), so no
        // branch merges a value that would have to be waited for here
        const uint32_t rk = (uint32_t)tid + (uint32_t)k * NT;
        const uint32_t e = rk < nspec ? L.sid[rk] : lo;
        sraw[k] = DT == AXS_DTYPE_BF16 ? (uint32_t)((const uint16_t*)rp)[e] : ((const uint32_t*)rp)[e];
        smw[k] = MASK ? a.mask[(size_t)r * a.mask_stride + (e >> 5)] : 0xFFFFFFFFu;
    }
    if (tid == 0) SL.ncand = 0;

    const uint32_t mode = c.mode;
    const float inv = __fdiv_rn(1.0f, c.p.temperature);
    const bool gather = mode == M_MINP && isfinite(inv);
    // the approximate greedy logprob of the stream (rows that take the exact
    // path for it need none)
    const bool gsum_on = mode == M_GREEDY && a.want_logprob && !a.exact_lp;
    const float thr = gather ? __fsub_rn(ln_f32(c.p.min_p), 1e-3f) : 0.0f;
    const uint32_t sflags = c.err ? CS_ERROR : ((c.any_proc && L.err) ? (CS_ERROR | CS_CAPACITY) : 0u);

    float tm = -INFINITY;             // thread maximum (non-special ids)
    uint32_t ta = NONE;               // its lowest id
    float gm = -INFINITY, gs = 0.0f;  // greedy logprob: sum of exp(l - gm)
    float mrun = -INFINITY;           // a lower bound of the row maximum (wave-uniform)
    float lpre = INFINITY;            // l < lpre ⇒ not a candidate (wave-uniform)

    auto set_pre = [&]() {
        // (l - mrun) * inv >= thr needs l >= mrun + thr / inv; the bound is
        // lowered by 0.01 nats and a few ulps so rounding never excludes one
        if (!isfinite(mrun)) {
            lpre = INFINITY;
        } else if (inv > 0.0f) {
            const double bnd = (double)mrun + ((double)thr - 0.01) / (double)inv;
            const double slack = 4.0 * fmax(fabs((double)mrun), fabs(bnd)) * 1.2e-7;
            lpre = (float)(bnd - slack);
        } else {
            lpre = -INFINITY;
        }
    };
    auto add_cand = [&](uint32_t e, float l) {
        const uint32_t slot = atomicAdd(&SL.ncand, 1u);
        if (slot < CAPC) {
            SL.cand[slot].id = e;
            SL.cand[slot].l = l;
        }
    };
    auto gsum_add = [&](float l) {
        if (isfinite(l)) {
            if (l > gm) {
                gs = __fmaf_rn(gs, __expf(gm - l), 1.0f);
                gm = l;
            } else {
                gs += __expf(l - gm);
            }
        }
    };
    // the EPV logits of a vector as the processors see them, with the special
    // ids as NaN: never a maximum, never gathered
    // (on the raw words: disallowed elements become -inf and special ones an
    // all-ones pattern, which is a NaN in both formats)
    constexpr uint32_t EMASK = (1u << EPV) - 1u;
    constexpr uint32_t NINF = DT == AXS_DTYPE_BF16 ? 0xFF80FF80u : 0xFF800000u;
    auto vec_vals = [&](u32x4 raw, uint32_t mw, uint32_t e0, float* v) {
        if (MASK) {
            const u32x4 m = SL.xt[(~mw >> (e0 & 31u)) & EMASK];
#pragma unroll
            for (int k = 0; k < 4; ++k) raw[k] = (m[k] & NINF) | (~m[k] & raw[k]);
        }
        if (special) {
            const uint32_t off0 = e0 - lo;
            const u32x4 m = SL.xt[(L.spec[off0 >> 5] >> (off0 & 31u)) & EMASK];
#pragma unroll
            for (int k = 0; k < 4; ++k) raw[k] |= m[k];
        }
#pragma unroll
        for (int q = 0; q < EPV; ++q) v[q] = unpack<DT>(raw, q);
    };
    // Per vector: its maximum decides everything.  The thread keeps the
    // lowest-id vector holding its running maximum; the element is resolved
    // once at the end.  Only vectors reaching the gather bound, and greedy
    // rows that want a logprob, look at single elements.
    uint32_t tj = NONE;  // first id of the best vector
    u32x4 traw = u32x4{0u, 0u, 0u, 0u};
    uint32_t tmw = 0xFFFFFFFFu;
    auto process = [&](Tile<DT, TV, MASK>& T, uint32_t ch) {
        const uint32_t t0 = chunk_t0(ch), sl = chunk_slot(ch);
#pragma unroll
        for (int j = 0; j < TV; ++j) {
            asm volatile("" : "+v"(T.raw[j]));
            const uint32_t e0 = t0 + ((uint32_t)j * NT + sl) * EPV;
            const uint32_t mw = MASK ? T.mw[j] : 0xFFFFFFFFu;
            float v[EPV];
            vec_vals(T.raw[j], mw, e0, v);
            float vm = v[0];
#pragma unroll
            for (int q = 1; q < EPV; ++q) vm = fmaxf(vm, v[q]);
            if (e0 >= hi) vm = __builtin_nanf("");  // a lane past the segment end
            if (vm > tm || (vm == tm && e0 < tj)) {
                tm = vm;
                tj = e0;
                traw = T.raw[j];
                tmw = mw;
            }
            if (gather && vm >= lpre) {
                // one slot reservation for all of the vector's candidates
                uint32_t qm = 0;
#pragma unroll
                for (int q = 0; q < EPV; ++q)
                    if (v[q] >= lpre && __fmul_rn(__fsub_rn(v[q], mrun), inv) >= thr) qm |= 1u << q;
                if (qm) {
                    uint32_t slot = atomicAdd(&SL.ncand, (uint32_t)__popc(qm));
#pragma unroll
                    for (int q = 0; q < EPV; ++q)
                        if ((qm >> q) & 1u) {
                            if (slot < CAPC) {
                                SL.cand[slot].id = e0 + q;
                                SL.cand[slot].l = v[q];
                            }
                            ++slot;
                        }
                }
            }
            if (gsum_on && e0 < hi) {
#pragma unroll
                for (int q = 0; q < EPV; ++q) gsum_add(v[q]);
            }
            // one vector at a time: interleaving them only raises register
            // pressure (the other waves hide the latencies)
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    // maximum of a tile (seeds the gather bound)
    auto tile_max = [&](Tile<DT, TV, MASK>& T, uint32_t ch) {
        const uint32_t t0 = chunk_t0(ch), sl = chunk_slot(ch);
        float pm = -INFINITY;
#pragma unroll
        for (int j = 0; j < TV; ++j) {
            const uint32_t e0 = t0 + ((uint32_t)j * NT + sl) * EPV;
            float v[EPV];
            vec_vals(T.raw[j], MASK ? T.mw[j] : 0xFFFFFFFFu, e0, v);
            if (e0 < hi)
#pragma unroll
                for (int q = 0; q < EPV; ++q) pm = fmaxf(pm, v[q]);
        }
        return pm;
    };
    // raises the wave's bound with its running maximum (no barrier)
    auto raise = [&]() {
        mrun = fmaxf(mrun, wave_max_dpp(tm));
        set_pre();
    };

    // chunk 0..NW-1 (tile 0) seeds the gather bound with its block maximum:
    // one barrier, then waves go alone; without a gather the barrier only
    // publishes the chunk counter
    if (gather) {
        const float v = wave_max_dpp(c0 < nchunk ? tile_max(b0, c0) : -INFINITY);
        if (lane == 0) SL.red[wv] = v;
    }
    __syncthreads();
    if (gather) {
        float mm = SL.red[0];
#pragma unroll
        for (int k = 1; k < NT / 64; ++k) mm = fmaxf(mm, SL.red[k]);
        mrun = mm;
        set_pre();
    }
    // claims the next chunk for this wave; a greedy logprob row takes every
    // NW-th chunk in order instead, so that each lane's sum runs over the same
    // elements in the same order on every call (a reproducible logprob)
    auto grab = [&](uint32_t cur) {
        if (gsum_on) return cur + 2u * NW;
        uint32_t ch = 0;
        if (lane == 0) ch = atomicAdd(&SL.next, 1u);
        return (uint32_t)__builtin_amdgcn_readfirstlane((int)ch);
    };
    // process a chunk (seeding the bound first if the wave has none yet),
    // claim the next one into the same buffer, raise the bound
    auto step = [&](Tile<DT, TV, MASK>& T, uint32_t& ch) __attribute__((always_inline)) {
        if (gather && mrun == -INFINITY) {
            mrun = wave_max_dpp(tile_max(T, ch));
            set_pre();
        }
        process(T, ch);
        ch = grab(ch);
        load(T, ch);
        if (gather) raise();
    };
    // Both buffers are refilled unconditionally (a claim past the end loads a
    // dummy line), so the compiler's wait for one buffer leaves the other's
    // loads in flight.  Claims only grow: once one is past the end, so are
    // all later ones.
    while (c0 < nchunk) {
        step(b0, c0);
        if (c1 >= nchunk) break;
        step(b1, c1);
    }
    // the first element of the best vector that attains the maximum
    if (tj != NONE) {
        float v[EPV];
        vec_vals(traw, tmw, tj, v);
        uint32_t q0 = NONE;
#pragma unroll
        for (int q = EPV - 1; q >= 0; --q)
            if (v[q] == tm) q0 = (uint32_t)q;
        ta = tj + q0;
    }
    // the special ids' processed values
    if (special) {
        auto visit = [&](uint32_t e, float l) {
            am_merge(tm, ta, l, isnan(l) ? NONE : e);
            if (gather && l > -INFINITY &&
                (mrun == -INFINITY || __fmul_rn(__fsub_rn(l, mrun), inv) >= thr))
                add_cand(e, l);
            if (gsum_on) gsum_add(l);
        };
#pragma unroll
        for (int k = 0; k < SPK; ++k) {
            const uint32_t rk = (uint32_t)tid + (uint32_t)k * NT;
            if (rk < nspec) {
                const uint32_t e = L.sid[rk];
                const float l = __uint_as_float(DT == AXS_DTYPE_BF16 ? sraw[k] << 16 : sraw[k]);
                visit(e, special_value(c, L, e, l, L.cnt[rk], smw[k]));
            }
        }
        if (!ranked || nspec > (uint32_t)SPK * NT)
            visit_specials<DT, NT, SEGMAX>(a, c, L, ranked, (uint32_t)SPK * NT, r, rp, lo, hi, visit);
    }

    // segment results
    __syncthreads();
    float bm = tm;
    uint32_t bi = ta;
    block_argmax<NT>(bm, bi, SL.redf, SL.redu);
    ChunkStat st;
    st.m = bi == NONE ? -INFINITY : bm;
    st.amax = bi;
    st.flags = sflags;
    st.gsum = 0.0f;
    if (gsum_on && isfinite(st.m)) {
        const float part = isfinite(gm) ? gs * __expf(gm - st.m) : 0.0f;
        st.gsum = block_sum_f<NT>(part, SL.redf);
    }
    const uint32_t n = gather ? SL.ncand : 0u;
    if (gather && n > CAPC) st.flags |= CS_OVERFLOW;

    if (nseg == 1) {
        // the whole row is here: decide it in place
        finish_decide<NT>(a, r, c.p, st.m, st.amax, st.flags, (double)st.gsum, n, SL.u.F, [&](auto&& f) {
            for (uint32_t i = tid; i < n; i += NT) f(SL.cand[i].id, SL.cand[i].l);
        });
        return;
    }

    if (gather && n <= CAPC) {
        // publish the candidates within the min-p window of the segment
        // maximum (<= the row maximum, so still every possible survivor)
        Cand mine[CPT];
        uint32_t keep = 0, cnt = 0;
#pragma unroll
        for (int k = 0; k < CPT; ++k) {
            const uint32_t i = (uint32_t)tid + (uint32_t)k * NT;
            mine[k].id = 0;
            mine[k].l = 0.0f;
            if (i < n) {
                const Cand cd = SL.cand[i];
                if (__fmul_rn(__fsub_rn(cd.l, st.m), inv) >= thr) {
                    mine[k] = cd;
                    keep |= 1u << k;
                    ++cnt;
                }
            }
        }
        uint32_t tot;
        uint32_t pre = block_excl_scan_u32<NT>(cnt, SL.redu, &tot);
        if (tot > CAPS) {
            st.flags |= CS_OVERFLOW;
        } else {
            Cand* dst = a.pool + ((size_t)r * nseg + si) * CAPS;
#pragma unroll
            for (int k = 0; k < CPT; ++k)
                if ((keep >> k) & 1u) pub_cand(&dst[pre++], mine[k]);
            st.flags |= tot << 8;
        }
    }
    if (tid == 0) pub_stat(&a.cstat[(size_t)r * nseg + si], st);

    // the last workgroup of the row to get here finishes it; the counter
    // wraps back to 0 for the next call
    wait_mem();
    __syncthreads();
    if (tid == 0) {
        const uint32_t old = atomicInc(&a.row_done[r], (uint32_t)nseg - 1u);
        SL.last = old == (uint32_t)nseg - 1u ? 1u : 0u;
    }
    __syncthreads();
    if (!SL.last) return;
    finish_row<NT>(a, r, nseg, SL.u.F);
}

// --------------------------------------------------------------------------
// k_row: one 1024-thread workgroup per row (large batches), the row decided
// in place.  The logits stream starts at once: every wave issues its first
// chunk's loads, reads the row's context, issues its share of the repetition
// window (which then queues behind one chunk per wave, not two) and then its
// second chunk; the window is staged in LDS.  The special-id tables are then
//   spec  a bit per id: in the window, biased or banned
//   hkey/hval  an open-addressing hash of the special ids: window count,
//         bias entry, n-gram ban
// A vector whose raw maximum reaches the running bound is rare; a wave queues
// such vectors in LDS and looks at them 64 at a time, one lane each.  The look
// reads special elements as NaN (never a maximum, never a candidate) and
// captures their raw values into a shared capture pool (a wave claims a run
// of slots with one LDS atomic, a ballot places its lanes); after the stream
// each captured element gets every processor from the hash and joins the
// maximum and the candidates.  No scattered loads.  The row's maximum is
// merged from per-wave DPP reductions, and a min-p row with at most 256
// candidates is decided by wave 0 alone (survivors by a precomputed exp edge,
// ranked by LDS broadcasts, no block barriers).
// --------------------------------------------------------------------------
constexpr int RT = 1024;               // threads of a row workgroup
constexpr int RWV = RT / 64;           // its waves
constexpr int HWAVES = 2;              // waves that fetch the window before their tiles
constexpr uint32_t HPRE = 2048;        // window tokens staged through LDS
constexpr uint32_t HBITS = 12;
constexpr uint32_t HSZ = 1u << HBITS;  // hash slots
constexpr uint32_t CAPP = 2048;        // captured special elements per row (shared pool)
constexpr uint32_t CANDP = 2048;       // min-p candidates per row (shared pool)
constexpr uint32_t QN = 64;            // relevant vectors a wave queues before looking at them
constexpr uint32_t RBCAP = 1024;       // bias entries per row
constexpr uint32_t HV_CNT = 0x000FFFFFu;  // window count
constexpr uint32_t HV_BSH = 20;           // bias entry index + 1, or HV_BMULTI
constexpr uint32_t HV_BMULTI = 0x7FFu;
constexpr uint32_t HV_BAN = 0x80000000u;
constexpr uint32_t CAP_OFF = 0x80000000u;  // captured element is masked off
constexpr uint32_t RERR_HASH = 1u;         // more special ids than hash slots
constexpr uint32_t RERR_BIAS = 2u;         // more bias entries than RBCAP
constexpr uint32_t RERR_CAP = 4u;          // more than CAPP captures

// LDS of the exact path's sort and running sums (one row per workgroup)
constexpr uint32_t NMIXW = NBUCKET / 32;
constexpr uint32_t NTAILB = 5120;                  // tail buckets: p in [2^-24, 2^-14)
constexpr uint32_t BEND_STRIDE = NBUCKET + NTAILB;  // per row: bucket ends, top-value counts
// LDS state of block_exact_sums
struct SumLds {
    Xd w[NT_EX / 64];
    float s;
    uint32_t cross, npc;
    uint32_t pc[32];  // predicted crossings of a tile
};

struct ExLds {
    uint32_t cnt[NBUCKET];  // bucket counts, then bucket ends; then sort scratch
    uint64_t stage[(NT_EX / 64) * 128];  // each wave's window of keys
    uint32_t mixed[NMIXW];  // buckets of more than 64 keys with two different p
    uint32_t topv[NMIXW];   // tail buckets holding their top value
    uint32_t done[NMIXW];   // tail buckets sorted and summed element by element
    uint32_t u[NT_EX / 64];
    uint32_t k, cross, err, xc;
    SumLds sum;  // the exact running sums' state
};

struct RowLds {
    union {
        struct {
            uint32_t spec[ROW_MAX / 32];
            uint32_t hkey[HSZ];
            uint32_t hval[HSZ];
        } p;
        FinLds<RT> F;
    } u;
    union {
        struct {
            Cand cand[CANDP];       // min-p candidates (a wave claims a run of slots per batch)
            uint32_t stage[HPRE];   // the window's first tokens (read by the hash build during the stream)
            Cand cap[CAPP];         // captured special elements (likewise)
            u32x4 qraw[RWV][QN];    // each wave's queue of relevant vectors ...
            uint32_t qe0[RWV][QN];  // ... their first ids ...
            uint32_t qmw[RWV][QN];  // ... and mask words
        };
        ExLds ex;  // a row that takes the exact path in place (the above are dead by then)
    };
    uint32_t ncand, ncap;  // pool claims (may exceed the pools: overflow)
    uint32_t bias_id[RBCAP];
    float bias_v[RBCAP];
    u32x4 xt[256];
    float wm[RWV];      // per-wave maximum ...
    uint32_t wa[RWV];   // ... and its lowest id
    float gm[RWV];      // per-wave greedy logprob partials: maximum ...
    float gs[RWV];      // ... and sum of exp(l - maximum)
    uint32_t next, nbias, err;
    uint32_t xn;    // exact path in place: compacted keys
    uint32_t bpos;  // some bias entry is not <= 0 (it may raise a logit)
    int gmax;       // shared lower bound of the row maximum (ordered-int encoding)
};

__device__ __forceinline__ int f2ord(float f) {
    const int k = __float_as_int(f);
    return k >= 0 ? k : k ^ 0x7FFFFFFF;
}
__device__ __forceinline__ float ord2f(int k) { return __int_as_float(k >= 0 ? k : k ^ 0x7FFFFFFF); }

// The smallest f32 x with exp_ref(x) >= min_p (+inf when none, min_p > 1):
// ln(min_p) rounded, moved by ulps; where exp rounds to the same value over
// many ulps (near 0), a bisection over the ordered encoding of [-FLT_MAX, 0].
__device__ __forceinline__ float minp_edge(float min_p) {
    if (!(min_p <= 1.0f)) return INFINITY;
    float x = (float)log((double)min_p);
    for (int it = 0; it < 4 && !(exp_ref(x) >= min_p); ++it) x = nextafterf(x, INFINITY);
    for (int it = 0; it < 4 && exp_ref(nextafterf(x, -INFINITY)) >= min_p; ++it) x = nextafterf(x, -INFINITY);
    if (exp_ref(x) >= min_p && !(exp_ref(nextafterf(x, -INFINITY)) >= min_p)) return x;
    int lo = f2ord(-__FLT_MAX__), hi = f2ord(0.0f);  // exp_ref(0) = 1 >= min_p
    while (hi - lo > 1) {
        const int mid = lo + (hi - lo) / 2;
        if (exp_ref(ord2f(mid)) >= min_p) hi = mid;
        else lo = mid;
    }
    return ord2f(hi);
}

// Bounds of a sorted row's exact path, on x = (l - m) * inv: the keys are the
// elements with x >= xe (p >= pmin: exp_ref is monotone), and the min-p
// boundary flag reads the elements with x in [xm0, xm1) (p within 2e-6
// relative of min_p; the flag's 1e-6 margin lies inside).
struct KeyEdge {
    float xe, xm0, xm1;
};
__device__ __forceinline__ KeyEdge key_edges(float pmin, bool minp, float min_p) {
    KeyEdge k;
    k.xe = minp_edge(pmin);
    k.xm0 = k.xm1 = INFINITY;
    if (minp) {
        k.xm0 = minp_edge(min_p * (1.0f - 2e-6f));
        k.xm1 = minp_edge(min_p * (1.0f + 2e-6f));
    }
    return k;
}

// home slot of id t: the murmur3 finalizer, so that arithmetic progressions
// of ids (a permuted vocabulary's top ranks, for one) do not cluster
__device__ __forceinline__ uint32_t hslot0(uint32_t t) {
    t ^= t >> 16;
    t *= 0x85EBCA6Bu;
    t ^= t >> 13;
    t *= 0xC2B2AE35u;
    t ^= t >> 16;
    return t & (HSZ - 1u);
}

// slot of special id t, inserting it if absent; NONE when HPROBE slots from
// its home are taken by other ids (the row then resolves its special ids
// from HBM)
constexpr uint32_t HPROBE = 256;
__device__ __forceinline__ uint32_t hash_insert(uint32_t* hkey, uint32_t t) {
    uint32_t h = hslot0(t);
    for (uint32_t k = 0; k < HPROBE; ++k) {
        const uint32_t old = atomicCAS(&hkey[h], NONE, t);
        if (old == NONE || old == t) return h;
        h = (h + 1u) & (HSZ - 1u);
    }
    return NONE;
}

// slot of special id t (present by construction unless an insert failed)
__device__ __forceinline__ uint32_t hash_find(const uint32_t* hkey, uint32_t t) {
    uint32_t h = hslot0(t);
    for (uint32_t k = 0; k < HPROBE; ++k) {
        const uint32_t key = hkey[h];
        if (key == t) return h;
        if (key == NONE) return NONE;
        h = (h + 1u) & (HSZ - 1u);
    }
    return NONE;
}

// Every processor in order for special id e with raw logit l: repetition →
// presence/frequency → bias → mask → n-gram ban (sampling.rs:875-920 for the
// first and last; the others are this build's extensions).  cnt is the id's
// window count, bcode its bias entry (index + 1, 0 for none, HV_BMULTI for
// several), off whether the mask disallows it.
__device__ __forceinline__ float row_special_value(const RowCtx& c, const RowLds& SL, uint32_t e, float l,
                                                  uint32_t cnt, uint32_t bcode, bool ban, bool off) {
    if (c.cnt_on && cnt) {
        if (c.rep_on) {
            const float rep = c.p.repetition_penalty;
            l = l < 0.0f ? __fmul_rn(l, rep) : __fdiv_rn(l, rep);
        }
        if (c.pf_on) {
            l = __fsub_rn(l, __fmul_rn(c.p.frequency_penalty, (float)cnt));
            l = __fsub_rn(l, c.p.presence_penalty);
        }
    }
    if (c.bias_on) {
        if (bcode == HV_BMULTI) {
            // several entries for this id: added one by one in list order
            for (uint32_t j = 0; j < SL.nbias; ++j)
                if (SL.bias_id[j] == e) l = __fadd_rn(l, SL.bias_v[j]);
        } else if (bcode) {
            l = __fadd_rn(l, SL.bias_v[bcode - 1u]);
        }
    }
    if (off) l = -INFINITY;
    if (ban) l = -INFINITY;
    return l;
}

template <uint32_t XI>
__device__ __forceinline__ void exact_row(const KArgs& a, int r, const RowState& rs, ExLds& X);

template <int DT, int TV, bool MASK, bool FAST>
__global__ __launch_bounds__(RT) void k_row(KArgs a) {
    constexpr int EPV = Ev<DT>::EPV;
    constexpr uint32_t TILE = (uint32_t)RT * TV * EPV;
    constexpr uint32_t NW = RWV;
    __shared__ RowLds SL;
    const int tid = threadIdx.x;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63;
    const int64_t w = xcd_item(a.nrows);
    if (w >= a.nrows) return;
    const int r = (int)w;
    const uint32_t lo = 0u, hi = (uint32_t)a.vocab;
    const uint32_t ntile = (hi + TILE - 1) / TILE;
    const char* rp = row_ptr(a, r);
    // rows start at different tiles so they do not all read the same HBM
    // channels at once (the order of visits does not matter: ties are broken
    // by id)
    const uint32_t rot = (uint32_t)(((uint64_t)w * 5u) % ntile);
    auto tbase = [&](uint32_t k) {
        uint32_t t = k + rot;
        if (t >= ntile) t -= ntile;
        return t * TILE;
    };
    // chunk ch = one wave's share of a tile: slot ch % NW of tile ch / NW
    const uint32_t nchunk = ntile * NW;
    auto chunk_t0 = [&](uint32_t ch) { return tbase(ch / NW); };
    auto chunk_slot = [&](uint32_t ch) { return (ch % NW) * 64u + (uint32_t)lane; };
    auto load = [&](Tile<DT, TV, MASK>& T, uint32_t ch) __attribute__((always_inline)) {
        const bool valid = ch < nchunk;  // wave-uniform
        if (FAST) {
            tile_load_fast<DT, TV, MASK, RT>(a, r, rp, valid ? chunk_t0(ch) : lo, hi, valid ? chunk_slot(ch) : 0u,
                                             valid, T);
        } else {
            const uint32_t t0 = valid ? chunk_t0(ch) : lo;
            tile_load<DT, TV, MASK, RT>(a, r, rp, t0, valid ? hi : t0, valid ? chunk_slot(ch) : 0u, T);
        }
    };
    uint32_t c0 = (uint32_t)wv, c1 = NW + (uint32_t)wv;
    // Every wave: its first chunk, the row's context, its share of the
    // window's first HPRE tokens, then its second chunk (the window's loads
    // queue behind one chunk per wave, not two).
    Tile<DT, TV, MASK> b0, b1;
    load(b0, c0);
    const RowCtx c = make_ctx(a, r);
    const bool special = c.cnt_on || c.bias_on || c.ban_on;
    constexpr int HK = (int)(HPRE / RT);
    uint32_t ht[HK];
#pragma unroll
    for (int k = 0; k < HK; ++k) {
        const int64_t i = c.w0 + tid + (int64_t)k * RT;
        ht[k] = (c.cnt_on && i < c.w1) ? a.hist[i] : NONE;
    }
    load(b1, c1);
    if (tid == 0) {
        SL.next = 2u * NW;
        SL.ncand = 0;
        SL.ncap = 0;
        SL.err = 0;
        SL.bpos = 0;
        SL.gmax = f2ord(-INFINITY);
        const int64_t nb = c.bias_on ? c.b1 - c.b0 : 0;
        SL.nbias = (uint32_t)(nb < (int64_t)RBCAP ? nb : (int64_t)RBCAP);
    }
    if (special || MASK) {
        // expansion table: bit q of an index marks element q of a vector; the
        // entry holds, per 32-bit word of the vector, all ones over the
        // marked elements
        for (uint32_t i = tid; i < 256u; i += RT) {
            u32x4 m;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                if (DT == AXS_DTYPE_BF16)
                    m[k] = (((i >> (2 * k)) & 1u) ? 0x0000FFFFu : 0u) | (((i >> (2 * k + 1)) & 1u) ? 0xFFFF0000u : 0u);
                else
                    m[k] = ((i >> k) & 1u) ? 0xFFFFFFFFu : 0u;
            }
            SL.xt[i] = m;
        }
    }
    if (special) {
        const uint32_t nw = (hi + 31u) / 32u;
        for (uint32_t i = tid; i < nw; i += RT) SL.u.p.spec[i] = 0u;
        for (uint32_t i = tid; i < HSZ; i += RT) {
            SL.u.p.hkey[i] = NONE;
            SL.u.p.hval[i] = 0u;
        }
        if (c.bias_on) {
            bool pos = false;
            for (int64_t i = c.b0 + tid; i < c.b1 && i < c.b0 + (int64_t)RBCAP; i += RT) {
                SL.bias_id[i - c.b0] = a.bias_ids[i];
                const float bv = a.bias_vals[i];
                SL.bias_v[i - c.b0] = bv;
                pos |= !(bv <= 0.0f);
            }
            if (pos) SL.bpos = 1u;
        }
#pragma unroll
        for (int k = 0; k < HK; ++k) SL.stage[tid + k * RT] = ht[k];
    }
    lds_barrier();
    // The bitmap, which the stream needs, is marked by every thread; the hash
    // (window counts, bias entries, bans), which only the specials' pass
    // after the stream needs, is built by the window waves while the others
    // already stream.
    uint32_t* spec = SL.u.p.spec;
    uint32_t* hkey = SL.u.p.hkey;
    uint32_t* hval = SL.u.p.hval;
    if (special) {
        auto mark = [&](uint32_t t) {
            if (t < hi) atomicOr(&spec[t >> 5], 1u << (t & 31u));  // ids outside the vocabulary are skipped
        };
        if (c.cnt_on) {
#pragma unroll
            for (int k = 0; k < (int)(HPRE / RT); ++k) {
                const uint32_t t = SL.stage[tid + k * RT];
                if (t != NONE) mark(t);
            }
            for (int64_t i = c.w0 + HPRE + tid; i < c.w1; i += RT) mark(a.hist[i]);
        }
        if (c.bias_on) {
            if (c.b1 - c.b0 > (int64_t)RBCAP && tid == 0) SL.err |= RERR_BIAS;
            for (uint32_t j = tid; j < SL.nbias; j += RT) mark(SL.bias_id[j]);
        }
        if (c.ban_on) ngram_each<RT>(a, c, lo, hi, mark);
        lds_barrier();
    }
    auto build_hash = [&]() {  // waves 0..HWAVES-1
        constexpr int HL = HWAVES * 64;
        bool full = false;
        auto count = [&](uint32_t t) {
            if (t >= hi || full) return;
            const uint32_t s = hash_insert(hkey, t);
            if (s == NONE) full = true;
            else atomicAdd(&hval[s], 1u);
        };
        if (c.cnt_on) {
            if (c.w1 - c.w0 > (int64_t)HV_CNT) full = true;  // counts would not fit
#pragma unroll
            for (int k = 0; k < (int)(HPRE / HL); ++k) {
                const uint32_t t = SL.stage[tid + k * HL];
                if (t != NONE) count(t);
            }
            for (int64_t i = c.w0 + HPRE + tid; i < c.w1; i += HL) count(a.hist[i]);
        }
        if (c.bias_on) {
            for (uint32_t j = tid; j < SL.nbias; j += HL) {
                const uint32_t t = SL.bias_id[j];
                if (t >= hi) continue;
                const uint32_t s = hash_insert(hkey, t);
                if (s == NONE) {
                    full = true;
                    continue;
                }
                uint32_t old = hval[s];
                while (true) {
                    const uint32_t b = (old >> HV_BSH) & HV_BMULTI;
                    const uint32_t nb = b == 0u ? j + 1u : HV_BMULTI;
                    const uint32_t nv = (old & ~(HV_BMULTI << HV_BSH)) | (nb << HV_BSH);
                    const uint32_t got = atomicCAS(&hval[s], old, nv);
                    if (got == old) break;
                    old = got;
                }
            }
        }
        if (c.ban_on)
            ngram_each_g(a, c, lo, hi, (int64_t)tid, (int64_t)HL, [&](uint32_t t) {
                const uint32_t s = hash_insert(hkey, t);
                if (s == NONE) full = true;
                else atomicOr(&hval[s], HV_BAN);
            });
        if (full) atomicOr(&SL.err, RERR_HASH);
    };

    const uint32_t mode = c.mode;
    const float inv = __fdiv_rn(1.0f, c.p.temperature);
    const bool gather = mode == M_MINP && isfinite(inv);
    // the approximate greedy logprob of the stream (rows that take the exact
    // path for it need none)
    const bool gsum_on = mode == M_GREEDY && a.want_logprob && !a.exact_lp;
    const float thr = gather ? __fsub_rn(ln_f32(c.p.min_p), 1e-3f) : 0.0f;
    const uint32_t sflags = c.err ? CS_ERROR : ((SL.err & RERR_BIAS) ? (CS_ERROR | CS_CAPACITY) : 0u);
    // Processors that can only lower a logit (repetition >= 1, presence and
    // frequency >= 0, biases <= 0, mask, ban) let the stream skip every
    // vector whose raw maximum is below rthr: none of its plain elements can
    // be the maximum or a min-p candidate, and none of its special ones either
    // (processed <= raw).  Otherwise, and for the greedy logprob sum, every
    // vector is looked at.
    const bool mono = (!c.rep_on || c.p.repetition_penalty > 1.0f) &&
                      (!c.pf_on || (c.p.presence_penalty >= 0.0f && c.p.frequency_penalty >= 0.0f)) &&
                      (!c.bias_on || SL.bpos == 0u);
    const bool fastp = mono && !gsum_on;
    const double dlow = gather ? ((double)thr - 0.01) / (double)inv : 0.0;

    float tm = -INFINITY;             // thread maximum (non-special ids)
    uint32_t ta = NONE;               // its lowest id
    float gm = -INFINITY, gs = 0.0f;  // greedy logprob: sum of exp(l - gm)
    float mrun = -INFINITY;           // a lower bound of the row maximum (wave-uniform)
    float lpre = INFINITY;            // l < lpre ⇒ not a candidate (wave-uniform)
    float rthr = -INFINITY;           // raw vector maximum < rthr ⇒ skipped (wave-uniform)

    auto set_pre = [&]() {
        // (l - mrun) * inv >= thr needs l >= mrun + thr / inv; the bound is
        // lowered by 0.01 nats and a few ulps so rounding never excludes one
        if (gather) {
            if (!isfinite(mrun)) {
                lpre = INFINITY;
            } else if (inv > 0.0f) {
                const double bnd = (double)mrun + dlow;
                const double slack = 4.0 * fmax(fabs((double)mrun), fabs(bnd)) * 1.2e-7;
                lpre = (float)(bnd - slack);
            } else {
                lpre = -INFINITY;
            }
        }
        rthr = !fastp ? -INFINITY : (gather ? fminf(lpre, mrun) : mrun);
    };
    // tot slots of a pool for the wave: one LDS atomic by lane 0 (every lane
    // of the wave calls it)
    auto claim = [&](uint32_t* ctr, uint32_t tot) -> uint32_t {
        uint32_t b = 0;
        if (lane == 0) b = atomicAdd(ctr, tot);
        return (uint32_t)__builtin_amdgcn_readfirstlane((int)b);
    };
    // The row's min-p candidates: a run of pool slots per call, lanes placed
    // by ballot (every lane of the wave calls these)
    auto append_one = [&](bool c, uint32_t e, float l) {
        const uint64_t m1 = __ballot(c);
        if (m1 == 0ull) return;
        const uint32_t pos = claim(&SL.ncand, (uint32_t)__popcll(m1)) + mbcnt64(m1);
        if (c && pos < CANDP) {
            SL.cand[pos].id = e;
            SL.cand[pos].l = l;
        }
    };
    auto gsum_add = [&](float l) {
        if (isfinite(l)) {
            if (l > gm) {
                gs = __fmaf_rn(gs, __expf(gm - l), 1.0f);
                gm = l;
            } else {
                gs += __expf(l - gm);
            }
        }
    };
    constexpr uint32_t EMASK = (1u << EPV) - 1u;
    constexpr uint32_t NINF = DT == AXS_DTYPE_BF16 ? 0xFF80FF80u : 0xFF800000u;
    // The special bits of the vector at e0
    auto spec_bits = [&](uint32_t e0) -> uint32_t {
        return special ? (SL.u.p.spec[e0 >> 5] >> (e0 & 31u)) & EMASK : 0u;
    };
    // The EPV logits of a vector as the stream sees them: disallowed elements
    // -inf, special ones (bits sk) NaN (an all-ones pattern in both formats)
    auto vec_vals = [&](u32x4 raw, uint32_t mw, uint32_t e0, uint32_t sk, float* v) {
        if (MASK) {
            const u32x4 m = SL.xt[(~mw >> (e0 & 31u)) & EMASK];
#pragma unroll
            for (int k = 0; k < 4; ++k) raw[k] = (m[k] & NINF) | (~m[k] & raw[k]);
        }
        if (special) {
            const u32x4 m = SL.xt[sk];
#pragma unroll
            for (int k = 0; k < 4; ++k) raw[k] |= m[k];
        }
#pragma unroll
        for (int q = 0; q < EPV; ++q) v[q] = unpack<DT>(raw, q);
    };
    // element q (lane-varying) of a vector, as f32
    auto elem = [&](const u32x4& raw, uint32_t q) -> float {
        if (DT == AXS_DTYPE_BF16) {
            const uint32_t wi = q >> 1;
            const uint32_t lo = (wi & 1u) ? raw[1] : raw[0];
            const uint32_t hi2 = (wi & 1u) ? raw[3] : raw[2];
            const uint32_t w = (wi & 2u) ? hi2 : lo;
            return __uint_as_float((q & 1u) ? (w & 0xFFFF0000u) : (w << 16));
        } else {
            const uint32_t lo = (q & 1u) ? raw[1] : raw[0];
            const uint32_t hi2 = (q & 1u) ? raw[3] : raw[2];
            return __uint_as_float((q & 2u) ? hi2 : lo);
        }
    };
    // The wave's lanes holding special elements (bits sk) append (id, raw
    // value) to the capture pool.
    auto capture = [&](const u32x4& raw, uint32_t mw, uint32_t e0, uint32_t sk) {
        const uint64_t m1 = __ballot(sk != 0u);
        if (m1 == 0ull) return;
        const uint64_t m2 = __ballot((sk & (sk - 1u)) != 0u);
        if (m2 == 0ull) {
            // at most one special element per lane (the common case)
            const uint32_t pos = claim(&SL.ncap, (uint32_t)__popcll(m1)) + mbcnt64(m1);
            if (sk != 0u && pos < CAPP) {
                const uint32_t q = (uint32_t)__ffs((int)sk) - 1u;
                const bool off = MASK && !((mw >> ((e0 + q) & 31u)) & 1u);
                SL.cap[pos].id = (e0 + q) | (off ? CAP_OFF : 0u);
                SL.cap[pos].l = elem(raw, q);
            }
        } else {
            // per-lane counts up to EPV: prefix from their bit slices
            const uint32_t c = (uint32_t)__popc(sk);
            uint32_t pre = 0, tot = 0;
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                const uint64_t mb = __ballot((c >> b) & 1u);
                pre += mbcnt64(mb) << b;
                tot += (uint32_t)__popcll(mb) << b;
            }
            uint32_t pos = claim(&SL.ncap, tot) + pre;
#pragma unroll
            for (int q = 0; q < EPV; ++q)
                if ((sk >> q) & 1u) {
                    if (pos < CAPP) {
                        const bool off = MASK && !((mw >> ((e0 + q) & 31u)) & 1u);
                        SL.cap[pos].id = (e0 + q) | (off ? CAP_OFF : 0u);
                        SL.cap[pos].l = unpack<DT>(raw, q);
                    }
                    ++pos;
                }
        }
    };
    // Per vector: its maximum decides everything.  The thread keeps the
    // lowest-id vector holding its running maximum; the element is resolved
    // once at the end.  Only vectors reaching the gather bound, and greedy
    // rows that want a logprob, look at single elements.
    uint32_t tj = NONE;  // first id of the best vector
    u32x4 traw = u32x4{0u, 0u, 0u, 0u};
    uint32_t tmw = 0xFFFFFFFFu;
    // The full look at one vector with special bits sk: special elements
    // read as NaN, disallowed ones -inf; the lane's maximum, min-p candidates
    // and the greedy logprob sum updated.  Runs with only the relevant lanes
    // active (the capture, whose ballots need the whole wave, is done before).
    auto look = [&](const u32x4& raw, uint32_t mw, uint32_t e0, uint32_t sk) __attribute__((always_inline)) -> uint32_t {
        float v[EPV];
        vec_vals(raw, mw, e0, sk, v);
        float vm = v[0];
#pragma unroll
        for (int q = 1; q < EPV; ++q) vm = fmaxf(vm, v[q]);
        if (vm > tm || (vm == tm && e0 < tj)) {
            tm = vm;
            tj = e0;
            traw = raw;
            tmw = mw;
        }
        uint32_t qm = 0;  // the vector's min-p candidates (a superset of the survivors)
        if (gather && vm >= lpre) {
#pragma unroll
            for (int q = 0; q < EPV; ++q)
                if (v[q] >= lpre) qm |= 1u << q;
        }
        if (gsum_on) {
#pragma unroll
            for (int q = 0; q < EPV; ++q) gsum_add(v[q]);
        }
        return qm;
    };
    // Appends the vector's candidates (bits qm; a candidate is neither special
    // nor disallowed, so its value is the raw element).  Whole wave.
    auto append = [&](const u32x4& raw, uint32_t e0, uint32_t qm) {
        const uint64_t m1 = __ballot(qm != 0u);
        if (m1 == 0ull) return;
        const uint64_t m2 = __ballot((qm & (qm - 1u)) != 0u);
        if (m2 == 0ull) {
            const uint32_t pos = claim(&SL.ncand, (uint32_t)__popcll(m1)) + mbcnt64(m1);
            if (qm != 0u && pos < CANDP) {
                const uint32_t q = (uint32_t)__ffs((int)qm) - 1u;
                SL.cand[pos].id = e0 + q;
                SL.cand[pos].l = elem(raw, q);
            }
        } else {
            const uint32_t c = (uint32_t)__popc(qm);
            uint32_t pre = 0, tot = 0;
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                const uint64_t mb = __ballot((c >> b) & 1u);
                pre += mbcnt64(mb) << b;
                tot += (uint32_t)__popcll(mb) << b;
            }
            uint32_t pos = claim(&SL.ncand, tot) + pre;
#pragma unroll
            for (int q = 0; q < EPV; ++q)
                if ((qm >> q) & 1u) {
                    if (pos < CANDP) {
                        SL.cand[pos].id = e0 + q;
                        SL.cand[pos].l = unpack<DT>(raw, q);
                    }
                    ++pos;
                }
        }
    };
    // With the skip (fastp), a wave queues its relevant vectors in LDS
    // (ballot slots) and looks at them 64 at a time, one lane per vector: a
    // relevant vector is rare, and a look costs the whole wave.
    uint32_t wq = 0;  // queued vectors (wave-uniform)
    auto flush = [&]() {
        if (wq == 0u) return;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        const bool v = (uint32_t)lane < wq;
        const u32x4 raw = v ? SL.qraw[wv][lane] : u32x4{0u, 0u, 0u, 0u};
        const uint32_t e0 = v ? SL.qe0[wv][lane] : 0u;
        const uint32_t mw = (MASK && v) ? SL.qmw[wv][lane] : 0xFFFFFFFFu;
        const uint32_t sk = v ? spec_bits(e0) : 0u;
        if (special) capture(raw, mw, e0, sk);
        uint32_t qm = 0;
        if (v) qm = look(raw, mw, e0, sk);
        if (gather) append(raw, e0, qm);
        wq = 0;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");  // read before the queue is refilled
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    };
    // Per vector: its raw maximum (special and disallowed elements included)
    // against rthr; only vectors that reach it are looked at closer.
    auto process = [&](Tile<DT, TV, MASK>& T, uint32_t ch) {
        const uint32_t t0 = chunk_t0(ch), sl = chunk_slot(ch);
#pragma unroll
        for (int j = 0; j < TV; ++j) {
            asm volatile("" : "+v"(T.raw[j]));
            const uint32_t e0 = t0 + ((uint32_t)j * RT + sl) * EPV;
            const uint32_t mw = MASK ? T.mw[j] : 0xFFFFFFFFu;
            const bool in = e0 < hi;  // lanes past the row end re-read a vector
            float vr = unpack<DT>(T.raw[j], 0);
#pragma unroll
            for (int q = 1; q < EPV; ++q) vr = fmaxf(vr, unpack<DT>(T.raw[j], q));
            // (an all-NaN vector is looked at: masked or banned, NaN is -inf)
            const bool rel = in && !(vr < rthr);
            const uint64_t bal = __ballot(rel);
            if (bal != 0ull) {
                if (fastp) {
                    const uint32_t cnt = (uint32_t)__popcll(bal);
                    if (wq + cnt > QN) flush();
                    if (rel) {
                        const uint32_t pos = wq + mbcnt64(bal);
                        SL.qraw[wv][pos] = T.raw[j];
                        SL.qe0[wv][pos] = e0;
                        if (MASK) SL.qmw[wv][pos] = mw;
                    }
                    wq += cnt;
                } else {
                    // every vector is relevant: looked at in place (whole wave)
                    const uint32_t sk = rel ? spec_bits(e0) : 0u;
                    if (special) capture(T.raw[j], mw, e0, sk);
                    uint32_t qm = 0;
                    if (rel) qm = look(T.raw[j], mw, e0, sk);
                    if (gather) append(T.raw[j], e0, qm);
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    // maximum of a chunk (seeds a wave's gather bound)
    auto tile_max = [&](Tile<DT, TV, MASK>& T, uint32_t ch) {
        const uint32_t t0 = chunk_t0(ch), sl = chunk_slot(ch);
        float pm = -INFINITY;
#pragma unroll
        for (int j = 0; j < TV; ++j) {
            const uint32_t e0 = t0 + ((uint32_t)j * RT + sl) * EPV;
            float v[EPV];
            vec_vals(T.raw[j], MASK ? T.mw[j] : 0xFFFFFFFFu, e0, spec_bits(e0), v);
            if (e0 < hi)
#pragma unroll
                for (int q = 0; q < EPV; ++q) pm = fmaxf(pm, v[q]);
        }
        return pm;
    };
    // raises the wave's bound: its own maximum, shared through SL.gmax
    auto raise = [&](float wm) {
        int g = 0;
        if (lane == 0) g = atomicMax(&SL.gmax, f2ord(wm));
        g = __builtin_amdgcn_readfirstlane(g);
        mrun = fmaxf(mrun, fmaxf(wm, ord2f(g)));
        set_pre();
    };
    // the next chunk for this wave: claimed, or, for a greedy logprob row,
    // every NW-th chunk in order (each lane's sum then runs over the same
    // elements in the same order on every call: a reproducible logprob)
    auto grab = [&](uint32_t cur) {
        if (gsum_on) return cur + 2u * NW;
        uint32_t ch = 0;
        if (lane == 0) ch = atomicAdd(&SL.next, 1u);
        return (uint32_t)__builtin_amdgcn_readfirstlane((int)ch);
    };
    const bool bound = gather || fastp;  // the stream keeps a lower bound of the maximum
    auto step = [&](Tile<DT, TV, MASK>& T, uint32_t& ch) __attribute__((always_inline)) {
        if (bound && mrun == -INFINITY) raise(wave_max_dpp(tile_max(T, ch)));
        process(T, ch);
        ch = grab(ch);
        load(T, ch);
        if (bound) raise(wave_max_dpp(tm));
    };
    if (special && wv < HWAVES) build_hash();
    // the decision's per-row constants, off its critical path
    double lnmin = 0.0;
    float urow = 0.0f, xstar = INFINITY;
    if (gather && wv == 0) {
        lnmin = log((double)c.p.min_p);
        xstar = minp_edge(c.p.min_p);
        urow = row_uniform(a, r, c.p);
        // computed here, while the first tiles load: the compiler would
        // otherwise sink them to their use after the stream
        asm volatile("" : "+v"(lnmin), "+v"(xstar), "+v"(urow));
    }
    // Both buffers are refilled unconditionally (a claim past the end loads a
    // dummy line), so the wait for one buffer leaves the other's loads in
    // flight.  Claims only grow: once one is past the end, so are all later.
    while (c0 < nchunk) {
        step(b0, c0);
        if (c1 >= nchunk) break;
        step(b1, c1);
    }
    flush();
    // the first element of the best vector that attains the maximum
    if (tj != NONE) {
        float v[EPV];
        vec_vals(traw, tmw, tj, spec_bits(tj), v);
        uint32_t q0 = NONE;
#pragma unroll
        for (int q = EPV - 1; q >= 0; --q)
            if (v[q] == tm) q0 = (uint32_t)q;
        ta = tj + q0;
    }
    lds_barrier();
    // the special ids' processed values
    if (special) {
        auto cand_ok = [&](float l) {
            return gather && l > -INFINITY && (mrun == -INFINITY || __fmul_rn(__fsub_rn(l, mrun), inv) >= thr);
        };
        const uint32_t ncap = SL.ncap;
        if (ncap <= CAPP && !(SL.err & RERR_HASH)) {
            // the captures, 64 per wave at a time (whole-wave loop: the
            // appends ballot)
            for (uint32_t base = (uint32_t)wv * 64u; base < ncap; base += RT) {
                const uint32_t i = base + (uint32_t)lane;
                const bool ok = i < ncap;
                uint32_t e = 0;
                float l = NAN;
                if (ok) {
                    const Cand cd = SL.cap[i];
                    e = cd.id & ~CAP_OFF;
                    const uint32_t s = hash_find(SL.u.p.hkey, e);
                    const uint32_t hv = s == NONE ? 0u : SL.u.p.hval[s];
                    l = row_special_value(c, SL, e, cd.l, hv & HV_CNT, (hv >> HV_BSH) & HV_BMULTI,
                                          (hv & HV_BAN) != 0u, (cd.id & CAP_OFF) != 0u);
                    am_merge(tm, ta, l, isnan(l) ? NONE : e);
                    if (gsum_on) gsum_add(l);
                }
                if (gather) append_one(ok && cand_ok(l), e, l);
            }
        } else {
            // a full hash or capture pool: every special id resolved from HBM
            // (raw logit; window count and ban from the hash, or, when it is
            // full, by scanning the history); candidates by LDS atomics
            const bool hok = !(SL.err & RERR_HASH);
            const uint32_t nw = (hi + 31u) / 32u;
            for (uint32_t wi = tid; wi < nw; wi += RT) {
                uint32_t bits = SL.u.p.spec[wi];
                while (bits) {
                    const uint32_t b = (uint32_t)__ffs((int)bits) - 1u;
                    bits &= bits - 1u;
                    const uint32_t e = wi * 32u + b;
                    uint32_t cnt, bcode;
                    bool ban;
                    if (hok) {
                        const uint32_t s = hash_find(SL.u.p.hkey, e);
                        const uint32_t hv = s == NONE ? 0u : SL.u.p.hval[s];
                        cnt = hv & HV_CNT;
                        bcode = (hv >> HV_BSH) & HV_BMULTI;
                        ban = (hv & HV_BAN) != 0u;
                    } else {
                        const uint32_t cw = count_word_hbm(a, c, e);
                        cnt = cw & ~CNT_BAN;
                        bcode = HV_BMULTI;
                        ban = (cw & CNT_BAN) != 0u;
                    }
                    const bool off = c.mask_on && !((a.mask[(size_t)r * a.mask_stride + (e >> 5)] >> (e & 31u)) & 1u);
                    const float l = row_special_value(c, SL, e, raw_at<DT>(rp, e), cnt, bcode, ban, off);
                    am_merge(tm, ta, l, isnan(l) ? NONE : e);
                    if (gsum_on) gsum_add(l);
                    if (cand_ok(l)) {
                        const uint32_t slot = atomicAdd(&SL.ncand, 1u);
                        if (slot < CANDP) {
                            SL.cand[slot].id = e;
                            SL.cand[slot].l = l;
                        }
                    }
                }
            }
        }
    }

    // row results: per-wave DPP reductions, merged by every thread
    float bm = tm;
    uint32_t bi = ta;
    wave_argmax_dpp(bm, bi);
    float wgm = -INFINITY, wgs = 0.0f;
    if (gsum_on) {
        wgm = wave_max_dpp(gm);
        const float part = (isfinite(gm) && isfinite(wgm)) ? gs * __expf(gm - wgm) : 0.0f;
        wgs = wave_sum_f(part);
    }
    if (lane == 0) {
        SL.wm[wv] = bm;
        SL.wa[wv] = bi;
        SL.gm[wv] = wgm;
        SL.gs[wv] = wgs;
    }
    lds_barrier();
    // the 16 results, one per lane, merged by DPP (every thread)
    float m = lane < RWV ? SL.wm[lane] : -INFINITY;
    uint32_t am = lane < RWV ? SL.wa[lane] : NONE;
    wave_argmax_dpp(m, am);
    if (am == NONE) m = -INFINITY;
    if (a.mtp_amax && tid == 0) a.mtp_amax[r] = am == NONE ? 0u : am;  // argmax_f32 (all-NaN: 0)
    double gsum = 0.0;
    if (gsum_on && isfinite(m)) {
#pragma unroll
        for (int k = 0; k < RWV; ++k)
            if (isfinite(SL.gm[k])) gsum += (double)SL.gs[k] * exp((double)SL.gm[k] - (double)m);
    }
    uint32_t flags = sflags;
    const uint32_t nc = gather ? SL.ncand : 0u;
    if (nc > CANDP) flags |= CS_OVERFLOW;
    const uint32_t n = nc < CANDP ? nc : CANDP;
    auto cand_at = [&](uint32_t k) -> Cand { return SL.cand[k]; };
    if (gather && !(flags & (CS_ERROR | CS_OVERFLOW)) && am != NONE && isfinite(m) && n <= 256u) {
        // min-p row with few candidates: wave 0 decides alone
        if (wv != 0) return;
        wave_decide_minp<RT>(a, r, c.p, m, inv, am, n, cand_at, (uint64_t*)SL.stage, SL.u.F, lnmin, xstar, urow);
        return;
    }
    RowState xs;
    const bool ex = finish_decide<RT, true>(
        a, r, c.p, m, am, flags, gsum, n, SL.u.F,
        [&](auto&& f) {
            for (uint32_t i = tid; i < n; i += RT) {
                const Cand cd = cand_at(i);
                f(cd.id, cd.l);
            }
        },
        &xs);
    if (!ex) return;
    if (!a.inplace) {  // listed for k_exact_mat / k_exact_row
        if (tid == 0) {
            a.rstate[r] = xs;
            a.exact_rows[atomicAdd(a.exact_count, 1u)] = (uint32_t)r;
        }
        return;
    }

    // The exact path in place (laws without min-p, candidate overflow): every
    // element's probability with the row maximum, from a second read of the
    // row (processors as in the stream: the bitmap and hash are intact), as a
    // dense row (index-order laws) or compacted (p desc, id asc) keys at or
    // above the floor (sorted laws); then exact_row sorts, sums and decides.
    if (tid == 0) {
        a.rstate[r] = xs;
        SL.xn = 0;
    }
    const bool xminp = xs.mode == M_MINP;
    const bool xsorted = xs.sorted != 0;
    // sorted laws: the exp only for keys and near the min-p boundary
    const KeyEdge ke = key_edges(xs.pmin, xminp, c.p.min_p);
    const float xstage = fminf(ke.xe, ke.xm0);
    // each wave's staging slots for the elements whose exp is computed
    static_assert(sizeof(ExLds) >= (size_t)RWV * 64u * EPV * sizeof(uint64_t), "staging slots");
    uint64_t* xstg = reinterpret_cast<uint64_t*>(&SL.ex) + (size_t)(tid >> 6) * 64u * EPV;
    const bool hok = !(SL.err & RERR_HASH);
    float* dense = a.dense + (size_t)r * a.vocab;
    uint64_t* ck = a.ckey + (size_t)r * a.vocab;
    float xmg = INFINITY;
    auto xval = [&](uint32_t e, float raw, bool off) -> float {
        uint32_t cnt, bcode;
        bool ban;
        if (hok) {
            const uint32_t s = hash_find(SL.u.p.hkey, e);
            const uint32_t hv = s == NONE ? 0u : SL.u.p.hval[s];
            cnt = hv & HV_CNT;
            bcode = (hv >> HV_BSH) & HV_BMULTI;
            ban = (hv & HV_BAN) != 0u;
        } else {
            const uint32_t cw = count_word_hbm(a, c, e);
            cnt = cw & ~CNT_BAN;
            bcode = HV_BMULTI;
            ban = (cw & CNT_BAN) != 0u;
        }
        return row_special_value(c, SL, e, raw, cnt, bcode, ban, off);
    };
    lds_barrier();
    constexpr int XV = 4;  // vectors per thread per tile
    constexpr uint32_t XTILE = (uint32_t)RT * XV * EPV;
    // The wave's exclusive prefix of per-lane slot bits (n slots per lane)
    // and its total.  Masked rows: one ballot per slot, and their tiles
    // double-buffered below (C4: -28 us).  Unmasked rows keep the
    // cross-lane scan and single tiles: the same changes there move the code
    // generation of the stream loop the kernel shares with them (C3 +2.5 us,
    // measured).
    auto wave_prefix = [&](uint32_t bits, int n, uint32_t& excl, uint32_t& total) {
        if constexpr (MASK) {
            excl = 0;
            total = 0;
#pragma unroll
            for (int q = 0; q < EPV; ++q) {
                if (q >= n) break;
                const uint64_t bq = __ballot((bits >> q) & 1u);
                excl += mbcnt64(bq);
                total += (uint32_t)__popcll(bq);
            }
        } else {
            const uint32_t nc = (uint32_t)__popc(bits);
            uint32_t incl = nc;
#pragma unroll
            for (int d = 1; d < 64; d <<= 1) {
                const uint32_t y = (uint32_t)__shfl_up((int)incl, d, 64);
                if (lane >= d) incl += y;
            }
            total = (uint32_t)__shfl((int)incl, 63, 64);
            excl = incl - nc;
        }
    };
    Tile<DT, XV, MASK> Tn;
    if constexpr (MASK) tile_load<DT, XV, MASK, RT>(a, r, rp, 0u, hi, (uint32_t)tid, Tn);
    for (uint32_t t0 = 0; t0 < hi; t0 += XTILE) {
        Tile<DT, XV, MASK> T;
        if constexpr (MASK) {
            T = Tn;
            if (t0 + XTILE < hi) tile_load<DT, XV, MASK, RT>(a, r, rp, t0 + XTILE, hi, (uint32_t)tid, Tn);
        } else {
            tile_load<DT, XV, MASK, RT>(a, r, rp, t0, hi, (uint32_t)tid, T);
        }
#pragma unroll
        for (int j = 0; j < XV; ++j) {
            const uint32_t e0 = t0 + ((uint32_t)j * RT + (uint32_t)tid) * EPV;
            const uint32_t mw = MASK ? T.mw[j] : 0xFFFFFFFFu;
            const uint32_t sk = e0 < hi ? spec_bits(e0) : 0u;
            float v[EPV];
            vec_vals(T.raw[j], mw, e0, sk, v);
            if (xsorted) {
                // x = (l - m) * inv of each element; the keys (x >= xe) and
                // those near the min-p boundary are staged (x, id) in the
                // wave's LDS slots, so that the exp runs on full waves
                uint32_t cm = 0;
                float xq[EPV];
#pragma unroll
                for (int q = 0; q < EPV; ++q) {
                    const uint32_t e = e0 + (uint32_t)q;
                    if ((sk >> q) & 1u) v[q] = xval(e, unpack<DT>(T.raw[j], q), MASK && !((mw >> (e & 31u)) & 1u));
                    xq[q] = __fmul_rn(__fsub_rn(v[q], xs.m), xs.inv);
                    if (e < hi && xq[q] >= xstage) cm |= 1u << q;
                }
                uint32_t so, tot;
                wave_prefix(cm, EPV, so, tot);
#pragma unroll
                for (int q = 0; q < EPV; ++q)
                    if ((cm >> q) & 1u) xstg[so++] = ((uint64_t)__float_as_uint(xq[q]) << 32) | (e0 + (uint32_t)q);
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                uint64_t kk[EPV];
                uint32_t km = 0;
#pragma unroll
                for (int i = 0; i < EPV; ++i) {
                    const uint32_t t = (uint32_t)lane + 64u * (uint32_t)i;
                    kk[i] = 0;
                    if (64u * (uint32_t)i >= tot) continue;  // wave-uniform
                    if (t < tot) {
                        const uint64_t w = xstg[t];
                        const float x = __uint_as_float((uint32_t)(w >> 32));
                        float pr = exp_ref(x);
                        if (!isfinite(pr)) pr = 0.0f;
                        if (x >= ke.xm0 && x < ke.xm1) xmg = fminf(xmg, fabsf(pr - c.p.min_p) / c.p.min_p);
                        if (x >= ke.xe) {
                            kk[i] = key_pdesc(pr, (uint32_t)w);
                            km |= 1u << i;
                        }
                    }
                }
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                // the wave's keys, at one LDS claim per vector
                uint32_t kex, ktot;
                wave_prefix(km, EPV, kex, ktot);
                uint32_t base = 0;
                if (lane == 0 && ktot) base = atomicAdd(&SL.xn, ktot);
                uint32_t o = (uint32_t)__shfl((int)base, 0, 64) + kex;
#pragma unroll
                for (int i = 0; i < EPV; ++i)
                    if ((km >> i) & 1u) ck[o++] = kk[i];
                continue;
            }
#pragma unroll
            for (int q = 0; q < EPV; ++q) {
                const uint32_t e = e0 + (uint32_t)q;
                if ((sk >> q) & 1u) v[q] = xval(e, unpack<DT>(T.raw[j], q), MASK && !((mw >> (e & 31u)) & 1u));
                const float pr = prob_of(v[q], xs.m, xs.inv);
                bool keep = true;
                if (xminp) {
                    if (!isnan(v[q]) && e < hi) xmg = fminf(xmg, fabsf(pr - c.p.min_p) / c.p.min_p);
                    keep = pr >= c.p.min_p;
                }
                if (e < hi) dense[e] = keep ? pr : 0.0f;
            }
        }
    }
    if (xminp) {
        const float wmg = -wave_max_dpp(-xmg);
        if (lane == 0) SL.wm[wv] = wmg;
    }
    __threadfence_block();
    __syncthreads();  // the row's keys / probabilities are complete
    if (xminp) {
        float g = SL.wm[0];
#pragma unroll
        for (int k = 1; k < RWV; ++k) g = fminf(g, SL.wm[k]);
        xs.minp_mg = __float_as_uint(g);
    }
    xs.ncompact = SL.xn;
    exact_row<8>(a, r, xs, SL.ex);
}

// --------------------------------------------------------------------------
// k_exact_mat: exact probabilities of the listed rows (second pass)
// --------------------------------------------------------------------------
template <int DT, int NV>
__global__ __launch_bounds__(NT_CHUNK) void k_exact_mat(KArgs a) {
    __shared__ ProcLds<NT_CHUNK, EX_SEGMAX> L;
    __shared__ uint32_t s_u[NT_CHUNK / 64];
    __shared__ float s_f[NT_CHUNK / 64];
    __shared__ uint32_t s_base, s_cur;
    constexpr int EPVC = Ev<DT>::EPV;
    __shared__ uint64_t s_stg[(NT_CHUNK / 64) * 64 * EPVC];  // each wave's staged (x, id)
    const int tid = threadIdx.x;
    const uint32_t nex = *a.exact_count;
    const int64_t total = (int64_t)nex * a.nch;
    for (int64_t w = blockIdx.x; w < total; w += gridDim.x) {
        const int r = (int)a.exact_rows[w / a.nch];
        const int ci = (int)(w % a.nch);
        const uint32_t lo = (uint32_t)ci * (uint32_t)a.chunk;
        const uint32_t hi = min(lo + (uint32_t)a.chunk, (uint32_t)a.vocab);
        const RowState rs = a.rstate[r];
        RowCtx c = make_ctx(a, r);
        Seg<DT, NV> S;
        seg_load<DT, NV>(a, r, lo, hi, a.vec != 0, c.mask_on, S);
        const bool special = c.cnt_on || c.bias_on || c.ban_on;
        const char* rp = row_ptr(a, r);
        bool ranked = true;
        HistPre<NT_CHUNK> hp;
        hist_prefetch<NT_CHUNK>(a, c, hp);
        if (c.any_proc) proc_build<NT_CHUNK, EX_SEGMAX>(a, c, lo, hi, L, hp);
        if (special) ranked = proc_rank<NT_CHUNK, EX_SEGMAX>(a, c, lo, hi, L, hp);
        const bool minp = rs.mode == M_MINP;
        const float minp_v = c.p.min_p;
        float mg = INFINITY;
        uint32_t cnt = 0;
        float* dense = a.dense + (size_t)r * a.vocab;
        if (!rs.sorted) {
            // index-order rows: every probability, written to the dense row
            auto pass_dense = [&](uint32_t e, float l) {
                const float pr = prob_of(l, rs.m, rs.inv);
                bool keep = true;
                if (minp) {
                    if (!isnan(l)) mg = fminf(mg, fabsf(pr - minp_v) / minp_v);
                    keep = pr >= minp_v;
                }
                if (e < hi) dense[e] = keep ? pr : 0.0f;
            };
            regs_visit<DT, NV>(c, L, lo, S, special, pass_dense);
            if (special) visit_specials<DT, NT_CHUNK, EX_SEGMAX>(a, c, L, ranked, 0u, r, rp, lo, hi, pass_dense);
        } else {
            // sorted rows: the keys are the elements with x >= xe; counted
            // first (no exp), then written with the exp run on full waves
            const KeyEdge ke = key_edges(rs.pmin, minp, minp_v);
            auto xof = [&](float l) { return __fmul_rn(__fsub_rn(l, rs.m), rs.inv); };
            auto margin = [&](float x) {
                if (x >= ke.xm0 && x < ke.xm1) {
                    float pr = exp_ref(x);
                    if (!isfinite(pr)) pr = 0.0f;
                    mg = fminf(mg, fabsf(pr - minp_v) / minp_v);
                }
            };
            auto pass1 = [&](uint32_t e, float l) {
                const float x = xof(l);
                if (e < hi && x >= ke.xe) ++cnt;
                if (minp && e < hi) margin(x);
            };
            regs_visit<DT, NV>(c, L, lo, S, special, pass1);
            if (special) visit_specials<DT, NT_CHUNK, EX_SEGMAX>(a, c, L, ranked, 0u, r, rp, lo, hi, pass1);
            uint32_t tot;
            block_excl_scan_u32<NT_CHUNK>(cnt, s_u, &tot);
            if (tid == 0) {
                s_base = tot ? atomicAdd(&a.rstate[r].ncompact, tot) : 0u;
                s_cur = 0;
            }
            __syncthreads();
            uint64_t* dst = a.ckey + (size_t)r * a.vocab + s_base;
            const int lane = tid & 63;
            uint64_t* stg = s_stg + (size_t)(tid >> 6) * 64u * EPVC;
            // pass 2, the elements held in registers: per vector, the wave's
            // keys staged (x, id), their exp, one LDS claim per wave
#pragma unroll
            for (int j = 0; j < NV; ++j) {
                asm volatile("" : "+v"(S.raw[j]));
                const uint32_t e0 = lo + ((uint32_t)j * NT_CHUNK + tid) * EPVC;
                const uint32_t off0 = e0 - lo;
                uint32_t sk = 0;
                if (special) sk = (L.spec[off0 >> 5] >> (off0 & 31u)) & ((1u << EPVC) - 1u);
                uint32_t cm = 0;
                float xq[EPVC];
#pragma unroll
                for (int q = 0; q < EPVC; ++q) {
                    float l = unpack<DT>(S.raw[j], q);
                    if (c.mask_on && !((S.mw[j] >> ((e0 + q) & 31u)) & 1u)) l = -INFINITY;
                    xq[q] = xof(l);
                    if (!((sk >> q) & 1u) && e0 + q < hi && xq[q] >= ke.xe) cm |= 1u << q;
                }
                // the wave's exclusive prefix of the keys, one ballot per
                // element slot (no cross-lane data movement); the wave's slot
                // claim goes out before the staging
                uint32_t so = 0, wt = 0;
#pragma unroll
                for (int q = 0; q < EPVC; ++q) {
                    const uint64_t bq = __ballot((cm >> q) & 1u);
                    so += mbcnt64(bq);
                    wt += (uint32_t)__popcll(bq);
                }
                if (!wt) continue;  // wave-uniform
                uint32_t base = 0;
                if (lane == 0) base = atomicAdd(&s_cur, wt);
#pragma unroll
                for (int q = 0; q < EPVC; ++q)
                    if ((cm >> q) & 1u) stg[so++] = ((uint64_t)__float_as_uint(xq[q]) << 32) | (e0 + (uint32_t)q);
                base = (uint32_t)__shfl((int)base, 0, 64);
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                for (uint32_t t = (uint32_t)lane; t < wt; t += 64u) {
                    const uint64_t w = stg[t];
                    const float pr = exp_ref(__uint_as_float((uint32_t)(w >> 32)));
                    dst[base + t] = key_pdesc(pr, (uint32_t)w);
                }
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            }
            // the special elements (their processed values), one claim each
            if (special) {
                auto pass2s = [&](uint32_t e, float l) {
                    const float x = xof(l);
                    if (e < hi && x >= ke.xe) dst[atomicAdd(&s_cur, 1u)] = key_pdesc(exp_ref(x), e);
                };
                visit_specials<DT, NT_CHUNK, EX_SEGMAX>(a, c, L, ranked, 0u, r, rp, lo, hi, pass2s);
            }
        }
        if (minp) {
            mg = block_max<NT_CHUNK>(-mg, s_f);
            if (tid == 0 && -mg < INFINITY) atomicMin(&a.rstate[r].minp_mg, __float_as_uint(-mg));
        }
        __syncthreads();
    }
}

// --------------------------------------------------------------------------
// k_exact_row: sort + exact running sums + decisions, one workgroup per row
// --------------------------------------------------------------------------
__device__ __forceinline__ Xd shfl_up_xd(Xd x, int d) {
    Xd y;
    y.inc0 = ((uint64_t)(uint32_t)__shfl_up((int)(uint32_t)(x.inc0 >> 32), d, 64) << 32) |
             (uint32_t)__shfl_up((int)(uint32_t)x.inc0, d, 64);
    y.inc1 = ((uint64_t)(uint32_t)__shfl_up((int)(uint32_t)(x.inc1 >> 32), d, 64) << 32) |
             (uint32_t)__shfl_up((int)(uint32_t)x.inc1, d, 64);
    y.par0 = (uint32_t)__shfl_up((int)x.par0, d, 64);
    y.par1 = (uint32_t)__shfl_up((int)x.par1, d, 64);
    return y;
}

// One DPP move of a transducer record (every dword); lanes without a source
// (outside the row, or rows the mask leaves out) get the identity.
template <int CTRL, int ROWS>
__device__ __forceinline__ Xd dpp_xd(const Xd& x) {
    auto mv = [](uint32_t old, uint32_t v) {
        return (uint32_t)__builtin_amdgcn_update_dpp((int)old, (int)v, CTRL, ROWS, 0xF, false);
    };
    Xd y;
    y.inc0 = ((uint64_t)mv(0u, (uint32_t)(x.inc0 >> 32)) << 32) | mv(0u, (uint32_t)x.inc0);
    y.inc1 = ((uint64_t)mv(0u, (uint32_t)(x.inc1 >> 32)) << 32) | mv(0u, (uint32_t)x.inc1);
    y.par0 = mv(0u, x.par0);
    y.par1 = mv(1u, x.par1);
    return y;
}

// Inclusive scan of transducer records over each 16-lane row (Hillis-Steele:
// row shifts 1, 2, 4, 8; composition is associative, not commutative, and
// the earlier lane's record goes first).
__device__ __forceinline__ Xd row_incl_scan_xd(Xd x) {
    x = xd_compose(dpp_xd<0x111, 0xF>(x), x);  // row_shr:1
    x = xd_compose(dpp_xd<0x112, 0xF>(x), x);  // row_shr:2
    x = xd_compose(dpp_xd<0x114, 0xF>(x), x);  // row_shr:4
    x = xd_compose(dpp_xd<0x118, 0xF>(x), x);  // row_shr:8
    return x;
}

__device__ __forceinline__ Xd readlane_xd(const Xd& x, int l) {
    Xd y;
    y.inc0 = ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(x.inc0 >> 32), l) << 32) |
             (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)x.inc0, l);
    y.inc1 = ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(x.inc1 >> 32), l) << 32) |
             (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)x.inc1, l);
    y.par0 = (uint32_t)__builtin_amdgcn_readlane((int)x.par0, l);
    y.par1 = (uint32_t)__builtin_amdgcn_readlane((int)x.par1, l);
    return y;
}

// Exclusive scan of transducer records over the block: within each wave by
// DPP (rows, then row_bcast:15 into rows 1 and 3, row_bcast:31 into rows 2
// and 3), across the waves by one DPP row scan of their totals.  Every
// thread of the block calls it; LDS-only barriers.
template <int NT>
__device__ __forceinline__ Xd block_excl_scan_xd(Xd x, Xd* s_w) {
    constexpr int NW = NT / 64;
    static_assert(NW <= 16, "wave totals are scanned in one row");
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    Xd inc = row_incl_scan_xd(x);
    inc = xd_compose(dpp_xd<0x142, 0xA>(inc), inc);  // row_bcast:15 into rows 1, 3
    inc = xd_compose(dpp_xd<0x143, 0xC>(inc), inc);  // row_bcast:31 into rows 2, 3
    if (lane == 63) s_w[w] = inc;
    Xd ex = shfl_up_xd(inc, 1);
    if (lane == 0) ex = xd_identity();
    lds_barrier();  // LDS only: the caller's global loads and stores stay in flight
    const Xd wt = row_incl_scan_xd(lane < NW ? s_w[lane] : xd_identity());
    const Xd wp = w > 0 ? readlane_xd(wt, w - 1) : xd_identity();
    lds_barrier();
    return xd_compose(wp, ex);
}

// first index i in [lo, hi) with S[i] >= t (S non-decreasing), hi if none
__device__ __forceinline__ uint32_t bucket_of(uint64_t key) {
    uint32_t pb = (uint32_t)(key >> 32);
    uint32_t d = pb <= 0x3F800000u ? 0x3F800000u - pb : 0u;
    uint32_t b = d >> 14;
    return b < NBUCKET ? b : NBUCKET - 1;
}

// Exact running sums S[k] = fl(S[k-1] + X(k)) over positions [k0, kend) from
// the sum s0, by the NT_EX threads of one workgroup (axs_exact_sum.h); S may
// be null when only the last sum is wanted.  Returns the last sum (every
// thread).  A range of up to 256 terms is summed by the reference's own loop
// on one thread (loads issued eight at a time: cheaper than the scan's
// barriers).  Otherwise a tile of IT terms per thread is loaded once; a scan
// adds the terms in the binade of the current sum, and the first term that
// would leave it (the earliest crossing over the block) is added directly by
// its thread; the rest of the tile is scanned again in the new binade.  Each
// scan covers a window of the tile that ends a margin after the next
// position where the real-valued prefix sum (fixed point, 2^-40) passes a
// power of two: the rounded sum crosses there or close by, and a window
// without a crossing only means one more scan.  The barriers are LDS-only:
// S is read only after the call.
template <uint32_t IT, typename XF>
__device__ float block_exact_sums(XF X, uint32_t k0, uint32_t kend, float s0, float* S, SumLds& L) {
    constexpr uint32_t WMARGIN = 128;
    const int tid = threadIdx.x;
    if (kend - k0 <= 256u) {
        if (tid == 0) {
            float s = s0;
            for (uint32_t i0 = k0; i0 < kend; i0 += 8u) {
                float xv[8];
#pragma unroll
                for (uint32_t j = 0; j < 8u; ++j) xv[j] = i0 + j < kend ? X(i0 + j) : 0.0f;
#pragma unroll
                for (uint32_t j = 0; j < 8u; ++j)
                    if (i0 + j < kend) {
                        s = __fadd_rn(s, xv[j]);
                        if (S) S[i0 + j] = s;
                    }
            }
            L.s = s;
        }
        __threadfence_block();
        __syncthreads();
        const float fin = L.s;
        __syncthreads();
        return fin;
    }
    if (tid == 0) L.cross = NONE;
    __syncthreads();
    float s = s0;
    for (uint32_t k = k0; k < kend;) {
        const uint32_t tile = min((uint32_t)NT_EX * IT, kend - k);
        const uint32_t i0 = k + (uint32_t)tid * IT;
        float xv[IT];
#pragma unroll
        for (uint32_t j = 0; j < IT; ++j) xv[j] = i0 + j < k + tile ? X(i0 + j) : 0.0f;
        // predicted crossings: the real prefix from the tile's start sum
        {
            uint64_t loc = 0;
#pragma unroll
            for (uint32_t j = 0; j < IT; ++j) loc += (uint64_t)((double)xv[j] * 0x1p40);
            Xd fx = xd_identity();
            fx.inc0 = fx.inc1 = loc;
            const uint64_t rb = block_excl_scan_xd<NT_EX>(fx, L.w).inc0;
            if (tid == 0) L.npc = 0;
            lds_barrier();
            double rs = (double)s + (double)rb * 0x1p-40;
            int eprev = ilogb(rs > 0.0 ? rs : 0x1p-1000);
#pragma unroll
            for (uint32_t j = 0; j < IT; ++j) {
                if (i0 + j >= k + tile) continue;
                rs += (double)(uint64_t)((double)xv[j] * 0x1p40) * 0x1p-40;
                const int e = ilogb(rs > 0.0 ? rs : 0x1p-1000);
                if (e > eprev) {
                    const uint32_t slot = atomicAdd(&L.npc, 1u);
                    if (slot < 32u) L.pc[slot] = i0 + j;
                }
                eprev = e;
            }
            lds_barrier();
        }
        const uint32_t npc = min(L.npc, 32u);
        uint32_t kk = k;  // the tile's first term not yet added
        while (true) {
            // the window [kk, we)
            uint32_t nxt = NONE;
            for (uint32_t q = 0; q < npc; ++q) {
                const uint32_t pq = L.pc[q];
                if (pq >= kk && pq < nxt) nxt = pq;
            }
            const uint32_t we = nxt == NONE ? k + tile : min(k + tile, nxt + 1u + WMARGIN);
            const Binade bd = binade_of(s);
            Term t[IT];
            Xd mine = xd_identity();
#pragma unroll
            for (uint32_t j = 0; j < IT; ++j) {
                t[j].c0 = t[j].c1 = 0u;
                if (i0 + j >= kk && i0 + j < we) {
                    t[j] = term_of(xv[j], bd.E);
                    mine = xd_compose(mine, xd_of(t[j]));
                }
            }
            Xd pre = block_excl_scan_xd<NT_EX>(mine, L.w);
            const uint32_t b0 = bd.A & 1u;
            uint64_t acc = (uint64_t)bd.A + (b0 ? pre.inc1 : pre.inc0);
            uint32_t par = b0 ? pre.par1 : pre.par0;
            uint32_t mycross = NONE;
            float xs = 0.0f, last = 0.0f;
#pragma unroll
            for (uint32_t j = 0; j < IT; ++j) {
                const uint32_t i = i0 + j;
                if (i < kk || i >= we || mycross != NONE) continue;
                const uint32_t cc = par ? t[j].c1 : t[j].c0;
                if (acc + cc >= (1ull << 24)) {
                    mycross = i;
                    xs = __fadd_rn(binade_value((uint32_t)acc, bd.E), xv[j]);  // the direct add
                    continue;
                }
                acc += cc;
                par = (uint32_t)(acc & 1u);
                last = binade_value((uint32_t)acc, bd.E);
                if (S) S[i] = last;
            }
            if (mycross != NONE) atomicMin(&L.cross, mycross);
            lds_barrier();
            const uint32_t kc = L.cross;
            if (kc == NONE) {
                if (we - 1u - i0 < IT) L.s = last;  // this thread holds the window's last term
            } else if (mycross == kc) {
                if (S) S[kc] = xs;
                L.s = xs;
            }
            lds_barrier();
            s = L.s;  // rewritten only after the next scan's barriers
            if (kc == NONE) {
                kk = we;
            } else {
                if (tid == 0) L.cross = NONE;  // read by every thread before the barrier above
                kk = kc + 1u;
            }
            if (kk >= k + tile) break;
        }
        k += tile;
        lds_barrier();  // L.pc read by every thread before the next tile rewrites it
    }
    __threadfence_block();
    __syncthreads();
    return s;
}

// Buckets of p >= 2^-14 (bucket 7168 holds 2^-14 itself) are the head:
// sorted and summed element by element.  The tail buckets [NHB, TB_END)
// (2^-24 <= p < 2^-14) hold one binade each except for a power-of-two top
// value.  Once the running sum is >= 1 (after the maximum, p = 1) its
// spacing U is >= 2^-23 and a tail term x has x / U = M / 2^d with M its
// significand and d >= 15, so the rounding boundaries of x / U fall on
// multiples of 2^14 of the bit pattern: every element below the bucket's top
// value adds the same number of units, in any order.  Such a bucket is one
// term (count x units) while the sum stays in its binade; a bucket that
// would leave the binade or that holds its top value is sorted and summed
// element by element.
constexpr uint32_t NHB = 7169;
constexpr uint32_t TB_END = 12289;  // bucket of 2^-24, the lowest floor, + 1
__device__ __forceinline__ uint32_t bucket_top(uint32_t b) { return 0x3F800000u - (b << 14); }

// Row r's exact path (rs: its state; X: LDS scratch).  Called by the NT_EX
// threads of one workgroup; XI = keys or terms per thread in flight at once
// (a register budget).
template <uint32_t XI>
__device__ __forceinline__ void exact_row(const KArgs& a, int r, const RowState& rs, ExLds& XL) {
    uint32_t* s_cnt = XL.cnt;
    Xd* s_w = XL.sum.w;
    uint32_t* s_u = XL.u;
    float& s_s = XL.sum.s;
    uint32_t &s_k = XL.k, &s_cross = XL.cross, &s_err = XL.err;
    const int tid = threadIdx.x;
    const axs_sampling_params p = row_params(a, r);
    const uint32_t V = (uint32_t)a.vocab;
    const bool sorted = rs.sorted != 0;
    const uint32_t n = sorted ? rs.ncompact : V;
    const uint64_t* src = a.ckey + (size_t)r * V;
    uint64_t* keys = a.ckey2 + (size_t)r * V;
    uint64_t* sorted_keys = a.ckey + (size_t)r * V;  // written once src is consumed
    uint32_t* bend = a.bend + (size_t)r * BEND_STRIDE;
    uint32_t* zc = bend + NBUCKET;  // copies of each tail bucket's top value
    const float* dense = a.dense + (size_t)r * V;
    float* S = a.sbuf + (size_t)r * V;
    if (tid == 0) s_err = 0;
    uint64_t* const ck2 = keys;  // the head grouped by bucket, then the tail keys in any order
    // block sort of kp[st, en) by (p desc, id asc): in LDS (s_cnt) up to
    // BIG_LDS_SORT keys, else in the row's HBM scratch.  Uniform control flow.
    auto sort_range_in = [&](uint64_t* kp, uint32_t st, uint32_t en) {
        const uint32_t mcount = en - st;
        if (mcount <= 1) return;
        if (mcount <= 64u) {
            // one wave: each lane's key goes to its rank, the number of
            // larger keys (keys are distinct: ids are)
            if (tid < 64) {
                const uint64_t mk = (uint32_t)tid < mcount ? kp[st + tid] : 0ull;
                uint32_t rk = 0;
                for (uint32_t j = 0; j < mcount; ++j) {
                    const uint64_t kj = ((uint64_t)(uint32_t)__shfl((int)(uint32_t)(mk >> 32), (int)j, 64) << 32) |
                                        (uint32_t)__shfl((int)(uint32_t)mk, (int)j, 64);
                    rk += kj > mk ? 1u : 0u;
                }
                if ((uint32_t)tid < mcount) kp[st + rk] = mk;
            }
            __threadfence_block();
            __syncthreads();
            return;
        }
        const uint32_t np2 = next_pow2(mcount);
        uint64_t* t = np2 <= BIG_LDS_SORT ? (uint64_t*)s_cnt : a.tmp64 + (size_t)r * a.tmp_stride;
        for (uint32_t i = tid; i < np2; i += NT_EX) t[i] = i < mcount ? kp[st + i] : 0ull;
        __threadfence_block();
        __syncthreads();
        block_sort_desc<NT_EX>(t, np2);
        for (uint32_t i = tid; i < mcount; i += NT_EX) kp[st + i] = t[i];
        __threadfence_block();
        __syncthreads();
    };
    auto sort_range = [&](uint32_t st, uint32_t en) { sort_range_in(keys, st, en); };
    // Each bucket of at most 64 keys among positions [p0, p1) of the grouped
    // keys gk is sorted by the wave whose window of 64 positions holds its
    // start: the window's 128 keys staged in LDS, each key's rank = the keys
    // of its bucket above it, written to dk.  Keys of larger buckets are
    // copied in place, and a large bucket holding two different p is marked
    // for a block sort; one whose p are all equal is already in p order, and
    // its ids are ordered later only where an output reads them.  Bucket
    // ends in s_cnt.
    auto window_sort = [&](const uint64_t* gk, uint64_t* dk, uint32_t p0, uint32_t p1) {
        const int wv = tid >> 6, lane = tid & 63;
        uint64_t* st = XL.stage + (uint32_t)wv * 128u;
        constexpr uint32_t WSTEP = 64u * (NT_EX / 64);
        auto wload = [&](uint32_t at) { return at < p1 ? gk[at] : 0ull; };
        uint64_t n0 = wload(p0 + (uint32_t)wv * 64u + lane), n1 = wload(p0 + (uint32_t)wv * 64u + 64u + lane);
        for (uint32_t s0 = p0 + (uint32_t)wv * 64u; s0 < p1; s0 += WSTEP) {
            const uint64_t k0 = n0, k1 = n1;
            n0 = wload(s0 + WSTEP + lane);  // the next window's keys, in flight meanwhile
            n1 = wload(s0 + WSTEP + 64u + lane);
            st[lane] = k0;
            st[64 + lane] = k1;
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const uint32_t pos = s0 + (uint32_t)h * 64u + (uint32_t)lane;
                const uint64_t key = h ? k1 : k0;
                if (pos >= p1) continue;
                const uint32_t b = bucket_of(key);
                const uint32_t bs = b ? s_cnt[b - 1] : 0u, be = s_cnt[b];
                if (be - bs <= 64u) {
                    if (bs >= s0 && bs < s0 + 64u) {
                        uint32_t rank = 0, q = bs;
                        for (; q + 4u <= be; q += 4u) {  // four LDS reads in flight
                            const uint64_t c0 = st[q - s0], c1 = st[q + 1u - s0];
                            const uint64_t c2 = st[q + 2u - s0], c3 = st[q + 3u - s0];
                            rank += (c0 > key ? 1u : 0u) + (c1 > key ? 1u : 0u) + (c2 > key ? 1u : 0u) +
                                    (c3 > key ? 1u : 0u);
                        }
                        for (; q < be; ++q) rank += st[q - s0] > key ? 1u : 0u;
                        dk[bs + rank] = key;
                    }
                } else {
                    if (h == 0) dk[pos] = key;
                    if (pdesc_p(key) != pdesc_p(gk[bs])) atomicOr(&XL.mixed[b >> 5], 1u << (b & 31u));
                }
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        }
        __threadfence_block();
        __syncthreads();
    };
    // large buckets with two different p (marked in XL.mixed): block sorts of
    // keys (uniform loop)
    auto mixed_sorts = [&]() {
        uint32_t anym = 0;
        for (uint32_t i = tid; i < NMIXW; i += NT_EX) anym |= XL.mixed[i];
        if (__syncthreads_or(anym != 0u))
        for (uint32_t wi = 0; wi < NMIXW; ++wi) {
            uint32_t bits = XL.mixed[wi];
            while (bits) {
                const uint32_t b = wi * 32u + (uint32_t)__ffs((int)bits) - 1u;
                bits &= bits - 1u;
                sort_range(b ? bend[b - 1] : 0u, bend[b]);
            }
        }
        __syncthreads();
    };

    // positions [0, n_head) are sorted in keys and summed element by element;
    // the tail keys stay unordered in ck2[n_head, n) unless tail_all
    uint32_t n_head = n;
    bool tail_all = true;
    if (sorted) {
        // counting sort by p bucket (descending p) into keys
        for (uint32_t i = tid; i < NBUCKET; i += NT_EX) s_cnt[i] = 0;
        for (uint32_t i = tid; i < NMIXW; i += NT_EX) {
            XL.mixed[i] = 0;
            XL.topv[i] = 0;
            XL.done[i] = 0;
        }
        if (tid == 0) s_k = 0;
        __syncthreads();
        constexpr uint32_t U = XI;  // keys per thread per round, every load issued first
        for (uint32_t i0 = tid; i0 < n; i0 += NT_EX * U) {
            uint64_t kk[U];
#pragma unroll
            for (uint32_t u = 0; u < U; ++u) kk[u] = i0 + u * NT_EX < n ? src[i0 + u * NT_EX] : 0ull;
#pragma unroll
            for (uint32_t u = 0; u < U; ++u)
                if (i0 + u * NT_EX < n) {
                    const uint32_t b = bucket_of(kk[u]);
                    atomicAdd(&s_cnt[b], 1u);
                    if (b >= NHB && (uint32_t)(kk[u] >> 32) == bucket_top(b)) {
                        atomicOr(&XL.topv[b >> 5], 1u << (b & 31u));
                        // zero before the call; waited for here, so that the
                        // count is complete before any later read
                        const uint32_t old = atomicAdd(&zc[b - NHB], 1u);
                        asm volatile("" ::"v"(old));
                    }
                }
        }
        __syncthreads();
        constexpr uint32_t PER = NBUCKET / NT_EX;
        uint32_t loc = 0;
        for (uint32_t q = 0; q < PER; ++q) loc += s_cnt[tid * PER + q];
        uint32_t tot;
        uint32_t pre = block_excl_scan_u32<NT_EX>(loc, s_u, &tot);
        for (uint32_t q = 0; q < PER; ++q) {
            uint32_t c = s_cnt[tid * PER + q];
            s_cnt[tid * PER + q] = pre;
            pre += c;
        }
        __syncthreads();
        // head keys to their bucket's range; tail keys appended after the
        // head in any order (one claim per wave and round)
        n_head = s_cnt[NHB];
        const int lane = tid & 63;
        for (uint32_t i0 = tid; i0 < n; i0 += NT_EX * U) {
            uint64_t kk[U];
#pragma unroll
            for (uint32_t u = 0; u < U; ++u) kk[u] = i0 + u * NT_EX < n ? src[i0 + u * NT_EX] : 0ull;
#pragma unroll
            for (uint32_t u = 0; u < U; ++u) {
                const bool ok = i0 + u * NT_EX < n;
                const uint32_t b = bucket_of(kk[u]);
                if (ok && b < NHB) keys[atomicAdd(&s_cnt[b], 1u)] = kk[u];
                const uint64_t tm = __ballot(ok && b >= NHB);
                if (tm) {
                    uint32_t base = 0;
                    if (lane == 0) base = atomicAdd(&s_k, (uint32_t)__popcll(tm));
                    base = (uint32_t)__shfl((int)base, 0, 64);
                    if (ok && b >= NHB)
                        keys[n_head + base + (uint32_t)__popcll(tm & ((1ull << lane) - 1ull))] = kk[u];
                }
            }
        }
        __threadfence_block();
        __syncthreads();
        // s_cnt[b] is now the end of head bucket b and the start of tail
        // bucket b; bucket ends kept in HBM for the phases that reuse s_cnt
        // as sort scratch
        for (uint32_t i = tid; i < NBUCKET; i += NT_EX)
            bend[i] = i < NHB ? s_cnt[i] : (i + 1u < NBUCKET ? s_cnt[i + 1u] : n);
        tail_all = n_head >= n;
        window_sort(keys, sorted_keys, 0u, n_head);
        keys = sorted_keys;
        mixed_sorts();
    }
    __syncthreads();

    // exact running sums of the keys' p (or the dense row), in parallel
    constexpr uint32_t IT = XI;
    auto elem_sums = [&](const uint64_t* kp, uint32_t k0, uint32_t kend, float s0) -> float {
        if (kp) return block_exact_sums<IT>([&](uint32_t i) { return pdesc_p(kp[i]); }, k0, kend, s0, S, XL.sum);
        return block_exact_sums<IT>([&](uint32_t i) { return dense[i]; }, k0, kend, s0, S, XL.sum);
    };
    // tail bucket b extracted to its range of keys, sorted, and summed element
    // by element from the sum before it (whole block, once per bucket)
    auto bucket_elems = [&](uint32_t b, float sb) -> float {
        const uint32_t bs = bend[b - 1], be = bend[b];
        if (!tail_all) {
            // the bucket's keys, from the unordered tail, to its range of keys
            if (tid == 0) XL.xc = 0;
            __syncthreads();
            const int lane = tid & 63;
            for (uint32_t i0 = n_head + (uint32_t)tid; i0 < n; i0 += NT_EX * IT) {
                uint64_t kk[IT];
#pragma unroll
                for (uint32_t u = 0; u < IT; ++u) kk[u] = i0 + u * NT_EX < n ? ck2[i0 + u * NT_EX] : 0ull;
#pragma unroll
                for (uint32_t u = 0; u < IT; ++u) {
                    const bool hit = i0 + u * NT_EX < n && bucket_of(kk[u]) == b;
                    const uint64_t hm = __ballot(hit);
                    if (hm) {
                        uint32_t base = 0;
                        if (lane == 0) base = atomicAdd(&XL.xc, (uint32_t)__popcll(hm));
                        base = (uint32_t)__shfl((int)base, 0, 64);
                        if (hit) keys[bs + base + (uint32_t)__popcll(hm & ((1ull << lane) - 1ull))] = kk[u];
                    }
                }
            }
            __threadfence_block();
            __syncthreads();
        }
        sort_range_in(keys, bs, be);
        const float se = elem_sums(keys, bs, be, sb);
        if (tid == 0) XL.done[b >> 5] |= 1u << (b & 31u);
        __syncthreads();
        return se;
    };
    // The tail buckets [NHB, TB_END) from the sum s0 (>= 1): a round takes IT
    // buckets per thread as terms: the copies of the top value first (counted
    // with the buckets; a possible tie makes that term parity-dependent),
    // then count x units for the rest.  The first bucket that would leave the
    // binade is sorted and summed element by element, and the next round
    // starts after it.  S is written at each bucket's last position.
    auto tail_sums = [&](float s0) {
        if (tid == 0) s_cross = NONE;
        __syncthreads();
        float s = s0;
        for (uint32_t k = NHB; k < TB_END;) {
            const Binade bd = binade_of(s);
            const uint32_t tile = min((uint32_t)NT_EX * IT, TB_END - k);
            const uint32_t i0 = k + (uint32_t)tid * IT;
            Xd bx[IT];
            uint32_t be[IT];
            uint32_t evm = 0, nem = 0;  // bit j: bucket i0 + j is an event / not empty
            uint32_t prev = i0 < k + tile ? bend[i0 - 1u] : 0u;
#pragma unroll
            for (uint32_t j = 0; j < IT; ++j) be[j] = i0 + j < k + tile ? bend[i0 + j] : 0u;
            Xd mine = xd_identity();
#pragma unroll
            for (uint32_t j = 0; j < IT; ++j) {
                const uint32_t b = i0 + j;
                bx[j] = xd_identity();
                if (b >= k + tile) continue;
                const uint32_t cnt = be[j] - prev;
                prev = be[j];
                if (!cnt) continue;
                nem |= 1u << j;
                const Term t = term_of(bits_f32(bucket_top(b) - 1u), bd.E);
                uint32_t z = 0;
                if ((XL.topv[b >> 5] >> (b & 31u)) & 1u) z = atomicAdd(&zc[b - NHB], 0u);
                if (t.c0 != t.c1) {  // not reached: the rest of a tail bucket has no tie
                    evm |= 1u << j;
                    continue;
                }
                const uint64_t ri = (uint64_t)(cnt - z) * t.c0;
                Xd rest;
                rest.inc0 = rest.inc1 = ri;
                rest.par0 = (uint32_t)(ri & 1u);
                rest.par1 = (uint32_t)((ri + 1u) & 1u);
                Xd top = xd_identity(), base = xd_of(term_of(bits_f32(bucket_top(b)), bd.E));
                for (uint32_t e = z; e; e >>= 1) {
                    if (e & 1u) top = xd_compose(top, base);
                    base = xd_compose(base, base);
                }
                bx[j] = xd_compose(top, rest);
                mine = xd_compose(mine, bx[j]);
            }
            const Xd pre = block_excl_scan_xd<NT_EX>(mine, s_w);
            const uint32_t b0 = bd.A & 1u;
            uint64_t acc = (uint64_t)bd.A + (b0 ? pre.inc1 : pre.inc0);
            uint32_t par = b0 ? pre.par1 : pre.par0;
            uint32_t mystop = NONE;
            float stopv = 0.0f, last = 0.0f;
#pragma unroll
            for (uint32_t j = 0; j < IT; ++j) {
                const uint32_t b = i0 + j;
                if (b >= k + tile || mystop != NONE) continue;
                const uint64_t inc = par ? bx[j].inc1 : bx[j].inc0;
                if (((evm >> j) & 1u) || acc + inc >= (1ull << 24)) {
                    mystop = b;
                    stopv = binade_value((uint32_t)acc, bd.E);
                    continue;
                }
                par = par ? bx[j].par1 : bx[j].par0;
                acc += inc;
                last = binade_value((uint32_t)acc, bd.E);
                if ((nem >> j) & 1u) S[be[j] - 1u] = last;
            }
            if (mystop != NONE) atomicMin(&s_cross, mystop);
            lds_barrier();
            const uint32_t kc = s_cross;
            if (kc == NONE) {
                if (k + tile - 1u - i0 < IT) s_s = last;  // this thread holds the tile's last bucket
            } else if (mystop == kc) {
                s_s = stopv;
            }
            lds_barrier();
            s = s_s;
            if (kc == NONE) {
                k += tile;
                continue;
            }
            __syncthreads();  // s_s and s_cross read by every thread
            if (tid == 0) s_cross = NONE;
            s = bucket_elems(kc, s);  // resets s_cross itself
            k = kc + 1u;
        }
        __threadfence_block();
        __syncthreads();
    };
    // the whole tail sorted into keys after the head, as the head is
    auto tail_sort_all = [&]() {
        // the unordered tail grouped by bucket into keys, then copied back to
        // ck2 as the window sort's source
        for (uint32_t i = tid; i < NBUCKET; i += NT_EX) s_cnt[i] = i ? bend[i - 1u] : 0u;
        __syncthreads();
        for (uint32_t i = n_head + (uint32_t)tid; i < n; i += NT_EX) {
            const uint64_t key = ck2[i];
            keys[atomicAdd(&s_cnt[bucket_of(key)], 1u)] = key;
        }
        __threadfence_block();
        __syncthreads();
        for (uint32_t i = n_head + (uint32_t)tid; i < n; i += NT_EX) ck2[i] = keys[i];
        for (uint32_t i = tid; i < NBUCKET; i += NT_EX) s_cnt[i] = bend[i];
        for (uint32_t i = tid; i < NMIXW; i += NT_EX) XL.mixed[i] = 0;
        __threadfence_block();
        __syncthreads();
        window_sort(ck2, keys, n_head, n);
        mixed_sorts();
        tail_all = true;
    };
    if (!sorted) {
        elem_sums(nullptr, 0u, V, 0.0f);
    } else if (n > 0) {
        // the top-value counts, left at zero for the next call once read
        auto reset_zc = [&]() {
            for (uint32_t wi = tid; wi < NMIXW; wi += NT_EX) {
                uint32_t bits = XL.topv[wi];
                while (bits) {
                    const uint32_t b = wi * 32u + (uint32_t)__ffs((int)bits) - 1u;
                    bits &= bits - 1u;
                    const uint32_t old = atomicExch(&zc[b - NHB], 0u);
                    asm volatile("" ::"v"(old));
                }
            }
        };
        const float sh = elem_sums(keys, 0u, n_head, 0.0f);
        if (!tail_all) {
            if (sh >= 1.0f) {
                tail_sums(sh);
            } else {  // not reached: the head holds the maximum (p = 1)
                tail_sort_all();
                elem_sums(keys, n_head, n, sh);
                n_head = n;
            }
        }
        reset_zc();
    }
    __threadfence_block();
    __syncthreads();  // every S store complete before the decisions read S

    if (a.lp_tokens && a.topn) {
        // top-N row: the n largest p (ties to the lower id) by a radix
        // select of the N-th largest p's bit pattern (4 passes of 8 bits over
        // the dense row; p >= 0, so the bits order as the values), those
        // above it and the lowest ids equal to it gathered, one wave's rank
        // sort; each with max(ln(max(p / S, 1e-37)), -30)
        const uint32_t n = a.topn < V ? a.topn : V;
        uint32_t* hist = s_cnt;            // 256 bins
        uint32_t* sel = s_cnt + 256;       // up to 64 selected ids
        uint32_t* eq = s_cnt + 512;        // ids equal to the cut, up to EQCAP
        constexpr uint32_t EQCAP = 4096;
        uint32_t prefix = 0, mask = 0, want = n;
        for (int shift = 24; shift >= 0; shift -= 8) {
            for (uint32_t i = tid; i < 256u; i += NT_EX) hist[i] = 0;
            __syncthreads();
            for (uint32_t i = tid; i < V; i += NT_EX) {
                const uint32_t b = __float_as_uint(dense[i]);
                if ((b & mask) == prefix) atomicAdd(&hist[(b >> shift) & 255u], 1u);
            }
            __syncthreads();
            if (tid == 0) {
                uint32_t cum = 0, d = 0;
                for (int q = 255; q >= 0; --q) {
                    if (cum + hist[q] >= want) {
                        d = (uint32_t)q;
                        break;
                    }
                    cum += hist[q];
                }
                s_k = d;
                s_cross = want - cum;
            }
            __syncthreads();
            prefix |= s_k << shift;
            mask |= 255u << shift;
            want = s_cross;
            __syncthreads();
        }
        // prefix: the N-th largest p; want: how many of its copies are listed
        if (tid == 0) {
            s_k = 0;     // ids above the cut
            s_cross = 0; // ids equal to it
        }
        __syncthreads();
        for (uint32_t i = tid; i < V; i += NT_EX) {
            const uint32_t b = __float_as_uint(dense[i]);
            if (b > prefix) sel[atomicAdd(&s_k, 1u)] = i;
            else if (b == prefix) {
                const uint32_t q = atomicAdd(&s_cross, 1u);
                if (q < EQCAP) eq[q] = i;
            }
        }
        __syncthreads();
        const uint32_t ngt = s_k, neq = s_cross;
        if (neq <= EQCAP) {
            // the `want` lowest ids among the copies: rank = smaller ids
            for (uint32_t q = tid; q < neq; q += NT_EX) {
                const uint32_t id = eq[q];
                uint32_t rk = 0;
                for (uint32_t j = 0; j < neq; ++j) rk += eq[j] < id ? 1u : 0u;
                if (rk < want) sel[ngt + rk] = id;
            }
        } else {
            // very many copies: the lowest ids one at a time
            uint32_t last = 0;
            for (uint32_t k = 0; k < want; ++k) {
                uint32_t best = NONE;
                for (uint32_t i = tid; i < V; i += NT_EX)
                    if (__float_as_uint(dense[i]) == prefix && (k == 0 || i > last) && i < best) best = i;
                if (tid == 0) s_k = NONE;
                __syncthreads();
                atomicMin(&s_k, best);
                __syncthreads();
                last = s_k;
                if (tid == 0) sel[ngt + k] = last;
                __syncthreads();
            }
        }
        __threadfence_block();
        __syncthreads();
        if (tid < 64) {
            // (p desc, id asc): each lane's entry goes to its rank
            const float F0 = S[V - 1];
            const bool okF = F0 > 0.0f && isfinite(F0);
            const uint32_t id = (uint32_t)tid < n ? sel[tid] : 0u;
            const float pv = (uint32_t)tid < n ? dense[id] : 0.0f;
            const uint64_t key = (uint32_t)tid < n ? (((uint64_t)__float_as_uint(pv) << 32) | (uint32_t)~id) : 0ull;
            uint32_t rk = 0;
            for (uint32_t j = 0; j < n; ++j) {
                const uint64_t kj = ((uint64_t)(uint32_t)__shfl((int)(uint32_t)(key >> 32), (int)j, 64) << 32) |
                                    (uint32_t)__shfl((int)(uint32_t)key, (int)j, 64);
                rk += kj > key ? 1u : 0u;
            }
            if ((uint32_t)tid < n) {
                a.topn_ids[(size_t)r * a.topn + rk] = id;
                a.topn_lp[(size_t)r * a.topn + rk] = okF ? logprob_of(__fdiv_rn(pv, F0)) : -30.0f;
            }
            for (uint32_t k = n + (uint32_t)tid; k < a.topn; k += 64u) {
                a.topn_ids[(size_t)r * a.topn + k] = NONE;
                a.topn_lp[(size_t)r * a.topn + k] = -INFINITY;
            }
            if (tid == 0) write_row(a, r, 0u, 0.0f, AXS_FLAG_EXACT_PATH);
        }
        return;
    }
    if (a.lp_tokens) {
        // token-logprob row: max(ln(max(p_t / S, 1e-37)), -30) with S the
        // index-order f32 sum (crates/ax-engine-mlx/src/sampling.rs:772-786)
        if (tid == 0) {
            const uint32_t t = a.lp_tokens[r];
            const float F0 = S[V - 1];
            float lp = -30.0f;
            if (F0 > 0.0f && isfinite(F0)) lp = logprob_of(__fdiv_rn(dense[t], F0));
            write_row(a, r, t, lp, AXS_FLAG_EXACT_PATH);
        }
        return;
    }
    if (rs.mode == M_GREEDY) {
        // greedy row listed for its logprob: -ln of the index-order sum
        // (crates/ax-engine-core/src/sampling.rs:179-190); the token is the
        // first maximum found by the stream
        if (tid == 0) {
            const float F0 = S[V - 1];
            const float lp = (F0 > 0.0f && isfinite(F0)) ? -ln_f32(F0) : NAN;
            const uint32_t flags = AXS_FLAG_GREEDY | AXS_FLAG_EXACT_PATH;
            write_row(a, r, rs.amax, lp, flags);
            write_single_kept(a, r, rs.amax);
            if (a.ws_kept_id) a.rstate[r].flags = flags;
        }
        return;
    }

    // index-order rows: the kept-set size and the ordered kept lists, by the
    // whole block
    uint32_t dkept = 0, dlist = 0, dpos = 0;
    if (!sorted) {
        const bool mp = rs.mode == M_MINP;
        uint32_t cnt = 0, cpos = 0;
        for (uint32_t i = tid; i < V; i += NT_EX) {
            cnt += (!mp || dense[i] > 0.0f) ? 1u : 0u;
            cpos += dense[i] > 0.0f ? 1u : 0u;
        }
        dkept = block_sum_u32<NT_EX>(cnt, s_u);
        // the distribution's entries (TokenDistribution::new keeps p > 0,
        // crates/ax-engine-mlx/src/sampling.rs:128-144)
        if (a.ws_kept_id) dpos = block_sum_u32<NT_EX>(cpos, s_u);
        // out_kept: ids with (!min-p || p > 0); ws lists: ids with p > 0
        const uint32_t cap_o = (a.out_kept && a.out_kept_cap > 0) ? (uint32_t)a.out_kept_cap : 0u;
        const uint32_t cap_w = a.ws_kept_id ? KEPT_CAP : 0u;
        uint32_t base_o = 0, base_w = 0;
        for (uint32_t c0 = 0; c0 < V && (base_o < cap_o || base_w < cap_w); c0 += NT_EX * 8u) {
            uint32_t fo = 0, fw = 0;
#pragma unroll
            for (uint32_t q = 0; q < 8; ++q) {
                const uint32_t i = c0 + (uint32_t)tid * 8u + q;
                const float pv = i < V ? dense[i] : 0.0f;
                if (i < V && (!mp || pv > 0.0f)) fo |= 1u << q;
                if (pv > 0.0f) fw |= 1u << q;
            }
            uint32_t to, tw;
            uint32_t po = base_o + block_excl_scan_u32<NT_EX>((uint32_t)__popc(fo), s_u, &to);
            uint32_t pw = base_w + block_excl_scan_u32<NT_EX>((uint32_t)__popc(fw), s_u, &tw);
#pragma unroll
            for (uint32_t q = 0; q < 8; ++q) {
                const uint32_t i = c0 + (uint32_t)tid * 8u + q;
                if ((fo >> q) & 1u) {
                    if (po < cap_o) a.out_kept[(size_t)r * cap_o + po] = i;
                    ++po;
                }
                if ((fw >> q) & 1u) {
                    if (pw < cap_w) {
                        a.ws_kept_id[(size_t)r * KEPT_CAP + pw] = i;
                        a.ws_kept_p[(size_t)r * KEPT_CAP + pw] = dense[i];
                    }
                    ++pw;
                }
            }
            base_o += to;
            base_w += tw;
        }
        dlist = base_w < cap_w ? base_w : cap_w;
    }

    // decisions (sampling.rs:283-316, 922-952) on the exact running sums,
    // computed by every thread (the same reads); one thread writes
    uint32_t flags = AXS_FLAG_DREW | AXS_FLAG_EXACT_PATH;
    if (s_err) flags |= AXS_FLAG_ERROR;
    const bool minp = rs.mode == M_MINP;
    if (minp && __uint_as_float(rs.minp_mg) < 1e-6f) flags |= AXS_FLAG_NEAR_MINP;
    uint32_t tok = 0;
    float F = 0.0f, pj = 0.0f;
    uint32_t kept = 0, Lk = 0;
    if (n == 0) {
        if (tid == 0) {
            tok = rs.amax;
            flags = AXS_FLAG_ARGMAX_FALLBACK | AXS_FLAG_EXACT_PATH;
            write_row(a, r, tok, NAN, flags);
            write_single_kept(a, r, tok);
            if (a.ws_kept_id) a.rstate[r].flags = flags;
        }
        return;
    }
    // Sorted rows: positions >= n_head lie in tail buckets, whose sums are
    // exact at each bucket's last position; a bucket that a decision reads
    // inside is sorted and summed element by element first (whole block:
    // every thread makes the same calls).
    auto tail_bucket_at = [&](uint32_t i) -> uint32_t {  // first b with bend[b] > i
        uint32_t lo = NHB, hi = TB_END - 1u;
        while (lo < hi) {
            const uint32_t mid = lo + (hi - lo) / 2;
            if (bend[mid] > i) hi = mid;
            else lo = mid + 1;
        }
        return lo;
    };
    auto ensure_bucket = [&](uint32_t b) {
        if ((XL.done[b >> 5] >> (b & 31u)) & 1u) return;
        const float sb = S[bend[b - 1] - 1u];
        __syncthreads();
        bucket_elems(b, sb);
    };
    auto S_at = [&](uint32_t i) -> float {
        if (i >= n_head) {
            const uint32_t b = tail_bucket_at(i);
            if (i + 1u != bend[b]) ensure_bucket(b);
        }
        return S[i];
    };
    auto key_at = [&](uint32_t i) -> uint64_t {
        if (i >= n_head && !tail_all) ensure_bucket(tail_bucket_at(i));
        return keys[i];
    };
    // first position in [0, lim) with S >= t, lim if none
    auto locate = [&](float t, uint32_t lim) -> uint32_t {
        const uint32_t hl = lim < n_head ? lim : n_head;
        const uint32_t j = first_ge(S, 0, hl, t);
        if (j < hl || lim <= n_head) return j;
        uint32_t lo = NHB, hi = TB_END;  // the first tail bucket whose sum reaches t
        while (lo < hi) {
            const uint32_t mid = lo + (hi - lo) / 2;
            if (S[bend[mid] - 1u] >= t) hi = mid;
            else lo = mid + 1;
        }
        if (lo >= TB_END || bend[lo - 1] >= lim) return lim;
        ensure_bucket(lo);
        const uint32_t jj = first_ge(S, bend[lo - 1], bend[lo], t);
        return jj < lim ? jj : lim;
    };
    if (sorted) {
        const uint32_t L = n;
        uint32_t nk = L;
        if (topp_active(p)) {
            float total = S[L - 1];  // the last bucket's end
            float cutoff = __fmul_rn(p.top_p, total);
            uint32_t j = locate(cutoff, L);
            nk = j < L ? j + 1 : L;
            double up = (double)S_at(nk - 1) - (double)cutoff;
            double lo = nk >= 2 ? (double)cutoff - (double)S_at(nk - 2) : INFINITY;
            if (fmin(up, lo) / (double)total < 1e-6 && (p.top_k == 0 || nk <= p.top_k))
                flags |= AXS_FLAG_NEAR_NUCLEUS;
            kept = nk;
        } else {
            // no nucleus cut: every candidate (all ids, or all min-p survivors)
            kept = minp ? 0xFFFFFFFFu : V;
        }
        if (p.top_k > 0 && kept > p.top_k) kept = p.top_k;
        Lk = kept < L ? kept : L;
        if (kept < L) {
            float pa = pdesc_p(key_at(kept - 1)), pb = pdesc_p(key_at(kept));
            if (pa != pb && (double)pa - (double)pb <= 2.0 * ulp_f(pa)) flags |= AXS_FLAG_NEAR_TIE;
        }
        F = S_at(Lk - 1);
        const float thr = __fmul_rn(rs.u, F);
        uint32_t j = locate(thr, Lk);
        if (j >= Lk) j = Lk - 1;  // unreachable: S[Lk-1] = F >= u*F
        double up = (double)S_at(j) - (double)thr;
        double lo = j > 0 ? (double)thr - (double)S_at(j - 1) : INFINITY;
        if (fmin(up, lo) / (double)F < 1e-6) flags |= AXS_FLAG_NEAR_DRAW;
        // ids are read at the draw position and in the kept prefixes; a
        // bucket of more than 64 keys with a single p is still in arbitrary
        // id order, so each one holding such a position is sorted first
        const uint32_t po = (a.out_kept && a.out_kept_cap > 0) ? min(Lk, (uint32_t)a.out_kept_cap) : 0u;
        // an MTP row's whole kept list is put in order: listed below when it
        // is short, read in place by the verify kernel otherwise
        const uint32_t pw = a.ws_kept_id ? Lk : 0u;
        const uint32_t P = max(po, pw);
        const uint64_t kj0 = key_at(j);  // a tail bucket read here is extracted and sorted
        if (P > n_head && !tail_all) tail_sort_all();
        auto order_ids = [&](uint32_t pos) -> uint32_t {  // returns the end of pos's bucket
            const uint32_t b = bucket_of(keys[pos]);
            const uint32_t bs = b ? bend[b - 1] : 0u, be = bend[b];
            if (be - bs > 64u) sort_range(bs, be);
            return be;
        };
        for (uint32_t pos = 0; pos < P;) pos = order_ids(pos);
        if (j >= P && (j < n_head || P > n_head)) order_ids(j);
        const uint64_t kj = (j < n_head || P > n_head) ? keys[j] : kj0;
        tok = pdesc_id(kj);
        pj = pdesc_p(kj);
        if (kept == 0xFFFFFFFFu) kept = L;  // min-p survivors below 2^-24 are not listed
    } else {
        F = S[V - 1];
        if (!(F > 0.0f)) {  // min_p > 1: no survivor (sampling.rs:290-293)
            if (tid == 0) empty_minp(a, r, rs.amax);
            return;
        }
        const float thr = __fmul_rn(rs.u, F);
        uint32_t j = first_ge(S, 0, V, thr);
        if (j >= V) j = V - 1;
        double up = (double)S[j] - (double)thr;
        double lo = j > 0 ? (double)thr - (double)S[j - 1] : INFINITY;
        if (fmin(up, lo) / (double)F < 1e-6) flags |= AXS_FLAG_NEAR_DRAW;
        tok = j;
        pj = dense[j];
        kept = dkept;
    }
    // the ordered kept lists (every thread)
    if (sorted && a.out_kept && a.out_kept_cap > 0) {
        // kept entries below the compaction floor (p < 2^-24 of the
        // maximum's: never drawn) are not ordered here; they are listed as
        // NONE after the ordered prefix
        const uint32_t cap = (uint32_t)a.out_kept_cap;
        const uint32_t nw = Lk < cap ? Lk : cap;
        const uint32_t ne = kept < cap ? kept : cap;
        for (uint32_t i = tid; i < ne; i += NT_EX) a.out_kept[(size_t)r * cap + i] = i < nw ? pdesc_id(keys[i]) : NONE;
    }
    const uint32_t nws = Lk <= KEPT_CAP ? Lk : 0u;
    if (sorted && a.ws_kept_id)
        for (uint32_t i = tid; i < nws; i += NT_EX) {
            a.ws_kept_id[(size_t)r * KEPT_CAP + i] = pdesc_id(keys[i]);
            a.ws_kept_p[(size_t)r * KEPT_CAP + i] = pdesc_p(keys[i]);
        }
    if (tid != 0) return;
    write_row(a, r, tok, logprob_of(__fdiv_rn(pj, F)), flags);
    if (a.out_kept_count) a.out_kept_count[r] = kept;
    if (a.ws_kept_id) {
        uint32_t o = 0;
        uint32_t rsf = 0;
        if (sorted) {
            o = nws;
            // ids below 2^-24 never carry normalised mass ≥ one f32 ulp of 1, but
            // they are entries of the reference's distribution: refuse to
            // truncate silently
            if (kept > Lk) flags |= AXS_FLAG_ERROR;
            if (Lk > KEPT_CAP) {  // the list is the row's sorted keys [0, Lk)
                o = Lk;
                rsf = RSF_LIST_IN_ROW;
            }
        } else {
            o = dlist;
            kept = dpos;  // an MTP distribution counts its p > 0 entries
            if (dpos > KEPT_CAP) {  // the list is the dense row's p > 0 entries
                o = dpos;
                rsf = RSF_LIST_IN_ROW;
            }
        }
        a.rstate[r].kept = kept;
        a.rstate[r].nlist = o;
        a.rstate[r].F = F;
        a.rstate[r].flags = flags | rsf;
    }
}

// One workgroup per listed row.  Every workgroup of the grid also counts
// itself out; the last one clears the exact-row list for the next call (all
// of them have read its length by then).
__global__ __launch_bounds__(NT_EX) void k_exact_row(KArgs a) {
    __shared__ ExLds X;
    const uint32_t nex = *a.exact_count;
    if (blockIdx.x < nex) {
        const int r = (int)a.exact_rows[blockIdx.x];
        const RowState rs = a.rstate[r];
        exact_row<8>(a, r, rs, X);
    }
    __syncthreads();
    if (threadIdx.x == 0 && atomicInc(a.ex_done, gridDim.x - 1u) == gridDim.x - 1u) *a.exact_count = 0u;
}

// --------------------------------------------------------------------------
// k_mtp_verify: accept / residual / bonus per sequence
// (crates/ax-engine-mlx/src/runner/mod.rs:12388-12431, sampling.rs:709-752)
// --------------------------------------------------------------------------
constexpr int NT_MTP = 1024;
// One 1024-thread workgroup per sequence.  Per draft position i, in order:
// a greedy comparison of the draft with the target's prediction (the mode
// gates, or no target probabilities / no finite draft log-prob), or the
// rejection test u < min(1, P_i(d) / q') with q' = max(exp(ln q * Td/Tt),
// 1e-37) (the temperature ratio for model drafts only, when the two differ)
// (runner/mod.rs:12355-12446).  A rejected test is corrected by the residual
// max(P_i - Q_i, 0) over the id-ascending union (Q_i = delta(draft) for an
// n-gram draft when delta_correction is set) or, for an n-gram draft
// without it, left to the target row's own draw; a failed comparison is
// corrected by the prediction.  The tail (runner/mod.rs:9732-9775): the
// correction, else the bonus draw of target row D, else the draw of the
// target row at the rejected position.  With a.mtp_stream the uniforms are
// taken in the reference's stream order; otherwise slot i for position i's
// test and slot D for the tail (axs_mtp_verify).
__global__ __launch_bounds__(NT_MTP) void k_mtp_verify(KArgs a, const uint32_t* draft_ids,
                                                       uint32_t* out_ids, uint32_t* out_count,
                                                       uint32_t* out_accept, uint32_t* out_flags,
                                                       const float* ptgt) {
    __shared__ uint64_t s_t[KEPT_CAP];
    __shared__ uint64_t s_d[KEPT_CAP];
    __shared__ float s_v[KEPT_CAP];     // residual terms (then their normalised values) in walk order
    __shared__ __align__(16) uint32_t s_id[KEPT_CAP]; // ... and their ids
    __shared__ int s_ft, s_fd;
    __shared__ float s_rsum, s_total;
    __shared__ uint32_t s_cr;
    __shared__ uint64_t s_mx;
    __shared__ SumLds s_sum;
    __shared__ uint32_t s_corr;
    const int b = blockIdx.x;
    const int tid = threadIdx.x;
    const int D = a.mtp_depth;
    const int Bm = a.mtp_batch;
    if (b >= Bm) return;
    const axs_sampling_params tp = a.params[b];
    const axs_sampling_params dp = a.params2[b];
    const float Tt = tp.temperature, Td = dp.temperature;
    const bool stream = a.mtp_stream != 0;
    constexpr uint32_t NEAR_DIST = AXS_FLAG_NEAR_NUCLEUS | AXS_FLAG_NEAR_MINP | AXS_FLAG_NEAR_TIE;
    constexpr uint32_t NEAR_ALL = NEAR_DIST | AXS_FLAG_NEAR_DRAW;
    uint32_t flags = 0;
    uint32_t count = 0;    // accepted drafts
    uint32_t nu = 0;       // uniforms consumed (stream order)
    uint32_t corr = NONE;  // the correction token
    int tail_row = -1;     // position whose target row's own draw is the tail
    bool stopped = false;
    for (int i = 0; i < D; ++i) {
        const int tr = b * (D + 1) + i;
        const int dr = Bm * (D + 1) + b * D + i;
        const uint32_t src = stream ? mtp_source(a, b, i) : (uint32_t)AXS_MTP_SRC_MTP;
        const bool has_dd = src != AXS_MTP_SRC_NGRAM;
        const uint32_t d = draft_ids[(size_t)b * D + i];
        if (stream && !mtp_is_test(a, b, i, Tt)) {
            // greedy comparison with the target's prediction
            const uint32_t pred = a.mtp_pred ? a.mtp_pred[(size_t)b * D + i] : a.mtp_amax[tr];
            if (pred == d) {
                if (tid == 0) out_ids[(size_t)b * (D + 1) + count] = d;
                ++count;
                continue;
            }
            corr = pred;
            flags |= AXS_MTP_FLAG_CORRECTION;
            stopped = true;
            break;
        }
        const RowState rt = a.rstate[tr];
        const RowState rd = has_dd ? a.rstate[dr] : rt;
        if ((rt.flags | rd.flags) & AXS_FLAG_ERROR || rt.nlist < rt.kept || rd.nlist < rd.kept) {
            flags |= AXS_MTP_FLAG_ERROR;
            stopped = true;
            break;
        }
        if ((rt.flags | rd.flags) & NEAR_DIST) flags |= AXS_MTP_FLAG_NEAR;
        const uint32_t* tid_l = a.ws_kept_id + (size_t)tr * KEPT_CAP;
        const float* tp_l = a.ws_kept_p + (size_t)tr * KEPT_CAP;
        const uint32_t* did_l = a.ws_kept_id + (size_t)dr * KEPT_CAP;
        const float* dp_l = a.ws_kept_p + (size_t)dr * KEPT_CAP;
        // every wave has read the previous position's s_ft / s_fd (an accept
        // continues straight here) before thread 0 clears them
        __syncthreads();
        if (tid == 0) {
            s_ft = -1;
            s_fd = -1;
        }
        __syncthreads();
        // d's entry in each list: a short list is a KEPT_CAP list, a long one
        // the row's sorted keys (found by scan) or its dense row (read by id)
        const size_t Vz = (size_t)a.vocab;
        const bool big_t = (rt.flags & RSF_LIST_IN_ROW) != 0u;
        const bool big_d = has_dd && (rd.flags & RSF_LIST_IN_ROW) != 0u;
        auto find = [&](int row, const RowState& rs_, bool big, const uint32_t* idl, int* slot) {
            if (!big) {
                for (uint32_t k = tid; k < rs_.nlist; k += NT_MTP)
                    if (idl[k] == d) atomicMax(slot, (int)k);
            } else if (rs_.sorted) {
                const uint64_t* kp = a.ckey + (size_t)row * Vz;
                for (uint32_t k = tid; k < rs_.nlist; k += NT_MTP)
                    if (pdesc_id(kp[k]) == d) atomicMax(slot, (int)k);
            }
        };
        // the raw p of d (-1 when d is not an entry)
        auto praw = [&](int row, const RowState& rs_, bool big, const float* pl, int slot) -> float {
            if (!big) return slot >= 0 ? pl[slot] : -1.0f;
            if (rs_.sorted) return slot >= 0 ? pdesc_p(a.ckey[(size_t)row * Vz + (uint32_t)slot]) : -1.0f;
            const float v = d < (uint32_t)a.vocab ? a.dense[(size_t)row * Vz + d] : 0.0f;
            return v > 0.0f ? v : -1.0f;
        };
        find(tr, rt, big_t, tid_l, &s_ft);
        if (has_dd) find(dr, rd, big_d, did_l, &s_fd);
        __syncthreads();
        const float rawt = praw(tr, rt, big_t, tp_l, s_ft);
        const float rawd = has_dd ? praw(dr, rd, big_d, dp_l, s_fd) : -1.0f;
        // normalised entries p / F (TokenDistribution::new, sampling.rs:128-144)
        float pt = fmaxf(rawt >= 0.0f ? __fdiv_rn(rawt, rt.F) : 0.0f, 0.0f);
        if (ptgt) pt = ptgt[(size_t)b * D + i];  // the production law's (k_mtp_prod), or P_i(d)
        float lnq;
        if (a.mtp_lnq_in) {
            lnq = a.mtp_lnq_in[(size_t)b * D + i];
        } else if (!has_dd) {
            lnq = 0.0f;  // an n-gram draft under the delta law
        } else if (a.mtp_lnq_full) {
            lnq = a.mtp_lnq_full[(size_t)b * D + i];
        } else {
            lnq = logprob_of(rawd >= 0.0f ? __fdiv_rn(rawd, rd.F) : 0.0f);
        }
        float lps = lnq;
        if (has_dd && Td > 0.0f && Tt > 0.0f && fabsf(__fsub_rn(Td, Tt)) > 1e-6f)
            lps = __fmul_rn(lnq, __fdiv_rn(Td, Tt));
        const float pdraft = fmaxf(exp_ref(lps), 1e-37f);
        const float accp = fminf(__fdiv_rn(pt, pdraft), 1.0f);
        const float u = mtp_uniform(a, b, tp, stream ? nu++ : (uint32_t)i);
        // u >= 1 never accepts, whatever accp <= 1 rounds to
        if (u < 1.0f && fabs((double)u - (double)accp) < 1e-6) flags |= AXS_MTP_FLAG_NEAR_ACCEPT;
        if (u < accp) {
            if (tid == 0) out_ids[(size_t)b * (D + 1) + count] = d;
            ++count;
            continue;
        }
        stopped = true;
        if (!has_dd && !a.mtp_delta) {
            tail_row = i;  // no correction: the target row's own draw (sample_logit_row)
            break;
        }
        // residual max(P - Q, 0) over the union of ids, ascending id order
        // (runner/mod.rs:12409-12431, sampling.rs:709-752; Q = delta(draft)
        // for an n-gram draft: runner/mod.rs:12161-12184).  An id only in Q
        // carries max(0 - q, 0) = 0 and is skipped, so the walk is over the
        // target's ids: both lists sorted by id, each target term with its
        // draft entry found by binary search, all in parallel; the
        // reference's sequential f32 sums run on one thread over LDS.
        const float ut = mtp_uniform(a, b, tp, stream ? nu : (uint32_t)D);
        if (big_t || big_d) {
            // A list too long for the KEPT_CAP lists: the residual over every
            // id in ascending order, in global memory — P and Q by id in the
            // rows' dense buffers (a sorted row's list scattered there first;
            // an index-order row's dense row is its distribution), the terms
            // and running sums in the target row's ckey2 buffer (free by now),
            // the reference's sequential sums by the exact block scan.
            const uint32_t V = (uint32_t)a.vocab;
            float* Pd = a.dense + (size_t)tr * Vz;
            float* Qd = has_dd ? a.dense + (size_t)dr * Vz : nullptr;
            float* W = reinterpret_cast<float*>(a.ckey2 + (size_t)tr * Vz);
            float* Cs = W + V;
            auto by_id = [&](int row, const RowState& rs_, bool big, const uint32_t* idl, const float* pl, float* dst) {
                if (!rs_.sorted) return;  // the dense row holds p; its entries are p > 0
                for (uint32_t k = tid; k < V; k += NT_MTP) dst[k] = 0.0f;
                __threadfence_block();
                __syncthreads();
                const uint64_t* kp = a.ckey + (size_t)row * Vz;
                for (uint32_t k = tid; k < rs_.nlist; k += NT_MTP) {
                    if (big) dst[pdesc_id(kp[k])] = pdesc_p(kp[k]);
                    else dst[idl[k]] = pl[k];
                }
                __threadfence_block();
                __syncthreads();
            };
            by_id(tr, rt, big_t, tid_l, tp_l, Pd);
            if (has_dd) by_id(dr, rd, big_d, did_l, dp_l, Qd);
            // residual terms over the target's entries; an id only in Q
            // carries max(0 - q, 0) = 0 and is no entry of the walk
            for (uint32_t k = tid; k < V; k += NT_MTP) {
                const float pr = Pd[k];
                float w = 0.0f;
                if (pr > 0.0f) {
                    const float ptk = __fdiv_rn(pr, rt.F);
                    float qk = 0.0f;
                    if (has_dd) qk = Qd[k] > 0.0f ? __fdiv_rn(Qd[k], rd.F) : 0.0f;
                    else if (k == d) qk = 1.0f;
                    const float v = fmaxf(__fsub_rn(ptk, qk), 0.0f);
                    w = (v > 0.0f && isfinite(v)) ? v : 0.0f;
                }
                W[k] = w;
            }
            __threadfence_block();
            __syncthreads();
            const float rsum = block_exact_sums<8>([&](uint32_t k) { return W[k]; }, 0u, V, 0.0f, nullptr, s_sum);
            // the walk: position k's id and normalised value (-1: no entry)
            const bool resid = rsum > 0.0f && isfinite(rsum);
            uint32_t nwalk = V;
            if (resid) {
                for (uint32_t k = tid; k < V; k += NT_MTP) W[k] = W[k] > 0.0f ? __fdiv_rn(W[k], rsum) : -1.0f;
            } else if (rt.sorted) {
                // empty residual: the target itself, in its kept order (sampling.rs:749)
                nwalk = rt.nlist;
                const uint64_t* kp = a.ckey + (size_t)tr * Vz;
                for (uint32_t k = tid; k < nwalk; k += NT_MTP)
                    W[k] = __fdiv_rn(big_t ? pdesc_p(kp[k]) : tp_l[k], rt.F);
            } else {
                for (uint32_t k = tid; k < V; k += NT_MTP) W[k] = Pd[k] > 0.0f ? __fdiv_rn(Pd[k], rt.F) : -1.0f;
            }
            if (tid == 0) {
                s_cr = NONE;
                s_mx = 0ull;
            }
            __threadfence_block();
            __syncthreads();
            const float total = block_exact_sums<8>([&](uint32_t k) { return W[k] < 0.0f ? 0.0f : W[k]; }, 0u, nwalk,
                                                    0.0f, Cs, s_sum);
            const float thr = __fmul_rn(ut, total);
            for (uint32_t k = tid; k < nwalk; k += NT_MTP) {
                const float q = W[k];
                if (q < 0.0f) continue;
                if (Cs[k] >= thr) atomicMin(&s_cr, k);
                atomicMax(&s_mx, ((uint64_t)__float_as_uint(q) << 32) | (k + 1u));
            }
            __syncthreads();
            if (tid == 0) {
                const uint32_t cr = s_cr;
                const uint64_t mx = s_mx;
                const uint32_t kpos = cr != NONE ? cr : (mx ? (uint32_t)mx - 1u : NONE);
                uint32_t id = kpos;
                if (kpos != NONE && !resid && rt.sorted)
                    id = big_t ? pdesc_id(a.ckey[(size_t)tr * Vz + kpos]) : tid_l[kpos];
                s_corr = id;
            }
            __syncthreads();
            corr = s_corr;
            flags |= AXS_MTP_FLAG_RESIDUAL;
            break;
        }
        const uint32_t nt = rt.nlist, nd = has_dd ? rd.nlist : 1u;
        // a kept list to ascending id order: each entry's position is the
        // number of smaller ids (the ids of a list are distinct), counted
        // over the list staged in LDS (broadcast reads, no sorting network)
        auto id_order = [&](const uint32_t* ids, const float* ps, float F, uint32_t n, uint64_t* dst) {
            for (uint32_t k = tid; k < n; k += NT_MTP) {
                s_id[k] = ids[k];
                s_v[k] = __fdiv_rn(ps[k], F);
            }
            __syncthreads();
            for (uint32_t k = tid; k < n; k += NT_MTP) {
                const uint32_t idk = s_id[k];
                uint32_t rk = 0, j = 0;
                for (; j + 16u <= n; j += 16u) {  // four 16-byte reads in flight
                    u32x4 w[4];
#pragma unroll
                    for (int h = 0; h < 4; ++h) w[h] = *reinterpret_cast<const u32x4*>(&s_id[j + 4u * (uint32_t)h]);
#pragma unroll
                    for (int h = 0; h < 4; ++h)
                        rk += (w[h][0] < idk ? 1u : 0u) + (w[h][1] < idk ? 1u : 0u) + (w[h][2] < idk ? 1u : 0u) +
                              (w[h][3] < idk ? 1u : 0u);
                }
                for (; j < n; ++j) rk += s_id[j] < idk ? 1u : 0u;
                dst[rk] = ((uint64_t)(~idk) << 32) | __float_as_uint(s_v[k]);
            }
            __syncthreads();
        };
        id_order(tid_l, tp_l, rt.F, nt, s_t);
        if (has_dd) {
            id_order(did_l, dp_l, rd.F, nd, s_d);
        } else {
            if (tid == 0) s_d[0] = ((uint64_t)(~d) << 32) | __float_as_uint(1.0f);
            __syncthreads();
        }
        for (uint32_t k = tid; k < nt; k += NT_MTP) {
            const uint32_t id = idasc_id(s_t[k]);
            uint32_t lo = 0, hi = nd;
            while (lo < hi) {
                const uint32_t mid = (lo + hi) >> 1;
                if (idasc_id(s_d[mid]) < id) lo = mid + 1u;
                else hi = mid;
            }
            const float ptk = idasc_p(s_t[k]);
            s_v[k] = (lo < nd && idasc_id(s_d[lo]) == id) ? fmaxf(__fsub_rn(ptk, idasc_p(s_d[lo])), 0.0f) : ptk;
            s_id[k] = id;
        }
        __syncthreads();
        // The reference's sequential f32 sums: the terms prepared by every
        // thread (a skipped term as +0, which leaves a non-negative f32 sum
        // unchanged), the adds on one thread with LDS reads issued eight at
        // a time (the residual's early terms leave the sum's binade almost
        // every time, which makes a parallel exact scan slower here).  The
        // id-ordered lists are no longer read: s_t holds the terms, s_d the
        // running sums of the draw.
        float* s_w = reinterpret_cast<float*>(s_t);
        float* s_c = reinterpret_cast<float*>(s_d);
        constexpr uint32_t RB = 8;
        auto seq_sum = [&](bool keep) -> float {  // thread 0; running sums to s_c if keep
            float sum = 0.0f;
            for (uint32_t k0 = 0; k0 < nt; k0 += RB) {
                float v[RB];
#pragma unroll
                for (uint32_t q = 0; q < RB; ++q) v[q] = k0 + q < nt ? s_w[k0 + q] : 0.0f;
#pragma unroll
                for (uint32_t q = 0; q < RB; ++q) {
                    sum = __fadd_rn(sum, v[q]);
                    if (keep && k0 + q < nt) s_c[k0 + q] = sum;
                }
            }
            return sum;
        };
        for (uint32_t k = tid; k < nt; k += NT_MTP) {
            const float v = s_v[k];
            s_w[k] = (v > 0.0f && isfinite(v)) ? v : 0.0f;
        }
        __syncthreads();
        if (tid == 0) s_rsum = seq_sum(false);
        __syncthreads();
        const float rsum = s_rsum;
        if (rsum > 0.0f && isfinite(rsum)) {  // some term is > 0
            // normalised residual, then sample_from_token_distribution
            for (uint32_t k = tid; k < nt; k += NT_MTP) {
                const float w = s_w[k];
                s_v[k] = w > 0.0f ? __fdiv_rn(w, rsum) : -1.0f;
            }
        } else {
            // empty residual: the target itself, in its kept order (sampling.rs:749)
            for (uint32_t k = tid; k < nt; k += NT_MTP) {
                s_v[k] = __fdiv_rn(tp_l[k], rt.F);
                s_id[k] = tid_l[k];
            }
        }
        __syncthreads();
        for (uint32_t k = tid; k < nt; k += NT_MTP) {
            const float q = s_v[k];
            s_w[k] = q < 0.0f ? 0.0f : q;
        }
        if (tid == 0) {
            s_cr = NONE;
            s_mx = 0ull;
        }
        __syncthreads();
        if (tid == 0) s_total = seq_sum(true);
        __syncthreads();
        // the draw: the first listed entry whose running sum reaches u *
        // total; else the last of the largest entries
        const float thr = __fmul_rn(ut, s_total);
        for (uint32_t k = tid; k < nt; k += NT_MTP) {
            const float q = s_v[k];
            if (q < 0.0f) continue;
            if (s_c[k] >= thr) atomicMin(&s_cr, k);
            atomicMax(&s_mx, ((uint64_t)__float_as_uint(q) << 32) | (k + 1u));
        }
        __syncthreads();
        if (tid == 0) {
            const uint32_t cr = s_cr;
            const uint64_t mx = s_mx;
            s_corr = cr != NONE ? s_id[cr] : (mx ? s_id[(uint32_t)mx - 1u] : NONE);
        }
        __syncthreads();
        corr = s_corr;
        flags |= AXS_MTP_FLAG_RESIDUAL;
        break;
    }
    if (tid != 0) return;
    uint32_t acc = count;
    if (!(flags & AXS_MTP_FLAG_ERROR)) {
        uint32_t tail = corr;
        if (!stopped || tail_row >= 0) {
            // all drafts accepted: the bonus draw of target row D; or the
            // target row at the rejected position
            const int j = stopped ? tail_row : D;
            const RowState rb = a.rstate[b * (D + 1) + j];
            if (rb.flags & AXS_FLAG_ERROR) flags |= AXS_MTP_FLAG_ERROR;
            if (rb.flags & NEAR_ALL) flags |= AXS_MTP_FLAG_NEAR;
            tail = a.out_ids[b * (D + 1) + j];
            flags |= stopped ? AXS_MTP_FLAG_TAIL_ROW : AXS_MTP_FLAG_BONUS;
        }
        out_ids[(size_t)b * (D + 1) + count] = tail;
        ++count;
    }
    if (flags & AXS_MTP_FLAG_ERROR) {
        count = 0;
        acc = 0;
    }
    out_count[b] = count;
    if (out_accept) out_accept[b] = acc;
    if (out_flags) out_flags[b] = flags;
}

// --------------------------------------------------------------------------
// k_mtp_prod: the production target law's p(d) of each draft token
// (axs_mtp_verify_ex with AXS_MTP_TARGET_FILTERED), one workgroup per target
// row r = b * d1 + i of the verify batch, run right after the index-order
// exact pass over those rows has left each row's softmax terms (dense) and
// their index-order sum (S[V - 1]) in the workspace.
// --------------------------------------------------------------------------
struct ProdArgs {
    const uint32_t* tokens;            // [rows] the draft token of each target row
    const axs_sampling_params* params; // [batch] the target's params
    float* out;                        // [batch, d1 - 1]
    uint32_t topk;                     // mtp_target_softmax_topk (0: none)
    int32_t d1;                        // depth + 1
};

__global__ __launch_bounds__(NT_EX) void k_mtp_prod(KArgs a, ProdArgs pa) {
    __shared__ ExLds XL;
    uint32_t* s_cnt = XL.cnt;
    uint32_t* s_u = XL.u;
    uint32_t &s_k = XL.k, &s_cross = XL.cross;
    const int tid = threadIdx.x;
    const int r = blockIdx.x;
    const uint32_t V = (uint32_t)a.vocab;
    const float* dense = a.dense + (size_t)r * V;
    const float* S = a.sbuf + (size_t)r * V;
    // a row the pass decided without the exact path (T <= 0, an id past the
    // vocabulary, no finite maximum) left S[V - 1] at the 0 it was given
    // before the pass, and its slot keeps 0
    // Production target law of a draft token (compute_mtp_target_probs,
    // runner/mod.rs:12025-12159, then extract_cpu_into, :11836-11937, and
    // filtered_target_token_probability, :11943-12001) over this row's
    // softmax p_j = q_j / S (full_vocab_token_logprob's terms and
    // index-order sum).  The filtered laws keep the K largest p
    // ((p desc, id asc)), those >= min_p * max p, cut where the f32
    // running sum in that order first reaches top_p, and divide p_t by the
    // kept sum in that order.  Only values enter the sums, so the sorted
    // values are walked in chunks of PROD_CAP: each chunk's values found
    // by a radix select of its last position's value (4 passes of 8 bits
    // over the row), gathered into LDS, sorted and summed by the exact
    // block scan from the previous chunk's sum, until the running sum
    // reaches top_p or the kept prefix ends; t's place in the order is
    // counted over the row.
    constexpr uint32_t PROD_CAP = 4096;
    const uint32_t d1 = (uint32_t)pa.d1, bq = (uint32_t)r / d1, iq = (uint32_t)r % d1;
    if (iq + 1u >= d1) return;  // the bonus row has no draft position
    const axs_sampling_params pp = pa.params[bq];
    const uint32_t t = pa.tokens[r];
    const float Z = S[V - 1];
    float* slot = pa.out + (size_t)bq * (d1 - 1u) + iq;
    if (!(Z > 0.0f) || !isfinite(Z) || t >= V) {
        if (tid == 0) *slot = 0.0f;
        return;
    }
    auto pv = [&](uint32_t j) { return __fdiv_rn(dense[j], Z); };
    const bool mp_on = pp.has_min_p && isfinite(pp.min_p) && pp.min_p > 0.0f;
    if (pa.topk == 0 && pp.top_k == 0 && !(pp.top_p < 1.0f) && !mp_on) {
        if (tid == 0) *slot = pv(t);  // the softmax value itself
        return;
    }
    uint32_t K = V;
    float tp = pp.top_p;
    if (pa.topk > 0) K = pa.topk < V ? pa.topk : V;
    else if (pp.top_k > 0 || pp.top_p < 1.0f) K = (pp.top_k > 0 && pp.top_k < V) ? pp.top_k : V;
    else tp = 1.0f;
    const bool cut = isfinite(tp) && tp > 0.0f && tp < 1.0f;
    const float ptok = pv(t);
    float lmax = 0.0f;
    for (uint32_t j = tid; j < V; j += NT_EX) lmax = fmaxf(lmax, pv(j));
    const float pmax = block_max<NT_EX>(lmax, reinterpret_cast<float*>(s_u));
    const float cutoff = mp_on ? __fmul_rn(pp.min_p, pmax) : 0.0f;
    uint32_t cm = 0, cgt = 0, ceq = 0;
    for (uint32_t j = tid; j < V; j += NT_EX) {
        const float q = pv(j);
        cm += (q > 0.0f && q >= cutoff) ? 1u : 0u;
        cgt += q > ptok ? 1u : 0u;
        ceq += (q == ptok && j < t) ? 1u : 0u;
    }
    const uint32_t n_m = block_sum_u32<NT_EX>(cm, s_u);
    const uint32_t rank_t = block_sum_u32<NT_EX>(cgt, s_u) + block_sum_u32<NT_EX>(ceq, s_u);
    const uint32_t Kp = n_m < K ? n_m : K;
    if (Kp == 0) {
        if (tid == 0) *slot = 0.0f;
        return;
    }
    // The sorted values in chunks of up to PROD_CAP: the chunk ending at
    // sorted position `end` is everything above the end-th largest bit
    // pattern th (p >= 0: bits order as values) plus `want` copies of it,
    // minus what the previous chunks took (above th0, plus want0 copies
    // of th0).
    uint32_t* hist = s_cnt;
    uint64_t* vk = reinterpret_cast<uint64_t*>(s_cnt + 512);           // PROD_CAP sort keys
    float* Ss = reinterpret_cast<float*>(s_cnt + 512 + 2 * PROD_CAP);  // running sums
    auto select = [&](uint32_t rank, uint32_t& th, uint32_t& want) {
        uint32_t prefix = 0, mask = 0;
        want = rank;
        for (int shift = 24; shift >= 0; shift -= 8) {
            for (uint32_t j = tid; j < 256u; j += NT_EX) hist[j] = 0;
            __syncthreads();
            for (uint32_t j = tid; j < V; j += NT_EX) {
                const uint32_t bb = __float_as_uint(pv(j));
                if ((bb & mask) == prefix && bb != 0u) atomicAdd(&hist[(bb >> shift) & 255u], 1u);
            }
            __syncthreads();
            if (tid == 0) {
                uint32_t cum = 0, dg = 0;
                for (int q = 255; q >= 0; --q) {
                    if (cum + hist[q] >= want) {
                        dg = (uint32_t)q;
                        break;
                    }
                    cum += hist[q];
                }
                s_k = dg;
                s_cross = want - cum;
            }
            __syncthreads();
            prefix |= s_k << shift;
            mask |= 255u << shift;
            want = s_cross;
            __syncthreads();
        }
        th = prefix;
    };
    uint32_t pos = 0, th0 = 0xFFFFFFFFu, want0 = 0, keep = Kp;
    float run = 0.0f, fsum = 0.0f;
    bool found = false;
    while (pos < Kp) {
        const uint32_t end = (Kp - pos > PROD_CAP) ? pos + PROD_CAP : Kp;
        const uint32_t nch = end - pos;
        uint32_t th, want;
        select(end, th, want);
        // copies of th0 left after the previous chunks
        if (tid == 0) s_k = 0;
        __syncthreads();
        uint32_t ce = 0;
        for (uint32_t j = tid; j < V; j += NT_EX) ce += __float_as_uint(pv(j)) == th0 ? 1u : 0u;
        const uint32_t n_th0 = block_sum_u32<NT_EX>(ce, s_u);
        // strictly between th and th0
        for (uint32_t j = tid; j < V; j += NT_EX) {
            const uint32_t bb = __float_as_uint(pv(j));
            if (bb > th && bb < th0) vk[atomicAdd(&s_k, 1u)] = (uint64_t)bb << 32;
        }
        __syncthreads();
        uint32_t ng = s_k;
        const uint32_t c_hi = th < th0 ? (pos > 0 ? n_th0 - want0 : 0u) : 0u;  // th0's remaining copies
        const uint32_t c_lo = th < th0 ? want : want - want0;                  // copies of th in this chunk
        const uint32_t np2 = next_pow2(nch);
        for (uint32_t j = ng + (uint32_t)tid; j < np2; j += NT_EX) {
            uint64_t kv = 0ull;
            if (j < ng + c_hi) kv = (uint64_t)th0 << 32;
            else if (j < ng + c_hi + c_lo) kv = (uint64_t)th << 32;
            vk[j] = kv;
        }
        __threadfence_block();
        __syncthreads();
        block_sort_desc<NT_EX>(vk, np2);
        block_exact_sums<8>([&](uint32_t k) { return __uint_as_float((uint32_t)(vk[k] >> 32)); }, 0u, nch,
                             run, Ss, XL.sum);
        __threadfence_block();
        __syncthreads();
        if (cut) {
            // the first running sum reaching top_p
            if (tid == 0) s_k = NONE;
            __syncthreads();
            uint32_t first = NONE;
            for (uint32_t k = tid; k < nch; k += NT_EX)
                if (Ss[k] >= tp) first = min(first, k);
            if (first != NONE) atomicMin(&s_k, first);
            __syncthreads();
            const uint32_t fk = s_k;
            __syncthreads();
            if (fk != NONE) {
                keep = pos + fk + 1u;
                fsum = Ss[fk];
                found = true;
                break;
            }
        }
        run = Ss[nch - 1u];
        th0 = th;
        want0 = want;  // copies of th among the first `end` positions
        pos = end;
    }
    if (!found) fsum = run;  // every kept value summed
    if (tid == 0)
        *slot = (ptok > 0.0f && rank_t < keep) ? fmaxf(__fdiv_rn(ptok, fmaxf(fsum, 1e-37f)), 0.0f) : 0.0f;
    return;
}

// --------------------------------------------------------------------------
// k_probe: think_soft_close_in_top_k per row
// (crates/ax-engine-mlx/src/ngram_accel.rs:1609-1640)
// --------------------------------------------------------------------------
constexpr int NT_PROBE = 1024;
constexpr uint32_t PROBE_RANK_CAP = 1024;  // ranks the exact replay holds
// The reference keeps a running top set over the raw logits: the first
// `rank` taken as they come and sorted by total order, afterwards a logit
// replaces the last entry only when it is greater (IEEE).  Without NaN, and
// without both signed zeros, that set is the top `rank` by (logit desc, id
// asc): the target is in it iff fewer than `rank` logits beat it (larger, or
// equal at a lower id) — one pass and a count.  A row with a NaN, or with
// both -0 and +0, is replayed literally on one thread (NaNs and signed zeros
// sort by total order but compare by IEEE).  out: 1 hit, 0 miss, NONE when a
// replay would need more than PROBE_RANK_CAP entries.
template <int DT>
__global__ __launch_bounds__(NT_PROBE) void k_probe(KArgs a, const uint32_t* think_ids, const uint32_t* ranks,
                                                      uint32_t* out_hit) {
    __shared__ uint32_t s_beats, s_flags;
    __shared__ uint32_t s_idx[PROBE_RANK_CAP];
    __shared__ float s_val[PROBE_RANK_CAP];
    const int r = blockIdx.x;
    const int tid = threadIdx.x;
    const uint32_t V = (uint32_t)a.vocab;
    const uint32_t t = think_ids[r], rank = ranks[r];
    if (rank == 0u || t >= V) {
        if (tid == 0) out_hit[r] = 0u;
        return;
    }
    const char* rp = row_ptr(a, r);
    auto at = [&](uint32_t i) -> float {
        if (DT == AXS_DTYPE_BF16) return __uint_as_float((uint32_t)((const uint16_t*)rp)[i] << 16);
        return ((const float*)rp)[i];
    };
    if (tid == 0) {
        s_beats = 0;
        s_flags = 0;
    }
    __syncthreads();
    const float vt = at(t);
    uint32_t beats = 0, fl = 0;
    constexpr uint32_t U = 8;  // loads in flight per thread
    for (uint32_t i0 = (uint32_t)tid; i0 < V; i0 += NT_PROBE * U) {
        float v[U];
#pragma unroll
        for (uint32_t u = 0; u < U; ++u) v[u] = i0 + u * NT_PROBE < V ? at(i0 + u * NT_PROBE) : -INFINITY;
#pragma unroll
        for (uint32_t u = 0; u < U; ++u) {
            const uint32_t i = i0 + u * NT_PROBE;
            if (i >= V) continue;
            beats += (v[u] > vt || (v[u] == vt && i < t)) ? 1u : 0u;
            if (isnan(v[u])) fl |= 1u;
            if (v[u] == 0.0f) fl |= signbit(v[u]) ? 2u : 4u;
        }
    }
    beats += __shfl_xor(beats, 32, 64);
    beats += __shfl_xor(beats, 16, 64);
    beats += __shfl_xor(beats, 8, 64);
    beats += __shfl_xor(beats, 4, 64);
    beats += __shfl_xor(beats, 2, 64);
    beats += __shfl_xor(beats, 1, 64);
    if ((tid & 63) == 0) atomicAdd(&s_beats, beats);
    if (fl) atomicOr(&s_flags, fl);
    __syncthreads();
    if (tid != 0) return;
    const uint32_t f = s_flags;
    if (!((f & 1u) || (f & 6u) == 6u)) {
        out_hit[r] = s_beats < rank ? 1u : 0u;
        return;
    }
    if (rank >= V) {  // every logit is in the set
        out_hit[r] = 1u;
        return;
    }
    if (rank > PROBE_RANK_CAP) {
        out_hit[r] = NONE;
        return;
    }
    // the reference's loop, literally
    auto tkey = [](float x) -> int32_t {
        int32_t k = __float_as_int(x);
        return k ^ (int32_t)(((uint32_t)(k >> 31)) >> 1);
    };
    uint32_t len = 0;
    for (uint32_t i = 0; i < V; ++i) {
        const float v = at(i);
        if (len < rank) {
            s_idx[len] = i;
            s_val[len] = v;
            ++len;
            if (len == rank)
                for (uint32_t q = 1; q < len; ++q) {  // stable, descending total order
                    const uint32_t ti = s_idx[q];
                    const float tv = s_val[q];
                    uint32_t b = q;
                    while (b > 0 && tkey(tv) > tkey(s_val[b - 1])) {
                        s_idx[b] = s_idx[b - 1];
                        s_val[b] = s_val[b - 1];
                        --b;
                    }
                    s_idx[b] = ti;
                    s_val[b] = tv;
                }
            continue;
        }
        if (v > s_val[rank - 1]) {
            uint32_t b = rank - 1;
            while (b > 0 && tkey(v) > tkey(s_val[b - 1])) {
                s_idx[b] = s_idx[b - 1];
                s_val[b] = s_val[b - 1];
                --b;
            }
            s_idx[b] = i;
            s_val[b] = v;
        }
    }
    uint32_t hit = 0;
    for (uint32_t q = 0; q < len; ++q) hit |= s_idx[q] == t ? 1u : 0u;
    out_hit[r] = hit;
}

}  // namespace axs

// ==========================================================================
// host side: context, validation, launches, C ABI
// ==========================================================================
using namespace axs;

namespace {

thread_local std::string g_last_error;
std::mutex g_handler_mu;
axs_error_handler_func g_handler = nullptr;
void* g_handler_data = nullptr;

// Records the message of a failed call for this thread and passes it to the
// registered error handler, on this thread.
int fail(int code, const std::string& msg) {
    g_last_error = msg;
    axs_error_handler_func h;
    void* hd;
    {
        std::lock_guard<std::mutex> lk(g_handler_mu);
        h = g_handler;
        hd = g_handler_data;
    }
    if (h) h(g_last_error.c_str(), hd);
    return code;
}

#define AXS_HIP_CHECK(expr)                                                        \
    do {                                                                           \
        hipError_t e_ = (expr);                                                    \
        if (e_ != hipSuccess)                                                      \
            return fail(AXS_E_HIP, std::string(#expr) + ": " + hipGetErrorString(e_)); \
    } while (0)

}  // namespace

struct axs_context {
    int device;
    int max_rows;
    int max_vocab;
    int max_chunks;
    int64_t tmp_stride;
    ChunkStat* cstat;
    Cand* pool;             // published candidates [rows, segments, CAPS]
    RowState* rstate;
    uint32_t* exact_rows;
    uint32_t* exact_count;
    uint32_t* row_done;     // per-row segment counters (atomicInc, wrap to 0)
    uint32_t* ex_done;      // k_exact_row workgroup counter (atomicInc, wrap to 0)
    float* dense;
    uint64_t* ckey;
    uint64_t* ckey2;
    uint64_t* tmp64;
    float* sbuf;
    uint32_t* bend;
    uint32_t* kept_id;
    float* kept_p;
    uint32_t* mtp_tok;  // per-row tokens of the MTP sampler pass
    uint32_t* mtp_amax; // per-row first argmax of the MTP sampler pass
    float* mtp_lnq;     // full-softmax draft log-probs [rows]
    uint32_t* lp_tok;   // token echo of the draft log-prob pass [rows]
    float* lp_temps;    // draft temperatures per draft row [rows]
    axs_sampling_params* draft_par;  // axs_mtp_draft: the draft law's params [rows]
    float* mtp_ptgt;    // production-law target probabilities of the draft tokens [rows]
    bool timing;
    std::vector<std::pair<hipEvent_t, hipEvent_t>> ev[AXS_KERNEL_COUNT];
    // Calls are serialised: the lock covers each call's enqueue, and a call
    // on another stream than the previous one first waits for the previous
    // stream's work (done_ev recorded there), so two streams never run on
    // the workspace at once.
    std::mutex mu;
    hipEvent_t done_ev;
    hipStream_t last_stream;
    bool has_last;
    // axs_sample_batch_host: the context's own stream and device staging
    // for host inputs and outputs, grown on demand
    hipStream_t own_stream;
    void* stage[16];
    size_t stage_cap[16];
};

namespace {

constexpr uint32_t MIN_CHUNK = 2048;  // smallest segment (bf16 x1, f32 x2)

struct DevGuard {
    int prev = -1;
    explicit DevGuard(int d) {
        if (hipGetDevice(&prev) != hipSuccess) prev = -1;
        if (prev != d) (void)hipSetDevice(d);
    }
    ~DevGuard() {
        int cur = -1;
        if (prev >= 0 && hipGetDevice(&cur) == hipSuccess && cur != prev) (void)hipSetDevice(prev);
    }
};

template <typename T>
int dalloc(T** p, size_t n) {
    void* q = nullptr;
    hipError_t e = hipMalloc(&q, n * sizeof(T) + 256);
    if (e != hipSuccess) return fail(AXS_E_HIP, std::string("hipMalloc: ") + hipGetErrorString(e));
    *p = (T*)q;
    return AXS_OK;
}

void clear_events(axs_context* c);

void free_ctx(axs_context* c) {
    clear_events(c);
    for (int i = 0; i < 16; ++i)
        if (c->stage[i]) (void)hipFree(c->stage[i]);
    if (c->done_ev) (void)hipEventDestroy(c->done_ev);
    if (c->own_stream) (void)hipStreamDestroy(c->own_stream);
    void* ptrs[] = {c->cstat, c->pool, c->rstate,  c->exact_rows, c->exact_count,
                    c->row_done, c->dense, c->ckey, c->ckey2, c->tmp64, c->sbuf, c->bend,
                    c->kept_id, c->kept_p, c->mtp_tok, c->mtp_amax, c->mtp_lnq, c->lp_tok, c->lp_temps,
                    c->draft_par, c->mtp_ptgt};
    for (void* q : ptrs)
        if (q) (void)hipFree(q);
    delete c;
}

// Launch geometry.  k_stream: segments of schunk ids (snch per row) streamed
// in tiles of 256*tv vectors; the exact path: segments of chunk ids (nch per
// row), nv vectors per thread, held in registers.
struct Plan {
    int nv;
    uint32_t chunk;
    int nch;
    int tv;
    bool wide;     // one 1024-thread workgroup per row
    bool inplace;  // ... which also takes the row's exact path
    uint32_t schunk;
    int snch;
    bool vec;
};

int env_int(const char* name, int dflt) {
    const char* e = getenv(name);
    int v = e ? atoi(e) : dflt;
    return v >= 1 ? v : dflt;
}

// Segment size: the largest per-thread vector count whose grid still has
// >= 1024 workgroups (four per CU), so each workgroup keeps up to 64 KB of
// loads in flight while the GPU stays full.
Plan make_plan(int dtype, int nrows, int vocab, const void* base, int64_t stride, const void* base2) {
    const int epv = dtype == AXS_DTYPE_BF16 ? 8 : 4;
    const int es = dtype == AXS_DTYPE_BF16 ? 2 : 4;
    static const int nvs_bf16[5] = {16, 8, 4, 2, 1};
    static const int nvs_f32[4] = {16, 8, 4, 2};
    const int* nvs = dtype == AXS_DTYPE_BF16 ? nvs_bf16 : nvs_f32;
    const int nn = dtype == AXS_DTYPE_BF16 ? 5 : 4;
    // AXS_SEG_NV_MAX caps the vectors per thread (tuning; default 8)
    static const int nv_cap = [] {
        const char* e = getenv("AXS_SEG_NV_MAX");
        int v = e ? atoi(e) : 8;
        return v >= 1 ? v : 8;
    }();
    Plan pl;
    pl.nv = nvs[nn - 1];
    for (int i = 0; i < nn; ++i) {
        if (nvs[i] > nv_cap && i + 1 < nn) continue;
        uint32_t ch = (uint32_t)(NT_CHUNK * nvs[i] * epv);
        int64_t nch = ((int64_t)vocab + ch - 1) / ch;
        if (nch > (int64_t)MAX_SEGS) break;  // keep the previous (larger) segment
        pl.nv = nvs[i];
        if ((int64_t)nrows * nch >= 1024) break;
    }
    pl.chunk = (uint32_t)(NT_CHUNK * pl.nv * epv);
    pl.nch = (int)((vocab + pl.chunk - 1) / pl.chunk);
    // k_stream: enough (row, segment) workgroups to fill the GPU
    // (AXS_STREAM_WGS, default 1024: four per CU), segments a multiple of
    // MIN_CHUNK ids and at most SEG_MAX
    static const int target = env_int("AXS_STREAM_WGS", 1024);
    // From 2 rows on, each row is one 1024-thread workgroup that decides it in
    // place (AXS_STREAM_WIDE_ROWS): with fewer rows than CUs, each row's CU
    // draws more than its 1/256 share of HBM bandwidth, and this beats the
    // segmented shape's cross-workgroup merge (min-p rows, 8 to 64 of them:
    // 2-4x).  A row that needs the exact second pass takes it in its own
    // workgroup from 64 rows on (AXS_INPLACE_ROWS: no further launch); below,
    // it is listed for k_exact_mat, which spreads the pass over the idle CUs
    // (one workgroup per row reading it again is slower: measured).
    static const int wide_rows = env_int("AXS_STREAM_WIDE_ROWS", 2);
    static const int inplace_rows = env_int("AXS_INPLACE_ROWS", 64);
    pl.tv = 4;
    pl.inplace = false;
    if (nrows >= wide_rows && (uint32_t)vocab <= ROW_MAX) {
        pl.wide = true;
        pl.inplace = nrows >= inplace_rows;
        pl.schunk = (uint32_t)vocab;
        pl.snch = 1;
        pl.vec = ((uintptr_t)base % 16 == 0) && ((stride * es) % 16 == 0) &&
                 (base2 == nullptr || (uintptr_t)base2 % 16 == 0);
        return pl;
    }
    pl.wide = false;
    int64_t s0 = ((int64_t)target + nrows - 1) / nrows;
    if (s0 < 1) s0 = 1;
    int64_t seg = ((int64_t)vocab + s0 - 1) / s0;
    seg = (seg + MIN_CHUNK - 1) / MIN_CHUNK * MIN_CHUNK;
    if (seg > (int64_t)SEG_MAX) seg = SEG_MAX;
    pl.schunk = (uint32_t)seg;
    pl.snch = (int)(((int64_t)vocab + seg - 1) / seg);
    pl.vec = ((uintptr_t)base % 16 == 0) && ((stride * es) % 16 == 0) &&
             (base2 == nullptr || (uintptr_t)base2 % 16 == 0);
    return pl;
}

template <int DT, int NV>
void launch_exact_nv(const KArgs& a, hipStream_t s) {
    const int64_t total = (int64_t)a.nrows * a.nch;
    int64_t g = total < 1024 ? total : 1024;
    dim3 grid((unsigned)(g > 0 ? g : 1));
    hipLaunchKernelGGL((k_exact_mat<DT, NV>), grid, dim3(NT_CHUNK), 0, s, a);
}

void launch_exact_mat(const Plan& pl, const KArgs& a, hipStream_t s) {
    if (a.dtype == AXS_DTYPE_BF16) {
        switch (pl.nv) {
            case 16: launch_exact_nv<AXS_DTYPE_BF16, 16>(a, s); break;
            case 8: launch_exact_nv<AXS_DTYPE_BF16, 8>(a, s); break;
            case 4: launch_exact_nv<AXS_DTYPE_BF16, 4>(a, s); break;
            case 2: launch_exact_nv<AXS_DTYPE_BF16, 2>(a, s); break;
            default: launch_exact_nv<AXS_DTYPE_BF16, 1>(a, s); break;
        }
    } else {
        switch (pl.nv) {
            case 16: launch_exact_nv<AXS_DTYPE_F32, 16>(a, s); break;
            case 8: launch_exact_nv<AXS_DTYPE_F32, 8>(a, s); break;
            case 4: launch_exact_nv<AXS_DTYPE_F32, 4>(a, s); break;
            default: launch_exact_nv<AXS_DTYPE_F32, 2>(a, s); break;
        }
    }
}

template <int DT, int NT, uint32_t SEGMAX, bool FAST>
void launch_stream_tv(const KArgs& a, hipStream_t s) {
    const int64_t total = (int64_t)a.nrows * a.snch;
    dim3 grid((unsigned)(((total + 7) / 8) * 8));
    if (a.mask) hipLaunchKernelGGL((k_stream<DT, 4, true, NT, SEGMAX, FAST>), grid, dim3(NT), 0, s, a);
    else hipLaunchKernelGGL((k_stream<DT, 4, false, NT, SEGMAX, FAST>), grid, dim3(NT), 0, s, a);
}

// one row per 1024-thread workgroup, 4 vectors per lane in each chunk (8:
// +4 us at C3, 2: +0.5 us, measured)
template <int DT, bool FAST>
void launch_row(const KArgs& a, hipStream_t s) {
    constexpr int TV = 4;
    dim3 grid((unsigned)(((a.nrows + 7) / 8) * 8));
    if (a.mask) hipLaunchKernelGGL((k_row<DT, TV, true, FAST>), grid, dim3(RT), 0, s, a);
    else hipLaunchKernelGGL((k_row<DT, TV, false, FAST>), grid, dim3(RT), 0, s, a);
}

// fast: 16-byte aligned rows of whole vectors (every segment end, a multiple
// of MIN_CHUNK or the vocabulary, is then a multiple of the vector width)
template <int DT>
void launch_stream_dt(const Plan& pl, const KArgs& a, hipStream_t s) {
    static_assert(RT == NT_EX, "k_row takes the exact path in place with its own workgroup");
    const bool fast = a.vec && a.vocab % (DT == AXS_DTYPE_BF16 ? 8 : 4) == 0;
    if (pl.wide) {
        if (fast) launch_row<DT, true>(a, s);
        else launch_row<DT, false>(a, s);
    } else {
        if (fast) launch_stream_tv<DT, NT_CHUNK, SEG_MAX, true>(a, s);
        else launch_stream_tv<DT, NT_CHUNK, SEG_MAX, false>(a, s);
    }
}

void launch_stream(const Plan& pl, const KArgs& a, hipStream_t s) {
    if (a.dtype == AXS_DTYPE_BF16) launch_stream_dt<AXS_DTYPE_BF16>(pl, a, s);
    else launch_stream_dt<AXS_DTYPE_F32>(pl, a, s);
}

// geometry fields of KArgs from the plan
int apply_plan(KArgs& a, const Plan& pl) {
    if (pl.nch > (int)MAX_SEGS || pl.snch > (int)MAX_SEGS)
        return fail(AXS_E_UNSUPPORTED, "vocab too large (more than 1024 segments)");
    a.nch = pl.nch;
    a.chunk = (int32_t)pl.chunk;
    a.snch = pl.snch;
    a.schunk = (int32_t)pl.schunk;
    a.vec = pl.vec ? 1 : 0;
    a.inplace = pl.inplace ? 1 : 0;
    return AXS_OK;
}

void clear_events(axs_context* c) {
    for (auto& v : c->ev) {
        for (auto& e : v) {
            (void)hipEventDestroy(e.first);
            (void)hipEventDestroy(e.second);
        }
        v.clear();
    }
}

// Brackets one launch with events on its stream when timing is enabled.
template <typename F>
void timed(axs_context* c, int kind, hipStream_t s, F&& launch) {
    if (!c->timing) {
        launch();
        return;
    }
    hipEvent_t a = nullptr, b = nullptr;
    (void)hipEventCreate(&a);
    (void)hipEventCreate(&b);
    (void)hipEventRecord(a, s);
    launch();
    (void)hipEventRecord(b, s);
    c->ev[kind].push_back({a, b});
}

void fill_ws(KArgs& a, axs_context* c) {
    a.cstat = c->cstat;
    a.pool = c->pool;
    a.rstate = c->rstate;
    a.exact_rows = c->exact_rows;
    a.exact_count = c->exact_count;
    a.row_done = c->row_done;
    a.ex_done = c->ex_done;
    a.dense = c->dense;
    a.ckey = c->ckey;
    a.ckey2 = c->ckey2;
    a.tmp64 = c->tmp64;
    a.sbuf = c->sbuf;
    a.bend = c->bend;
    a.tmp_stride = c->tmp_stride;
}

// the three-kernel pipeline over a.nrows rows
int run_pipeline(axs_context* c, KArgs& a, const Plan& pl, hipStream_t s) {
    int rc = apply_plan(a, pl);
    if (rc) return rc;
    fill_ws(a, c);
    timed(c, AXS_KERNEL_STREAM, s, [&] { launch_stream(pl, a, s); });
    if (pl.wide && pl.inplace) {  // k_row takes the exact path in place
        AXS_HIP_CHECK(hipGetLastError());
        return AXS_OK;
    }
    timed(c, AXS_KERNEL_EXACT_MAT, s, [&] { launch_exact_mat(pl, a, s); });
    timed(c, AXS_KERNEL_EXACT_ROW, s, [&] {
        hipLaunchKernelGGL(k_exact_row, dim3((unsigned)a.nrows), dim3(NT_EX), 0, s, a);
    });
    AXS_HIP_CHECK(hipGetLastError());
    return AXS_OK;
}

// A call's work on stream s follows the previous call's when that ran on
// another stream: an event recorded on the previous stream now (after its
// enqueued work) and waited for on s.  Consecutive calls on one stream cost
// nothing here.  A stream being captured into a graph is not recorded as the
// previous stream (its work runs at replay).
int order_begin(axs_context* c, hipStream_t s) {
    if (c->has_last && c->last_stream != s) {
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        AXS_HIP_CHECK(hipStreamIsCapturing(c->last_stream, &cs));
        if (cs == hipStreamCaptureStatusNone) {
            AXS_HIP_CHECK(hipEventRecord(c->done_ev, c->last_stream));
            AXS_HIP_CHECK(hipStreamWaitEvent(s, c->done_ev, 0));
        }
    }
    return AXS_OK;
}
int order_end(axs_context* c, hipStream_t s) {
    c->last_stream = s;
    c->has_last = true;
    return AXS_OK;
}

// Device staging slot i of at least n bytes (grown, never shrunk).
int stage_at(axs_context* c, int i, size_t n, void** out) {
    if (n == 0) n = 16;
    if (c->stage_cap[i] < n) {
        if (c->stage[i]) {
            AXS_HIP_CHECK(hipStreamSynchronize(c->own_stream));
            AXS_HIP_CHECK(hipFree(c->stage[i]));
            c->stage[i] = nullptr;
            c->stage_cap[i] = 0;
        }
        void* q = nullptr;
        hipError_t e = hipMalloc(&q, n + 256);
        if (e != hipSuccess) return fail(AXS_E_HIP, std::string("hipMalloc (staging): ") + hipGetErrorString(e));
        c->stage[i] = q;
        c->stage_cap[i] = n;
    }
    *out = c->stage[i];
    return AXS_OK;
}

// ---------------------------------------------------------------------------
// Scratch of axs_argmax_batch_noalloc: a file-scope device array instead of a
// context.  The one-row (segmented) argmax publishes per-segment results
// (ChunkStat), candidates (Cand) and an arrival counter there; batches of 2
// rows or more (k_row) use none of it.  NA_SEGS segments cover the one-row
// plan up to ROW_MAX ids (2,048-id segments).  Each GPU holds its own copy for
// the life of the process; calls that overlap on one GPU race on it.
// ---------------------------------------------------------------------------
constexpr uint32_t NA_SEGS = 128;
constexpr size_t NA_CSTAT_OFF = 0;
constexpr size_t NA_POOL_OFF = NA_CSTAT_OFF + (size_t)NA_SEGS * sizeof(ChunkStat);
constexpr size_t NA_DONE_OFF = NA_POOL_OFF + (size_t)NA_SEGS * CAPS * sizeof(Cand);
constexpr size_t NA_DONE_WORDS = 2;  // row_done[0] and the (unused) exact-path counter
constexpr size_t NA_SCRATCH_BYTES = NA_DONE_OFF + NA_DONE_WORDS * sizeof(uint32_t);
static_assert(NA_POOL_OFF % 16 == 0 && NA_DONE_OFF % 16 == 0, "scratch carve-up alignment");

static __device__ __align__(256) unsigned char scratch[NA_SCRATCH_BYTES];

constexpr int NA_MAX_DEVICES = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[NA_MAX_DEVICES];  // device address of `scratch` on each GPU

// Device address of this GPU's `scratch` (device must be current); looked up
// once per device.
int scratch_ptr(int device, void** out) {
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_ptr[device]) {
        void* ptr = nullptr;
        hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !ptr)
            return fail(AXS_E_HIP, std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e));
        g_scratch_ptr[device] = ptr;
    }
    *out = g_scratch_ptr[device];
    return AXS_OK;
}

__global__ void k_fill_u32(uint32_t* p, uint32_t n, uint32_t v) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = v;
}

uint32_t next_pow2_h(uint32_t n) {
    uint32_t p = 1;
    while (p < n) p <<= 1;
    return p;
}

}  // namespace

extern "C" {

int axs_abi_version(void) { return AXS_ABI_VERSION; }

const char* axs_last_error(void) { return g_last_error.c_str(); }

void axs_set_error_handler(axs_error_handler_func handler, void* data) {
    std::lock_guard<std::mutex> lk(g_handler_mu);
    g_handler = handler;
    g_handler_data = data;
}

int axs_context_create(int device, int max_batch, int max_vocab, axs_context** out) {
    if (!out) return fail(AXS_E_INVALID, "out is NULL");
    *out = nullptr;
    if (max_batch < 1 || max_vocab < 1) return fail(AXS_E_INVALID, "max_batch and max_vocab must be >= 1");
    int ndev = 0;
    if (hipGetDeviceCount(&ndev) != hipSuccess || device < 0 || device >= ndev)
        return fail(AXS_E_INVALID, "no such HIP device");
    DevGuard g(device);
    axs_context* c = new (std::nothrow) axs_context();
    if (!c) return fail(AXS_E_INVALID, "out of host memory");
    c->device = device;
    c->max_rows = max_batch;
    c->max_vocab = max_vocab;
    c->max_chunks = (int)((max_vocab + MIN_CHUNK - 1) / MIN_CHUNK);
    c->tmp_stride = next_pow2_h((uint32_t)max_vocab);
    size_t R = (size_t)max_batch, Vv = (size_t)max_vocab;
    int rc = AXS_OK;
    if ((rc = dalloc(&c->cstat, R * c->max_chunks)) ||
        (rc = dalloc(&c->pool, R * c->max_chunks * CAPS)) || (rc = dalloc(&c->rstate, R)) ||
        (rc = dalloc(&c->exact_rows, R)) || (rc = dalloc(&c->exact_count, 1)) ||
        (rc = dalloc(&c->row_done, R + 1)) ||
        (rc = dalloc(&c->dense, R * Vv)) || (rc = dalloc(&c->ckey, R * Vv)) ||
        (rc = dalloc(&c->ckey2, R * Vv)) || (rc = dalloc(&c->tmp64, R * (size_t)c->tmp_stride)) ||
        (rc = dalloc(&c->sbuf, R * Vv)) || (rc = dalloc(&c->bend, R * BEND_STRIDE)) ||
        (rc = dalloc(&c->kept_id, R * KEPT_CAP)) || (rc = dalloc(&c->kept_p, R * KEPT_CAP)) ||
        (rc = dalloc(&c->mtp_tok, R)) || (rc = dalloc(&c->mtp_amax, R)) || (rc = dalloc(&c->mtp_lnq, R)) ||
        (rc = dalloc(&c->lp_tok, R)) || (rc = dalloc(&c->lp_temps, R)) || (rc = dalloc(&c->draft_par, R)) ||
        (rc = dalloc(&c->mtp_ptgt, R))) {
        free_ctx(c);
        return rc;
    }
    c->ex_done = c->row_done + R;
    if (hipStreamCreateWithFlags(&c->own_stream, hipStreamNonBlocking) != hipSuccess ||
        hipEventCreateWithFlags(&c->done_ev, hipEventDisableTiming) != hipSuccess) {
        free_ctx(c);
        return fail(AXS_E_HIP, "creating the context's stream and event failed");
    }
    // the counters start at zero; every call leaves them at zero again
    if (hipMemset(c->row_done, 0, (R + 1) * sizeof(uint32_t)) != hipSuccess ||
        hipMemset(c->exact_count, 0, sizeof(uint32_t)) != hipSuccess ||
        hipMemset(c->bend, 0, R * BEND_STRIDE * sizeof(uint32_t)) != hipSuccess ||
        hipDeviceSynchronize() != hipSuccess) {
        free_ctx(c);
        return fail(AXS_E_HIP, "clearing the workspace counters failed");
    }
    *out = c;
    return AXS_OK;
}

int axs_context_destroy(axs_context* ctx) {
    if (!ctx) return fail(AXS_E_INVALID, "ctx is NULL");
    DevGuard g(ctx->device);
    (void)hipDeviceSynchronize();
    free_ctx(ctx);
    return AXS_OK;
}

}  // extern "C"

namespace {

// Validation shared by the device- and host-pointer sampling entry points.
int check_batch(axs_context* ctx, const axs_batch_desc* d, const axs_outputs* o) {
    if (!ctx || !d || !o) return fail(AXS_E_INVALID, "ctx, desc and outputs must be non-NULL");
    if (!d->logits || !d->params || !o->token_ids)
        return fail(AXS_E_INVALID, "logits, params and token_ids must be non-NULL");
    if (d->dtype != AXS_DTYPE_F32 && d->dtype != AXS_DTYPE_BF16) return fail(AXS_E_INVALID, "bad dtype");
    if (d->batch < 1 || d->vocab < 1) return fail(AXS_E_INVALID, "batch and vocab must be >= 1");
    if (d->row_stride < d->vocab) return fail(AXS_E_INVALID, "row_stride < vocab");
    if (d->batch > ctx->max_rows || d->vocab > ctx->max_vocab)
        return fail(AXS_E_CAPACITY, "batch or vocab larger than the context");
    if (d->history && (!d->history_offsets || d->history_len < 0))
        return fail(AXS_E_INVALID, "history needs history_offsets and history_len");
    if (d->mask_words && d->mask_stride < (d->vocab + 31) / 32)
        return fail(AXS_E_INVALID, "mask_stride < ceil(vocab / 32)");
    if (d->bias_ids && (!d->bias_values || !d->bias_offsets || d->bias_len < 0))
        return fail(AXS_E_INVALID, "bias_ids needs bias_values, bias_offsets and bias_len");
    if (o->kept_ids && o->kept_cap < 1) return fail(AXS_E_INVALID, "kept_ids needs kept_cap >= 1");
    return AXS_OK;
}

int sample_batch_locked(axs_context* ctx, const axs_batch_desc* d, const axs_outputs* o, hipStream_t s);

}  // namespace

extern "C" {

int axs_sample_batch(axs_context* ctx, const axs_batch_desc* d, const axs_outputs* o, void* stream) {
    int rc = check_batch(ctx, d, o);
    if (rc) return rc;
    std::lock_guard<std::mutex> lk(ctx->mu);
    DevGuard g(ctx->device);
    hipStream_t s = (hipStream_t)stream;
    if ((rc = order_begin(ctx, s))) return rc;
    if ((rc = sample_batch_locked(ctx, d, o, s))) return rc;
    return order_end(ctx, s);
}

int axs_sample_batch_host(axs_context* ctx, const axs_batch_desc* hd, const axs_outputs* ho) {
    int rc = check_batch(ctx, hd, ho);
    if (rc) return rc;
    std::lock_guard<std::mutex> lk(ctx->mu);
    DevGuard g(ctx->device);
    hipStream_t s = ctx->own_stream;
    if ((rc = order_begin(ctx, s))) return rc;
    const int B = hd->batch, V = hd->vocab;
    const size_t es = hd->dtype == AXS_DTYPE_BF16 ? 2 : 4;
    axs_batch_desc d = *hd;
    axs_outputs o = *ho;
    void* p = nullptr;
    auto up = [&](int slot, const void* src, size_t n, void** dst) -> int {
        int r = stage_at(ctx, slot, n, dst);
        if (r) return r;
        if (n) AXS_HIP_CHECK(hipMemcpyAsync(*dst, src, n, hipMemcpyHostToDevice, s));
        return AXS_OK;
    };
    // logits, packed to row stride = vocab
    if ((rc = stage_at(ctx, 0, (size_t)B * V * es, &p))) return rc;
    AXS_HIP_CHECK(hipMemcpy2DAsync(p, (size_t)V * es, hd->logits, (size_t)hd->row_stride * es, (size_t)V * es,
                                   (size_t)B, hipMemcpyHostToDevice, s));
    d.logits = p;
    d.row_stride = V;
    if ((rc = up(1, hd->params, (size_t)B * sizeof(axs_sampling_params), &p))) return rc;
    d.params = (const axs_sampling_params*)p;
    if (hd->history) {
        if ((rc = up(2, hd->history, (size_t)hd->history_len * 4, &p))) return rc;
        d.history = (const uint32_t*)p;
        if ((rc = up(3, hd->history_offsets, (size_t)(B + 1) * 8, &p))) return rc;
        d.history_offsets = (const int64_t*)p;
    }
    if (hd->mask_words) {
        if ((rc = up(4, hd->mask_words, (size_t)B * hd->mask_stride * 4, &p))) return rc;
        d.mask_words = (const uint32_t*)p;
    }
    if (hd->bias_ids && B >= 2) {
        for (int r = 0; r < B; ++r)
            if (hd->bias_offsets[r + 1] - hd->bias_offsets[r] > (int64_t)RBCAP)
                return fail(AXS_E_CAPACITY, "a row has more than 1024 bias entries (AXS_BIAS_ROW_MAX)");
    }
    if (hd->bias_ids) {
        if ((rc = up(5, hd->bias_ids, (size_t)hd->bias_len * 4, &p))) return rc;
        d.bias_ids = (const uint32_t*)p;
        if ((rc = up(6, hd->bias_values, (size_t)hd->bias_len * 4, &p))) return rc;
        d.bias_values = (const float*)p;
        if ((rc = up(7, hd->bias_offsets, (size_t)(B + 1) * 8, &p))) return rc;
        d.bias_offsets = (const int64_t*)p;
    }
    if (hd->uniforms) {
        if ((rc = up(8, hd->uniforms, (size_t)B * 4, &p))) return rc;
        d.uniforms = (const float*)p;
    }
    // device outputs
    void *dt = nullptr, *dl = nullptr, *df = nullptr, *dk = nullptr, *dc = nullptr;
    if ((rc = stage_at(ctx, 9, (size_t)B * 4, &dt))) return rc;
    o.token_ids = (uint32_t*)dt;
    if (ho->logprobs) {
        if ((rc = stage_at(ctx, 10, (size_t)B * 4, &dl))) return rc;
        o.logprobs = (float*)dl;
    }
    if (ho->flags) {
        if ((rc = stage_at(ctx, 11, (size_t)B * 4, &df))) return rc;
        o.flags = (uint32_t*)df;
    }
    if (ho->kept_ids) {
        if ((rc = stage_at(ctx, 12, (size_t)B * ho->kept_cap * 4, &dk))) return rc;
        o.kept_ids = (uint32_t*)dk;
    }
    if (ho->kept_count) {
        if ((rc = stage_at(ctx, 13, (size_t)B * 4, &dc))) return rc;
        o.kept_count = (uint32_t*)dc;
    }
    if ((rc = sample_batch_locked(ctx, &d, &o, s))) return rc;
    AXS_HIP_CHECK(hipMemcpyAsync(ho->token_ids, dt, (size_t)B * 4, hipMemcpyDeviceToHost, s));
    if (ho->logprobs) AXS_HIP_CHECK(hipMemcpyAsync(ho->logprobs, dl, (size_t)B * 4, hipMemcpyDeviceToHost, s));
    if (ho->flags) AXS_HIP_CHECK(hipMemcpyAsync(ho->flags, df, (size_t)B * 4, hipMemcpyDeviceToHost, s));
    if (ho->kept_ids)
        AXS_HIP_CHECK(hipMemcpyAsync(ho->kept_ids, dk, (size_t)B * ho->kept_cap * 4, hipMemcpyDeviceToHost, s));
    if (ho->kept_count) AXS_HIP_CHECK(hipMemcpyAsync(ho->kept_count, dc, (size_t)B * 4, hipMemcpyDeviceToHost, s));
    if ((rc = order_end(ctx, s))) return rc;
    AXS_HIP_CHECK(hipStreamSynchronize(s));
    return AXS_OK;
}

}  // extern "C"

namespace {

int sample_batch_locked(axs_context* ctx, const axs_batch_desc* d, const axs_outputs* o, hipStream_t s) {
    KArgs a{};
    a.logits = d->logits;
    a.logits2 = nullptr;
    a.dtype = d->dtype;
    a.nrows = d->batch;
    a.vocab = d->vocab;
    a.mtp_depth = 0;
    a.mtp_batch = 0;
    a.want_logprob = o->logprobs != nullptr;
    a.exact_lp = 1;
    a.stride = d->row_stride;
    a.params = d->params;
    a.params2 = nullptr;
    a.hist = d->history;
    a.hist_off = d->history ? d->history_offsets : nullptr;
    a.hist_len = d->history_len;
    a.mask = d->mask_words;
    a.mask_stride = d->mask_stride;
    a.bias_ids = d->bias_ids;
    a.bias_vals = d->bias_values;
    a.bias_off = d->bias_ids ? d->bias_offsets : nullptr;
    a.bias_len = d->bias_len;
    a.uniforms = d->uniforms;
    a.ws_kept_id = nullptr;
    a.ws_kept_p = nullptr;
    a.out_ids = o->token_ids;
    a.out_lp = o->logprobs;
    a.out_flags = o->flags;
    a.out_kept = o->kept_ids;
    a.out_kept_count = o->kept_count;
    a.out_kept_cap = o->kept_ids ? o->kept_cap : 0;
    Plan pl = make_plan(d->dtype, d->batch, d->vocab, d->logits, d->row_stride, nullptr);
    return run_pipeline(ctx, a, pl, s);
}

}  // namespace

extern "C" {

int axs_argmax_batch(axs_context* ctx, const void* logits, int dtype, int batch, int vocab,
                     int64_t row_stride, uint32_t* out_ids, float* out_logprob, void* stream) {
    if (!ctx || !logits || !out_ids) return fail(AXS_E_INVALID, "ctx, logits and out_ids must be non-NULL");
    if (dtype != AXS_DTYPE_F32 && dtype != AXS_DTYPE_BF16) return fail(AXS_E_INVALID, "bad dtype");
    if (batch < 1 || vocab < 1 || row_stride < vocab) return fail(AXS_E_INVALID, "bad shape");
    if (batch > ctx->max_rows || vocab > ctx->max_vocab)
        return fail(AXS_E_CAPACITY, "batch or vocab larger than the context");
    std::lock_guard<std::mutex> lk(ctx->mu);
    DevGuard g(ctx->device);
    KArgs a{};
    a.logits = logits;
    a.dtype = dtype;
    a.nrows = batch;
    a.vocab = vocab;
    a.stride = row_stride;
    a.params = nullptr;
    a.want_logprob = out_logprob != nullptr;
    a.out_ids = out_ids;
    a.out_lp = out_logprob;
    Plan pl = make_plan(dtype, batch, vocab, logits, row_stride, nullptr);
    int rc = apply_plan(a, pl);
    if (rc) return rc;
    fill_ws(a, ctx);
    hipStream_t s = (hipStream_t)stream;
    if ((rc = order_begin(ctx, s))) return rc;
    timed(ctx, AXS_KERNEL_STREAM, s, [&] { launch_stream(pl, a, s); });
    AXS_HIP_CHECK(hipGetLastError());
    return order_end(ctx, s);
}

int axs_argmax_batch_noalloc(int device, const void* logits, int dtype, int batch, int vocab,
                             int64_t row_stride, uint32_t* out_ids, float* out_logprob, void* stream) {
    if (!logits || !out_ids) return fail(AXS_E_INVALID, "logits and out_ids must be non-NULL");
    if (dtype != AXS_DTYPE_F32 && dtype != AXS_DTYPE_BF16) return fail(AXS_E_INVALID, "bad dtype");
    if (batch < 1 || vocab < 1 || row_stride < vocab) return fail(AXS_E_INVALID, "bad shape");
    if ((uint32_t)vocab > ROW_MAX)
        return fail(AXS_E_CAPACITY, "axs_argmax_batch_noalloc: vocab above 262144 (its scratch limit)");
    int ndev = 0;
    if (hipGetDeviceCount(&ndev) != hipSuccess || device < 0 || device >= ndev || device >= NA_MAX_DEVICES)
        return fail(AXS_E_INVALID, "no such HIP device");
    DevGuard g(device);
    KArgs a{};
    a.logits = logits;
    a.dtype = dtype;
    a.nrows = batch;
    a.vocab = vocab;
    a.stride = row_stride;
    a.params = nullptr;
    a.want_logprob = out_logprob != nullptr;
    a.out_ids = out_ids;
    a.out_lp = out_logprob;
    Plan pl = make_plan(dtype, batch, vocab, logits, row_stride, nullptr);
    if (!pl.wide && (int64_t)batch * pl.snch > (int64_t)NA_SEGS)
        return fail(AXS_E_CAPACITY, "axs_argmax_batch_noalloc: more segments than its scratch holds (128)");
    int rc = apply_plan(a, pl);
    if (rc) return rc;
    void* base = nullptr;
    if ((rc = scratch_ptr(device, &base))) return rc;
    char* sp = (char*)base;
    a.cstat = (ChunkStat*)(sp + NA_CSTAT_OFF);
    a.pool = (Cand*)(sp + NA_POOL_OFF);
    a.row_done = (uint32_t*)(sp + NA_DONE_OFF);
    a.ex_done = a.row_done + 1;
    hipStream_t s = (hipStream_t)stream;
    // the arrival counters start at zero (a fill kernel, not a memset node,
    // so that the call can be captured in a graph)
    hipLaunchKernelGGL(k_fill_u32, dim3(1), dim3(64), 0, s, a.row_done, (uint32_t)NA_DONE_WORDS, 0u);
    launch_stream(pl, a, s);
    AXS_HIP_CHECK(hipGetLastError());
    return AXS_OK;
}

int axs_token_logprob_batch(axs_context* ctx, const void* logits, int dtype, int batch, int vocab,
                            int64_t row_stride, const uint32_t* tokens, const float* temperatures,
                            float* out_logprob, void* stream) {
    if (!ctx || !logits || !tokens || !temperatures || !out_logprob)
        return fail(AXS_E_INVALID, "ctx, logits, tokens, temperatures and out_logprob must be non-NULL");
    if (dtype != AXS_DTYPE_F32 && dtype != AXS_DTYPE_BF16) return fail(AXS_E_INVALID, "bad dtype");
    if (batch < 1 || vocab < 1 || row_stride < vocab) return fail(AXS_E_INVALID, "bad shape");
    if (batch > ctx->max_rows || vocab > ctx->max_vocab)
        return fail(AXS_E_CAPACITY, "batch or vocab larger than the context");
    std::lock_guard<std::mutex> lk(ctx->mu);
    DevGuard g(ctx->device);
    hipStream_t s = (hipStream_t)stream;
    int rc = order_begin(ctx, s);
    if (rc) return rc;
    KArgs a{};
    a.logits = logits;
    a.dtype = dtype;
    a.nrows = batch;
    a.vocab = vocab;
    a.stride = row_stride;
    a.params = nullptr;
    a.lp_tokens = tokens;
    a.lp_temps = temperatures;
    a.out_ids = ctx->mtp_tok;  // the rows' tokens echoed: scratch
    a.out_lp = out_logprob;
    Plan pl = make_plan(dtype, batch, vocab, logits, row_stride, nullptr);
    if ((rc = run_pipeline(ctx, a, pl, s))) return rc;
    return order_end(ctx, s);
}

int axs_top_logprobs(axs_context* ctx, const void* logits, int dtype, int batch, int vocab,
                     int64_t row_stride, const float* temperatures, int n, uint32_t* out_ids, float* out_logprob,
                     void* stream) {
    if (!ctx || !logits || !temperatures || !out_ids || !out_logprob)
        return fail(AXS_E_INVALID, "ctx, logits, temperatures, out_ids and out_logprob must be non-NULL");
    if (dtype != AXS_DTYPE_F32 && dtype != AXS_DTYPE_BF16) return fail(AXS_E_INVALID, "bad dtype");
    if (batch < 1 || vocab < 1 || row_stride < vocab) return fail(AXS_E_INVALID, "bad shape");
    if (n < 1 || n > AXS_TOP_LOGPROBS_MAX) return fail(AXS_E_INVALID, "n must be 1..AXS_TOP_LOGPROBS_MAX");
    if (batch > ctx->max_rows || vocab > ctx->max_vocab)
        return fail(AXS_E_CAPACITY, "batch or vocab larger than the context");
    std::lock_guard<std::mutex> lk(ctx->mu);
    DevGuard g(ctx->device);
    hipStream_t s = (hipStream_t)stream;
    int rc = order_begin(ctx, s);
    if (rc) return rc;
    // the rows' token list (unused by top-N rows): zeros
    hipLaunchKernelGGL(k_fill_u32, dim3((batch + 255) / 256), dim3(256), 0, s, ctx->lp_tok, (uint32_t)batch, 0u);
    AXS_HIP_CHECK(hipGetLastError());
    KArgs a{};
    a.logits = logits;
    a.dtype = dtype;
    a.nrows = batch;
    a.vocab = vocab;
    a.stride = row_stride;
    a.params = nullptr;
    a.lp_tokens = ctx->lp_tok;
    a.lp_temps = temperatures;
    a.topn = (uint32_t)n;
    a.topn_ids = out_ids;
    a.topn_lp = out_logprob;
    a.out_ids = ctx->mtp_tok;  // scratch
    Plan pl = make_plan(dtype, batch, vocab, logits, row_stride, nullptr);
    if ((rc = run_pipeline(ctx, a, pl, s))) return rc;
    return order_end(ctx, s);
}

int axs_soft_close_probe(axs_context* ctx, const void* logits, int dtype, int batch, int vocab,
                         int64_t row_stride, const uint32_t* think_ids, const uint32_t* ranks,
                         uint32_t* out_hit, void* stream) {
    if (!ctx || !logits || !think_ids || !ranks || !out_hit)
        return fail(AXS_E_INVALID, "ctx, logits, think_ids, ranks and out_hit must be non-NULL");
    if (dtype != AXS_DTYPE_F32 && dtype != AXS_DTYPE_BF16) return fail(AXS_E_INVALID, "bad dtype");
    if (batch < 1 || vocab < 1 || row_stride < vocab) return fail(AXS_E_INVALID, "bad shape");
    if (batch > ctx->max_rows || vocab > ctx->max_vocab)
        return fail(AXS_E_CAPACITY, "batch or vocab larger than the context");
    std::lock_guard<std::mutex> lk(ctx->mu);
    DevGuard g(ctx->device);
    hipStream_t s = (hipStream_t)stream;
    int rc = order_begin(ctx, s);
    if (rc) return rc;
    KArgs a{};
    a.logits = logits;
    a.dtype = dtype;
    a.nrows = batch;
    a.vocab = vocab;
    a.stride = row_stride;
    if (dtype == AXS_DTYPE_BF16)
        hipLaunchKernelGGL((k_probe<AXS_DTYPE_BF16>), dim3(batch), dim3(NT_PROBE), 0, s, a, think_ids, ranks, out_hit);
    else
        hipLaunchKernelGGL((k_probe<AXS_DTYPE_F32>), dim3(batch), dim3(NT_PROBE), 0, s, a, think_ids, ranks, out_hit);
    AXS_HIP_CHECK(hipGetLastError());
    return order_end(ctx, s);
}

int axs_lm_head(axs_context* ctx, const void* hidden, int64_t hidden_stride, const void* weight,
                int64_t weight_stride, int batch, int hidden_size, int vocab, float scale, float softcap,
                float* out_logits, int64_t out_stride, uint32_t* out_argmax, void* stream) {
    if (!ctx || !hidden || !weight) return fail(AXS_E_INVALID, "ctx, hidden and weight must be non-NULL");
    if (!out_logits && !out_argmax) return fail(AXS_E_INVALID, "out_logits and out_argmax are both NULL");
    if (batch < 1 || vocab < 1 || hidden_size < 32 || hidden_size % 32 != 0)
        return fail(AXS_E_INVALID, "bad shape (hidden_size must be a positive multiple of 32)");
    if (hidden_stride < hidden_size || weight_stride < hidden_size || hidden_stride % 8 || weight_stride % 8)
        return fail(AXS_E_INVALID, "hidden_stride and weight_stride must be >= hidden_size and multiples of 8");
    if (((uintptr_t)hidden | (uintptr_t)weight) & 15)
        return fail(AXS_E_INVALID, "hidden and weight must be 16-byte aligned");
    if (out_logits && out_stride < vocab) return fail(AXS_E_INVALID, "out_stride < vocab");
    if (!std::isfinite(scale) || std::isnan(softcap)) return fail(AXS_E_INVALID, "scale must be finite");
    if (batch > ctx->max_rows) return fail(AXS_E_CAPACITY, "batch larger than the context");
    std::lock_guard<std::mutex> lk(ctx->mu);
    DevGuard g(ctx->device);
    hipStream_t s = (hipStream_t)stream;
    int rc = order_begin(ctx, s);
    if (rc) return rc;
    axs_lmh::LmArgs a{};
    a.hidden = (const uint16_t*)hidden;
    a.hs = hidden_stride;
    a.w = (const uint16_t*)weight;
    a.ws = weight_stride;
    a.B = batch;
    a.H = hidden_size;
    a.V = vocab;
    a.scale = scale;
    a.cap = softcap > 0.0f ? softcap : 0.0f;
    a.inv_cap = softcap > 0.0f ? 1.0f / softcap : 0.0f;
    a.out = out_logits;
    a.os = out_stride;
    a.out_vec = (out_logits && ((uintptr_t)out_logits & 15) == 0 && out_stride % 4 == 0) ? 1 : 0;
    a.keys = out_argmax ? (unsigned long long*)ctx->tmp64 : nullptr;
    if (a.keys) {
        hipLaunchKernelGGL(k_fill_u32, dim3((2 * batch + 255) / 256), dim3(256), 0, s, (uint32_t*)a.keys,
                           (uint32_t)(2 * batch), 0u);
        AXS_HIP_CHECK(hipGetLastError());
    }
    using namespace axs_lmh;
    timed(ctx, AXS_KERNEL_LM_HEAD, s, [&] {
        if (batch <= DOT_BMAX) {
            // B = 1: two vocabulary rows per wave, 2 K pieces of each in
            // flight; B = 2: four rows per wave, one piece
            const int rows = batch == 1 ? 2 : 4;
            const dim3 grid((unsigned)((vocab + (NT / 64) * rows - 1) / ((NT / 64) * rows)));
            if (batch == 1)
                hipLaunchKernelGGL((k_lm_head_dot<1, 2, 2>), grid, dim3(NT), 0, s, a);
            else
                hipLaunchKernelGGL((k_lm_head_dot<2, 4, 1>), grid, dim3(NT), 0, s, a);
        } else {
            // up to 48 batch rows: 64 vocabulary rows per workgroup, 512-byte
            // K chunks; above: 128 rows per workgroup (each hidden fragment
            // feeds two matrix-core steps), 256-byte chunks.  A launch slice
            // covers 16 * nb batch rows (nb 1-4; 6 for 65-96 rows, 8 above),
            // so W is read once per 128 batch rows.
            const int need = batch < BMAX ? (batch + 15) / 16 : BMAX / 16;  // 16-row batch blocks
            const int nb = need <= 4 ? need : (need <= 6 ? 6 : 8);
            const int rows = nb <= 3 ? 64 : 128;
            const dim3 grid((unsigned)((vocab + rows - 1) / rows), (unsigned)((batch + 16 * nb - 1) / (16 * nb)));
            switch (nb) {
                case 1: hipLaunchKernelGGL((k_lm_head_mfma<1, 1, 256>), grid, dim3(NT), 0, s, a); break;
                case 2: hipLaunchKernelGGL((k_lm_head_mfma<2, 1, 256>), grid, dim3(NT), 0, s, a); break;
                case 3: hipLaunchKernelGGL((k_lm_head_mfma<3, 1, 256>), grid, dim3(NT), 0, s, a); break;
                case 4: hipLaunchKernelGGL((k_lm_head_mfma<4, 2, 128>), grid, dim3(NT), 0, s, a); break;
                case 6: hipLaunchKernelGGL((k_lm_head_mfma<6, 2, 128>), grid, dim3(NT), 0, s, a); break;
                default: hipLaunchKernelGGL((k_lm_head_mfma<8, 2, 128>), grid, dim3(NT), 0, s, a); break;
            }
        }
    });
    AXS_HIP_CHECK(hipGetLastError());
    if (out_argmax) {
        hipLaunchKernelGGL(axs_lmh::k_lm_head_ids, dim3((batch + 255) / 256), dim3(256), 0, s, a.keys, batch,
                           out_argmax);
        AXS_HIP_CHECK(hipGetLastError());
    }
    return order_end(ctx, s);
}

}  // extern "C"

namespace {

// The draft law of one MTP depth per row (no processors, no filters): the
// sampled mode's argmax is the greedy law (T = 0), the stochastic mode's
// draw is sample_categorical_into at T with top_p 1 and top_k 0; lp_temps
// gets the temperature of the full-softmax log-prob.
__global__ void k_draft_prep(const axs_sampling_params* in, int n, int mode, axs_sampling_params* out,
                             float* lp_temps) {
    const int r = blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= n) return;
    const float T = in[r].temperature;
    axs_sampling_params p{};
    p.temperature = mode == AXS_MTP_DRAFT_SAMPLED ? 0.0f : T;
    p.top_p = 1.0f;
    p.top_k = 0;
    p.min_p = 0.0f;
    p.has_min_p = 0;
    p.repetition_penalty = 1.0f;
    p.repetition_context_size = AXS_NONE_U32;
    p.no_repeat_ngram_size = 0;
    p.ngram_window = 128;
    p.presence_penalty = 0.0f;
    p.frequency_penalty = 0.0f;
    p.seed = in[r].seed;
    p.step = in[r].step;
    out[r] = p;
    lp_temps[r] = (mode == AXS_MTP_DRAFT_SAMPLED || T > 0.0f) ? T : 1.0f;
}

}  // namespace

extern "C" {

int axs_mtp_draft(axs_context* ctx, const void* logits, int dtype, int batch, int vocab, int64_t row_stride,
                  const axs_sampling_params* params, int mode, const float* uniforms, uint32_t* out_ids,
                  float* out_lnq, void* stream) {
    if (!ctx || !logits || !params || !out_ids || !out_lnq)
        return fail(AXS_E_INVALID, "ctx, logits, params, out_ids and out_lnq must be non-NULL");
    if (dtype != AXS_DTYPE_F32 && dtype != AXS_DTYPE_BF16) return fail(AXS_E_INVALID, "bad dtype");
    if (mode != AXS_MTP_DRAFT_SAMPLED && mode != AXS_MTP_DRAFT_STOCHASTIC) return fail(AXS_E_INVALID, "bad mode");
    if (batch < 1 || vocab < 1 || row_stride < vocab) return fail(AXS_E_INVALID, "bad shape");
    if (batch > ctx->max_rows || vocab > ctx->max_vocab)
        return fail(AXS_E_CAPACITY, "batch or vocab larger than the context");
    std::lock_guard<std::mutex> lk(ctx->mu);
    DevGuard g(ctx->device);
    hipStream_t s = (hipStream_t)stream;
    int rc = order_begin(ctx, s);
    if (rc) return rc;
    hipLaunchKernelGGL(k_draft_prep, dim3((unsigned)((batch + 255) / 256)), dim3(256), 0, s, params, batch, mode,
                       ctx->draft_par, ctx->lp_temps);
    AXS_HIP_CHECK(hipGetLastError());
    // the draw (or argmax) of every draft row
    KArgs a{};
    a.logits = logits;
    a.dtype = dtype;
    a.nrows = batch;
    a.vocab = vocab;
    a.stride = row_stride;
    a.params = ctx->draft_par;
    a.exact_lp = 1;
    a.uniforms = uniforms;
    a.out_ids = out_ids;
    Plan pl = make_plan(dtype, batch, vocab, logits, row_stride, nullptr);
    if ((rc = run_pipeline(ctx, a, pl, s))) return rc;
    // ln softmax(l / T)[token] of the drawn tokens, axs_token_logprob_batch's pass
    KArgs l{};
    l.logits = logits;
    l.dtype = dtype;
    l.nrows = batch;
    l.vocab = vocab;
    l.stride = row_stride;
    l.params = nullptr;
    l.lp_tokens = out_ids;
    l.lp_temps = ctx->lp_temps;
    l.out_ids = ctx->lp_tok;  // the tokens echoed: scratch
    l.out_lp = out_lnq;
    if ((rc = run_pipeline(ctx, l, pl, s))) return rc;
    return order_end(ctx, s);
}

}  // extern "C"

namespace {

// target temperatures of the draft rows (row b * depth + i: sequence b's
// draft temperature) for the full-softmax draft log-prob pass
__global__ void k_draft_temps(const axs_sampling_params* dp, int depth, int n, float* out) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = dp[i / depth].temperature;
}

// the production target law's pass over the target rows q = b * (D + 1) + i:
// the draft token of position i (the bonus row gets vocab, which the stream
// pass decides directly) and the target temperature
__global__ void k_prod_prep(const uint32_t* draft_ids, const axs_sampling_params* tp, int depth, int n,
                            uint32_t vocab, uint32_t* tok, float* temps) {
    const int q = blockIdx.x * blockDim.x + threadIdx.x;
    if (q >= n) return;
    const int b = q / (depth + 1), i = q % (depth + 1);
    tok[q] = i < depth ? draft_ids[(size_t)b * depth + i] : vocab;
    temps[q] = tp[b].temperature;
}

// the last running-sum slot of rows [0, n) set to 0: a row the exact path
// does not reach keeps it
__global__ void k_zero_last(float* S, int n, uint32_t V) {
    const int q = blockIdx.x * blockDim.x + threadIdx.x;
    if (q < n) S[(size_t)q * V + V - 1u] = 0.0f;
}

int mtp_verify_impl(axs_context* ctx, const axs_mtp_desc* d, const axs_mtp_options* op,
                    const axs_mtp_outputs* o, void* stream) {
    if (!ctx || !d || !o) return fail(AXS_E_INVALID, "ctx, desc and outputs must be non-NULL");
    if (!d->target_logits || !d->draft_logits || !d->draft_ids || !d->target_params ||
        !d->draft_params || !o->out_ids || !o->out_count)
        return fail(AXS_E_INVALID, "missing required pointer");
    if (d->dtype != AXS_DTYPE_F32 && d->dtype != AXS_DTYPE_BF16) return fail(AXS_E_INVALID, "bad dtype");
    if (d->batch < 1 || d->vocab < 1 || d->depth < 1 || d->depth > 7 || d->row_stride < d->vocab)
        return fail(AXS_E_INVALID, "bad shape (depth must be 1..7)");
    if (op && (op->model_mode < AXS_MTP_MODEL_GREEDY || op->model_mode > AXS_MTP_MODEL_REJECTION ||
               op->ngram_mode < AXS_MTP_NGRAM_CONFIDENCE || op->ngram_mode > AXS_MTP_NGRAM_GREEDY ||
               op->lnq_mode < AXS_MTP_LNQ_DISTRIBUTION || op->lnq_mode > AXS_MTP_LNQ_FULL_SOFTMAX ||
               op->target_law < AXS_MTP_TARGET_DISTRIBUTION || op->target_law > AXS_MTP_TARGET_FILTERED))
        return fail(AXS_E_INVALID, "bad MTP option mode");
    const int64_t rows = (int64_t)d->batch * (2 * d->depth + 1);
    if (rows > ctx->max_rows || d->vocab > ctx->max_vocab)
        return fail(AXS_E_CAPACITY, "batch*(2*depth+1) rows or vocab larger than the context");
    std::lock_guard<std::mutex> lk(ctx->mu);
    DevGuard g(ctx->device);
    hipStream_t s = (hipStream_t)stream;
    int rc = order_begin(ctx, s);
    if (rc) return rc;
    const bool ex = op != nullptr;
    const bool full_lnq = ex && op->lnq_mode == AXS_MTP_LNQ_FULL_SOFTMAX && !op->pending_log_probs;
    const bool prod = ex && op->target_law == AXS_MTP_TARGET_FILTERED;
    if (prod) {
        // the production law's target probability of every draft token, from
        // the target rows' softmax (before the pipeline reuses the workspace)
        const int nt = d->batch * (d->depth + 1), nd = d->batch * d->depth;
        hipLaunchKernelGGL(k_fill_u32, dim3((unsigned)((nd + 255) / 256)), dim3(256), 0, s,
                           reinterpret_cast<uint32_t*>(ctx->mtp_ptgt), (uint32_t)nd, 0u);
        hipLaunchKernelGGL(k_prod_prep, dim3((unsigned)((nt + 255) / 256)), dim3(256), 0, s, d->draft_ids,
                           d->target_params, d->depth, nt, (uint32_t)d->vocab, ctx->lp_tok, ctx->lp_temps);
        AXS_HIP_CHECK(hipGetLastError());
        KArgs l{};
        l.logits = d->target_logits;
        l.dtype = d->dtype;
        l.nrows = nt;
        l.vocab = d->vocab;
        l.stride = d->row_stride;
        l.params = nullptr;
        l.lp_tokens = ctx->lp_tok;
        l.lp_temps = ctx->lp_temps;
        l.out_ids = ctx->mtp_amax;  // the rows' tokens echoed: scratch
        hipLaunchKernelGGL(k_zero_last, dim3((unsigned)((nt + 255) / 256)), dim3(256), 0, s, ctx->sbuf, nt,
                           (uint32_t)d->vocab);
        Plan lpp = make_plan(d->dtype, nt, d->vocab, d->target_logits, d->row_stride, nullptr);
        if ((rc = run_pipeline(ctx, l, lpp, s))) return rc;
        ProdArgs pa{};
        pa.tokens = ctx->lp_tok;
        pa.params = d->target_params;
        pa.out = ctx->mtp_ptgt;
        pa.topk = op->target_topk;
        pa.d1 = d->depth + 1;
        hipLaunchKernelGGL(k_mtp_prod, dim3((unsigned)nt), dim3(NT_EX), 0, s, l, pa);
        AXS_HIP_CHECK(hipGetLastError());
    }
    if (full_lnq) {
        // ln softmax(draft row / T_d)[d] of every draft row, the draft's own
        // temperature per sequence (axs_token_logprob_batch's pass)
        const int nd = d->batch * d->depth;
        hipLaunchKernelGGL(k_draft_temps, dim3((unsigned)((nd + 255) / 256)), dim3(256), 0, s, d->draft_params,
                           d->depth, nd, ctx->lp_temps);
        KArgs l{};
        l.logits = d->draft_logits;
        l.dtype = d->dtype;
        l.nrows = nd;
        l.vocab = d->vocab;
        l.stride = d->row_stride;
        l.params = nullptr;
        l.lp_tokens = d->draft_ids;
        l.lp_temps = ctx->lp_temps;
        l.out_ids = ctx->lp_tok;
        l.out_lp = ctx->mtp_lnq;
        Plan lp = make_plan(d->dtype, nd, d->vocab, d->draft_logits, d->row_stride, nullptr);
        if ((rc = run_pipeline(ctx, l, lp, s))) return rc;
    }
    KArgs a{};
    a.logits = d->target_logits;
    a.logits2 = d->draft_logits;
    a.dtype = d->dtype;
    a.nrows = (int32_t)rows;
    a.vocab = d->vocab;
    a.mtp_depth = d->depth;
    a.mtp_batch = d->batch;
    a.want_logprob = 0;
    a.stride = d->row_stride;
    a.params = d->target_params;
    a.params2 = d->draft_params;
    a.uniforms = d->uniforms;
    a.ws_kept_id = ctx->kept_id;
    a.ws_kept_p = ctx->kept_p;
    a.out_ids = ctx->mtp_tok;
    a.mtp_amax = ctx->mtp_amax;
    if (ex) {
        a.mtp_stream = 1;
        a.mtp_sources = op->sources;
        a.mtp_lnq_in = op->pending_log_probs;
        a.mtp_pred = op->predicted;
        a.mtp_lnq_full = full_lnq ? ctx->mtp_lnq : nullptr;
        a.mtp_model_mode = op->model_mode;
        a.mtp_ngram_mode = op->ngram_mode;
        a.mtp_delta = op->delta_correction ? 1 : 0;
    } else {
        a.mtp_model_mode = AXS_MTP_MODEL_REJECTION;
    }
    Plan pl = make_plan(d->dtype, (int)rows, d->vocab, d->target_logits, d->row_stride, d->draft_logits);
    if ((rc = run_pipeline(ctx, a, pl, s))) return rc;
    timed(ctx, AXS_KERNEL_MTP, s, [&] {
        hipLaunchKernelGGL(k_mtp_verify, dim3((unsigned)d->batch), dim3(NT_MTP), 0, s, a, d->draft_ids,
                           o->out_ids, o->out_count, o->accept_count, o->flags, prod ? ctx->mtp_ptgt : nullptr);
    });
    AXS_HIP_CHECK(hipGetLastError());
    return order_end(ctx, s);
}

}  // namespace

extern "C" {

int axs_mtp_verify(axs_context* ctx, const axs_mtp_desc* d, const axs_mtp_outputs* o, void* stream) {
    return mtp_verify_impl(ctx, d, nullptr, o, stream);
}

int axs_mtp_verify_ex(axs_context* ctx, const axs_mtp_desc* d, const axs_mtp_options* opts,
                      const axs_mtp_outputs* o, void* stream) {
    axs_mtp_options dflt{};
    dflt.model_mode = AXS_MTP_MODEL_REJECTION;
    return mtp_verify_impl(ctx, d, opts ? opts : &dflt, o, stream);
}

int axs_timing_enable(axs_context* ctx, int enable) {
    if (!ctx) return fail(AXS_E_INVALID, "ctx is NULL");
    std::lock_guard<std::mutex> lk(ctx->mu);
    DevGuard g(ctx->device);
    clear_events(ctx);
    ctx->timing = enable != 0;
    return AXS_OK;
}

int axs_timing_read(axs_context* ctx, int kernel, double* total_ms, int* launches) {
    if (!ctx || !total_ms || !launches) return fail(AXS_E_INVALID, "NULL argument");
    if (kernel < 0 || kernel >= AXS_KERNEL_COUNT) return fail(AXS_E_INVALID, "bad kernel id");
    std::lock_guard<std::mutex> lk(ctx->mu);
    DevGuard g(ctx->device);
    double t = 0.0;
    for (auto& e : ctx->ev[kernel]) {
        AXS_HIP_CHECK(hipEventSynchronize(e.second));
        float ms = 0.0f;
        AXS_HIP_CHECK(hipEventElapsedTime(&ms, e.first, e.second));
        t += ms;
    }
    *total_ms = t;
    *launches = (int)ctx->ev[kernel].size();
    return AXS_OK;
}

}  // extern "C"
