// axs_sampler.hip — MI355X (gfx950) per-step token sampler behind the C ABI
// of include/ax_hip_sampler.h.
//
// One sampling step over [rows, V] logits in HBM runs as four kernels on the
// caller's stream:
//
//   k_chunk     one pass over the logits (the HBM-bound kernel).  Work item =
//               (row, chunk of <= 8192 ids); the chunks of a row are placed on
//               one XCD.  Per chunk: the logits processors (repetition,
//               presence/frequency, bias, mask, n-gram ban) from LDS tables,
//               max/argmax, and — for min-p and top-k rows — every element
//               that can still be in the row's kept set, plus the largest
//               value it left out.
//   k_finish    one workgroup per row.  Merges the chunk results; greedy,
//               fallback, min-p and top-k rows are decided here exactly when
//               the gathered candidates provably contain the needed prefix.
//               Other rows join the exact-path list.
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
// -ffp-contract=off), correctly rounded division.

#include <hip/hip_runtime.h>

#include <cstdlib>
#include <mutex>
#include <new>
#include <string>
#include <vector>

#include "axs_device.h"

namespace axs {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int NT_CHUNK = 256;
constexpr uint32_t SEG_MAX = 32768;   // ids per segment (upper bound)
constexpr uint32_t MAX_SEGS = 1024;   // segments per row (upper bound)
constexpr uint32_t CAPC = 512;        // candidates kept per chunk
constexpr int NT_FIN = 256;
constexpr uint32_t FIN_CAP = 2048;    // candidates merged per row in k_finish
constexpr int NT_EX = 1024;
constexpr uint32_t NBUCKET = 13312;   // 13 per thread; covers p in [2^-24, 1]
constexpr uint32_t BIAS_LDS = 256;    // bias entries per chunk
constexpr uint32_t NBIN = 2048;       // top-k histogram bins (1/32 nat each)
constexpr uint32_t KEPT_CAP = 2048;   // kept entries per MTP distribution row
constexpr uint32_t BIG_LDS_SORT = 4096;
constexpr float P_FLOOR = 0x1p-24f;   // smaller terms never change a sum >= 1

// chunk-stat flags
constexpr uint32_t CS_OVERFLOW = 1u;
constexpr uint32_t CS_ERROR = 2u;

struct ChunkStat {
    float m;        // max processed logit (-inf if the chunk has no non-NaN)
    uint32_t amax;  // lowest id attaining m, NONE if none
    float lx;       // largest non-NaN logit NOT gathered (-inf if none)
    uint32_t count; // gathered candidates
    uint32_t flags;
    float gsum;     // sum of exp(l - m) over finite l (greedy logprob)
    uint32_t pad0, pad1;
};

struct Cand {
    uint32_t id;
    float l;
};

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
    int32_t nch;
    int32_t chunk;
    int32_t mtp_depth;    // > 0: MTP layout
    int32_t mtp_batch;
    int32_t want_logprob;
    int32_t vec;          // rows are 16-byte aligned: vector loads
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
    Cand* cand;
    RowState* rstate;
    uint32_t* exact_rows;
    uint32_t* exact_count;
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
    if (a.params == nullptr) {  // plain argmax entry point
        axs_sampling_params p;
        p.temperature = 0.0f;
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

// the uniform a row's draw consumes: supplied, or Philox(seed, row, step)
__device__ __forceinline__ float row_uniform(const KArgs& a, int r, const axs_sampling_params& p) {
    if (a.mtp_depth > 0) {
        int D = a.mtp_depth;
        int nt = a.mtp_batch * (D + 1);
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
//   spec  bit per id of the segment: the id has a history count or a bias entry
//   ban   bit per id: banned by the no-repeat n-gram rule
//   hash  open-addressing table offset → occurrence count in the repetition
//         window (only ids that occur); if it ever fills, counts are taken by
//         scanning the window in HBM for the (few) flagged ids
// --------------------------------------------------------------------------
constexpr uint32_t HSLOTS = 2048;
constexpr uint32_t HBITS = 11;

struct ProcLds {
    uint32_t spec[SEG_MAX / 32];
    uint32_t ban[SEG_MAX / 32];
    uint32_t hkey[HSLOTS];   // offset + 1, 0 = empty
    uint32_t hval[HSLOTS];   // occurrence count
    uint32_t bias_id[BIAS_LDS];
    float bias_v[BIAS_LDS];
    uint32_t nbias;
    uint32_t err;    // bias entries beyond BIAS_LDS in one segment
    uint32_t hfull;  // the hash filled up
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

__device__ __forceinline__ uint32_t hslot(uint32_t off) { return (off * 2654435761u) >> (32 - HBITS); }

__device__ __forceinline__ void hash_add(ProcLds& L, uint32_t off) {
    const uint32_t key = off + 1u;
    uint32_t h = hslot(off);
    for (uint32_t probe = 0; probe < HSLOTS; ++probe) {
        uint32_t k = L.hkey[h];
        if (k == 0u) {
            uint32_t prev = atomicCAS(&L.hkey[h], 0u, key);
            k = prev == 0u ? key : prev;
        }
        if (k == key) {
            atomicAdd(&L.hval[h], 1u);
            return;
        }
        h = (h + 1u) & (HSLOTS - 1u);
    }
    L.hfull = 1u;
}

// Builds the segment's LDS tables for ids in [lo, hi).  Block-uniform control.
__device__ __forceinline__ void proc_setup(const KArgs& a, const RowCtx& c, uint32_t lo, uint32_t hi,
                                           ProcLds& L) {
    const int tid = threadIdx.x;
    const uint32_t nw = (hi - lo + 31u) / 32u;
    if (tid == 0) {
        L.nbias = 0;
        L.err = 0;
        L.hfull = 0;
    }
    for (uint32_t i = tid; i < nw; i += NT_CHUNK) {
        L.spec[i] = 0u;
        L.ban[i] = 0u;
    }
    if (c.cnt_on)
        for (uint32_t i = tid; i < HSLOTS; i += NT_CHUNK) {
            L.hkey[i] = 0u;
            L.hval[i] = 0u;
        }
    __syncthreads();
    if (c.cnt_on) {
        for (int64_t i = c.w0 + tid; i < c.w1; i += NT_CHUNK) {
            uint32_t t = a.hist[i];
            if (t >= lo && t < hi) {
                uint32_t off = t - lo;
                hash_add(L, off);
                atomicOr(&L.spec[off >> 5], 1u << (off & 31u));
            }
        }
    }
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
                if (slot < BIAS_LDS) {
                    L.bias_id[slot] = t;
                    L.bias_v[slot] = v;
                    atomicOr(&L.spec[(t - lo) >> 5], 1u << ((t - lo) & 31u));
                } else {
                    L.err = 1;
                }
            }
            base += __popcll(m);
        }
        if (lane == 0) L.nbias = base < BIAS_LDS ? base : BIAS_LDS;
    }
    if (c.ban_on) {
        // logits_with_no_repeat_ngram_in_place (sampling.rs:896-920)
        int64_t nhist = c.w1 - c.h0;
        uint32_t ng = c.p.no_repeat_ngram_size;
        int64_t keep = (int64_t)(c.p.ngram_window > ng ? c.p.ngram_window : ng);
        if (keep > nhist) keep = nhist;
        int64_t hs = c.w1 - keep;
        int64_t plen = (int64_t)ng - 1;
        for (int64_t s = tid; s + (int64_t)ng <= keep; s += NT_CHUNK) {
            bool match = true;
            for (int64_t j = 0; j < plen; ++j)
                if (a.hist[hs + s + j] != a.hist[c.w1 - plen + j]) {
                    match = false;
                    break;
                }
            if (match) {
                uint32_t t = a.hist[hs + s + plen];
                if (t >= lo && t < hi) atomicOr(&L.ban[(t - lo) >> 5], 1u << ((t - lo) & 31u));
            }
        }
    }
    __syncthreads();
}

// Processor flags of a row
constexpr uint32_t PF_REP = 1u, PF_PF = 2u, PF_CNT = 4u, PF_BIAS = 8u;

// Repetition → presence/frequency → bias for one id that carries a history
// count or a bias entry (mask and n-gram ban are applied by the caller).
__device__ __forceinline__ float proc_special(const uint32_t* __restrict__ hist, const ProcLds& L,
                                              uint32_t off, uint32_t e, float l, uint32_t pfl,
                                              float rep, float freq, float pres, int64_t w0,
                                              int64_t w1) {
    if (pfl & PF_CNT) {
        // occurrences of e in the repetition window, from the LDS hash
        const uint32_t key = off + 1u;
        uint32_t h = hslot(off);
        uint32_t cnt = 0;
        bool found = false;
        for (uint32_t probe = 0; probe < HSLOTS; ++probe) {
            uint32_t k = L.hkey[h];
            if (k == key) {
                cnt = L.hval[h];
                found = true;
                break;
            }
            if (k == 0u) break;
            h = (h + 1u) & (HSLOTS - 1u);
        }
        if (!found && L.hfull) {  // the table overflowed: count in HBM
            for (int64_t i = w0; i < w1; ++i) cnt += hist[i] == e ? 1u : 0u;
        }
        if (cnt) {
            if (pfl & PF_REP) l = l < 0.0f ? __fmul_rn(l, rep) : __fdiv_rn(l, rep);
            if (pfl & PF_PF) {
                l = __fsub_rn(l, __fmul_rn(freq, (float)cnt));
                l = __fsub_rn(l, pres);
            }
        }
    }
    if (pfl & PF_BIAS)
        for (uint32_t j = 0; j < L.nbias; ++j)
            if (L.bias_id[j] == e) l = __fadd_rn(l, L.bias_v[j]);
    return l;
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

// Visits every id of the segment once, with its processed logit: f(id, l).
// Ids without a special bit come from the thread's registers (mask applied
// inline); ids with a history count, a bias entry or an n-gram ban are
// visited in a second loop over the segment's bitmaps, which re-reads their
// raw logits (a few per segment) and applies every processor in order.
template <int DT, int NV, typename F>
__device__ __forceinline__ void seg_visit(const KArgs& a, const RowCtx& c, const ProcLds& L, int r,
                                          uint32_t lo, uint32_t hi, Seg<DT, NV>& S, F&& f) {
    constexpr int EPV = Ev<DT>::EPV;
    const int tid = threadIdx.x;
    const uint32_t pfl = (c.rep_on ? PF_REP : 0u) | (c.pf_on ? PF_PF : 0u) |
                         (c.cnt_on ? PF_CNT : 0u) | (c.bias_on ? PF_BIAS : 0u);
    const bool special = pfl != 0u || c.ban_on;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        // recompute from the raw registers in every pass (keeps the unpacked
        // values out of the register budget)
        asm volatile("" : "+v"(S.raw[j]));
        const uint32_t e0 = lo + ((uint32_t)j * NT_CHUNK + tid) * EPV;
        const uint32_t off0 = e0 - lo;
        uint32_t skip = 0;
        if (special)
            skip = ((L.spec[off0 >> 5] | L.ban[off0 >> 5]) >> (off0 & 31u)) & ((1u << EPV) - 1u);
#pragma unroll
        for (int q = 0; q < EPV; ++q) {
            if ((skip >> q) & 1u) continue;
            float l = unpack<DT>(S.raw[j], q);
            if (c.mask_on && !((S.mw[j] >> ((e0 + q) & 31u)) & 1u)) l = -INFINITY;
            f(e0 + q, l);
        }
    }
    if (special) {
        const char* rp = row_ptr(a, r);
        const uint32_t nw = (hi - lo + 31u) / 32u;
        for (uint32_t wi = tid; wi < nw; wi += NT_CHUNK) {
            uint32_t bits = L.spec[wi] | L.ban[wi];
            while (bits) {
                const uint32_t b = (uint32_t)__ffs((int)bits) - 1u;
                bits &= bits - 1u;
                const uint32_t off = wi * 32u + b;
                const uint32_t e = lo + off;
                float l = DT == AXS_DTYPE_BF16 ? __uint_as_float((uint32_t)((const uint16_t*)rp)[e] << 16)
                                               : ((const float*)rp)[e];
                if ((L.spec[wi] >> b) & 1u)
                    l = proc_special(a.hist, L, off, e, l, pfl, c.p.repetition_penalty,
                                     c.p.frequency_penalty, c.p.presence_penalty, c.w0, c.w1);
                if (c.mask_on) {
                    uint32_t mw = a.mask[(size_t)r * a.mask_stride + (e >> 5)];
                    if (!((mw >> (e & 31u)) & 1u)) l = -INFINITY;
                }
                if ((L.ban[wi] >> b) & 1u) l = -INFINITY;
                f(e, l);
            }
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

// wave-aggregated append of a candidate into LDS (one LDS atomic per wave)
__device__ __forceinline__ void cand_append(bool in, uint32_t id, float l, uint32_t* s_n, Cand* s_cand) {
    const int lane = threadIdx.x & 63;
    uint64_t m = __ballot(in);
    if (m == 0ull) return;
    uint32_t base = 0;
    int leader = __ffsll((long long)m) - 1;
    if (lane == leader) base = atomicAdd(s_n, (uint32_t)__popcll(m));
    base = (uint32_t)__shfl((int)base, leader, 64);
    if (in) {
        uint32_t slot = base + (uint32_t)__popcll(m & ((1ull << lane) - 1ull));
        if (slot < CAPC) {
            s_cand[slot].id = id;
            s_cand[slot].l = l;
        }
    }
}

// --------------------------------------------------------------------------
// k_chunk: the single pass over the logits, one segment per workgroup
// --------------------------------------------------------------------------
template <int DT, int NV>
__global__ __launch_bounds__(NT_CHUNK) void k_chunk(KArgs a) {
    __shared__ ProcLds L;
    __shared__ Cand s_cand[CAPC];
    __shared__ uint32_t s_hist[NBIN];
    __shared__ float s_f[NT_CHUNK / 64];
    __shared__ uint32_t s_u[NT_CHUNK / 64];
    __shared__ uint32_t s_n;
    __shared__ uint32_t s_bstar;

    const int tid = threadIdx.x;
    if (blockIdx.x == 0 && tid == 0) *a.exact_count = 0;
    const int64_t total = (int64_t)a.nrows * a.nch;
    const int64_t w = xcd_item(total);
    if (w >= total) return;
    const int r = (int)(w / a.nch);
    const int ci = (int)(w % a.nch);
    const uint32_t lo = (uint32_t)ci * (uint32_t)a.chunk;
    const uint32_t hi = min(lo + (uint32_t)a.chunk, (uint32_t)a.vocab);

    RowCtx c = make_ctx(a, r);
    Seg<DT, NV> S;
    seg_load<DT, NV>(a, r, lo, hi, a.vec != 0, c.mask_on, S);  // in flight during the setup
    if (c.any_proc) proc_setup(a, c, lo, hi, L);

    // max and first argmax (NaN skipped)
    float bm = -INFINITY;
    uint32_t bi = NONE;
    seg_visit<DT, NV>(a, c, L, r, lo, hi, S, [&](uint32_t e, float l) {
        if (!isnan(l)) am_merge(bm, bi, l, e);
    });
    block_argmax<NT_CHUNK>(bm, bi, s_f, s_u);
    const float mc = bi == NONE ? -INFINITY : bm;

    ChunkStat st;
    st.m = mc;
    st.amax = bi;
    st.lx = -INFINITY;
    st.count = 0;
    st.flags = (c.err || (c.any_proc && L.err)) ? CS_ERROR : 0u;
    st.gsum = 0.0f;
    st.pad0 = st.pad1 = 0;

    const uint32_t mode = c.mode;
    if (mode == M_GREEDY) {
        if (a.want_logprob && isfinite(mc)) {
            float s = 0.0f;
            seg_visit<DT, NV>(a, c, L, r, lo, hi, S, [&](uint32_t, float l) {
                if (isfinite(l)) s += __expf(l - mc);
            });
            st.gsum = block_sum_f<NT_CHUNK>(s, s_f);
        }
    } else if ((mode == M_MINP || mode == M_TOPK) && isfinite(mc)) {
        const float inv = __fdiv_rn(1.0f, c.p.temperature);
        if (isfinite(inv)) {
            if (tid == 0) s_n = 0;
            const bool use_bins = mode == M_TOPK;
            uint32_t bstar = 0;
            float thr = 0.0f;
            if (use_bins) {
                if (c.p.top_k > CAPC) {
                    st.flags |= CS_OVERFLOW;
                } else {
                    for (uint32_t i = tid; i < NBIN; i += NT_CHUNK) s_hist[i] = 0;
                    __syncthreads();
                    seg_visit<DT, NV>(a, c, L, r, lo, hi, S, [&](uint32_t, float l) {
                        float x = __fmul_rn(__fsub_rn(mc, l), inv);
                        if (x < 64.0f) atomicAdd(&s_hist[(uint32_t)(x * 32.0f)], 1u);
                    });
                    __syncthreads();
                    uint32_t loc = 0;
#pragma unroll
                    for (int q = 0; q < NBIN / NT_CHUNK; ++q) loc += s_hist[tid * (NBIN / NT_CHUNK) + q];
                    uint32_t tot;
                    uint32_t pre = block_excl_scan_u32<NT_CHUNK>(loc, s_u, &tot);
                    const uint32_t K = c.p.top_k;
                    if (tid == 0) {
                        s_bstar = NBIN - 1;
                        s_n = tot;  // gathered-set size when every binned id is taken
                    }
                    __syncthreads();
                    if (tot >= K && pre < K && pre + loc >= K) {
                        uint32_t acc = pre;
                        for (int q = 0; q < NBIN / NT_CHUNK; ++q) {
                            acc += s_hist[tid * (NBIN / NT_CHUNK) + q];
                            if (acc >= K) {
                                s_bstar = tid * (NBIN / NT_CHUNK) + q;
                                s_n = acc;
                                break;
                            }
                        }
                    }
                    __syncthreads();
                    bstar = s_bstar;
                    if (s_n > CAPC) st.flags |= CS_OVERFLOW;
                    __syncthreads();
                    if (tid == 0) s_n = 0;
                }
            } else {
                thr = __fsub_rn(ln_f32(c.p.min_p), 1e-3f);
            }
            __syncthreads();
            if (!(st.flags & CS_OVERFLOW)) {
                float lx = -INFINITY;
                seg_visit<DT, NV>(a, c, L, r, lo, hi, S, [&](uint32_t e, float l) {
                    bool in = false;
                    if (!isnan(l)) {
                        if (use_bins) {
                            float x = __fmul_rn(__fsub_rn(mc, l), inv);
                            in = x < 64.0f && (uint32_t)(x * 32.0f) <= bstar;
                        } else {
                            in = __fmul_rn(__fsub_rn(l, mc), inv) >= thr;
                        }
                        if (!in) lx = fmaxf(lx, l);
                    }
                    cand_append(in, e, l, &s_n, s_cand);
                });
                lx = block_max<NT_CHUNK>(lx, s_f);
                uint32_t n = s_n;
                if (n > CAPC) {
                    st.flags |= CS_OVERFLOW;
                } else {
                    Cand* dst = a.cand + ((size_t)r * a.nch + ci) * CAPC;
                    for (uint32_t i = tid; i < n; i += NT_CHUNK) dst[i] = s_cand[i];
                    st.count = n;
                    st.lx = lx;
                }
            }
        }
    }
    if (tid == 0) a.cstat[(size_t)r * a.nch + ci] = st;
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

// --------------------------------------------------------------------------
// k_finish: one workgroup per row
// --------------------------------------------------------------------------
__global__ __launch_bounds__(NT_FIN) void k_finish(KArgs a) {
    __shared__ uint64_t s_key[FIN_CAP];
    __shared__ float s_f[NT_FIN / 64];
    __shared__ uint32_t s_u[NT_FIN / 64];
    __shared__ double s_d[NT_FIN / 64];
    __shared__ uint32_t s_n;
    __shared__ float s_mg;
    __shared__ uint32_t s_coff[MAX_SEGS + 1];
    const int r = blockIdx.x;
    const int tid = threadIdx.x;
    if (r >= a.nrows) return;
    const axs_sampling_params p = row_params(a, r);
    const uint32_t mode = row_mode(p);
    const int nch = a.nch;

    float m = -INFINITY;
    uint32_t am = NONE;
    float lx = -INFINITY;
    uint32_t fl = 0;
    for (int c = tid; c < nch; c += NT_FIN) {
        ChunkStat st = a.cstat[(size_t)r * nch + c];
        am_merge(m, am, st.m, st.amax);
        lx = fmaxf(lx, st.lx);
        fl |= st.flags;
    }
    block_argmax<NT_FIN>(m, am, s_f, s_u);
    lx = block_max<NT_FIN>(lx, s_f);
    fl = block_or_u32<NT_FIN>(fl, s_u);
    if (am == NONE) {  // all-NaN row: argmax_f32 → 0 (sampling.rs:966)
        am = 0;
        m = -INFINITY;
    }

    if (fl & CS_ERROR) {
        if (tid == 0) {
            write_row(a, r, 0u, NAN, AXS_FLAG_ERROR);
            if (a.out_kept_count) a.out_kept_count[r] = 0;
            if (a.ws_kept_id) {
                a.rstate[r].kept = 0;
                a.rstate[r].nlist = 0;
                a.rstate[r].flags = AXS_FLAG_ERROR;
            }
        }
        return;
    }

    if (mode == M_GREEDY) {
        float lp = NAN;
        if (a.want_logprob) {
            double gs = 0.0;
            for (int c = tid; c < nch; c += NT_FIN) {
                ChunkStat st = a.cstat[(size_t)r * nch + c];
                if (isfinite(st.m) && st.amax != NONE) gs += (double)st.gsum * exp((double)st.m - (double)m);
            }
            gs = block_sum_d<NT_FIN>(gs, s_d);
            if (isfinite(m) && gs > 0.0) lp = (float)(-log(gs));
        }
        if (tid == 0) {
            write_row(a, r, am, lp, AXS_FLAG_GREEDY);
            write_single_kept(a, r, am);
            if (a.ws_kept_id) a.rstate[r].flags = AXS_FLAG_GREEDY;
        }
        return;
    }

    const float inv = __fdiv_rn(1.0f, p.temperature);
    if (!(isfinite(m) && isfinite(inv))) {
        // every probability is zero or NaN → argmax (sampling.rs:264-266,279-281)
        if (tid == 0) {
            write_row(a, r, am, NAN, AXS_FLAG_ARGMAX_FALLBACK);
            write_single_kept(a, r, am);
            if (a.ws_kept_id) a.rstate[r].flags = AXS_FLAG_ARGMAX_FALLBACK;
        }
        return;
    }

    const bool minp = mode == M_MINP;
    const bool sorted = minp ? filters_enabled(p) : (mode != M_FAST);
    bool exact = !(mode == M_MINP || mode == M_TOPK) || (fl & CS_OVERFLOW);

    // candidate merge: every gathered id above the global exclusion level lx
    float plx = -1.0f;
    if (!exact) {
        if (tid == 0) {
            s_n = 0;
            s_mg = INFINITY;
        }
        __syncthreads();
        float mg = INFINITY;
        // candidate counts of every segment → prefix offsets, then one flat
        // parallel loop over all candidates of the row
        uint32_t loc = 0;
        constexpr uint32_t PER = MAX_SEGS / NT_FIN;
        for (uint32_t q = 0; q < PER; ++q) {
            uint32_t c = (uint32_t)tid * PER + q;
            uint32_t cnt = c < (uint32_t)nch ? a.cstat[(size_t)r * nch + c].count : 0u;
            s_coff[c] = cnt;
            loc += cnt;
        }
        uint32_t ntot;
        uint32_t pre = block_excl_scan_u32<NT_FIN>(loc, s_u, &ntot);
        for (uint32_t q = 0; q < PER; ++q) {
            uint32_t c = (uint32_t)tid * PER + q;
            uint32_t cnt = s_coff[c];
            s_coff[c] = pre;
            pre += cnt;
        }
        if (tid == 0) s_coff[MAX_SEGS] = ntot;
        __syncthreads();
        for (uint32_t i = tid; i < ntot; i += NT_FIN) {
            uint32_t lo_c = 0, hi_c = (uint32_t)nch;  // last c with s_coff[c] <= i
            while (hi_c - lo_c > 1) {
                uint32_t mid = (lo_c + hi_c) / 2;
                if (s_coff[mid] <= i) lo_c = mid;
                else hi_c = mid;
            }
            {
                const uint32_t c = lo_c;
                Cand cd = a.cand[((size_t)r * nch + c) * CAPC + (i - s_coff[c])];
                if (!(cd.l > lx)) continue;
                float pr = prob_of(cd.l, m, inv);
                uint64_t key;
                if (minp) {
                    float d = fabsf(pr - p.min_p) / p.min_p;
                    mg = fminf(mg, d);
                    if (!(pr >= p.min_p)) continue;  // cutoff = min_p * max_prob, max_prob = 1
                    key = sorted ? key_pdesc(pr, cd.id) : key_idasc(pr, cd.id);
                } else {
                    key = key_pdesc(pr, cd.id);
                }
                uint32_t slot = atomicAdd(&s_n, 1u);
                if (slot < FIN_CAP) s_key[slot] = key;
            }
        }
        mg = block_max<NT_FIN>(-mg, s_f);  // min via max of negatives
        if (tid == 0) s_mg = -mg;
        __syncthreads();
        uint32_t n = s_n;
        if (lx > -INFINITY) plx = prob_of(lx, m, inv);
        if (n > FIN_CAP || n == 0) exact = true;
        // min-p: complete iff every id left out has p < min_p
        if (minp && plx >= p.min_p) exact = true;
        if (!exact) {
            uint32_t np2 = next_pow2(n);
            for (uint32_t i = n + tid; i < np2; i += NT_FIN) s_key[i] = 0;
            __syncthreads();
            block_sort_desc<NT_FIN>(s_key, np2);
            if (mode == M_TOPK) {
                uint32_t K = p.top_k < (uint32_t)a.vocab ? p.top_k : (uint32_t)a.vocab;
                if (n < K) exact = true;
                else {
                    float pk = pdesc_p(s_key[K - 1]);
                    if (!(pk > plx) || !(pk > 0.0f)) exact = true;
                }
            }
        }
        if (!exact && tid == 0) {
            // sequential decisions over the sorted candidates — the reference's
            // own f32 loops (sampling.rs:283-316, 922-952)
            const uint32_t L = n;
            uint32_t flags = AXS_FLAG_DREW;
            if (minp && s_mg < 1e-6f) flags |= AXS_FLAG_NEAR_MINP;
            auto P = [&](uint32_t i) { return sorted ? pdesc_p(s_key[i]) : idasc_p(s_key[i]); };
            auto ID = [&](uint32_t i) { return sorted ? pdesc_id(s_key[i]) : idasc_id(s_key[i]); };
            uint32_t nk = L;
            if (sorted && topp_active(p)) {
                float total = 0.0f;
                for (uint32_t i = 0; i < L; ++i) total = __fadd_rn(total, P(i));
                float cutoff = __fmul_rn(p.top_p, total);
                float cum = 0.0f, prev = 0.0f;
                uint32_t keep = 0;
                for (uint32_t i = 0; i < L; ++i) {
                    prev = cum;
                    cum = __fadd_rn(cum, P(i));
                    keep += 1;
                    if (cum >= cutoff) break;
                }
                nk = keep > 1 ? keep : 1;
                double up = (double)cum - (double)cutoff;
                double lo = keep > 1 ? (double)cutoff - (double)prev : INFINITY;
                double mgn = fmin(up, lo) / (double)total;
                if (mgn < 1e-6 && (p.top_k == 0 || nk <= p.top_k)) flags |= AXS_FLAG_NEAR_NUCLEUS;
            }
            uint32_t kept = nk;
            if (sorted && p.top_k > 0 && kept > p.top_k) kept = p.top_k;
            if (sorted && (kept < L || mode == M_TOPK)) {
                float nextp = kept < L ? P(kept) : -1.0f;
                if (mode == M_TOPK) nextp = fmaxf(nextp, plx);
                // near but not identical probabilities across the cut (identical
                // ones come from equal logits and are ordered by id everywhere)
                if (nextp >= 0.0f && P(kept - 1) != nextp &&
                    (double)P(kept - 1) - (double)nextp <= 2.0 * ulp_f(P(kept - 1)))
                    flags |= AXS_FLAG_NEAR_TIE;
            }
            float F = 0.0f;
            for (uint32_t i = 0; i < kept; ++i) F = __fadd_rn(F, P(i));
            const float u = row_uniform(a, r, p);
            const float thr = __fmul_rn(u, F);
            float cum = 0.0f, prev = 0.0f;
            uint32_t j = kept;
            for (uint32_t i = 0; i < kept; ++i) {
                prev = cum;
                cum = __fadd_rn(cum, P(i));
                if (cum >= thr) {
                    j = i;
                    break;
                }
            }
            if (j == kept) {  // last maximum (sampling.rs:310-315)
                float bp = -1.0f;
                for (uint32_t i = 0; i < kept; ++i)
                    if (P(i) >= bp) {
                        bp = P(i);
                        j = i;
                    }
            } else {
                double up = (double)cum - (double)thr;
                double lo = j > 0 ? (double)thr - (double)prev : INFINITY;
                if (fmin(up, lo) / (double)F < 1e-6) flags |= AXS_FLAG_NEAR_DRAW;
            }
            const uint32_t tok = ID(j);
            write_row(a, r, tok, logprob_of(__fdiv_rn(P(j), F)), flags);
            if (a.out_kept) {
                uint32_t nw = kept < (uint32_t)a.out_kept_cap ? kept : (uint32_t)a.out_kept_cap;
                for (uint32_t i = 0; i < nw; ++i) a.out_kept[(size_t)r * a.out_kept_cap + i] = ID(i);
            }
            if (a.out_kept_count) a.out_kept_count[r] = kept;
            if (a.ws_kept_id) {
                uint32_t nw = kept < KEPT_CAP ? kept : KEPT_CAP;
                for (uint32_t i = 0; i < nw; ++i) {
                    a.ws_kept_id[(size_t)r * KEPT_CAP + i] = ID(i);
                    a.ws_kept_p[(size_t)r * KEPT_CAP + i] = P(i);
                }
                a.rstate[r].kept = kept;
                a.rstate[r].nlist = nw;
                a.rstate[r].F = F;
                a.rstate[r].flags = flags;
            }
        }
    }
    if (exact && tid == 0) {
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
        a.rstate[r] = rs;
        uint32_t idx = atomicAdd(a.exact_count, 1u);
        a.exact_rows[idx] = (uint32_t)r;
    }
}

// --------------------------------------------------------------------------
// k_exact_mat: exact probabilities of the listed rows (second pass)
// --------------------------------------------------------------------------
template <int DT, int NV>
__global__ __launch_bounds__(NT_CHUNK) void k_exact_mat(KArgs a) {
    __shared__ ProcLds L;
    __shared__ uint32_t s_u[NT_CHUNK / 64];
    __shared__ float s_f[NT_CHUNK / 64];
    __shared__ uint32_t s_base;
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
        if (c.any_proc) proc_setup(a, c, lo, hi, L);
        const bool minp = rs.mode == M_MINP;
        const float minp_v = c.p.min_p;
        float mg = INFINITY;
        uint32_t cnt = 0;
        float* dense = a.dense + (size_t)r * a.vocab;
        // pass 1: exact probabilities; dense rows are written here, sorted rows
        // only counted
        seg_visit<DT, NV>(a, c, L, r, lo, hi, S, [&](uint32_t e, float l) {
            float pr = prob_of(l, rs.m, rs.inv);
            bool keep = true;
            if (minp) {
                if (!isnan(l)) mg = fminf(mg, fabsf(pr - minp_v) / minp_v);
                keep = pr >= minp_v;
            }
            float v = keep ? pr : 0.0f;
            if (!rs.sorted) {
                if (e < hi) dense[e] = v;
            } else if (v >= rs.pmin) {
                ++cnt;
            }
        });
        if (rs.sorted) {
            uint32_t tot;
            uint32_t pre = block_excl_scan_u32<NT_CHUNK>(cnt, s_u, &tot);
            if (tid == 0) s_base = tot ? atomicAdd(&a.rstate[r].ncompact, tot) : 0u;
            __syncthreads();
            uint64_t* dst = a.ckey + (size_t)r * a.vocab + s_base + pre;
            uint32_t o = 0;
            // pass 2: write the compacted (p desc, id asc) keys
            seg_visit<DT, NV>(a, c, L, r, lo, hi, S, [&](uint32_t e, float l) {
                float pr = prob_of(l, rs.m, rs.inv);
                if (minp && !(pr >= minp_v)) pr = 0.0f;
                if (pr >= rs.pmin) dst[o++] = key_pdesc(pr, e);
            });
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

template <int NT>
__device__ __forceinline__ Xd block_excl_scan_xd(Xd x, Xd* s_w) {
    constexpr int NW = NT / 64;
    int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    Xd inc = x;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        Xd y = shfl_up_xd(inc, d);
        if (lane >= d) inc = xd_compose(y, inc);
    }
    if (lane == 63) s_w[w] = inc;
    Xd ex = shfl_up_xd(inc, 1);
    if (lane == 0) ex = xd_identity();
    __syncthreads();
    Xd wp = xd_identity();
    for (int k = 0; k < NW; ++k)
        if (k < w) wp = xd_compose(wp, s_w[k]);
    __syncthreads();
    return xd_compose(wp, ex);
}

// first index i in [lo, hi) with S[i] >= t (S non-decreasing), hi if none
__device__ __forceinline__ uint32_t first_ge(const float* S, uint32_t lo, uint32_t hi, float t) {
    uint32_t a = lo, b = hi;
    while (a < b) {
        uint32_t mid = a + (b - a) / 2;
        if (S[mid] >= t) b = mid;
        else a = mid + 1;
    }
    return a;
}

__device__ __forceinline__ uint32_t bucket_of(uint64_t key) {
    uint32_t pb = (uint32_t)(key >> 32);
    uint32_t d = pb <= 0x3F800000u ? 0x3F800000u - pb : 0u;
    uint32_t b = d >> 14;
    return b < NBUCKET ? b : NBUCKET - 1;
}

__global__ __launch_bounds__(NT_EX) void k_exact_row(KArgs a) {
    __shared__ uint32_t s_cnt[NBUCKET];
    __shared__ Xd s_w[NT_EX / 64];
    __shared__ uint32_t s_u[NT_EX / 64];
    __shared__ float s_s;
    __shared__ uint32_t s_k, s_cross, s_nbig, s_err;
    __shared__ uint32_t s_big[256];
    const int tid = threadIdx.x;
    if (blockIdx.x >= *a.exact_count) return;
    const int r = (int)a.exact_rows[blockIdx.x];
    const RowState rs = a.rstate[r];
    const axs_sampling_params p = row_params(a, r);
    const uint32_t V = (uint32_t)a.vocab;
    const bool sorted = rs.sorted != 0;
    const uint32_t n = sorted ? rs.ncompact : V;
    const uint64_t* src = a.ckey + (size_t)r * V;
    uint64_t* keys = a.ckey2 + (size_t)r * V;
    const float* dense = a.dense + (size_t)r * V;
    float* S = a.sbuf + (size_t)r * V;
    if (tid == 0) {
        s_err = 0;
        s_nbig = 0;
    }

    if (sorted) {
        // counting sort by p bucket (descending p), then each bucket sorted
        // by (p desc, id asc)
        for (uint32_t i = tid; i < NBUCKET; i += NT_EX) s_cnt[i] = 0;
        __syncthreads();
        for (uint32_t i = tid; i < n; i += NT_EX) atomicAdd(&s_cnt[bucket_of(src[i])], 1u);
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
        for (uint32_t i = tid; i < n; i += NT_EX) {
            uint64_t k = src[i];
            uint32_t pos = atomicAdd(&s_cnt[bucket_of(k)], 1u);
            keys[pos] = k;
        }
        __syncthreads();
        uint32_t* bend = a.bend + (size_t)r * NBUCKET;
        for (uint32_t i = tid; i < NBUCKET; i += NT_EX) bend[i] = s_cnt[i];
        __threadfence_block();
        __syncthreads();
        const int wv = tid >> 6, lane = tid & 63;
        for (uint32_t b = wv; b < NBUCKET; b += NT_EX / 64) {
            uint32_t st = b ? bend[b - 1] : 0u, en = bend[b];
            uint32_t mcount = en - st;
            if (mcount <= 1) continue;
            if (mcount <= 64) {
                uint64_t k = lane < (int)mcount ? keys[st + lane] : 0ull;
                k = wave_sort_desc(k);
                if (lane < (int)mcount) keys[st + lane] = k;
            } else if (lane == 0) {
                uint32_t slot = atomicAdd(&s_nbig, 1u);
                if (slot < 256) s_big[slot] = b;
                else s_err = 1;
            }
        }
        __threadfence_block();
        __syncthreads();
        const uint32_t nbig = s_nbig < 256 ? s_nbig : 256;
        uint64_t* lds = (uint64_t*)s_cnt;  // bucket counts no longer needed
        for (uint32_t q = 0; q < nbig; ++q) {
            uint32_t b = s_big[q];
            uint32_t st = b ? bend[b - 1] : 0u, en = bend[b];
            uint32_t mcount = en - st;
            uint32_t np2 = next_pow2(mcount);
            if (np2 <= BIG_LDS_SORT) {
                for (uint32_t i = tid; i < np2; i += NT_EX) lds[i] = i < mcount ? keys[st + i] : 0ull;
                __syncthreads();
                block_sort_desc<NT_EX>(lds, np2);
                for (uint32_t i = tid; i < mcount; i += NT_EX) keys[st + i] = lds[i];
                __syncthreads();
            } else {
                uint64_t* t = a.tmp64 + (size_t)r * a.tmp_stride;
                for (uint32_t i = tid; i < np2; i += NT_EX) t[i] = i < mcount ? keys[st + i] : 0ull;
                __threadfence_block();
                __syncthreads();
                block_sort_desc<NT_EX>(t, np2);
                for (uint32_t i = tid; i < mcount; i += NT_EX) keys[st + i] = t[i];
                __threadfence_block();
                __syncthreads();
            }
        }
    }
    __syncthreads();

    // exact running sums S[k] = fl(S[k-1] + x_k), in parallel (axs_exact_sum.h)
    auto X = [&](uint32_t i) -> float { return sorted ? pdesc_p(keys[i]) : dense[i]; };
    if (tid == 0) {
        s_s = 0.0f;
        s_k = 0;
    }
    __syncthreads();
    constexpr uint32_t IT = 4;
    while (true) {
        const float s = s_s;
        const uint32_t k = s_k;
        if (k >= n) break;
        const Binade bd = binade_of(s);
        const uint32_t tile = min((uint32_t)NT_EX * IT, n - k);
        const uint32_t i0 = k + (uint32_t)tid * IT;
        Term t[IT];
        Xd mine = xd_identity();
#pragma unroll
        for (uint32_t j = 0; j < IT; ++j) {
            uint32_t i = i0 + j;
            if (i < k + tile) {
                t[j] = term_of(X(i), bd.E);
                mine = xd_compose(mine, xd_of(t[j]));
            }
        }
        Xd pre = block_excl_scan_xd<NT_EX>(mine, s_w);
        const uint32_t b0 = bd.A & 1u;
        uint64_t acc = (uint64_t)bd.A + (b0 ? pre.inc1 : pre.inc0);
        uint32_t par = b0 ? pre.par1 : pre.par0;
        uint32_t mycross = NONE;
#pragma unroll
        for (uint32_t j = 0; j < IT; ++j) {
            uint32_t i = i0 + j;
            if (i >= k + tile || mycross != NONE) continue;
            uint32_t cc = par ? t[j].c1 : t[j].c0;
            if (acc + cc >= (1ull << 24)) {
                mycross = i;
                continue;
            }
            acc += cc;
            par = (uint32_t)(acc & 1u);
            S[i] = binade_value((uint32_t)acc, bd.E);
        }
        if (tid == 0) s_cross = NONE;
        __syncthreads();
        if (mycross != NONE) atomicMin(&s_cross, mycross);
        __threadfence_block();
        __syncthreads();
        if (tid == 0) {
            const uint32_t kc = s_cross;
            if (kc == NONE) {
                s_s = S[k + tile - 1];
                s_k = k + tile;
            } else {
                float prev = kc == k ? s : S[kc - 1];
                float ns = __fadd_rn(prev, X(kc));
                S[kc] = ns;
                s_s = ns;
                s_k = kc + 1;
            }
        }
        __threadfence_block();
        __syncthreads();
    }

    if (tid != 0) return;
    // decisions (sampling.rs:283-316, 922-952) on the exact running sums
    uint32_t flags = AXS_FLAG_DREW | AXS_FLAG_EXACT_PATH;
    if (s_err) flags |= AXS_FLAG_ERROR;
    const bool minp = rs.mode == M_MINP;
    if (minp && __uint_as_float(rs.minp_mg) < 1e-6f) flags |= AXS_FLAG_NEAR_MINP;
    uint32_t tok = 0;
    float F = 0.0f, pj = 0.0f;
    uint32_t kept = 0, Lk = 0;
    if (n == 0) {
        tok = rs.amax;
        flags = AXS_FLAG_ARGMAX_FALLBACK | AXS_FLAG_EXACT_PATH;
        write_row(a, r, tok, NAN, flags);
        write_single_kept(a, r, tok);
        if (a.ws_kept_id) a.rstate[r].flags = flags;
        return;
    }
    if (sorted) {
        const uint32_t L = n;
        uint32_t nk = L;
        if (topp_active(p)) {
            float total = S[L - 1];
            float cutoff = __fmul_rn(p.top_p, total);
            uint32_t j = first_ge(S, 0, L, cutoff);
            nk = j < L ? j + 1 : L;
            double up = (double)S[nk - 1] - (double)cutoff;
            double lo = nk >= 2 ? (double)cutoff - (double)S[nk - 2] : INFINITY;
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
            float pa = pdesc_p(keys[kept - 1]), pb = pdesc_p(keys[kept]);
            if (pa != pb && (double)pa - (double)pb <= 2.0 * ulp_f(pa)) flags |= AXS_FLAG_NEAR_TIE;
        }
        F = S[Lk - 1];
        const float thr = __fmul_rn(rs.u, F);
        uint32_t j = first_ge(S, 0, Lk, thr);
        if (j >= Lk) j = Lk - 1;  // unreachable: S[Lk-1] = F >= u*F
        double up = (double)S[j] - (double)thr;
        double lo = j > 0 ? (double)thr - (double)S[j - 1] : INFINITY;
        if (fmin(up, lo) / (double)F < 1e-6) flags |= AXS_FLAG_NEAR_DRAW;
        tok = pdesc_id(keys[j]);
        pj = pdesc_p(keys[j]);
        if (kept == 0xFFFFFFFFu) kept = L;  // min-p survivors below 2^-24 are not listed
    } else {
        F = S[V - 1];
        const float thr = __fmul_rn(rs.u, F);
        uint32_t j = first_ge(S, 0, V, thr);
        if (j >= V) j = V - 1;
        double up = (double)S[j] - (double)thr;
        double lo = j > 0 ? (double)thr - (double)S[j - 1] : INFINITY;
        if (fmin(up, lo) / (double)F < 1e-6) flags |= AXS_FLAG_NEAR_DRAW;
        tok = j;
        pj = dense[j];
        kept = 0;
        for (uint32_t i = 0; i < V; ++i) kept += dense[i] > 0.0f || !minp ? 1u : 0u;
    }
    write_row(a, r, tok, logprob_of(__fdiv_rn(pj, F)), flags);
    if (a.out_kept_count) a.out_kept_count[r] = kept;
    if (a.out_kept && a.out_kept_cap > 0) {
        uint32_t cap = (uint32_t)a.out_kept_cap;
        if (sorted) {
            uint32_t nw = Lk < cap ? Lk : cap;
            for (uint32_t i = 0; i < nw; ++i) a.out_kept[(size_t)r * cap + i] = pdesc_id(keys[i]);
        } else {
            uint32_t o = 0;
            for (uint32_t i = 0; i < V && o < cap; ++i)
                if (!minp || dense[i] > 0.0f) a.out_kept[(size_t)r * cap + o++] = i;
        }
    }
    if (a.ws_kept_id) {
        uint32_t o = 0;
        if (sorted) {
            for (uint32_t i = 0; i < Lk && o < KEPT_CAP; ++i) {
                a.ws_kept_id[(size_t)r * KEPT_CAP + o] = pdesc_id(keys[i]);
                a.ws_kept_p[(size_t)r * KEPT_CAP + o] = pdesc_p(keys[i]);
                ++o;
            }
            // ids below 2^-24 never carry normalised mass ≥ one f32 ulp of 1, but
            // they are entries of the reference's distribution: refuse to
            // truncate silently
            if (kept > Lk) flags |= AXS_FLAG_ERROR;
        } else {
            for (uint32_t i = 0; i < V && o < KEPT_CAP; ++i)
                if (dense[i] > 0.0f) {
                    a.ws_kept_id[(size_t)r * KEPT_CAP + o] = i;
                    a.ws_kept_p[(size_t)r * KEPT_CAP + o] = dense[i];
                    ++o;
                }
        }
        if (kept > KEPT_CAP) flags |= AXS_FLAG_ERROR;
        a.rstate[r].kept = kept;
        a.rstate[r].nlist = o;
        a.rstate[r].F = F;
        a.rstate[r].flags = flags;
    }
}

// --------------------------------------------------------------------------
// k_mtp_verify: accept / residual / bonus per sequence
// (crates/ax-engine-mlx/src/runner/mod.rs:12388-12431, sampling.rs:709-752)
// --------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_mtp_verify(KArgs a, const uint32_t* draft_ids,
                                                    uint32_t* out_ids, uint32_t* out_count,
                                                    uint32_t* out_accept, uint32_t* out_flags) {
    __shared__ uint64_t s_t[KEPT_CAP];
    __shared__ uint64_t s_d[KEPT_CAP];
    __shared__ int s_ft, s_fd;
    const int b = blockIdx.x;
    const int tid = threadIdx.x;
    const int D = a.mtp_depth;
    const int Bm = a.mtp_batch;
    if (b >= Bm) return;
    const axs_sampling_params tp = a.params[b];
    const axs_sampling_params dp = a.params2[b];
    const float Tt = tp.temperature, Td = dp.temperature;
    uint32_t flags = 0;
    uint32_t count = 0;
    for (int i = 0; i < D; ++i) {
        const int tr = b * (D + 1) + i;
        const int dr = Bm * (D + 1) + b * D + i;
        const RowState rt = a.rstate[tr];
        const RowState rd = a.rstate[dr];
        if ((rt.flags | rd.flags) & AXS_FLAG_ERROR || rt.nlist < rt.kept || rd.nlist < rd.kept) {
            flags |= AXS_MTP_FLAG_ERROR;
            break;
        }
        if ((rt.flags | rd.flags) & (AXS_FLAG_NEAR_DRAW | AXS_FLAG_NEAR_NUCLEUS | AXS_FLAG_NEAR_MINP |
                                     AXS_FLAG_NEAR_TIE))
            flags |= AXS_MTP_FLAG_NEAR;
        const uint32_t d = draft_ids[(size_t)b * D + i];
        const uint32_t* tid_l = a.ws_kept_id + (size_t)tr * KEPT_CAP;
        const float* tp_l = a.ws_kept_p + (size_t)tr * KEPT_CAP;
        const uint32_t* did_l = a.ws_kept_id + (size_t)dr * KEPT_CAP;
        const float* dp_l = a.ws_kept_p + (size_t)dr * KEPT_CAP;
        if (tid == 0) {
            s_ft = -1;
            s_fd = -1;
        }
        __syncthreads();
        for (uint32_t k = tid; k < rt.nlist; k += 256)
            if (tid_l[k] == d) atomicMax(&s_ft, (int)k);
        for (uint32_t k = tid; k < rd.nlist; k += 256)
            if (did_l[k] == d) atomicMax(&s_fd, (int)k);
        __syncthreads();
        // normalised entries p / F (TokenDistribution::new, sampling.rs:128-144)
        float qd = s_fd >= 0 ? __fdiv_rn(dp_l[s_fd], rd.F) : 0.0f;
        float pt = s_ft >= 0 ? __fdiv_rn(tp_l[s_ft], rt.F) : 0.0f;
        pt = fmaxf(pt, 0.0f);
        float lnq = logprob_of(qd);
        float lps = lnq;
        if (Td > 0.0f && Tt > 0.0f && fabsf(__fsub_rn(Td, Tt)) > 1e-6f)
            lps = __fmul_rn(lnq, __fdiv_rn(Td, Tt));
        float pdraft = fmaxf(exp_cr(lps), 1e-37f);
        float accp = fminf(__fdiv_rn(pt, pdraft), 1.0f);
        float u = a.uniforms ? a.uniforms[(size_t)b * (D + 1) + i]
                             : philox_uniform(tp.seed, (uint32_t)b, tp.step, 1u + (uint32_t)i / 4u,
                                              (uint32_t)i & 3u);
        if (fabs((double)u - (double)accp) < 1e-6) flags |= AXS_MTP_FLAG_NEAR_ACCEPT;
        if (u < accp) {
            if (tid == 0) out_ids[(size_t)b * (D + 1) + count] = d;
            ++count;
            continue;
        }
        // residual max(P - Q, 0) over the union of ids, ascending id order
        const float ut = a.uniforms ? a.uniforms[(size_t)b * (D + 1) + D]
                                    : philox_uniform(tp.seed, (uint32_t)b, tp.step,
                                                     1u + (uint32_t)D / 4u, (uint32_t)D & 3u);
        const uint32_t nt = rt.nlist, nd = rd.nlist;
        uint32_t npt = next_pow2(nt > 0 ? nt : 1), npd = next_pow2(nd > 0 ? nd : 1);
        for (uint32_t k = tid; k < npt; k += 256)
            s_t[k] = k < nt ? (((uint64_t)(~tid_l[k]) << 32) |
                               __float_as_uint(__fdiv_rn(tp_l[k], rt.F)))
                            : 0ull;
        for (uint32_t k = tid; k < npd; k += 256)
            s_d[k] = k < nd ? (((uint64_t)(~did_l[k]) << 32) |
                               __float_as_uint(__fdiv_rn(dp_l[k], rd.F)))
                            : 0ull;
        __syncthreads();
        block_sort_desc<256>(s_t, npt);  // descending ~id = ascending id
        block_sort_desc<256>(s_d, npd);
        if (tid == 0) {
            // pass 1: residual sum in ascending id order
            auto merged = [&](auto&& visit) {
                uint32_t x = 0, y = 0;
                while (x < nt || y < nd) {
                    uint32_t ix = x < nt ? idasc_id(s_t[x]) : NONE;
                    uint32_t iy = y < nd ? idasc_id(s_d[y]) : NONE;
                    float v;
                    if (ix == iy) {
                        v = fmaxf(__fsub_rn(idasc_p(s_t[x]), idasc_p(s_d[y])), 0.0f);
                        visit(ix, v);
                        ++x;
                        ++y;
                    } else if (ix < iy) {
                        v = idasc_p(s_t[x]);
                        visit(ix, v);
                        ++x;
                    } else {
                        ++y;  // only in the draft: max(0 - q, 0) = 0
                    }
                }
            };
            float rsum = 0.0f;
            uint32_t rn = 0;
            merged([&](uint32_t, float v) {
                if (v > 0.0f && isfinite(v)) {
                    rsum = __fadd_rn(rsum, v);
                    ++rn;
                }
            });
            uint32_t corr = NONE;
            if (rn > 0 && rsum > 0.0f && isfinite(rsum)) {
                // normalised residual, then sample_from_token_distribution
                float total = 0.0f;
                merged([&](uint32_t, float v) {
                    if (v > 0.0f && isfinite(v)) total = __fadd_rn(total, __fdiv_rn(v, rsum));
                });
                float thr = __fmul_rn(ut, total);
                float cum = 0.0f;
                uint32_t last_id = NONE;
                float bp = -1.0f;
                merged([&](uint32_t id, float v) {
                    if (!(v > 0.0f && isfinite(v)) || corr != NONE) return;
                    float q = __fdiv_rn(v, rsum);
                    cum = __fadd_rn(cum, q);
                    if (q >= bp) {
                        bp = q;
                        last_id = id;
                    }
                    if (cum >= thr) corr = id;
                });
                if (corr == NONE) corr = last_id;
            } else {
                // empty residual: the target itself (sampling.rs:749)
                float total = 0.0f;
                for (uint32_t k = 0; k < nt; ++k) total = __fadd_rn(total, __fdiv_rn(tp_l[k], rt.F));
                float thr = __fmul_rn(ut, total);
                float cum = 0.0f, bp = -1.0f;
                uint32_t last_id = NONE;
                for (uint32_t k = 0; k < nt; ++k) {
                    float q = __fdiv_rn(tp_l[k], rt.F);
                    cum = __fadd_rn(cum, q);
                    if (q >= bp) {
                        bp = q;
                        last_id = tid_l[k];
                    }
                    if (cum >= thr) {
                        corr = tid_l[k];
                        break;
                    }
                }
                if (corr == NONE) corr = last_id;
            }
            out_ids[(size_t)b * (D + 1) + count] = corr;
        }
        ++count;
        flags |= AXS_MTP_FLAG_RESIDUAL;
        break;
    }
    if (tid == 0) {
        uint32_t acc = 0;
        if (!(flags & (AXS_MTP_FLAG_RESIDUAL | AXS_MTP_FLAG_ERROR))) {
            // all drafts accepted: the bonus token of target row D
            const int br = b * (D + 1) + D;
            const RowState rb = a.rstate[br];
            if (rb.flags & AXS_FLAG_ERROR) flags |= AXS_MTP_FLAG_ERROR;
            if (rb.flags & (AXS_FLAG_NEAR_DRAW | AXS_FLAG_NEAR_NUCLEUS | AXS_FLAG_NEAR_MINP |
                            AXS_FLAG_NEAR_TIE))
                flags |= AXS_MTP_FLAG_NEAR;
            out_ids[(size_t)b * (D + 1) + count] = a.out_ids[br];
            acc = count;
            ++count;
            flags |= AXS_MTP_FLAG_BONUS;
        } else {
            acc = count > 0 ? count - 1 : 0;
        }
        if (flags & AXS_MTP_FLAG_ERROR) count = 0;
        out_count[b] = count;
        if (out_accept) out_accept[b] = acc;
        if (out_flags) out_flags[b] = flags;
    }
}

}  // namespace axs

// ==========================================================================
// host side: context, validation, launches, C ABI
// ==========================================================================
using namespace axs;

namespace {

thread_local std::string g_last_error;

int fail(int code, const std::string& msg) {
    g_last_error = msg;
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
    Cand* cand;
    RowState* rstate;
    uint32_t* exact_rows;
    uint32_t* exact_count;
    float* dense;
    uint64_t* ckey;
    uint64_t* ckey2;
    uint64_t* tmp64;
    float* sbuf;
    uint32_t* bend;
    uint32_t* kept_id;
    float* kept_p;
    uint32_t* mtp_tok;  // per-row tokens of the MTP sampler pass
    bool timing;
    std::vector<std::pair<hipEvent_t, hipEvent_t>> ev[AXS_KERNEL_COUNT];
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
    void* ptrs[] = {c->cstat, c->cand,  c->rstate, c->exact_rows, c->exact_count, c->dense,  c->ckey,
                    c->ckey2, c->tmp64, c->sbuf,   c->bend,       c->kept_id,     c->kept_p, c->mtp_tok};
    for (void* q : ptrs)
        if (q) (void)hipFree(q);
    delete c;
}

// elements per thread-vector and the chunk size for a launch
struct Plan {
    int nv;
    uint32_t chunk;
    int nch;
    bool vec;
};

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
    pl.vec = ((uintptr_t)base % 16 == 0) && ((stride * es) % 16 == 0) &&
             (base2 == nullptr || (uintptr_t)base2 % 16 == 0);
    return pl;
}

template <int DT, int NV>
void launch_pair_nv(const KArgs& a, hipStream_t s, bool exact_pass) {
    const int64_t total = (int64_t)a.nrows * a.nch;
    if (!exact_pass) {
        dim3 grid((unsigned)(((total + 7) / 8) * 8));
        hipLaunchKernelGGL((k_chunk<DT, NV>), grid, dim3(NT_CHUNK), 0, s, a);
    } else {
        int64_t g = total < 1024 ? total : 1024;
        dim3 grid((unsigned)(g > 0 ? g : 1));
        hipLaunchKernelGGL((k_exact_mat<DT, NV>), grid, dim3(NT_CHUNK), 0, s, a);
    }
}

void launch_chunkish(const Plan& pl, const KArgs& a, hipStream_t s, bool exact_pass) {
    if (a.dtype == AXS_DTYPE_BF16) {
        switch (pl.nv) {
            case 16: launch_pair_nv<AXS_DTYPE_BF16, 16>(a, s, exact_pass); break;
            case 8: launch_pair_nv<AXS_DTYPE_BF16, 8>(a, s, exact_pass); break;
            case 4: launch_pair_nv<AXS_DTYPE_BF16, 4>(a, s, exact_pass); break;
            case 2: launch_pair_nv<AXS_DTYPE_BF16, 2>(a, s, exact_pass); break;
            default: launch_pair_nv<AXS_DTYPE_BF16, 1>(a, s, exact_pass); break;
        }
    } else {
        switch (pl.nv) {
            case 16: launch_pair_nv<AXS_DTYPE_F32, 16>(a, s, exact_pass); break;
            case 8: launch_pair_nv<AXS_DTYPE_F32, 8>(a, s, exact_pass); break;
            case 4: launch_pair_nv<AXS_DTYPE_F32, 4>(a, s, exact_pass); break;
            default: launch_pair_nv<AXS_DTYPE_F32, 2>(a, s, exact_pass); break;
        }
    }
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
    a.cand = c->cand;
    a.rstate = c->rstate;
    a.exact_rows = c->exact_rows;
    a.exact_count = c->exact_count;
    a.dense = c->dense;
    a.ckey = c->ckey;
    a.ckey2 = c->ckey2;
    a.tmp64 = c->tmp64;
    a.sbuf = c->sbuf;
    a.bend = c->bend;
    a.tmp_stride = c->tmp_stride;
}

// the four-kernel pipeline over a.nrows rows
int run_pipeline(axs_context* c, KArgs& a, const Plan& pl, hipStream_t s) {
    if (pl.nch > (int)MAX_SEGS) return fail(AXS_E_UNSUPPORTED, "vocab too large (more than 1024 segments)");
    a.nch = pl.nch;
    a.chunk = (int32_t)pl.chunk;
    a.vec = pl.vec ? 1 : 0;
    fill_ws(a, c);
    timed(c, AXS_KERNEL_CHUNK, s, [&] { launch_chunkish(pl, a, s, false); });
    timed(c, AXS_KERNEL_FINISH, s, [&] {
        hipLaunchKernelGGL(k_finish, dim3((unsigned)a.nrows), dim3(NT_FIN), 0, s, a);
    });
    timed(c, AXS_KERNEL_EXACT_MAT, s, [&] { launch_chunkish(pl, a, s, true); });
    timed(c, AXS_KERNEL_EXACT_ROW, s, [&] {
        hipLaunchKernelGGL(k_exact_row, dim3((unsigned)a.nrows), dim3(NT_EX), 0, s, a);
    });
    AXS_HIP_CHECK(hipGetLastError());
    return AXS_OK;
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
        (rc = dalloc(&c->cand, R * c->max_chunks * CAPC)) || (rc = dalloc(&c->rstate, R)) ||
        (rc = dalloc(&c->exact_rows, R)) || (rc = dalloc(&c->exact_count, 1)) ||
        (rc = dalloc(&c->dense, R * Vv)) || (rc = dalloc(&c->ckey, R * Vv)) ||
        (rc = dalloc(&c->ckey2, R * Vv)) || (rc = dalloc(&c->tmp64, R * (size_t)c->tmp_stride)) ||
        (rc = dalloc(&c->sbuf, R * Vv)) || (rc = dalloc(&c->bend, R * NBUCKET)) ||
        (rc = dalloc(&c->kept_id, R * KEPT_CAP)) || (rc = dalloc(&c->kept_p, R * KEPT_CAP)) ||
        (rc = dalloc(&c->mtp_tok, R))) {
        free_ctx(c);
        return rc;
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

int axs_sample_batch(axs_context* ctx, const axs_batch_desc* d, const axs_outputs* o, void* stream) {
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
    DevGuard g(ctx->device);
    hipStream_t s = (hipStream_t)stream;
    KArgs a{};
    a.logits = d->logits;
    a.logits2 = nullptr;
    a.dtype = d->dtype;
    a.nrows = d->batch;
    a.vocab = d->vocab;
    a.mtp_depth = 0;
    a.mtp_batch = 0;
    a.want_logprob = o->logprobs != nullptr;
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

int axs_argmax_batch(axs_context* ctx, const void* logits, int dtype, int batch, int vocab,
                     int64_t row_stride, uint32_t* out_ids, float* out_logprob, void* stream) {
    if (!ctx || !logits || !out_ids) return fail(AXS_E_INVALID, "ctx, logits and out_ids must be non-NULL");
    if (dtype != AXS_DTYPE_F32 && dtype != AXS_DTYPE_BF16) return fail(AXS_E_INVALID, "bad dtype");
    if (batch < 1 || vocab < 1 || row_stride < vocab) return fail(AXS_E_INVALID, "bad shape");
    if (batch > ctx->max_rows || vocab > ctx->max_vocab)
        return fail(AXS_E_CAPACITY, "batch or vocab larger than the context");
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
    if (pl.nch > (int)MAX_SEGS) return fail(AXS_E_UNSUPPORTED, "vocab too large (more than 1024 segments)");
    a.nch = pl.nch;
    a.chunk = (int32_t)pl.chunk;
    a.vec = pl.vec ? 1 : 0;
    fill_ws(a, ctx);
    hipStream_t s = (hipStream_t)stream;
    timed(ctx, AXS_KERNEL_CHUNK, s, [&] { launch_chunkish(pl, a, s, false); });
    timed(ctx, AXS_KERNEL_FINISH, s, [&] {
        hipLaunchKernelGGL(k_finish, dim3((unsigned)batch), dim3(NT_FIN), 0, s, a);
    });
    AXS_HIP_CHECK(hipGetLastError());
    return AXS_OK;
}

int axs_mtp_verify(axs_context* ctx, const axs_mtp_desc* d, const axs_mtp_outputs* o, void* stream) {
    if (!ctx || !d || !o) return fail(AXS_E_INVALID, "ctx, desc and outputs must be non-NULL");
    if (!d->target_logits || !d->draft_logits || !d->draft_ids || !d->target_params ||
        !d->draft_params || !o->out_ids || !o->out_count)
        return fail(AXS_E_INVALID, "missing required pointer");
    if (d->dtype != AXS_DTYPE_F32 && d->dtype != AXS_DTYPE_BF16) return fail(AXS_E_INVALID, "bad dtype");
    if (d->batch < 1 || d->vocab < 1 || d->depth < 1 || d->depth > 7 || d->row_stride < d->vocab)
        return fail(AXS_E_INVALID, "bad shape (depth must be 1..7)");
    int64_t rows = (int64_t)d->batch * (2 * d->depth + 1);
    if (rows > ctx->max_rows || d->vocab > ctx->max_vocab)
        return fail(AXS_E_CAPACITY, "batch*(2*depth+1) rows or vocab larger than the context");
    DevGuard g(ctx->device);
    hipStream_t s = (hipStream_t)stream;
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
    Plan pl = make_plan(d->dtype, (int)rows, d->vocab, d->target_logits, d->row_stride, d->draft_logits);
    int rc = run_pipeline(ctx, a, pl, s);
    if (rc) return rc;
    timed(ctx, AXS_KERNEL_MTP, s, [&] {
        hipLaunchKernelGGL(k_mtp_verify, dim3((unsigned)d->batch), dim3(256), 0, s, a, d->draft_ids,
                           o->out_ids, o->out_count, o->accept_count, o->flags);
    });
    AXS_HIP_CHECK(hipGetLastError());
    return AXS_OK;
}

int axs_timing_enable(axs_context* ctx, int enable) {
    if (!ctx) return fail(AXS_E_INVALID, "ctx is NULL");
    DevGuard g(ctx->device);
    clear_events(ctx);
    ctx->timing = enable != 0;
    return AXS_OK;
}

int axs_timing_read(axs_context* ctx, int kernel, double* total_ms, int* launches) {
    if (!ctx || !total_ms || !launches) return fail(AXS_E_INVALID, "NULL argument");
    if (kernel < 0 || kernel >= AXS_KERNEL_COUNT) return fail(AXS_E_INVALID, "bad kernel id");
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
