/*
 * ax_oracle.c — CPU restatement of AX Engine's per-step sampling law.
 *
 * TEST INFRASTRUCTURE ONLY: the parity checker for the HIP sampler (see
 * ax_oracle.h).  Compiled with gcc -O2 -ffp-contract=off, no fast-math.
 * Every function cites the reference lines it restates; line numbers are in
 * /root/reference (defai-digital/ax-engine).
 */
#define _GNU_SOURCE
#include "ax_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* RNGs                                                                      */
/* ------------------------------------------------------------------------ */

/* Xorshift64::new (crates/ax-engine-mlx/src/sampling.rs:19-23) */
uint64_t axo_xorshift64_new(uint64_t seed) {
    uint64_t s = seed + 0x9e3779b97f4a7c15ull;
    return s == 0 ? 1 : s;
}

/* Xorshift64::next_u64 (sampling.rs:26-31) */
uint64_t axo_xorshift64_next_u64(uint64_t* state) {
    uint64_t x = *state;
    x ^= x << 13;
    x ^= x >> 7;
    x ^= x << 17;
    *state = x;
    return x;
}

/* Xorshift64::next_f32 (sampling.rs:34-36): the u64 → f32 conversion rounds
 * to nearest, so the result can be exactly 1.0. */
float axo_xorshift64_next_f32(uint64_t* state) {
    uint64_t v = axo_xorshift64_next_u64(state) >> 11;
    return (float)v * (1.0f / (float)(1ull << 53));
}

/* Philox4x32-10: Salmon et al., "Parallel random numbers: as easy as 1, 2,
 * 3", SC'11, multipliers 0xD2511F53 / 0xCD9E8D57, Weyl key increments
 * 0x9E3779B9 / 0xBB67AE85, ten rounds, the first with the unbumped key. */
void axo_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]) {
    uint32_t c0 = ctr[0], c1 = ctr[1], c2 = ctr[2], c3 = ctr[3];
    uint32_t k0 = key[0], k1 = key[1];
    for (int r = 0; r < 10; ++r) {
        if (r > 0) {
            k0 += 0x9E3779B9u;
            k1 += 0xBB67AE85u;
        }
        uint64_t p0 = (uint64_t)0xD2511F53u * c0;
        uint64_t p1 = (uint64_t)0xCD9E8D57u * c2;
        uint32_t hi0 = (uint32_t)(p0 >> 32), lo0 = (uint32_t)p0;
        uint32_t hi1 = (uint32_t)(p1 >> 32), lo1 = (uint32_t)p1;
        uint32_t n0 = hi1 ^ c1 ^ k0;
        uint32_t n1 = lo1;
        uint32_t n2 = hi0 ^ c3 ^ k1;
        uint32_t n3 = lo0;
        c0 = n0; c1 = n1; c2 = n2; c3 = n3;
    }
    out[0] = c0; out[1] = c1; out[2] = c2; out[3] = c3;
}

float axo_philox_uniform(uint64_t seed, uint32_t row, uint64_t step,
                         uint32_t purpose, uint32_t word) {
    uint32_t ctr[4] = {row, (uint32_t)step, (uint32_t)(step >> 32), purpose};
    uint32_t key[2] = {(uint32_t)seed, (uint32_t)(seed >> 32)};
    uint32_t out[4];
    axo_philox4x32_10(ctr, key, out);
    return (float)(out[word & 3] >> 8) * 0x1p-24f;
}

/* ------------------------------------------------------------------------ */
/* helpers                                                                   */
/* ------------------------------------------------------------------------ */

void axo_bf16_to_f32(const uint16_t* in, float* out, uint64_t n) {
    for (uint64_t i = 0; i < n; ++i) {
        uint32_t b = (uint32_t)in[i] << 16;
        memcpy(&out[i], &b, 4);
    }
}

/* argmax_index_f32 / argmax_f32 (sampling.rs:954-970): first strictly
 * greater value wins (lowest id on ties), NaN skipped, all-NaN → 0. */
uint32_t axo_argmax_f32(const float* logits, uint32_t n) {
    int have = 0;
    uint32_t best_i = 0;
    float best = 0.0f;
    for (uint32_t i = 0; i < n; ++i) {
        float l = logits[i];
        if (isnan(l)) continue;
        if (!have || l > best) {
            have = 1;
            best = l;
            best_i = i;
        }
    }
    return have ? best_i : 0;
}

/* MlxSamplingParams::uses_min_p (sampling.rs:86-89) */
static int uses_min_p(const axs_sampling_params* p) {
    return p->has_min_p && isfinite(p->min_p) && p->min_p > 0.0f;
}

/* MlxSamplingParams::uses_repetition_penalty (sampling.rs:91-95) */
static int uses_rep(const axs_sampling_params* p) {
    return isfinite(p->repetition_penalty) && p->repetition_penalty > 0.0f &&
           p->repetition_penalty != 1.0f;
}

static int uses_presence_freq(const axs_sampling_params* p) {
    return p->presence_penalty != 0.0f || p->frequency_penalty != 0.0f;
}

typedef struct {
    uint32_t V;
    float* row;         /* processed copy of the logits */
    float* probs;       /* fast-path probabilities      */
    uint32_t* cid;      /* candidate ids                */
    float* cp;          /* candidate probabilities      */
    uint32_t* counts;   /* per-id counts (zeroed)       */
    uint8_t* seen;      /* per-id marks (zeroed)        */
    uint32_t* order;    /* sort permutation             */
} workspace;

static int ws_init(workspace* w, uint32_t V) {
    memset(w, 0, sizeof(*w));
    w->V = V;
    size_t n = V ? V : 1;
    w->row = (float*)malloc(n * sizeof(float));
    w->probs = (float*)malloc(n * sizeof(float));
    w->cid = (uint32_t*)malloc(n * sizeof(uint32_t));
    w->cp = (float*)malloc(n * sizeof(float));
    w->counts = (uint32_t*)calloc(n, sizeof(uint32_t));
    w->seen = (uint8_t*)calloc(n, 1);
    w->order = (uint32_t*)malloc(n * sizeof(uint32_t));
    return w->row && w->probs && w->cid && w->cp && w->counts && w->seen && w->order;
}

static void ws_free(workspace* w) {
    free(w->row); free(w->probs); free(w->cid); free(w->cp);
    free(w->counts); free(w->seen); free(w->order);
}

/* recent_repetition_tokens (sampling.rs:809-815): the last
 * min(context_size or len, len) tokens. */
static uint32_t repetition_window(uint32_t nhist, uint32_t context_size, uint32_t* start) {
    uint32_t keep = context_size == AXS_NONE_U32 ? nhist : context_size;
    if (keep > nhist) keep = nhist;
    *start = nhist - keep;
    return keep;
}

/* logits_with_repetition_penalty_in_place (sampling.rs:875-894): each unique
 * id (first occurrence) below V is divided (l >= 0) or multiplied (l < 0). */
static void repetition_penalty(float* row, uint32_t V, float penalty,
                               const uint32_t* toks, uint32_t n, uint8_t* seen) {
    for (uint32_t i = 0; i < n; ++i) {
        uint32_t t = toks[i];
        if (t >= V) continue;          /* HashSet insert then get_mut → None */
        if (seen[t]) continue;
        seen[t] = 1;
        if (row[t] < 0.0f) row[t] = row[t] * penalty;
        else row[t] = row[t] / penalty;
    }
    for (uint32_t i = 0; i < n; ++i)
        if (toks[i] < V) seen[toks[i]] = 0;
}

/* logits_with_no_repeat_ngram_in_place (sampling.rs:896-920) */
static void no_repeat_ngram(float* row, uint32_t V, uint32_t ngram_size,
                            uint32_t window, const uint32_t* hist, uint32_t nhist) {
    if (ngram_size == 0 || nhist < ngram_size) return;
    uint32_t keep = window > ngram_size ? window : ngram_size;
    if (keep > nhist) keep = nhist;
    const uint32_t* h = hist + (nhist - keep);
    if (keep < ngram_size) return;
    uint32_t prefix_len = ngram_size - 1;
    const uint32_t* cur = h + (keep - prefix_len);
    for (uint32_t start = 0; start + ngram_size <= keep; ++start) {
        int match = 1;
        for (uint32_t j = 0; j < prefix_len; ++j)
            if (h[start + j] != cur[j]) { match = 0; break; }
        if (match) {
            uint32_t t = h[start + prefix_len];
            if (t < V) row[t] = -INFINITY;
        }
    }
}

static int apply_processors_ws(float* row, uint32_t V, const axs_sampling_params* p,
                               const uint32_t* hist, uint32_t nhist,
                               const uint32_t* mask_words,
                               const uint32_t* bias_ids, const float* bias_vals,
                               uint32_t nbias, workspace* w) {
    int applied = 0;
    /* the reference applies its processors only with a non-empty history
     * (sampling.rs:216) */
    int ref_proc = (uses_rep(p) || p->no_repeat_ngram_size > 0) && nhist > 0;
    uint32_t wstart = 0;
    uint32_t wlen = repetition_window(nhist, p->repetition_context_size, &wstart);
    const uint32_t* win = hist ? hist + wstart : NULL;
    if (ref_proc && uses_rep(p) && wlen > 0) {
        repetition_penalty(row, V, p->repetition_penalty, win, wlen, w->seen);
        applied = 1;
    }
    /* build extension: presence / frequency over the same window */
    if (uses_presence_freq(p) && wlen > 0) {
        for (uint32_t i = 0; i < wlen; ++i)
            if (win[i] < V) w->counts[win[i]]++;
        for (uint32_t i = 0; i < wlen; ++i) {
            uint32_t t = win[i];
            if (t >= V || w->counts[t] == 0) continue;
            float c = (float)w->counts[t];
            row[t] = row[t] - p->frequency_penalty * c;
            row[t] = row[t] - p->presence_penalty;
            w->counts[t] = 0;
        }
        applied = 1;
    }
    /* build extension: logit bias, entries in list order */
    if (bias_ids && nbias > 0) {
        for (uint32_t i = 0; i < nbias; ++i)
            if (bias_ids[i] < V) row[bias_ids[i]] = row[bias_ids[i]] + bias_vals[i];
        applied = 1;
    }
    /* build extension: allowed-token bitmask, LSB = lowest id */
    if (mask_words) {
        for (uint32_t t = 0; t < V; ++t)
            if (!((mask_words[t >> 5] >> (t & 31)) & 1u)) row[t] = -INFINITY;
        applied = 1;
    }
    if (ref_proc && p->no_repeat_ngram_size > 0) {
        no_repeat_ngram(row, V, p->no_repeat_ngram_size, p->ngram_window, hist, nhist);
        applied = 1;
    }
    return applied;
}

int axo_apply_processors(float* row, uint32_t V, const axs_sampling_params* p,
                         const uint32_t* hist, uint32_t nhist,
                         const uint32_t* mask_words,
                         const uint32_t* bias_ids, const float* bias_vals,
                         uint32_t nbias) {
    workspace w;
    if (!ws_init(&w, V)) return -1;
    int r = apply_processors_ws(row, V, p, hist, nhist, mask_words, bias_ids,
                                bias_vals, nbias, &w);
    ws_free(&w);
    return r;
}

/* sort order of apply_top_k_top_p (sampling.rs:928-932):
 * probability descending (f32::total_cmp; probabilities are non-negative and
 * never NaN here), then id ascending. */
static __thread const float* t_sort_p;
static __thread const uint32_t* t_sort_id;
static int cmp_cand(const void* a, const void* b) {
    uint32_t ia = *(const uint32_t*)a, ib = *(const uint32_t*)b;
    float pa = t_sort_p[ia], pb = t_sort_p[ib];
    if (pa > pb) return -1;
    if (pa < pb) return 1;
    uint32_t ta = t_sort_id[ia], tb = t_sort_id[ib];
    return ta < tb ? -1 : (ta > tb ? 1 : 0);
}

static void sort_candidates(uint32_t* cid, float* cp, uint32_t n, workspace* w) {
    for (uint32_t i = 0; i < n; ++i) w->order[i] = i;
    t_sort_p = cp;
    t_sort_id = cid;
    qsort(w->order, n, sizeof(uint32_t), cmp_cand);
    /* apply the permutation through the free buffers */
    uint32_t* tid = w->counts;  /* borrowed: restored to zero below */
    float* tp = w->probs;
    for (uint32_t i = 0; i < n; ++i) {
        tid[i] = cid[w->order[i]];
        tp[i] = cp[w->order[i]];
    }
    memcpy(cid, tid, n * sizeof(uint32_t));
    memcpy(cp, tp, n * sizeof(float));
    memset(tid, 0, n * sizeof(uint32_t));
}

static double ulp_of(float x) {
    float a = fabsf(x);
    float nx = nextafterf(a, INFINITY);
    return (double)nx - (double)a;
}

/* apply_top_k_top_p (sampling.rs:922-952), recording the nucleus margins. */
static uint32_t apply_top_k_top_p(uint32_t* cid, float* cp, uint32_t n, uint32_t top_k,
                                  float top_p, workspace* w, axo_explain* ex,
                                  int* sorted, const float* L) {
    *sorted = 0;
    int filters_enabled = top_k > 0 || top_p < 1.0f;
    if (!filters_enabled) {
        if (ex) ex->n_nucleus = n;
        return n;
    }
    sort_candidates(cid, cp, n, w);
    *sorted = 1;
    uint32_t keep_n = n;
    if (isfinite(top_p) && top_p > 0.0f && top_p < 1.0f) {
        float total = 0.0f;
        for (uint32_t i = 0; i < n; ++i) total += cp[i];
        float cutoff = top_p * total;
        float cum = 0.0f, prev = 0.0f;
        uint32_t keep = 0;
        for (uint32_t i = 0; i < n; ++i) {
            prev = cum;
            cum += cp[i];
            keep += 1;
            if (cum >= cutoff) break;
        }
        keep_n = keep > 1 ? keep : 1;
        if (ex) {
            ex->total = total;
            ex->cutoff = cutoff;
            double up = (double)cum - (double)cutoff;
            double lo = keep > 1 ? (double)cutoff - (double)prev : INFINITY;
            double mg = (up < lo ? up : lo) / (double)total;
            ex->margin_nucleus = mg;
        }
    }
    if (ex) ex->n_nucleus = keep_n;
    uint32_t kept = keep_n;
    if (top_k > 0) {
        uint32_t k = top_k > 1 ? top_k : 1;
        if (kept > k) kept = k;
    }
    if (ex) {
        if (ex->margin_nucleus < 1e-6 && (top_k == 0 || keep_n <= top_k))
            ex->boundary |= AXS_FLAG_NEAR_NUCLEUS;
        /* probabilities within 2 ulp across the cut, from DIFFERENT logits:
         * a one-ulp difference between two exp implementations could swap
         * them.  Equal logits give equal probabilities everywhere and are
         * ordered by id on both sides, so they are not a boundary. */
        if (kept < n && L && L[cid[kept - 1]] != L[cid[kept]]) {
            double d = (double)cp[kept - 1] - (double)cp[kept];
            double u = ulp_of(cp[kept - 1]);
            ex->margin_tie = u > 0 ? d / u : INFINITY;
            if (d <= 2.0 * u) ex->boundary |= AXS_FLAG_NEAR_TIE;
        }
    }
    return kept;
}

typedef struct {
    const float* supplied;
    uint64_t* rng;
    int used;
} usrc;

static float next_uniform(usrc* s) {
    s->used = 1;
    if (s->supplied) return *s->supplied;
    return axo_xorshift64_next_f32(s->rng);
}

static float logprob_of(float prob) {
    return fmaxf(logf(fmaxf(prob, 1e-37f)), -30.0f);
}

float axo_logprob_of(float prob) { return logprob_of(prob); }

static void ex_init(axo_explain* ex) {
    memset(ex, 0, sizeof(*ex));
    ex->margin_draw = INFINITY;
    ex->margin_nucleus = INFINITY;
    ex->margin_minp = INFINITY;
    ex->margin_tie = INFINITY;
    ex->logprob = NAN;
}

/* The draw scan shared by both branches: first index whose running f32 sum
 * reaches u * F (sampling.rs:256-263, :302-309), else the last maximum
 * (max_by total_cmp, :264-269, :310-315). */
static uint32_t draw_scan(const uint32_t* ids, const float* ps, uint32_t n, float F,
                          float u, axo_explain* ex) {
    float thr = u * F;
    float cum = 0.0f, prev = 0.0f;
    for (uint32_t i = 0; i < n; ++i) {
        prev = cum;
        cum += ps[i];
        if (cum >= thr) {
            if (ex) {
                double up = (double)cum - (double)thr;
                double lo = i > 0 ? (double)thr - (double)prev : INFINITY;
                ex->margin_draw = (up < lo ? up : lo) / (double)F;
                if (ex->margin_draw < 1e-6) ex->boundary |= AXS_FLAG_NEAR_DRAW;
                ex->thr = thr;
                ex->logprob = logprob_of(ps[i] / F);
            }
            return ids ? ids[i] : i;
        }
    }
    uint32_t best = 0;
    float bp = -INFINITY;
    for (uint32_t i = 0; i < n; ++i)
        if (ps[i] >= bp) { bp = ps[i]; best = i; }
    if (ex) ex->thr = thr;
    return ids ? ids[best] : best;
}

static uint32_t sample_row_ws(const float* logits, uint32_t V, const axs_sampling_params* p,
                              const uint32_t* hist, uint32_t nhist,
                              const uint32_t* mask_words, const uint32_t* bias_ids,
                              const float* bias_vals, uint32_t nbias, usrc* us,
                              axo_explain* ex, uint32_t* kept_ids, uint32_t kept_cap,
                              workspace* w) {
    axo_explain dummy;
    if (!ex) ex = &dummy;
    ex_init(ex);
    if (V == 0) {
        ex->path = AXO_PATH_EMPTY;
        return 0;
    }
    const float* L = logits;
    /* copy-on-write processors (sampling.rs:216-235) */
    int any = ((uses_rep(p) || p->no_repeat_ngram_size > 0) && nhist > 0) ||
              (uses_presence_freq(p) && nhist > 0) || (bias_ids && nbias > 0) ||
              mask_words != NULL;
    if (any) {
        memcpy(w->row, logits, (size_t)V * sizeof(float));
        apply_processors_ws(w->row, V, p, hist, nhist, mask_words, bias_ids, bias_vals,
                            nbias, w);
        L = w->row;
    }
    if (p->temperature <= 0.0f) {            /* sampling.rs:236-238 */
        ex->path = AXO_PATH_GREEDY;
        ex->token = axo_argmax_f32(L, V);
        ex->n_kept = 1;
        if (kept_ids && kept_cap) kept_ids[0] = ex->token;
        return ex->token;
    }
    float inv = 1.0f / p->temperature;        /* sampling.rs:240 */
    float m = -INFINITY;                      /* sampling.rs:241 */
    for (uint32_t i = 0; i < V; ++i) m = fmaxf(m, L[i]);
    ex->m = m;

    if (p->top_k == 0 && p->top_p >= 1.0f && !uses_min_p(p)) {   /* :246-270 */
        float S = 0.0f;
        for (uint32_t i = 0; i < V; ++i) {
            float q = expf((L[i] - m) * inv);
            w->probs[i] = isfinite(q) ? q : 0.0f;
            S += w->probs[i];
        }
        if (S == 0.0f || !isfinite(S)) {
            ex->path = AXO_PATH_FALLBACK;
            ex->token = axo_argmax_f32(L, V);
            ex->n_kept = 1;
            if (kept_ids && kept_cap) kept_ids[0] = ex->token;
            return ex->token;
        }
        ex->path = AXO_PATH_FAST;
        ex->n_cand = ex->n_nucleus = ex->n_kept = V;
        ex->F = S;
        float u = next_uniform(us);
        ex->drew = 1;
        ex->u = u;
        if (kept_ids)
            for (uint32_t i = 0; i < V && i < kept_cap; ++i) kept_ids[i] = i;
        ex->token = draw_scan(NULL, w->probs, V, S, u, ex);
        return ex->token;
    }

    /* filtered path (:273-316) */
    float S = 0.0f;
    for (uint32_t i = 0; i < V; ++i) {
        float q = expf((L[i] - m) * inv);
        w->cid[i] = i;
        w->cp[i] = isfinite(q) ? q : 0.0f;
        S += w->cp[i];
    }
    if (S == 0.0f || !isfinite(S)) {
        ex->path = AXO_PATH_FALLBACK;
        ex->token = axo_argmax_f32(L, V);
        ex->n_kept = 1;
        if (kept_ids && kept_cap) kept_ids[0] = ex->token;
        return ex->token;
    }
    uint32_t n = V;
    if (uses_min_p(p)) {                          /* :283-294 */
        float maxp = 0.0f;
        for (uint32_t i = 0; i < n; ++i) maxp = fmaxf(maxp, w->cp[i]);
        float cutoff = p->min_p * maxp;
        double mg = INFINITY;
        uint32_t k = 0;
        for (uint32_t i = 0; i < n; ++i) {
            double d = fabs((double)w->cp[i] - (double)cutoff) / (double)cutoff;
            if (d < mg) mg = d;
            if (w->cp[i] >= cutoff) {
                w->cid[k] = w->cid[i];
                w->cp[k] = w->cp[i];
                ++k;
            }
        }
        ex->margin_minp = mg;
        if (mg < 1e-6) ex->boundary |= AXS_FLAG_NEAR_MINP;
        n = k;
        if (n == 0) {
            ex->path = AXO_PATH_FALLBACK;
            ex->token = axo_argmax_f32(L, V);
            ex->n_kept = 1;
            if (kept_ids && kept_cap) kept_ids[0] = ex->token;
            return ex->token;
        }
    }
    ex->n_cand = n;
    int sorted = 0;
    uint32_t kept = apply_top_k_top_p(w->cid, w->cp, n, p->top_k, p->top_p, w, ex, &sorted, L);
    ex->sorted = (uint32_t)sorted;
    ex->n_kept = kept;
    float F = 0.0f;                               /* :297-300 */
    for (uint32_t i = 0; i < kept; ++i) F += w->cp[i];
    if (F == 0.0f || !isfinite(F)) {
        ex->path = AXO_PATH_FALLBACK;
        ex->token = axo_argmax_f32(L, V);
        ex->n_kept = 1;
        if (kept_ids && kept_cap) kept_ids[0] = ex->token;
        return ex->token;
    }
    ex->path = AXO_PATH_FILTERED;
    ex->F = F;
    if (kept_ids)
        for (uint32_t i = 0; i < kept && i < kept_cap; ++i) kept_ids[i] = w->cid[i];
    float u = next_uniform(us);
    ex->drew = 1;
    ex->u = u;
    ex->token = draw_scan(w->cid, w->cp, kept, F, u, ex);
    return ex->token;
}

uint32_t axo_sample_row(const float* logits, uint32_t V, const axs_sampling_params* p,
                        const uint32_t* hist, uint32_t nhist, const uint32_t* mask_words,
                        const uint32_t* bias_ids, const float* bias_vals, uint32_t nbias,
                        const float* u_supplied, uint64_t* rng, axo_explain* explain,
                        uint32_t* kept_ids, uint32_t kept_cap) {
    workspace w;
    if (!ws_init(&w, V)) return AXS_NONE_U32;
    usrc us = {u_supplied, rng, 0};
    uint32_t t = sample_row_ws(logits, V, p, hist, nhist, mask_words, bias_ids, bias_vals,
                               nbias, &us, explain, kept_ids, kept_cap, &w);
    ws_free(&w);
    return t;
}

/* ------------------------------------------------------------------------ */
/* batched host sampler                                                      */
/* ------------------------------------------------------------------------ */

typedef struct {
    const void* logits; int dtype; uint32_t B, V; uint64_t stride;
    const axs_sampling_params* params;
    const uint32_t* hist; const int64_t* hist_off;
    const uint32_t* mask; uint64_t mask_stride;
    const uint32_t* bias_ids; const float* bias_vals; const int64_t* bias_off;
    const float* uniforms;
    uint32_t* out_ids; axo_explain* explain; uint32_t* kept_ids; uint32_t kept_cap;
    int tid, nthreads; int err;
} batch_job;

static void* batch_worker(void* arg) {
    batch_job* j = (batch_job*)arg;
    workspace w;
    if (!ws_init(&w, j->V)) { j->err = 1; return NULL; }
    float* rowbuf = NULL;
    if (j->dtype == AXS_DTYPE_BF16) rowbuf = (float*)malloc((size_t)(j->V ? j->V : 1) * 4);
    uint32_t per = (j->B + j->nthreads - 1) / j->nthreads;
    uint32_t r0 = per * j->tid, r1 = r0 + per;
    if (r1 > j->B) r1 = j->B;
    for (uint32_t r = r0; r < r1; ++r) {
        const float* row;
        if (j->dtype == AXS_DTYPE_BF16) {
            axo_bf16_to_f32((const uint16_t*)j->logits + r * j->stride, rowbuf, j->V);
            row = rowbuf;
        } else {
            row = (const float*)j->logits + r * j->stride;
        }
        const axs_sampling_params* p = &j->params[r];
        const uint32_t* h = NULL; uint32_t nh = 0;
        if (j->hist && j->hist_off) {
            h = j->hist + j->hist_off[r];
            nh = (uint32_t)(j->hist_off[r + 1] - j->hist_off[r]);
        }
        const uint32_t* bi = NULL; const float* bv = NULL; uint32_t nb = 0;
        if (j->bias_ids && j->bias_off) {
            bi = j->bias_ids + j->bias_off[r];
            bv = j->bias_vals + j->bias_off[r];
            nb = (uint32_t)(j->bias_off[r + 1] - j->bias_off[r]);
        }
        const uint32_t* mk = j->mask ? j->mask + r * j->mask_stride : NULL;
        float u = j->uniforms ? j->uniforms[r] : axo_philox_uniform(p->seed, r, p->step, 0, 0);
        usrc us = {&u, NULL, 0};
        j->out_ids[r] = sample_row_ws(row, j->V, p, h, nh, mk, bi, bv, nb, &us,
                                      j->explain ? &j->explain[r] : NULL,
                                      j->kept_ids ? j->kept_ids + (uint64_t)r * j->kept_cap : NULL,
                                      j->kept_cap, &w);
    }
    free(rowbuf);
    ws_free(&w);
    return NULL;
}

int axo_sample_batch(const void* logits, int dtype, uint32_t B, uint32_t V, uint64_t stride,
                     const axs_sampling_params* params, const uint32_t* hist,
                     const int64_t* hist_off, const uint32_t* mask_words,
                     uint64_t mask_stride, const uint32_t* bias_ids, const float* bias_vals,
                     const int64_t* bias_off, const float* uniforms, uint32_t* out_ids,
                     axo_explain* explain, uint32_t* kept_ids, uint32_t kept_cap,
                     int nthreads) {
    if (nthreads < 1) nthreads = 1;
    if ((uint32_t)nthreads > B && B > 0) nthreads = (int)B;
    batch_job* jobs = (batch_job*)calloc((size_t)nthreads, sizeof(batch_job));
    pthread_t* th = (pthread_t*)calloc((size_t)nthreads, sizeof(pthread_t));
    if (!jobs || !th) { free(jobs); free(th); return 1; }
    for (int t = 0; t < nthreads; ++t) {
        batch_job* j = &jobs[t];
        j->logits = logits; j->dtype = dtype; j->B = B; j->V = V; j->stride = stride;
        j->params = params; j->hist = hist; j->hist_off = hist_off;
        j->mask = mask_words; j->mask_stride = mask_stride;
        j->bias_ids = bias_ids; j->bias_vals = bias_vals; j->bias_off = bias_off;
        j->uniforms = uniforms; j->out_ids = out_ids; j->explain = explain;
        j->kept_ids = kept_ids; j->kept_cap = kept_cap; j->tid = t; j->nthreads = nthreads;
    }
    int err = 0;
    if (nthreads == 1) {
        batch_worker(&jobs[0]);
    } else {
        for (int t = 0; t < nthreads; ++t) pthread_create(&th[t], NULL, batch_worker, &jobs[t]);
        for (int t = 0; t < nthreads; ++t) pthread_join(th[t], NULL);
    }
    for (int t = 0; t < nthreads; ++t) err |= jobs[t].err;
    free(jobs);
    free(th);
    return err;
}

/* ------------------------------------------------------------------------ */
/* token distributions (MTP)                                                 */
/* ------------------------------------------------------------------------ */

/* TokenDistribution::new (sampling.rs:128-144): keep positive finite
 * entries, divide by their f32 sum in entry order.  Returns count or -1. */
static int distribution_new(uint32_t* ids, float* probs, uint32_t n) {
    uint32_t k = 0;
    for (uint32_t i = 0; i < n; ++i)
        if (probs[i] > 0.0f && isfinite(probs[i])) { ids[k] = ids[i]; probs[k] = probs[i]; ++k; }
    if (k == 0) return -1;
    float sum = 0.0f;
    for (uint32_t i = 0; i < k; ++i) sum += probs[i];
    if (sum <= 0.0f || !isfinite(sum)) return -1;
    for (uint32_t i = 0; i < k; ++i) probs[i] = probs[i] / sum;
    return (int)k;
}

int axo_distribution_new(uint32_t* ids, float* probs, uint32_t n) {
    return distribution_new(ids, probs, n);
}

static int single_entry(uint32_t id, uint32_t* ids, float* probs, uint32_t cap) {
    if (cap < 1) return -2;
    ids[0] = id;
    probs[0] = 1.0f;
    return distribution_new(ids, probs, 1);
}

static int token_distribution_ws(const float* logits, uint32_t V, const axs_sampling_params* p,
                                 uint32_t* ids, float* probs, uint32_t cap, workspace* w) {
    if (V == 0) return -1;
    if (p->temperature <= 0.0f) return single_entry(axo_argmax_f32(logits, V), ids, probs, cap);
    float inv = 1.0f / p->temperature;
    float m = -INFINITY;
    for (uint32_t i = 0; i < V; ++i) m = fmaxf(m, logits[i]);
    float total = 0.0f;
    for (uint32_t i = 0; i < V; ++i) {
        float q = expf((logits[i] - m) * inv);
        w->cid[i] = i;
        w->cp[i] = isfinite(q) ? q : 0.0f;
        total += w->cp[i];
    }
    if (total == 0.0f || !isfinite(total))
        return single_entry(axo_argmax_f32(logits, V), ids, probs, cap);
    uint32_t n = V;
    if (uses_min_p(p)) {
        float maxp = 0.0f;
        for (uint32_t i = 0; i < n; ++i) maxp = fmaxf(maxp, w->cp[i]);
        float cutoff = p->min_p * maxp;
        uint32_t k = 0;
        for (uint32_t i = 0; i < n; ++i)
            if (w->cp[i] >= cutoff) { w->cid[k] = w->cid[i]; w->cp[k] = w->cp[i]; ++k; }
        n = k;
        if (n == 0) return single_entry(axo_argmax_f32(logits, V), ids, probs, cap);
    }
    int sorted = 0;
    if (p->top_k > 0 || p->top_p < 1.0f)
        n = apply_top_k_top_p(w->cid, w->cp, n, p->top_k, p->top_p, w, NULL, &sorted, NULL);
    float fs = 0.0f;
    for (uint32_t i = 0; i < n; ++i) fs += w->cp[i];
    if (fs == 0.0f || !isfinite(fs))
        return single_entry(axo_argmax_f32(logits, V), ids, probs, cap);
    /* TokenDistribution::new drops non-positive entries first */
    uint32_t k = 0;
    for (uint32_t i = 0; i < n; ++i)
        if (w->cp[i] > 0.0f && isfinite(w->cp[i])) ++k;
    if (k > cap) return -2;
    k = 0;
    for (uint32_t i = 0; i < n; ++i)
        if (w->cp[i] > 0.0f && isfinite(w->cp[i])) { ids[k] = w->cid[i]; probs[k] = w->cp[i]; ++k; }
    return distribution_new(ids, probs, k);
}

int axo_token_distribution(const float* logits, uint32_t V, const axs_sampling_params* p,
                           uint32_t* ids, float* probs, uint32_t cap) {
    workspace w;
    if (!ws_init(&w, V)) return -3;
    int r = token_distribution_ws(logits, V, p, ids, probs, cap, &w);
    ws_free(&w);
    return r;
}

/* sample_from_token_distribution (sampling.rs:709-731) */
uint32_t axo_sample_from_distribution(const uint32_t* ids, const float* probs, uint32_t n,
                                      float u) {
    float total = 0.0f;
    for (uint32_t i = 0; i < n; ++i) total += probs[i];
    if (total <= 0.0f || !isfinite(total)) return AXS_NONE_U32;
    float thr = u * total;
    float cum = 0.0f;
    for (uint32_t i = 0; i < n; ++i) {
        cum += probs[i];
        if (cum >= thr) return ids[i];
    }
    uint32_t best = AXS_NONE_U32;
    float bp = -INFINITY;
    for (uint32_t i = 0; i < n; ++i)
        if (probs[i] >= bp) { bp = probs[i]; best = ids[i]; }
    return best;
}

float axo_distribution_prob(const uint32_t* ids, const float* probs, uint32_t n,
                            uint32_t token) {
    for (uint32_t i = 0; i < n; ++i)
        if (ids[i] == token) return probs[i];
    return 0.0f;
}

static int cmp_u32_pair(const void* a, const void* b) {
    uint32_t x = *(const uint32_t*)a, y = *(const uint32_t*)b;
    return x < y ? -1 : (x > y ? 1 : 0);
}

/* sample_residual_token_distribution (sampling.rs:733-752): BTreeMap over the
 * union of ids (ascending), r = max(P - Q, 0), positive finite entries,
 * normalised; an empty residual falls back to the target. */
uint32_t axo_sample_residual(const uint32_t* t_ids, const float* t_probs, uint32_t tn,
                             const uint32_t* d_ids, const float* d_probs, uint32_t dn,
                             float u) {
    uint32_t cap = tn + dn;
    uint32_t (*pairs)[2] = malloc((size_t)(cap ? cap : 1) * sizeof(*pairs));
    float* val = malloc((size_t)(cap ? cap : 1) * sizeof(float));
    uint32_t* rid = malloc((size_t)(cap ? cap : 1) * sizeof(uint32_t));
    float* rp = malloc((size_t)(cap ? cap : 1) * sizeof(float));
    /* the map keys: union of target and draft ids, sorted */
    uint32_t* keys = malloc((size_t)(cap ? cap : 1) * sizeof(uint32_t));
    uint32_t nk = 0;
    for (uint32_t i = 0; i < tn; ++i) keys[nk++] = t_ids[i];
    for (uint32_t i = 0; i < dn; ++i) keys[nk++] = d_ids[i];
    qsort(keys, nk, sizeof(uint32_t), cmp_u32_pair);
    uint32_t nu = 0;
    for (uint32_t i = 0; i < nk; ++i)
        if (nu == 0 || keys[nu - 1] != keys[i]) keys[nu++] = keys[i];
    (void)pairs;
    for (uint32_t k = 0; k < nu; ++k) {
        /* insert(target) — later duplicates overwrite, as BTreeMap::insert */
        int present = 0;
        float v = 0.0f;
        for (uint32_t i = 0; i < tn; ++i)
            if (t_ids[i] == keys[k]) { v = t_probs[i]; present = 1; }
        for (uint32_t i = 0; i < dn; ++i)
            if (d_ids[i] == keys[k]) {
                if (!present) { v = 0.0f; present = 1; }
                v = fmaxf(v - d_probs[i], 0.0f);
            }
        val[k] = v;
    }
    uint32_t n = 0;
    for (uint32_t k = 0; k < nu; ++k)
        if (val[k] > 0.0f && isfinite(val[k])) { rid[n] = keys[k]; rp[n] = val[k]; ++n; }
    int dn2 = n > 0 ? distribution_new(rid, rp, n) : -1;
    uint32_t tok;
    if (dn2 < 0) {
        tok = axo_sample_from_distribution(t_ids, t_probs, tn, u);
    } else {
        tok = axo_sample_from_distribution(rid, rp, (uint32_t)dn2, u);
    }
    free(pairs); free(val); free(rid); free(rp); free(keys);
    return tok;
}

/* full_vocab_token_logprob (sampling.rs:761-787) */
float axo_full_vocab_token_logprob(const float* logits, uint32_t n, uint32_t token,
                                   float temperature) {
    if (n == 0 || token >= n) return -30.0f;
    if (temperature <= 0.0f) return axo_argmax_f32(logits, n) == token ? 0.0f : -INFINITY;
    float inv = 1.0f / temperature;
    float m = -INFINITY;
    for (uint32_t i = 0; i < n; ++i) m = fmaxf(m, logits[i]);
    float unnorm = expf((logits[token] - m) * inv);
    float sum = 0.0f;
    for (uint32_t i = 0; i < n; ++i) {
        float q = expf((logits[i] - m) * inv);
        sum += isfinite(q) ? q : 0.0f;
    }
    if (sum <= 0.0f || !isfinite(sum)) return -30.0f;
    return fmaxf(logf(fmaxf(unnorm / sum, 1e-37f)), -30.0f);
}

/* Top-N log-probabilities (a build extension over full_vocab_token_logprob,
 * sampling.rs:761-787; the reference's server rejects top_logprobs,
 * crates/ax-engine-server/src/openai/requests.rs:1283-1298): the n ids with
 * the largest unnormalised p = exp((l - max) / T) (non-finite p as 0), ties
 * to the lower id, each with full_vocab_token_logprob.  T <= 0 lists only
 * the first maximum (log-probability 0); unused slots hold id 0xFFFFFFFF and
 * -inf. */
typedef struct { float p; uint32_t id; } topn_ent;

static int topn_cmp(const void* a, const void* b) {
    const topn_ent* x = (const topn_ent*)a;
    const topn_ent* y = (const topn_ent*)b;
    if (x->p != y->p) return x->p > y->p ? -1 : 1;
    return x->id < y->id ? -1 : (x->id > y->id ? 1 : 0);
}

void axo_top_logprobs(const float* logits, uint32_t V, float temperature, uint32_t n, uint32_t* out_ids,
                      float* out_lp) {
    for (uint32_t k = 0; k < n; ++k) {
        out_ids[k] = 0xFFFFFFFFu;
        out_lp[k] = -INFINITY;
    }
    if (V == 0 || n == 0) return;
    if (temperature <= 0.0f) {
        out_ids[0] = axo_argmax_f32(logits, V);
        out_lp[0] = 0.0f;
        return;
    }
    float inv = 1.0f / temperature;
    float m = -INFINITY;
    for (uint32_t i = 0; i < V; ++i) m = fmaxf(m, logits[i]);
    topn_ent* e = (topn_ent*)malloc(sizeof(topn_ent) * V);
    for (uint32_t i = 0; i < V; ++i) {
        float q = expf((logits[i] - m) * inv);
        e[i].p = isfinite(q) ? q : 0.0f;
        e[i].id = i;
    }
    qsort(e, V, sizeof(topn_ent), topn_cmp);
    uint32_t k_n = n < V ? n : V;
    for (uint32_t k = 0; k < k_n; ++k) {
        out_ids[k] = e[k].id;
        out_lp[k] = axo_full_vocab_token_logprob(logits, V, e[k].id, temperature);
    }
    free(e);
}

/* The target probability of one draft token under the production MTP law:
 * compute_mtp_target_probs (runner/mod.rs:12025-12159) followed by
 * LazyTargetProbs::extract_cpu_into (runner/mod.rs:11836-11937) and
 * filtered_target_token_probability (runner/mod.rs:11943-12001).  Returns NaN
 * when the reference computes none (T <= 0: greedy comparisons).
 *
 * The row's softmax is full_vocab_token_logprob's statement of it
 * (sampling.rs:761-787): q_j = exp((l_j - max) / T) with non-finite q as 0,
 * S their f32 sum in index order, p_j = q_j / S (MLX's softmax reduction
 * order is not reproducible; this is the reference's own CPU statement).
 * Then, as compute_mtp_target_probs chooses:
 *   topk_opt > 0 (mtp_target_softmax_topk): the topk_opt largest p, top_p and
 *     min_p of the target (LazyTargetProbs::TopK);
 *   else target top_k > 0 or top_p < 1 (the draft filter is the target's
 *     own, runner/mod.rs:8643-8646): the top_k (or V) largest p, top_p,
 *     min_p (TopK);
 *   else min_p in use: every p, min_p (FullRows ->
 *     filtered_target_token_probability(row, t, min_p, 1.0, 0));
 *   else p_t itself (Full).
 * The filtered cases keep p > 0, then p >= min_p * max p, order by
 * (p desc, id asc), cut where the f32 running sum first reaches top_p
 * (0 < top_p < 1; at least one entry) and return p_t over the kept set's
 * f32 sum in that order, 0 for a token outside it.  The top-k set is taken
 * in the same order (MLX's argpartition leaves ties at the k-th value in an
 * unspecified order; here the lower id wins). */
static int prodp_cmp(const void* a, const void* b) {
    const topn_ent* x = (const topn_ent*)a;
    const topn_ent* y = (const topn_ent*)b;
    if (x->p != y->p) return x->p > y->p ? -1 : 1;
    return x->id < y->id ? -1 : (x->id > y->id ? 1 : 0);
}

float axo_mtp_target_prob(const float* logits, uint32_t V, float temperature, float top_p, uint32_t top_k,
                          int has_min_p, float min_p, uint32_t topk_opt, uint32_t token) {
    if (!(temperature > 0.0f)) return NAN;
    if (V == 0) return 0.0f;
    const float inv = 1.0f / temperature;
    float m = -INFINITY;
    for (uint32_t i = 0; i < V; ++i) m = fmaxf(m, logits[i]);
    float* q = (float*)malloc(sizeof(float) * V);
    float S = 0.0f;
    for (uint32_t i = 0; i < V; ++i) {
        const float e = expf((logits[i] - m) * inv);
        q[i] = isfinite(e) ? e : 0.0f;
        S += q[i];
    }
    float out = 0.0f;
    const int uses_min_p = has_min_p && isfinite(min_p) && min_p > 0.0f;
    if (!(S > 0.0f) || !isfinite(S)) {
        free(q);
        return 0.0f;
    }
    if (topk_opt == 0 && top_k == 0 && !(top_p < 1.0f) && !uses_min_p) {
        out = token < V ? q[token] / S : 0.0f;  /* Full: the softmax value itself */
        free(q);
        return out;
    }
    uint32_t K = V;
    float tp = top_p;
    if (topk_opt > 0) K = topk_opt < V ? topk_opt : V;
    else if (top_k > 0 || top_p < 1.0f) K = (top_k > 0 && top_k < V) ? top_k : V;
    else tp = 1.0f;  /* FullRows: min_p only */
    topn_ent* c = (topn_ent*)malloc(sizeof(topn_ent) * V);
    uint32_t n = 0;
    for (uint32_t i = 0; i < V; ++i) {
        const float p = q[i] / S;
        if (p > 0.0f && isfinite(p)) { c[n].p = p; c[n].id = i; ++n; }
    }
    qsort(c, n, sizeof(topn_ent), prodp_cmp);
    if (n > K) n = K;  /* the top-k set */
    if (uses_min_p && n > 0) {
        const float cutoff = min_p * c[0].p;  /* c[0].p: the largest */
        uint32_t w = 0;
        for (uint32_t k = 0; k < n; ++k)
            if (c[k].p >= cutoff) c[w++] = c[k];
        n = w;
    }
    if (isfinite(tp) && tp > 0.0f && tp < 1.0f) {
        float cum = 0.0f;
        uint32_t keep = 0;
        for (uint32_t k = 0; k < n; ++k) {
            cum += c[k].p;
            ++keep;
            if (cum >= tp) break;
        }
        n = keep > 0 ? keep : (n > 0 ? 1 : 0);
    }
    float sum = 0.0f;
    for (uint32_t k = 0; k < n; ++k) sum += c[k].p;
    for (uint32_t k = 0; k < n; ++k)
        if (c[k].id == token) {
            out = fmaxf(c[k].p / fmaxf(sum, 1e-37f), 0.0f);
            break;
        }
    free(c);
    free(q);
    return out;
}

/* think_soft_close_in_top_k (crates/ax-engine-mlx/src/ngram_accel.rs:1609-1640):
 * the reference's single pass, kept literally: the first `rank` logits taken
 * as they come and stably sorted descending by total order (f32::total_cmp);
 * afterwards a logit replaces the last entry only when it is greater (IEEE
 * `>`), the array re-sorted stably; membership of the target at the end. */
static int32_t total_key(float x);

int axo_soft_close_in_top_k(const float* logits, uint32_t n, uint32_t target, uint32_t rank) {
    if (rank == 0 || n == 0) return 0;
    if (target >= n) return 0;
    uint32_t* idx = (uint32_t*)malloc(sizeof(uint32_t) * rank);
    float* val = (float*)malloc(sizeof(float) * rank);
    uint32_t len = 0;
    for (uint32_t i = 0; i < n; ++i) {
        float v = logits[i];
        if (len < rank) {
            idx[len] = i;
            val[len] = v;
            ++len;
            if (len == rank) {
                /* stable insertion sort, descending by total order */
                for (uint32_t a = 1; a < len; ++a) {
                    uint32_t ti = idx[a];
                    float tv = val[a];
                    uint32_t b = a;
                    while (b > 0 && total_key(tv) > total_key(val[b - 1])) {
                        idx[b] = idx[b - 1];
                        val[b] = val[b - 1];
                        --b;
                    }
                    idx[b] = ti;
                    val[b] = tv;
                }
            }
            continue;
        }
        if (v > val[rank - 1]) {
            /* the new last entry, moved up past every entry it exceeds in
             * total order (a stable re-sort of an otherwise sorted array) */
            uint32_t b = rank - 1;
            while (b > 0 && total_key(v) > total_key(val[b - 1])) {
                idx[b] = idx[b - 1];
                val[b] = val[b - 1];
                --b;
            }
            idx[b] = i;
            val[b] = v;
        }
    }
    int hit = 0;
    for (uint32_t a = 0; a < len; ++a) hit |= idx[a] == target;
    free(idx);
    free(val);
    return hit;
}

/* ------------------------------------------------------------------------ */
/* MTP acceptance                                                            */
/* ------------------------------------------------------------------------ */

#define SRC_NONE 0
#define SRC_MTP 1
#define SRC_GEMMA 2
#define SRC_NGRAM 3
#define SRC_HYBRID 4

typedef struct { uint64_t* rng; const float* u; uint32_t n, i; } ustream;

static float ustream_next(ustream* s) {
    if (s->rng) return axo_xorshift64_next_f32(s->rng);
    if (s->i < s->n) return s->u[s->i++];
    return 1.0f;
}

uint32_t axo_mtp_accept_count(uint32_t n, const uint32_t* pending,
                              const float* pending_log_probs, uint32_t n_log_probs,
                              const uint32_t* d_ids, const float* d_probs,
                              const int64_t* d_off, uint32_t n_draft_dists,
                              const uint32_t* sources, uint32_t n_sources,
                              const float* target_probs,
                              const uint32_t* t_ids, const float* t_probs,
                              const int64_t* t_off, uint32_t n_target_dists,
                              const uint32_t* predicted, uint64_t* rng,
                              const float* uniforms, uint32_t n_uniforms,
                              float draft_temperature, float target_temperature,
                              int model_mode, int ngram_mode,
                              uint32_t* all_accepted, uint32_t* correction) {
    ustream us = {rng, uniforms, n_uniforms, 0};
    uint32_t ac = 0;
    uint32_t dist_index = 0;
    for (uint32_t i = 0; i < n; ++i) {
        uint32_t source = (i < n_sources && sources[i] != SRC_NONE) ? sources[i] : SRC_MTP;
        int has_draft_distribution = source == SRC_MTP || source == SRC_GEMMA || source == SRC_HYBRID;
        if (source == SRC_NGRAM && ngram_mode == 2) {
            if (predicted[i] == pending[i]) { ac++; continue; }
            *all_accepted = 0;
            *correction = predicted[i];
            return ac;
        }
        if (has_draft_distribution && model_mode == 0) {
            if (predicted[i] == pending[i]) { ac++; dist_index++; continue; }
            *all_accepted = 0;
            *correction = predicted[i];
            return ac;
        }
        int can_rs = i < n_log_probs && isfinite(pending_log_probs[i]) && target_probs != NULL;
        if (can_rs) {
            float p_target = fmaxf(target_probs[i], 0.0f);
            float lp = pending_log_probs[i];
            int is_mtp_source = source != SRC_NGRAM;
            float lps = lp;
            if (is_mtp_source && draft_temperature > 0.0f && target_temperature > 0.0f &&
                fabsf(draft_temperature - target_temperature) > 1e-6f)
                lps = lp * (draft_temperature / target_temperature);
            float p_draft = fmaxf(expf(lps), 1e-37f);
            float accept_prob = fminf(p_target / p_draft, 1.0f);
            if (ustream_next(&us) < accept_prob) {
                ac++;
                if (has_draft_distribution) dist_index++;
            } else {
                uint32_t corr = AXS_NONE_U32;
                if (has_draft_distribution && t_ids && i < n_target_dists &&
                    dist_index < n_draft_dists) {
                    float u = ustream_next(&us);
                    corr = axo_sample_residual(
                        t_ids + t_off[i], t_probs + t_off[i], (uint32_t)(t_off[i + 1] - t_off[i]),
                        d_ids + d_off[dist_index], d_probs + d_off[dist_index],
                        (uint32_t)(d_off[dist_index + 1] - d_off[dist_index]), u);
                }
                *all_accepted = 0;
                *correction = corr;
                return ac;
            }
        } else {
            if (predicted[i] == pending[i]) {
                ac++;
                if (has_draft_distribution) dist_index++;
            } else {
                *all_accepted = 0;
                *correction = predicted[i];
                return ac;
            }
        }
    }
    *all_accepted = ac == n;
    *correction = AXS_NONE_U32;
    return ac;
}

#define DIST_CAP_MAX (1u << 20)

uint32_t axo_mtp_verify_seq(const float* target, const float* draft, uint32_t V,
                            uint32_t depth, const uint32_t* draft_ids,
                            const axs_sampling_params* tparams,
                            const axs_sampling_params* dparams, const float* uniforms,
                            uint32_t* out_ids, uint32_t* accept_count, uint32_t* flags) {
    workspace w;
    uint32_t fl = 0;
    if (!ws_init(&w, V)) { *flags = AXS_MTP_FLAG_ERROR; return 0; }
    uint32_t cap = V ? V : 1;
    uint32_t* tid = malloc(cap * sizeof(uint32_t));
    float* tp = malloc(cap * sizeof(float));
    uint32_t* did = malloc(cap * sizeof(uint32_t));
    float* dp = malloc(cap * sizeof(float));
    uint32_t count = 0;
    uint32_t ac = 0;
    float Td = dparams->temperature, Tt = tparams->temperature;
    for (uint32_t i = 0; i < depth; ++i) {
        const float* trow = target + (uint64_t)i * V;
        const float* drow = draft + (uint64_t)i * V;
        int nt = token_distribution_ws(trow, V, tparams, tid, tp, cap, &w);
        int nd = token_distribution_ws(drow, V, dparams, did, dp, cap, &w);
        if (nt < 0 || nd < 0) { fl |= AXS_MTP_FLAG_ERROR; break; }
        uint32_t d = draft_ids[i];
        float lnq = logprob_of(axo_distribution_prob(did, dp, (uint32_t)nd, d));
        float p_target = fmaxf(axo_distribution_prob(tid, tp, (uint32_t)nt, d), 0.0f);
        float lps = lnq;
        if (Td > 0.0f && Tt > 0.0f && fabsf(Td - Tt) > 1e-6f) lps = lnq * (Td / Tt);
        float p_draft = fmaxf(expf(lps), 1e-37f);
        float accept_prob = fminf(p_target / p_draft, 1.0f);
        float u = uniforms[i];
        /* u >= 1 never accepts, whatever accept_prob <= 1 rounds to */
        if (u < 1.0f && fabs((double)u - (double)accept_prob) < 1e-6) fl |= AXS_MTP_FLAG_NEAR_ACCEPT;
        if (u < accept_prob) {
            out_ids[count++] = d;
            ac++;
            continue;
        }
        uint32_t corr = axo_sample_residual(tid, tp, (uint32_t)nt, did, dp, (uint32_t)nd,
                                            uniforms[depth]);
        if (corr == AXS_NONE_U32) {
            usrc us = {&uniforms[depth], NULL, 0};
            corr = sample_row_ws(trow, V, tparams, NULL, 0, NULL, NULL, NULL, 0, &us, NULL,
                                 NULL, 0, &w);
        }
        out_ids[count++] = corr;
        fl |= AXS_MTP_FLAG_RESIDUAL;
        goto done;
    }
    if (!(fl & AXS_MTP_FLAG_ERROR)) {
        axo_explain ex;
        usrc us = {&uniforms[depth], NULL, 0};
        uint32_t bonus = sample_row_ws(target + (uint64_t)depth * V, V, tparams, NULL, 0, NULL,
                                       NULL, NULL, 0, &us, &ex, NULL, 0, &w);
        if (ex.boundary) fl |= AXS_MTP_FLAG_NEAR;
        out_ids[count++] = bonus;
        fl |= AXS_MTP_FLAG_BONUS;
    }
done:
    free(tid); free(tp); free(did); free(dp);
    ws_free(&w);
    *accept_count = ac;
    *flags = fl;
    return count;
}

typedef struct {
    const void* target; const void* draft; int dtype; uint32_t B, depth, V; uint64_t stride;
    const uint32_t* draft_ids; const axs_sampling_params* tparams; const axs_sampling_params* dparams;
    const float* uniforms; uint32_t* out_ids; uint32_t* out_count; uint32_t* accept_count;
    uint32_t* flags; int tid, nthreads;
} mtp_job;

static void* mtp_worker(void* arg) {
    mtp_job* j = (mtp_job*)arg;
    uint64_t V = j->V;
    float* tbuf = malloc((j->depth + 1) * V * sizeof(float) + 4);
    float* dbuf = malloc((j->depth ? j->depth : 1) * V * sizeof(float) + 4);
    float* ubuf = malloc((j->depth + 1) * sizeof(float));
    uint32_t per = (j->B + j->nthreads - 1) / j->nthreads;
    uint32_t r0 = per * j->tid, r1 = r0 + per;
    if (r1 > j->B) r1 = j->B;
    for (uint32_t r = r0; r < r1; ++r) {
        for (uint32_t i = 0; i <= j->depth; ++i) {
            uint64_t off = ((uint64_t)r * (j->depth + 1) + i) * j->stride;
            if (j->dtype == AXS_DTYPE_BF16)
                axo_bf16_to_f32((const uint16_t*)j->target + off, tbuf + i * V, V);
            else
                memcpy(tbuf + i * V, (const float*)j->target + off, V * 4);
        }
        for (uint32_t i = 0; i < j->depth; ++i) {
            uint64_t off = ((uint64_t)r * j->depth + i) * j->stride;
            if (j->dtype == AXS_DTYPE_BF16)
                axo_bf16_to_f32((const uint16_t*)j->draft + off, dbuf + i * V, V);
            else
                memcpy(dbuf + i * V, (const float*)j->draft + off, V * 4);
        }
        const axs_sampling_params* tp = &j->tparams[r];
        for (uint32_t i = 0; i <= j->depth; ++i) {
            if (j->uniforms) ubuf[i] = j->uniforms[(uint64_t)r * (j->depth + 1) + i];
            else ubuf[i] = axo_philox_uniform(tp->seed, r, tp->step, 1 + i / 4, i & 3);
        }
        uint32_t ac = 0, fl = 0;
        uint32_t cnt = axo_mtp_verify_seq(tbuf, dbuf, j->V, j->depth,
                                          j->draft_ids + (uint64_t)r * j->depth, tp,
                                          &j->dparams[r], ubuf,
                                          j->out_ids + (uint64_t)r * (j->depth + 1), &ac, &fl);
        j->out_count[r] = cnt;
        if (j->accept_count) j->accept_count[r] = ac;
        if (j->flags) j->flags[r] = fl;
    }
    free(tbuf); free(dbuf); free(ubuf);
    return NULL;
}

int axo_mtp_verify_batch(const void* target, const void* draft, int dtype, uint32_t B,
                         uint32_t depth, uint32_t V, uint64_t stride,
                         const uint32_t* draft_ids, const axs_sampling_params* tparams,
                         const axs_sampling_params* dparams, const float* uniforms,
                         uint32_t* out_ids, uint32_t* out_count, uint32_t* accept_count,
                         uint32_t* flags, int nthreads) {
    if (nthreads < 1) nthreads = 1;
    if ((uint32_t)nthreads > B && B > 0) nthreads = (int)B;
    mtp_job* jobs = calloc((size_t)nthreads, sizeof(mtp_job));
    pthread_t* th = calloc((size_t)nthreads, sizeof(pthread_t));
    for (int t = 0; t < nthreads; ++t) {
        mtp_job* j = &jobs[t];
        j->target = target; j->draft = draft; j->dtype = dtype; j->B = B; j->depth = depth;
        j->V = V; j->stride = stride; j->draft_ids = draft_ids; j->tparams = tparams;
        j->dparams = dparams; j->uniforms = uniforms; j->out_ids = out_ids;
        j->out_count = out_count; j->accept_count = accept_count; j->flags = flags;
        j->tid = t; j->nthreads = nthreads;
    }
    if (nthreads == 1) mtp_worker(&jobs[0]);
    else {
        for (int t = 0; t < nthreads; ++t) pthread_create(&th[t], NULL, mtp_worker, &jobs[t]);
        for (int t = 0; t < nthreads; ++t) pthread_join(th[t], NULL);
    }
    free(jobs);
    free(th);
    return 0;
}

/* ------------------------------------------------------------------------ */
/* core DeterministicSampler                                                 */
/* ------------------------------------------------------------------------ */

/* f32::total_cmp key: order -NaN < -inf < ... < -0 < +0 < ... < inf < NaN */
static int32_t total_key(float x) {
    int32_t k;
    memcpy(&k, &x, 4);
    k ^= (int32_t)(((uint32_t)(k >> 31)) >> 1);
    return k;
}

/* sample_argmax_with_logprob_and_logits_processors
 * (crates/ax-engine-core/src/sampling.rs:142-191): repetition over ALL recent
 * tokens, n-gram ban, last maximum by total_cmp, logprob = -ln sum exp(l - best)
 * over finite l. */
int axo_core_argmax_logprob(const float* logits, uint32_t n, const axs_sampling_params* p,
                            const uint32_t* recent, uint32_t nrecent, uint32_t* token,
                            float* logprob) {
    int rep_applies = isfinite(p->repetition_penalty) && p->repetition_penalty > 0.0f &&
                      p->repetition_penalty != 1.0f && nrecent > 0;
    int ngram_applies = p->no_repeat_ngram_size > 0 && nrecent >= p->no_repeat_ngram_size;
    float* buf = NULL;
    const float* L = logits;
    if (rep_applies || ngram_applies) {
        buf = malloc((size_t)(n ? n : 1) * sizeof(float));
        memcpy(buf, logits, (size_t)n * sizeof(float));
        if (rep_applies) {
            uint8_t* seen = calloc(n ? n : 1, 1);
            repetition_penalty(buf, n, p->repetition_penalty, recent, nrecent, seen);
            free(seen);
        }
        no_repeat_ngram(buf, n, p->no_repeat_ngram_size, p->ngram_window, recent, nrecent);
        L = buf;
    }
    if (n == 0) { free(buf); return 0; }
    uint32_t bi = 0;
    int32_t bk = total_key(L[0]);
    for (uint32_t i = 1; i < n; ++i) {
        int32_t k = total_key(L[i]);
        if (k >= bk) { bk = k; bi = i; }
    }
    float best = L[bi];
    if (!isfinite(best)) { free(buf); return 0; }
    float norm = 0.0f;
    for (uint32_t i = 0; i < n; ++i)
        if (isfinite(L[i])) norm += expf(L[i] - best);
    free(buf);
    if (!isfinite(norm) || norm <= 0.0f) return 0;
    *token = bi;
    *logprob = -logf(norm);
    return 1;
}
