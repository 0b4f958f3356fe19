// axs_device.h — device-side building blocks of the gfx950 sampler:
// row-parameter decoding, Philox, the reference's exp, wave/block reductions and sorts.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/ax_hip_sampler.h"
#include "axs_exact_sum.h"
#include "axs_expf.h"

namespace axs {

constexpr uint32_t NONE = 0xFFFFFFFFu;

// ---------------------------------------------------------------------------
// Row modes.  The branch structure of sample_categorical_into
// (crates/ax-engine-mlx/src/sampling.rs:236-316):
//   temperature <= 0                          → GREEDY   (:236-238)
//   min-p active                              → MINP     (:283-294), draw in
//        sorted order iff top_k > 0 || top_p < 1 (:923-926), else index order
//   top_k == 0 && !(top_p < 1)                → FAST     (:246-270; also the
//        filtered path with no effective filter when top_p is NaN)
//   0 < top_p < 1 (finite)                    → TOPP     (sorted, full-vocab total)
//   top_k > 0                                 → TOPK     (sorted, top-k prefix)
//   otherwise (top_k == 0, top_p <= 0)        → SORTALL  (sorted, no truncation)
// ---------------------------------------------------------------------------
enum RowMode : uint32_t {
    M_GREEDY = 0,
    M_FAST = 1,
    M_MINP = 2,
    M_TOPK = 3,
    M_TOPP = 4,
    M_SORTALL = 5,
};

__device__ __forceinline__ bool uses_min_p(const axs_sampling_params& p) {
    return p.has_min_p && isfinite(p.min_p) && p.min_p > 0.0f;
}

__device__ __forceinline__ bool uses_rep(const axs_sampling_params& p) {
    return isfinite(p.repetition_penalty) && p.repetition_penalty > 0.0f &&
           p.repetition_penalty != 1.0f;
}

__device__ __forceinline__ bool topp_active(const axs_sampling_params& p) {
    return isfinite(p.top_p) && p.top_p > 0.0f && p.top_p < 1.0f;
}

__device__ __forceinline__ bool filters_enabled(const axs_sampling_params& p) {
    return p.top_k > 0u || p.top_p < 1.0f;
}

__device__ __forceinline__ uint32_t row_mode(const axs_sampling_params& p) {
    if (p.temperature <= 0.0f) return M_GREEDY;
    if (uses_min_p(p)) return M_MINP;
    if (!filters_enabled(p)) return M_FAST;
    if (topp_active(p)) return M_TOPP;
    if (p.top_k > 0u) return M_TOPK;
    return M_SORTALL;
}

// ---------------------------------------------------------------------------
// Philox4x32-10 (Salmon et al., SC'11): counter (row, step_lo, step_hi,
// purpose), key (seed_lo, seed_hi); uniform = (word >> 8) * 2^-24.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void philox4x32_10(uint32_t c[4], uint32_t k0, uint32_t k1) {
#pragma unroll
    for (int r = 0; r < 10; ++r) {
        if (r > 0) {
            k0 += 0x9E3779B9u;
            k1 += 0xBB67AE85u;
        }
        uint32_t hi0 = __umulhi(0xD2511F53u, c[0]);
        uint32_t lo0 = 0xD2511F53u * c[0];
        uint32_t hi1 = __umulhi(0xCD9E8D57u, c[2]);
        uint32_t lo1 = 0xCD9E8D57u * c[2];
        uint32_t n0 = hi1 ^ c[1] ^ k0;
        uint32_t n2 = hi0 ^ c[3] ^ k1;
        c[0] = n0;
        c[1] = lo1;
        c[2] = n2;
        c[3] = lo0;
    }
}

__device__ __forceinline__ float philox_uniform(uint64_t seed, uint32_t row, uint64_t step,
                                                uint32_t purpose, uint32_t word) {
    uint32_t c[4] = {row, (uint32_t)step, (uint32_t)(step >> 32), purpose};
    philox4x32_10(c, (uint32_t)seed, (uint32_t)(seed >> 32));
    return (float)(c[word & 3u] >> 8) * 0x1p-24f;
}

// ---------------------------------------------------------------------------
// exp as the reference computes it: f32::exp is the host libm's expf, which
// axs_expf.h restates bit for bit (checked over all 2^32 inputs on the CPU).
// ---------------------------------------------------------------------------
__device__ __forceinline__ float exp_ref(float x) { return expf_libm(x); }

// the reference's probability of a logit: exp((l - m) * inv), non-finite → 0
// (sampling.rs:248-251, 274-277)
__device__ __forceinline__ float prob_of(float l, float m, float inv) {
    float x = __fmul_rn(__fsub_rn(l, m), inv);
    float p = exp_ref(x);
    return isfinite(p) ? p : 0.0f;
}

// ln x rounded once to f32 (glibc's logf, which the reference calls, is
// correctly rounded for nearly all inputs)
__device__ __forceinline__ float ln_f32(float x) { return (float)log((double)x); }

// ln(max(prob, 1e-37)) floored at -30 (sampling.rs:156-160)
__device__ __forceinline__ float logprob_of(float prob) {
    float q = fmaxf(prob, 1e-37f);
    return fmaxf((float)log((double)q), -30.0f);
}

// ---------------------------------------------------------------------------
// wave (64-lane) and block helpers
// ---------------------------------------------------------------------------
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int d = 32; d > 0; d >>= 1) v = fmaxf(v, __shfl_xor(v, d, 64));
    return v;
}

// Maximum over the 64 lanes with DPP row operations instead of LDS
// permutes: pairs, quads, half rows, rows, then rows 1 and 3 take the rows
// below them and row 3 the first half; lane 63 holds the result, returned
// wave-uniform.  Every lane must be active.
template <int CTRL, int ROWS>
__device__ __forceinline__ float dpp_f(float x) {
    const int v = __float_as_int(x);
    return __int_as_float(__builtin_amdgcn_update_dpp(v, v, CTRL, ROWS, 0xF, false));
}
__device__ __forceinline__ float wave_max_dpp(float x) {
    x = fmaxf(x, dpp_f<0xB1, 0xF>(x));   // quad_perm [1,0,3,2]
    x = fmaxf(x, dpp_f<0x4E, 0xF>(x));   // quad_perm [2,3,0,1]
    x = fmaxf(x, dpp_f<0x141, 0xF>(x));  // row_half_mirror
    x = fmaxf(x, dpp_f<0x140, 0xF>(x));  // row_mirror
    x = fmaxf(x, dpp_f<0x142, 0xA>(x));  // row_bcast:15 into rows 1, 3
    x = fmaxf(x, dpp_f<0x143, 0xC>(x));  // row_bcast:31 into rows 2, 3
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 63));
}

// Unsigned minimum over the 64 lanes, the same DPP pattern; returned
// wave-uniform.  Every lane must be active.
template <int CTRL, int ROWS>
__device__ __forceinline__ uint32_t dpp_u(uint32_t x) {
    return (uint32_t)__builtin_amdgcn_update_dpp((int)x, (int)x, CTRL, ROWS, 0xF, false);
}
__device__ __forceinline__ uint32_t wave_min_u32_dpp(uint32_t x) {
    x = min(x, dpp_u<0xB1, 0xF>(x));
    x = min(x, dpp_u<0x4E, 0xF>(x));
    x = min(x, dpp_u<0x141, 0xF>(x));
    x = min(x, dpp_u<0x140, 0xF>(x));
    x = min(x, dpp_u<0x142, 0xA>(x));
    x = min(x, dpp_u<0x143, 0xC>(x));
    return (uint32_t)__builtin_amdgcn_readlane((int)x, 63);
}

// (value, index) argmax over the wave with the reference's rule (larger
// value, then lower index; NONE never wins), wave-uniform result.  v is
// never NaN.  Every lane must be active.
__device__ __forceinline__ void wave_argmax_dpp(float& v, uint32_t& i) {
    const float m = wave_max_dpp(i == NONE ? -INFINITY : v);
    const uint32_t c = (i != NONE && v == m) ? i : NONE;
    i = wave_min_u32_dpp(c);
    v = m;
}

// exclusive count of the set bits of a 64-lane mask below this lane
__device__ __forceinline__ uint32_t mbcnt64(uint64_t m) {
    return __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v) {
#pragma unroll
    for (int d = 32; d > 0; d >>= 1) v = min(v, (uint32_t)__shfl_xor((int)v, d, 64));
    return v;
}

__device__ __forceinline__ uint32_t wave_sum_u32(uint32_t v) {
#pragma unroll
    for (int d = 32; d > 0; d >>= 1) v += (uint32_t)__shfl_xor((int)v, d, 64);
    return v;
}

__device__ __forceinline__ float wave_sum_f(float v) {
#pragma unroll
    for (int d = 32; d > 0; d >>= 1) v += __shfl_xor(v, d, 64);
    return v;
}

// (value, index) argmax with the reference's rule: larger value wins, equal
// values keep the lower index, NaN never wins (sampling.rs:954-966).
__device__ __forceinline__ void am_merge(float& v, uint32_t& i, float v2, uint32_t i2) {
    bool take;
    if (i2 == NONE) take = false;
    else if (i == NONE) take = true;
    else take = (v2 > v) || (v2 == v && i2 < i);
    if (take) {
        v = v2;
        i = i2;
    }
}

__device__ __forceinline__ void wave_argmax(float& v, uint32_t& i) {
#pragma unroll
    for (int d = 32; d > 0; d >>= 1) {
        float v2 = __shfl_xor(v, d, 64);
        uint32_t i2 = (uint32_t)__shfl_xor((int)i, d, 64);
        am_merge(v, i, v2, i2);
    }
}

// Block-wide argmax; every thread gets the result.  `sv`/`si` are LDS
// scratch of nwaves entries.
template <int NT>
__device__ __forceinline__ void block_argmax(float& v, uint32_t& i, float* sv, uint32_t* si) {
    constexpr int NW = NT / 64;
    wave_argmax(v, i);
    int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    if (lane == 0) {
        sv[w] = v;
        si[w] = i;
    }
    __syncthreads();
    v = sv[0];
    i = si[0];
#pragma unroll
    for (int k = 1; k < NW; ++k) am_merge(v, i, sv[k], si[k]);
    __syncthreads();
}

template <int NT>
__device__ __forceinline__ float block_max(float v, float* sv) {
    constexpr int NW = NT / 64;
    v = wave_max(v);
    int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    if (lane == 0) sv[w] = v;
    __syncthreads();
    v = sv[0];
#pragma unroll
    for (int k = 1; k < NW; ++k) v = fmaxf(v, sv[k]);
    __syncthreads();
    return v;
}

__device__ __forceinline__ uint32_t wave_or_u32(uint32_t v) {
#pragma unroll
    for (int d = 32; d > 0; d >>= 1) v |= (uint32_t)__shfl_xor((int)v, d, 64);
    return v;
}

template <int NT>
__device__ __forceinline__ uint32_t block_or_u32(uint32_t v, uint32_t* sv) {
    constexpr int NW = NT / 64;
    v = wave_or_u32(v);
    int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    if (lane == 0) sv[w] = v;
    __syncthreads();
    v = 0;
#pragma unroll
    for (int k = 0; k < NW; ++k) v |= sv[k];
    __syncthreads();
    return v;
}

template <int NT>
__device__ __forceinline__ double block_sum_d(double v, double* sv) {
    constexpr int NW = NT / 64;
#pragma unroll
    for (int d = 32; d > 0; d >>= 1) v += __shfl_xor(v, d, 64);
    int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    if (lane == 0) sv[w] = v;
    __syncthreads();
    v = 0.0;
#pragma unroll
    for (int k = 0; k < NW; ++k) v += sv[k];
    __syncthreads();
    return v;
}

template <int NT>
__device__ __forceinline__ uint32_t block_min_u32(uint32_t v, uint32_t* sv) {
    constexpr int NW = NT / 64;
    v = wave_min_u32(v);
    int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    if (lane == 0) sv[w] = v;
    __syncthreads();
    v = sv[0];
#pragma unroll
    for (int k = 1; k < NW; ++k) v = min(v, sv[k]);
    __syncthreads();
    return v;
}

template <int NT>
__device__ __forceinline__ float block_sum_f(float v, float* sv) {
    constexpr int NW = NT / 64;
    v = wave_sum_f(v);
    int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    if (lane == 0) sv[w] = v;
    __syncthreads();
    v = 0.0f;
#pragma unroll
    for (int k = 0; k < NW; ++k) v += sv[k];
    __syncthreads();
    return v;
}

template <int NT>
__device__ __forceinline__ uint32_t block_sum_u32(uint32_t v, uint32_t* sv) {
    constexpr int NW = NT / 64;
    v = wave_sum_u32(v);
    int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    if (lane == 0) sv[w] = v;
    __syncthreads();
    v = 0;
#pragma unroll
    for (int k = 0; k < NW; ++k) v += sv[k];
    __syncthreads();
    return v;
}

// exclusive scan of u32 over the block; returns the exclusive prefix and
// writes the total to *total.
template <int NT>
__device__ __forceinline__ uint32_t block_excl_scan_u32(uint32_t v, uint32_t* sv, uint32_t* total) {
    constexpr int NW = NT / 64;
    int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    uint32_t x = v;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        uint32_t y = (uint32_t)__shfl_up((int)x, d, 64);
        if (lane >= d) x += y;
    }
    if (lane == 63) sv[w] = x;
    __syncthreads();
    uint32_t base = 0, tot = 0;
#pragma unroll
    for (int k = 0; k < NW; ++k) {
        if (k < w) base += sv[k];
        tot += sv[k];
    }
    __syncthreads();
    *total = tot;
    return base + x - v;
}

// ---------------------------------------------------------------------------
// Sort keys.  (p desc, id asc) ≡ descending order of
//   key = (bits(p) << 32) | ~id        (p >= 0, so its bits order like p)
// and ascending id ≡ descending order of
//   key = (~id << 32) | bits(p).
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint64_t key_pdesc(float p, uint32_t id) {
    return ((uint64_t)__float_as_uint(p) << 32) | (uint64_t)(~id);
}
__device__ __forceinline__ uint64_t key_idasc(float p, uint32_t id) {
    return ((uint64_t)(~id) << 32) | (uint64_t)__float_as_uint(p);
}
__device__ __forceinline__ float pdesc_p(uint64_t k) { return __uint_as_float((uint32_t)(k >> 32)); }
__device__ __forceinline__ uint32_t pdesc_id(uint64_t k) { return ~(uint32_t)k; }
__device__ __forceinline__ float idasc_p(uint64_t k) { return __uint_as_float((uint32_t)k); }
__device__ __forceinline__ uint32_t idasc_id(uint64_t k) { return ~(uint32_t)(k >> 32); }

// Descending bitonic sort of n (a power of two) keys in memory `s` (LDS or
// global) by the whole block.
template <int NT>
__device__ void block_sort_desc(uint64_t* s, uint32_t n) {
    for (uint32_t k = 2; k <= n; k <<= 1) {
        for (uint32_t j = k >> 1; j > 0; j >>= 1) {
            for (uint32_t i = threadIdx.x; i < n; i += NT) {
                uint32_t ixj = i ^ j;
                if (ixj > i) {
                    uint64_t a = s[i], b = s[ixj];
                    bool desc = (i & k) == 0;
                    if (desc ? (a < b) : (a > b)) {
                        s[i] = b;
                        s[ixj] = a;
                    }
                }
            }
            __threadfence_block();
            __syncthreads();
        }
    }
}

__device__ __forceinline__ uint32_t next_pow2(uint32_t n) {
    uint32_t p = 1;
    while (p < n) p <<= 1;
    return p;
}

}  // namespace axs
