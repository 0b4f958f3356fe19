// axs_lm_head.h — the LM-head projection with the greedy decision in its
// epilogue (gfx950, bf16 MFMA).
//
// logits[b, v] = softcap(scale * f32(bf16(sum_k hidden[b, k] * W[v, k])))
//
// as the reference's final projection forms them
// (crates/ax-engine-mlx/src/model/mod.rs:1771-1775): a bf16 x bf16 product
// whose bf16 result is widened to f32, then the optional output multiplier
// and logit softcap of apply_final_logit_softcap
// (crates/ax-engine-mlx/src/model/shared/utils.rs:1826-1845), each an f32
// operation: x * scale, then tanh(x * (1 / cap)) * cap.  W is the LM-head
// weight [V, H] (a linear layer's [out, in] layout), hidden the final-norm
// output [B, H].
//
// The product is HBM-bound for every decode batch (W is read once per 128
// batch rows; at B <= 128 a launch does at most 2B flops per weight byte,
// below gfx950's bf16 matrix-core-to-HBM ratio of ~312), so both kernels are
// laid out for streaming W in long contiguous pieces:
//
//   * k_lm_head_dot (B <= 2): each load is 1 KB of one W row, products on
//     the vector ALUs;
//   * k_lm_head_mfma (B > 2): W and hidden K chunks staged through LDS by
//     1 KB contiguous loads, double-buffered through registers, then
//     v_mfma_f32_16x16x32_bf16 with W as the A operand.
//
// The epilogue rounds each f32 accumulator to bf16 (round to nearest even),
// applies scale and softcap, writes the f32 logit when the caller wants the
// row, and folds it into the row's argmax under the reference's rule
// (argmax_f32, crates/ax-engine-mlx/src/sampling.rs:954-970: larger value
// wins, ties keep the lower id, NaN never wins, -0 equals +0, an all-NaN row
// gives 0).  The argmax is carried as a 64-bit key, order-preserving float
// bits above the complemented id, so at most one atomicMax per (workgroup,
// batch row) merges workgroups in any order to the same result.  A greedy
// row therefore gets its token without its logits ever being written or
// read again.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace axs_lmh {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int NT = 256;                  // threads per workgroup (4 waves)
constexpr int BMAX = 128;                // batch rows per launch slice at most (NB <= 8)

// f32 -> bf16 -> f32, round to nearest even; NaN stays NaN (quieted).
__device__ __forceinline__ float bf16_round(float x) {
    uint32_t u = __float_as_uint(x);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return __uint_as_float((u | 0x00400000u) & 0xFFFF0000u);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return __uint_as_float(u & 0xFFFF0000u);
}

// argmax key: 0 for NaN (never wins), otherwise order-preserving bits of x
// (-0 mapped to +0) above ~id, so that the larger key is the larger value,
// then the lower id.
__device__ __forceinline__ unsigned long long am_key(float x, uint32_t id) {
    uint32_t u = __float_as_uint(x);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0ull;
    if (u == 0x80000000u) u = 0u;
    u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((unsigned long long)u << 32) | (unsigned long long)(~id);
}

__device__ __forceinline__ unsigned long long shfl_xor_u64(unsigned long long v, int m) {
    const uint32_t lo = (uint32_t)__shfl_xor((int)(uint32_t)v, m, 64);
    const uint32_t hi = (uint32_t)__shfl_xor((int)(uint32_t)(v >> 32), m, 64);
    return ((unsigned long long)hi << 32) | lo;
}

__device__ __forceinline__ f32x4 mfma16(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b),
                                                   c, 0, 0, 0);
}

struct LmArgs {
    const uint16_t* hidden;  // [B, hs] bf16 bits
    int64_t hs;
    const uint16_t* w;       // [V, ws] bf16 bits
    int64_t ws;
    int B, H, V;
    float scale;             // 1: off
    float inv_cap, cap;      // cap <= 0: off
    float* out;              // [B, os] f32 or null
    int64_t os;
    int out_vec;             // out 16-byte aligned and os % 4 == 0: 16-byte stores
    unsigned long long* keys;  // [B] argmax keys (zeroed by the caller) or null
};

// Epilogue shared by both kernels: bf16 rounding, scale and softcap of one
// logit.
__device__ __forceinline__ float logit_of(const LmArgs& a, float acc) {
    float x = bf16_round(acc);
    if (a.scale != 1.0f) x = x * a.scale;
    if (a.cap > 0.0f) x = tanhf(x * a.inv_cap) * a.cap;
    return x;
}

// ... with its store and its argmax key (0 when v is past V).
__device__ __forceinline__ unsigned long long finish_logit(const LmArgs& a, float acc, int v, float* orow) {
    const float x = logit_of(a, acc);
    if (v >= a.V) return 0ull;
    if (orow) orow[v] = x;
    return am_key(x, (uint32_t)v);
}

// Folds a workgroup's best key for one batch row into the global key.  The
// global key only grows, so a workgroup whose key is not above the value it
// reads cannot change the result and issues no atomic: every workgroup of a
// launch targets the same B keys, and unconditional atomics on one address
// serialise at L2 (at B = 1 they cost more than the weight stream).
__device__ __forceinline__ void fold_key(unsigned long long* g, unsigned long long k) {
    if (k > __hip_atomic_load(g, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) atomicMax(g, k);
}

// Merges a workgroup's per-wave keys (s_key[wave][j] for batch row b0 + j)
// into the global keys, at most one atomicMax per batch row.
template <int NW>
__device__ __forceinline__ void merge_keys(const LmArgs& a, unsigned long long (*s_key)[BMAX], int b0, int nrows) {
    __syncthreads();
    const int t = threadIdx.x;
    if (t < nrows && b0 + t < a.B) {
        unsigned long long k = s_key[0][t];
#pragma unroll
        for (int w = 1; w < NW; ++w) k = s_key[w][t] > k ? s_key[w][t] : k;
        fold_key(a.keys + b0 + t, k);
    }
}

// ---------------------------------------------------------------------------
// B <= DOT_BMAX: one wave per ROWS vocabulary rows, each load a 1 KB
// contiguous piece of one W row (lane l: 8 elements at k0 + 8l), DEPTH such
// pieces per row in flight, products on the vector ALUs (a bf16 x bf16
// product is exact in f32; per lane the H/512 * 8 products of a row
// accumulate in K order, then a 64-lane tree sum, so every ROWS x DEPTH
// shape gives the same bits).  With at most 2 batch rows a matrix-core step
// would be >= 7/8 padding; the bound is HBM either way, and this load shape
// reaches more of it.  Measured at H = 4096, V = 151936 on normally
// distributed weights: the shapes tried (1, 2 or 4 rows x 4, 2 or 1 pieces)
// lie within 3% of one another; B = 1 is fastest with 2 rows and 2 pieces,
// B = 2 with 4 rows and 1 piece.
constexpr int DOT_BMAX = 2;
constexpr int DOT_KC = 512;   // K per load (64 lanes x 8 elements)

template <int NBR, int ROWS, int DEPTH>
__global__ __launch_bounds__(NT) void k_lm_head_dot(LmArgs a) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int vbase = (blockIdx.x * (NT / 64) + wave) * ROWS;
    const uint16_t* wrow[ROWS];
#pragma unroll
    for (int r = 0; r < ROWS; ++r) wrow[r] = a.w + (int64_t)min(vbase + r, a.V - 1) * a.ws + 8 * lane;
    const uint16_t* hrow[NBR];
#pragma unroll
    for (int b = 0; b < NBR; ++b) hrow[b] = a.hidden + (int64_t)min(b, a.B - 1) * a.hs + 8 * lane;
    float acc[ROWS][NBR];
#pragma unroll
    for (int r = 0; r < ROWS; ++r)
#pragma unroll
        for (int b = 0; b < NBR; ++b) acc[r][b] = 0.0f;
    auto dot8 = [](u32x4 w, u32x4 h, float s) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            s = s + __uint_as_float(w[q] << 16) * __uint_as_float(h[q] << 16);
            s = s + __uint_as_float(w[q] & 0xFFFF0000u) * __uint_as_float(h[q] & 0xFFFF0000u);
        }
        return s;
    };
    const int hmain = a.H - a.H % DOT_KC;
    const int hdeep = hmain - hmain % (DOT_KC * DEPTH);
    int k0 = 0;
    for (; k0 < hdeep; k0 += DOT_KC * DEPTH) {
        u32x4 wv[DEPTH][ROWS], hv[DEPTH][NBR];
#pragma unroll
        for (int d = 0; d < DEPTH; ++d) {
#pragma unroll
            for (int r = 0; r < ROWS; ++r) wv[d][r] = *(const u32x4*)(wrow[r] + k0 + DOT_KC * d);
#pragma unroll
            for (int b = 0; b < NBR; ++b) hv[d][b] = *(const u32x4*)(hrow[b] + k0 + DOT_KC * d);
        }
#pragma unroll
        for (int d = 0; d < DEPTH; ++d)
#pragma unroll
            for (int r = 0; r < ROWS; ++r)
#pragma unroll
                for (int b = 0; b < NBR; ++b) acc[r][b] = dot8(wv[d][r], hv[d][b], acc[r][b]);
    }
    for (; k0 < hmain; k0 += DOT_KC) {  // whole 512-element pieces past the last DEPTH group
        u32x4 wv[ROWS], hv[NBR];
#pragma unroll
        for (int r = 0; r < ROWS; ++r) wv[r] = *(const u32x4*)(wrow[r] + k0);
#pragma unroll
        for (int b = 0; b < NBR; ++b) hv[b] = *(const u32x4*)(hrow[b] + k0);
#pragma unroll
        for (int r = 0; r < ROWS; ++r)
#pragma unroll
            for (int b = 0; b < NBR; ++b) acc[r][b] = dot8(wv[r], hv[b], acc[r][b]);
    }
    if (hmain + 8 * lane < a.H) {  // the last H % 512 (a multiple of 32): lanes below it
        u32x4 wv[ROWS], hv[NBR];
#pragma unroll
        for (int r = 0; r < ROWS; ++r) wv[r] = *(const u32x4*)(wrow[r] + hmain);
#pragma unroll
        for (int b = 0; b < NBR; ++b) hv[b] = *(const u32x4*)(hrow[b] + hmain);
#pragma unroll
        for (int r = 0; r < ROWS; ++r)
#pragma unroll
            for (int b = 0; b < NBR; ++b) acc[r][b] = dot8(wv[r], hv[b], acc[r][b]);
    }
    // tree sums: every lane ends with the row totals
#pragma unroll
    for (int r = 0; r < ROWS; ++r)
#pragma unroll
        for (int b = 0; b < NBR; ++b)
#pragma unroll
            for (int d = 32; d > 0; d >>= 1) acc[r][b] = acc[r][b] + __shfl_xor(acc[r][b], d, 64);
    // lane r * NBR + b finishes (row r, batch b)
    unsigned long long key = 0ull;
    int mine_b = -1;
#pragma unroll
    for (int r = 0; r < ROWS; ++r)
#pragma unroll
        for (int b = 0; b < NBR; ++b)
            if (lane == r * NBR + b && b < a.B) {
                key = finish_logit(a, acc[r][b], vbase + r, a.out ? a.out + (int64_t)b * a.os : nullptr);
                mine_b = b;
            }
    if (!a.keys) return;
    __shared__ unsigned long long s_key[NT / 64][BMAX];
    // per batch row: the best of the wave's rows (lanes b, NBR + b, ...)
#pragma unroll
    for (int b = 0; b < NBR; ++b) {
        unsigned long long k = mine_b == b ? key : 0ull;
#pragma unroll
        for (int d = 32; d > 0; d >>= 1) {
            const unsigned long long o = shfl_xor_u64(k, d);
            k = o > k ? o : k;
        }
        if (lane == 0) s_key[wave][b] = k;
    }
    merge_keys<NT / 64>(a, s_key, 0, NBR);
}

// ---------------------------------------------------------------------------
// B > DOT_BMAX: matrix cores.  A workgroup owns 64 * WR vocabulary rows and
// up to 128 batch rows (NB 16-row blocks); wave w computes vocabulary blocks
// w, w + 4, ... (WR blocks of 16 rows) against every batch block with
// v_mfma_f32_16x16x32_bf16 (W as the A operand: row = vocabulary id; hidden
// as the B operand: column = batch row), so each hidden fragment read from
// LDS feeds WR matrix-core steps.  Each K chunk of KC is staged through LDS:
// every load instruction brings 1 KB of contiguous W or hidden (rows of
// KC * 2 bytes), the next chunk's loads are in flight while the matrix cores
// work on this one, and the fragments are read back in MFMA layout (lane
// (r, g) of K step s: 8 elements at 32s + 8g of row r).  16-byte chunks are
// XOR-swizzled by row so that the 16 rows of a fragment read fall in
// different LDS banks.
template <int NB, int WR, int KC>
__global__ __launch_bounds__(NT) void k_lm_head_mfma(LmArgs a) {
    constexpr int ROWS = 64 * WR;          // vocabulary rows per workgroup
    constexpr int CH = KC * 2 / 16;        // 16-byte chunks per row and K chunk
    constexpr int SW = CH - 1;             // swizzle mask
    constexpr int WLD = ROWS * CH / NT;    // W loads per thread per K chunk
    constexpr int HLD = 16 * NB * CH / NT; // hidden loads per thread per K chunk
    static_assert(WLD * NT == ROWS * CH && HLD * NT == 16 * NB * CH, "load plan");
    __shared__ u32x4 s_w[ROWS * CH];
    __shared__ u32x4 s_h[16 * NB * CH];
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int r16 = lane & 15, g = lane >> 4;
    const int v0 = blockIdx.x * ROWS, b0 = blockIdx.y * 16 * NB;
    // load plan: flat 16-byte chunk index q = i * NT + t -> (row q / CH, chunk q % CH)
    const uint16_t* wsrc[WLD];
#pragma unroll
    for (int i = 0; i < WLD; ++i) {
        const int q = i * NT + t;
        wsrc[i] = a.w + (int64_t)min(v0 + q / CH, a.V - 1) * a.ws + 8 * (q % CH);
    }
    const uint16_t* hsrc[HLD];
#pragma unroll
    for (int i = 0; i < HLD; ++i) {
        const int q = i * NT + t;
        hsrc[i] = a.hidden + (int64_t)min(b0 + q / CH, a.B - 1) * a.hs + 8 * (q % CH);
    }
    auto slot = [](int q) { return (q / CH) * CH + ((q % CH) ^ ((q / CH) & SW)); };
    f32x4 acc[WR][NB];
#pragma unroll
    for (int m = 0; m < WR; ++m)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) acc[m][nb] = f32x4{0.f, 0.f, 0.f, 0.f};
    u32x4 wreg[WLD], hreg[HLD];
    auto load = [&](int k0) {
#pragma unroll
        for (int i = 0; i < WLD; ++i) wreg[i] = *(const u32x4*)(wsrc[i] + k0);
#pragma unroll
        for (int i = 0; i < HLD; ++i) hreg[i] = *(const u32x4*)(hsrc[i] + k0);
    };
    auto stage = [&]() {
#pragma unroll
        for (int i = 0; i < WLD; ++i) s_w[slot(i * NT + t)] = wreg[i];
#pragma unroll
        for (int i = 0; i < HLD; ++i) s_h[slot(i * NT + t)] = hreg[i];
    };
    auto compute = [&](int nsteps) {
        for (int s = 0; s < nsteps; ++s) {
            const int ch = 4 * s + g;
            u32x4 wf[WR];
#pragma unroll
            for (int m = 0; m < WR; ++m) {
                const int wr = 16 * (wave + 4 * m) + r16;
                wf[m] = s_w[wr * CH + (ch ^ (wr & SW))];
            }
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) {
                const int hr = 16 * nb + r16;
                const u32x4 hf = s_h[hr * CH + (ch ^ (hr & SW))];
#pragma unroll
                for (int m = 0; m < WR; ++m) acc[m][nb] = mfma16(wf[m], hf, acc[m][nb]);
            }
        }
    };
    const int hmain = a.H - a.H % KC;
    if (hmain > 0) load(0);
    for (int k0 = 0; k0 < hmain; k0 += KC) {
        stage();
        __syncthreads();
        if (k0 + KC < hmain) load(k0 + KC);
        compute(KC / 32);
        __syncthreads();
    }
    if (hmain < a.H) {
        // the last H % KC (a multiple of 32): chunks past it are not loaded
        // and not read
        const int nch = (a.H - hmain) / 8;
#pragma unroll
        for (int i = 0; i < WLD; ++i)
            if ((i * NT + t) % CH < nch) wreg[i] = *(const u32x4*)(wsrc[i] + hmain);
#pragma unroll
        for (int i = 0; i < HLD; ++i)
            if ((i * NT + t) % CH < nch) hreg[i] = *(const u32x4*)(hsrc[i] + hmain);
        stage();
        __syncthreads();
        compute((a.H - hmain) / 32);
    }

    // epilogue: lane (r16, g) holds C[4g + i][r16] of each block
    unsigned long long best[NB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
        best[nb] = 0ull;
        const int b = b0 + 16 * nb + r16;
        float* orow = (a.out && b < a.B) ? a.out + (int64_t)b * a.os : nullptr;
#pragma unroll
        for (int m = 0; m < WR; ++m) {
            // this lane's 4 consecutive ids of the block: one 16-byte store
            // when the row allows it
            const int vq = v0 + 16 * (wave + 4 * m) + 4 * g;
            float x[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                x[i] = logit_of(a, acc[m][nb][i]);
                const unsigned long long k = vq + i < a.V ? am_key(x[i], (uint32_t)(vq + i)) : 0ull;
                best[nb] = (b < a.B && k > best[nb]) ? k : best[nb];
            }
            if (orow) {
                if (a.out_vec && vq + 4 <= a.V) {
                    *reinterpret_cast<f32x4*>(orow + vq) = f32x4{x[0], x[1], x[2], x[3]};
                } else {
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        if (vq + i < a.V) orow[vq + i] = x[i];
                }
            }
        }
    }
    if (!a.keys) return;
    __shared__ unsigned long long s_key[NT / 64][BMAX];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
        unsigned long long k = best[nb];
        unsigned long long o = shfl_xor_u64(k, 16);
        k = o > k ? o : k;
        o = shfl_xor_u64(k, 32);
        k = o > k ? o : k;
        if (g == 0) s_key[wave][16 * nb + r16] = k;
    }
    merge_keys<NT / 64>(a, s_key, b0, 16 * NB);
}

// ids[b] = the id under the row's key (0 for a row of NaN only)
__global__ void k_lm_head_ids(const unsigned long long* keys, int B, uint32_t* ids) {
    const int b = blockIdx.x * blockDim.x + threadIdx.x;
    if (b < B) {
        const unsigned long long k = keys[b];
        ids[b] = k ? ~(uint32_t)k : 0u;
    }
}

}  // namespace axs_lmh
