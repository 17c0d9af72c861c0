// top_probability (crates/rust-llm/src/forward.rs:1671-1680): for a row of
// logits, the argmax and (1 / sum) as f32, where sum is the f64 sum, in id
// order, of exp(l_i - l_best). The MTP draft loop compares it with MTP_P_MIN
// (forward.rs:341, :1014-1015), so the bits matter.
//
// Three launches: the argmax per chunk (and whether a NaN occurs), the f64
// sum of the terms per chunk in any order, then per row a certificate: the
// reference's sequential sum and the chunked one are each within
// gamma_(V-1) * sum of the exact sum, and (float)(1.0 / s) is monotone in s,
// so when both ends of that interval round to the same f32 that is the answer.
// Otherwise (about one row in a few hundred) the row's sequential sum is
// replayed exactly (rl_seqsum.h).
#pragma once
#include "full_kernels.h"

namespace rl {

// grid (chunks, rows), FAST_THREADS: per chunk the argmax composite (argmax's
// order, sample.rs:118-128, which top_probability's loop shares) and whether a
// NaN occurs.
template <bool VEC>
__global__ __launch_bounds__(FAST_THREADS) void k_tp_max(const float *logits, uint64_t stride, uint32_t vocab,
                                                         uint32_t chunks, uint64_t *part_am, uint32_t *part_nan) {
    __shared__ uint64_t red[FAST_WAVES];
    __shared__ uint32_t red_n[FAST_WAVES];
    const uint32_t row = blockIdx.y, chunk = blockIdx.x;
    const float *rowp = logits + (uint64_t)row * stride;
    const uint32_t n4 = vocab / 4;
    const uint32_t q0 = chunk_lo(n4, chunk, chunks), q1 = chunk_lo(n4, chunk + 1, chunks);
    uint64_t best = 0;
    uint32_t nan = 0;
    // Tiles of UNROLL float4 per thread, the next in flight while one is
    // scanned; loads past the chunk are clamped and their values skipped.
    constexpr uint32_t STEP = FAST_THREADS * UNROLL;
    if (q1 > q0) {
        f32x4 A[UNROLL], B[UNROLL];
        load_tile_clamped<VEC>(A, rowp, q0, q1);
        for (uint32_t b = q0; b < q1; b += STEP) {
            load_tile_clamped<VEC>(B, rowp, b + STEP, q1);
#pragma unroll
            for (uint32_t u = 0; u < UNROLL; ++u) {
                const uint32_t q = b + u * FAST_THREADS + threadIdx.x;
                const float x[4] = {A[u].x, A[u].y, A[u].z, A[u].w};
#pragma unroll
                for (uint32_t c = 0; c < 4; ++c) {
                    const uint64_t cc = q < q1 ? composite(argmax_key(x[c]), 4 * q + c) : 0ull;
                    best = cc > best ? cc : best;
                    nan |= (q < q1 && x[c] != x[c]) ? 1u : 0u;
                }
            }
#pragma unroll
            for (uint32_t u = 0; u < UNROLL; ++u) A[u] = B[u];
        }
    }
    if (chunk == chunks - 1) {
        const uint32_t e = 4 * n4 + threadIdx.x;
        if (e < vocab) {
            const float x = ((const RL_GLB float *)rowp)[e];
            const uint64_t cc = composite(argmax_key(x), e);
            best = cc > best ? cc : best;
            nan |= x != x ? 1u : 0u;
        }
    }
    best = wave_max_u64(best);
    nan = ballot(nan != 0) != 0 ? 1u : 0u;
    const uint32_t wave = threadIdx.x / WAVE;
    if (lane_id() == 0) {
        red[wave] = best;
        red_n[wave] = nan;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (uint32_t w = 1; w < FAST_WAVES; ++w) {
            best = red[w] > best ? red[w] : best;
            nan |= red_n[w];
        }
        part_am[(uint64_t)row * chunks + chunk] = best;
        part_nan[(uint64_t)row * chunks + chunk] = nan;
    }
}

// The row's argmax composite and whether the reference's sum is NaN: a NaN
// logit gives a NaN term; no value above -inf leaves best at -inf, and
// -inf - -inf is NaN; a +inf best gives +inf - +inf = NaN for itself.
__device__ __forceinline__ bool tp_row(const uint64_t *part_am, const uint32_t *part_nan, uint32_t row,
                                       uint32_t chunks, uint64_t *am) {
    uint64_t best = 0;
    uint32_t nan = 0;
    for (uint32_t c = 0; c < chunks; ++c) {
        const uint64_t x = part_am[(uint64_t)row * chunks + c];
        best = x > best ? x : best;
        nan |= part_nan[(uint64_t)row * chunks + c];
    }
    *am = best;
    const uint32_t key = comp_key(best);
    return nan != 0 || key == 0 || key_value(key) == __builtin_inff();
}

// grid (chunks, rows), FAST_THREADS: per chunk the f64 sum of exp(l_i - best)
// (forward.rs:1678), in any order.
template <bool VEC>
__global__ __launch_bounds__(FAST_THREADS) void k_tp_sum(const float *logits, uint64_t stride, uint32_t vocab,
                                                         uint32_t chunks, const uint64_t *part_am,
                                                         const uint32_t *part_nan, double *part_sum) {
    __shared__ uint64_t exp_tab[32];
    __shared__ double red[FAST_WAVES];
    const uint32_t row = blockIdx.y, chunk = blockIdx.x;
    uint64_t am;
    if (tp_row(part_am, part_nan, row, chunks, &am)) return;
    const float *rowp = logits + (uint64_t)row * stride;
    const float best = ((const RL_GLB float *)rowp)[comp_id(am)];
    copy_exp_table((RL_LDS uint64_t *)exp_tab);
    const LdsExpTable etab{(RL_LDS uint64_t *)exp_tab};
    const uint32_t n4 = vocab / 4;
    const uint32_t q0 = chunk_lo(n4, chunk, chunks), q1 = chunk_lo(n4, chunk + 1, chunks);
    double sum = 0.0;
    // Tiles as in k_tp_max: the next tile's loads overlap this tile's exps.
    constexpr uint32_t STEP = FAST_THREADS * UNROLL;
    if (q1 > q0) {
        f32x4 A[UNROLL], B[UNROLL];
        load_tile_clamped<VEC>(A, rowp, q0, q1);
        for (uint32_t b = q0; b < q1; b += STEP) {
            load_tile_clamped<VEC>(B, rowp, b + STEP, q1);
#pragma unroll
            for (uint32_t u = 0; u < UNROLL; ++u) {
                if (b + u * FAST_THREADS + threadIdx.x < q1) {
                    sum += (double)expf_libm_t(A[u].x - best, etab);
                    sum += (double)expf_libm_t(A[u].y - best, etab);
                    sum += (double)expf_libm_t(A[u].z - best, etab);
                    sum += (double)expf_libm_t(A[u].w - best, etab);
                }
            }
#pragma unroll
            for (uint32_t u = 0; u < UNROLL; ++u) A[u] = B[u];
        }
    }
    if (chunk == chunks - 1) {
        const uint32_t e = 4 * n4 + threadIdx.x;
        if (e < vocab) sum += (double)expf_libm_t(((const RL_GLB float *)rowp)[e] - best, etab);
    }
    for (int m = 32; m >= 1; m >>= 1) sum += __shfl_xor(sum, m);
    const uint32_t wave = threadIdx.x / WAVE;
    if (lane_id() == 0) red[wave] = sum;
    __syncthreads();
    if (threadIdx.x == 0) {
        for (uint32_t w = 1; w < FAST_WAVES; ++w) sum += red[w];
        part_sum[(uint64_t)row * chunks + chunk] = sum;
    }
}

// grid (rows), REPLAY_THREADS: the token, and 1 / sum certified from the
// chunk sums or from the replayed sequential sum.
__global__ __launch_bounds__(REPLAY_THREADS) void k_tp_final(const float *logits, uint64_t stride, uint32_t vocab,
                                                             uint32_t chunks, const uint64_t *part_am,
                                                             const uint32_t *part_nan, const double *part_sum,
                                                             uint32_t *out_token, float *out_prob) {
    __shared__ SeqLds<REPLAY_THREADS> seq;
    __shared__ uint64_t exp_tab[32];
    const uint32_t row = blockIdx.x;
    uint64_t am;
    const bool nan = tp_row(part_am, part_nan, row, chunks, &am);
    const uint32_t tok = comp_key(am) == 0 ? 0u : comp_id(am);
    if (nan) {
        if (threadIdx.x == 0) {
            out_token[row] = tok;
            out_prob[row] = __builtin_nanf("");
        }
        return;
    }
    double S = 0.0;
    for (uint32_t c = 0; c < chunks; ++c) S += part_sum[(uint64_t)row * chunks + c];
    // Both the sequential sum and S are within gamma_(V-1) of the exact sum
    // (gamma_n = n 2^-53 / (1 - n 2^-53)); d bounds their distance, with margin.
    const double d = 2.25 * ((double)vocab + 64.0) * 0x1p-53;
    const float lo = (float)(1.0 / (S * (1.0 + d))), hi = (float)(1.0 / (S * (1.0 - d)));
    float prob = lo;
    if (lo != hi) {
        const float *rowp = logits + (uint64_t)row * stride;
        const float best = ((const RL_GLB float *)rowp)[tok];
        copy_exp_table((RL_LDS uint64_t *)exp_tab);
        const LdsExpTable etab{(RL_LDS uint64_t *)exp_tab};
        double sum;
        seq_replay<53, REPLAY_THREADS, SEQ_ITEMS>(
            [rowp](uint32_t j) { return ((const RL_GLB uint32_t *)rowp)[j]; },
            [best, etab](uint32_t bits) { return expf_libm_t(__uint_as_float(bits) - best, etab); }, vocab,
            NeverStop{}, &seq, &sum);
        prob = (float)(1.0 / sum);
    }
    if (threadIdx.x == 0) {
        out_token[row] = tok;
        out_prob[row] = prob;
    }
}

}  // namespace rl
