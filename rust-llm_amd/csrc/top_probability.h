// top_probability (crates/rust-llm/src/forward.rs:1671-1680): for a row of
// logits, the argmax and (1 / sum) as f32, where sum is the f64 sum, in id
// order, of exp(l_i - l_best). The MTP draft loop compares it with MTP_P_MIN
// (forward.rs:341, :1014-1015), so the bits matter.
//
// Two launches: the argmax per chunk (and whether a NaN occurs), then the f64
// sum of the terms per chunk in any order, whose last chunk of a row to finish
// computes a certificate: an interval that holds both the chunked sum's exact
// value and the reference's sequential sum; (float)(1.0 / s) is monotone in s,
// so when both ends of the interval give the same f32 that is the answer.
// Otherwise that workgroup replays the row's sequential sum exactly
// (rl_seqsum.h).
//
// The interval. Every term is at most 1 (exp of a value <= 0) and the best
// one is exactly 1, so the sum S is at least 1; let E >= 0 be its binade and
// G = 2^(E-52) the grid of f64 values there. A step s + x of the sequential
// sum rounds only if x is not a multiple of the grid of the new partial sum
// (at most G), or if the partial sum enters a new binade. An f32 term
// x >= 2^(E-29) has its lowest bit at or above 2^(E-52) = G, so only terms
// below 2^(E-29) can round outside binade changes, and there are at most
// E + 150 binade changes above the smallest f32. Each rounding is at most
// G / 2: the sequential sum is within (small + 200) * G / 2 of the exact sum,
// where small counts the nonzero terms below 2^(E-29). The sum pass counts
// every term below 2^-26, zeros too (a zero term adds without rounding, so
// counting it only widens the bound), which serves every E <= 3; a larger E
// falls back to the
// general bound gamma_(V-1) * S. The chunked sum adds every term
// into a 32-term sum, those in order per thread, then a tree and the chunks in
// order: its relative error is at most the depth of that summation times
// 2^-53. For the rows of a peaked distribution this interval is about a
// thousand times narrower than gamma_(V-1) * S, and a row almost never needs
// the replay.
#pragma once
#include "full_kernels.h"

namespace rl {

// The argmax of (value, index) pairs merged from another lane or wave: the
// larger value, and on equal values (-0 equals +0) the lower index, as the
// reference's strict `v > best` over ascending indices keeps the first.
__device__ __forceinline__ void tp_take(float &bv, uint32_t &bi, float ov, uint32_t oi) {
    if (ov > bv || (ov == bv && oi < bi)) {
        bv = ov;
        bi = oi;
    }
}

// grid (chunks, rows), FAST_THREADS: per chunk the argmax composite (argmax's
// order, sample.rs:118-128, which top_probability's loop shares) and whether a
// NaN occurs. Each lane follows the reference's loop over its own elements,
// which it sees in ascending index order: a value replaces the lane's best
// only when strictly greater (so NaN and -inf never do, and the first of
// equal values stays); lanes and waves then merge (tp_take). Three vector
// operations per element, against a 64-bit composite compare.
template <bool VEC>
__global__ __launch_bounds__(FAST_THREADS) void k_tp_max(const float *logits, uint64_t stride, uint32_t vocab,
                                                         uint32_t chunks, uint64_t *part_am, uint32_t *part_nan) {
    __shared__ float red_v[FAST_WAVES];
    __shared__ uint32_t red_i[FAST_WAVES], red_n[FAST_WAVES];
    const uint32_t row = blockIdx.y, chunk = blockIdx.x;
    const float *rowp = logits + (uint64_t)row * stride;
    const uint32_t n4 = vocab / 4;
    const uint32_t q0 = chunk_lo(n4, chunk, chunks), q1 = chunk_lo(n4, chunk + 1, chunks);
    float bv = -__builtin_inff();
    uint32_t bi = 0xFFFFFFFFu;
    bool nan = false;
    // Tiles of UNROLL float4 per thread, the next in flight while one is
    // scanned; loads past the chunk are clamped and their values skipped.
    constexpr uint32_t STEP = FAST_THREADS * UNROLL;
    if (q1 > q0) {
        f32x4 A[UNROLL], B[UNROLL];
        load_tile_clamped<VEC>(A, rowp, q0, q1);
        for (uint32_t b = q0; b < q1; b += STEP) {
            load_tile_clamped<VEC>(B, rowp, b + STEP, q1);
            if (b + STEP <= q1) {
#pragma unroll
                for (uint32_t u = 0; u < UNROLL; ++u) {
                    const uint32_t q = b + u * FAST_THREADS + threadIdx.x;
                    const float x[4] = {A[u].x, A[u].y, A[u].z, A[u].w};
#pragma unroll
                    for (uint32_t c = 0; c < 4; ++c) {
                        if (x[c] > bv) {
                            bv = x[c];
                            bi = 4 * q + c;
                        }
                        nan |= x[c] != x[c];
                    }
                }
            } else {
#pragma unroll
                for (uint32_t u = 0; u < UNROLL; ++u) {
                    const uint32_t q = b + u * FAST_THREADS + threadIdx.x;
                    const float x[4] = {A[u].x, A[u].y, A[u].z, A[u].w};
#pragma unroll
                    for (uint32_t c = 0; c < 4; ++c) {
                        if (q < q1 && x[c] > bv) {
                            bv = x[c];
                            bi = 4 * q + c;
                        }
                        nan |= q < q1 && x[c] != x[c];
                    }
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
            if (x > bv) {  // past every other element of the chunk
                bv = x;
                bi = e;
            }
            nan |= x != x;
        }
    }
    // Butterfly over the lane exchanges, strides 32 down to 1.
    const auto step = [&](float ov, uint32_t oi) { tp_take(bv, bi, ov, oi); };
    step(__uint_as_float(lane_xor<32>(__float_as_uint(bv))), lane_xor<32>(bi));
    step(__uint_as_float(lane_xor<16>(__float_as_uint(bv))), lane_xor<16>(bi));
    step(__uint_as_float(lane_xor<8>(__float_as_uint(bv))), lane_xor<8>(bi));
    step(__uint_as_float(lane_xor<4>(__float_as_uint(bv))), lane_xor<4>(bi));
    step(__uint_as_float(lane_xor<2>(__float_as_uint(bv))), lane_xor<2>(bi));
    step(__uint_as_float(lane_xor<1>(__float_as_uint(bv))), lane_xor<1>(bi));
    const uint32_t anynan = ballot(nan) != 0 ? 1u : 0u;
    const uint32_t wave = threadIdx.x / WAVE;
    if (lane_id() == 0) {
        red_v[wave] = bv;
        red_i[wave] = bi;
        red_n[wave] = anynan;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t n = anynan;
        for (uint32_t w = 1; w < FAST_WAVES; ++w) {
            tp_take(bv, bi, red_v[w], red_i[w]);
            n |= red_n[w];
        }
        // As a composite (argmax_key: nothing above -inf gives key 0).
        part_am[(uint64_t)row * chunks + chunk] = bv > -__builtin_inff() ? composite(argmax_key(bv), bi) : 0ull;
        part_nan[(uint64_t)row * chunks + chunk] = n;
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

// Terms counted by the sum pass: below 2^-26 (bits 0x32800000).
constexpr uint32_t TP_SMALL = 0x32800000u;

// The depth of k_tp_sum's summation (the additions any term's value passes
// through): 32 within a tile, one per tile of the thread, the tail element,
// six across the wave and three across its waves, then the chunks in the
// row's finishing workgroup.
__host__ __device__ inline uint32_t tp_sum_depth(uint32_t vocab, uint32_t chunks) {
    const uint32_t n4 = vocab / 4;
    const uint32_t per = (n4 + chunks - 1) / chunks;
    const uint32_t tiles = (per + FAST_THREADS * UNROLL - 1) / (FAST_THREADS * UNROLL);
    return 32 + tiles + 1 + 6 + (FAST_WAVES - 1) + chunks;
}

// load_tile_clamped for the sum pass. With aligned rows the loads go through
// a buffer resource over the row (n4 float4, under 2^21 * 4 bytes, so byte
// offsets fit 32 bits): the tile's base is a scalar offset, each lane's
// offset is min(lane * 16, a scalar limit), one vector operation a load
// instead of the index, clamp and 64-bit address of a global load. Indices
// at or past `end` are clamped to end - 1 as in load_tile_clamped (a base at
// or past end loads element end - 1 in every lane), so every access stays
// inside the row.
template <bool VEC>
__device__ __forceinline__ void load_sum_tile(f32x4 *dst, const float *row, uint32_t n4, uint32_t base,
                                              uint32_t end) {
    if constexpr (VEC) {
        const __amdgpu_buffer_rsrc_t rsrc =
            __builtin_amdgcn_make_buffer_rsrc((void *)row, (short)0, (int)(n4 * 16u), 0x00020000);
        const uint32_t bb = base < end ? base : end - 1;
        const uint32_t lim = (end - 1 - bb) * 16u;  // the last element's byte offset from bb
        const uint32_t lane16 = threadIdx.x * 16u;
#pragma unroll
        for (uint32_t u = 0; u < UNROLL; ++u) {
            const uint32_t su = u * FAST_THREADS * 16u < lim ? u * FAST_THREADS * 16u : lim;
            const uint32_t vl = lim - su;
            const uint32_t voff = lane16 < vl ? lane16 : vl;
            dst[u] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, (int)voff,
                                                                                 (int)(bb * 16u + su), 2));
        }
    } else {
        load_tile_clamped<VEC>(dst, row, base, end);
    }
}

// The row's result from its chunk sums S and small-term counts (the
// interval of the file's header), or, when the interval does not decide the
// f32 of 1 / s, from the row's sequential sum replayed exactly by the
// workgroup. Every thread of the workgroup calls it; thread 0 writes.
__device__ __forceinline__ void tp_finish(const float *rowp, uint32_t vocab, uint32_t chunks, uint32_t tok,
                                          float best, double S, uint32_t small, const LdsExpTable &etab,
                                          SeqLds<FAST_THREADS> *seq, uint32_t *out_token, float *out_prob) {
    // S is within dS of the exact sum, the sequential sum within dq of it.
    const double dS = 2.0 * (double)tp_sum_depth(vocab, chunks) * 0x1p-53 * S;
    const double S_up = S * (1.0 + 4.0 * ((double)vocab + 64.0) * 0x1p-53);  // above both sums
    const int E = (int)((f64_bits(S_up) >> 52) & 0x7FF) - 1023;
    double dq;
    if (E <= 3) {
        dq = ((double)small + 200.0) * mul_pow2(1.0, E - 53);
    } else {
        dq = 2.0 * ((double)vocab + 64.0) * 0x1p-53 * S_up;  // gamma_(V-1) * S, with margin
    }
    const double D = dS + dq;
    const double s_lo = (S - D) * (1.0 - 0x1p-50), s_hi = (S + D) * (1.0 + 0x1p-50);
    const float lo = (float)(1.0 / s_hi), hi = (float)(1.0 / s_lo);
    float prob = lo;
    if (lo != hi) {
        double sum;
        seq_replay<53, FAST_THREADS, SEQ_ITEMS>(
            [rowp](uint32_t j) { return ((const RL_GLB uint32_t *)rowp)[j]; },
            [best, etab](uint32_t bits) { return expf_libm_nonpos_t(__uint_as_float(bits) - best, etab); }, vocab,
            NeverStop{}, seq, &sum);
        prob = (float)(1.0 / sum);
    }
    if (threadIdx.x == 0) {
        *out_token = tok;
        *out_prob = prob;
    }
}

// grid (chunks, rows), FAST_THREADS: per chunk the f64 sum of exp(l_i - best)
// (forward.rs:1678), in any order, and how many terms are small (above). The
// row's last chunk to publish its sum (a per-row arrival counter, zero
// between calls) finishes the row (tp_finish); a row whose sum is NaN is
// written by its chunk 0 (every chunk reaches the same verdict).
template <bool VEC>
__global__ __launch_bounds__(FAST_THREADS) void k_tp_sum(const float *logits, uint64_t stride, uint32_t vocab,
                                                         uint32_t chunks, const uint64_t *part_am,
                                                         const uint32_t *part_nan, double *part_sum,
                                                         uint32_t *part_small, uint32_t *arrive,
                                                         uint32_t *out_token, float *out_prob) {
    __shared__ uint64_t exp_tab[32];
    __shared__ double red[FAST_WAVES];
    __shared__ uint32_t red_c[FAST_WAVES];
    __shared__ SeqLds<FAST_THREADS> seq;
    __shared__ uint32_t s_last;
    const uint32_t row = blockIdx.y, chunk = blockIdx.x;
    const float *rowp = logits + (uint64_t)row * stride;
    const uint32_t n4 = vocab / 4;
    const uint32_t q0 = chunk_lo(n4, chunk, chunks), q1 = chunk_lo(n4, chunk + 1, chunks);
    // The first tile is loaded before the row's argmax partials, so the two
    // round trips overlap (vector loads complete in order: waiting for the
    // partials waits for the tile too). A chunk with no float4 (a row of
    // fewer than 4 logits) loads 16 bytes of the partials instead, with no
    // branch around the loads.
    f32x4 A[UNROLL], B[UNROLL];
    {
        const bool any = q1 > q0;
        load_sum_tile<VEC>(A, any ? rowp : (const float *)part_am, any ? n4 : 1u, any ? q0 : 0u, any ? q1 : 1u);
    }
    uint64_t am;
    if (tp_row(part_am, part_nan, row, chunks, &am)) {
        // The reference's sum is NaN (tp_row).
        if (chunk == 0 && threadIdx.x == 0) {
            out_token[row] = comp_key(am) == 0 ? 0u : comp_id(am);
            out_prob[row] = __builtin_nanf("");
        }
        return;
    }
    const uint32_t tok = comp_id(am);
    // The best value from its composite: argmax_key(v) = total_key(v + 0), so
    // this is the logit itself, or +0 where it is -0; x - best then differs
    // only in the sign of a zero result (x = -0), whose exp is 1 either way.
    const float best = key_value(comp_key(am));
    copy_exp_table((RL_LDS uint64_t *)exp_tab);
    const LdsExpTable etab{(RL_LDS uint64_t *)exp_tab};
    double sum = 0.0;
    uint32_t small = 0;   // this lane's count: the last, partial tile and the tail element
    uint32_t wsmall = 0;  // the wave's count over the full tiles (the same in every lane)
    // x - best <= 0 and is not NaN: tp_row has returned for rows holding a
    // NaN and for a best at +-inf.
    auto term = [&](double &acc, float x) {
        const float t = expf_libm_nonpos_t(x - best, etab);
        acc += (double)t;
        return __float_as_uint(t) < TP_SMALL;
    };
    auto add = [&](double &acc, float x) { small += term(acc, x) ? 1u : 0u; };
    // In a full tile every lane of the workgroup is active, so a term's count
    // can be a ballot, which the wave keeps in scalar registers.
    auto add_full = [&](double &acc, float x) { wsmall += (uint32_t)__builtin_popcountll(ballot(term(acc, x))); };
    // Tiles as in k_tp_max: the next tile's loads overlap this tile's exps.
    // Each tile's terms are summed on their own, then added to the thread's
    // sum, which bounds the depth of the summation (tp_sum_depth).
    constexpr uint32_t STEP = FAST_THREADS * UNROLL;
    if (q1 > q0) {
        for (uint32_t b = q0; b < q1; b += STEP) {
            load_sum_tile<VEC>(B, rowp, n4, b + STEP, q1);
            double ts = 0.0;
            if (b + STEP <= q1) {
#pragma unroll
                for (uint32_t u = 0; u < UNROLL; ++u) {
                    add_full(ts, A[u].x);
                    add_full(ts, A[u].y);
                    add_full(ts, A[u].z);
                    add_full(ts, A[u].w);
                }
            } else {
#pragma unroll
                for (uint32_t u = 0; u < UNROLL; ++u) {
                    if (b + u * FAST_THREADS + threadIdx.x < q1) {
                        add(ts, A[u].x);
                        add(ts, A[u].y);
                        add(ts, A[u].z);
                        add(ts, A[u].w);
                    }
                }
            }
            sum += ts;
#pragma unroll
            for (uint32_t u = 0; u < UNROLL; ++u) A[u] = B[u];
        }
    }
    if (chunk == chunks - 1) {
        const uint32_t e = 4 * n4 + threadIdx.x;
        if (e < vocab) add(sum, ((const RL_GLB float *)rowp)[e]);
    }
    // Butterfly over the lane exchanges, strides 32 down to 1 (f64 additions
    // in the same order as a shuffle butterfly).
    sum += lane_xor_f64<32>(sum);
    sum += lane_xor_f64<16>(sum);
    sum += lane_xor_f64<8>(sum);
    sum += lane_xor_f64<4>(sum);
    sum += lane_xor_f64<2>(sum);
    sum += lane_xor_f64<1>(sum);
    small = wave_sum_u32(small) + wsmall;
    const uint32_t wave = threadIdx.x / WAVE;
    if (lane_id() == 0) {
        red[wave] = sum;
        red_c[wave] = small;
    }
    __syncthreads();
    // The chunk's sum, waves in order (the same in every thread).
    sum = red[0];
    small = red_c[0];
    for (uint32_t w = 1; w < FAST_WAVES; ++w) {
        sum += red[w];
        small += red_c[w];
    }
    if (chunks == 1) {  // the row's only chunk: its sum is the row's
        tp_finish(rowp, vocab, 1, tok, best, sum, small, etab, &seq, out_token + row, out_prob + row);
        return;
    }
    if (threadIdx.x == 0) {
        // Publish: device-scope stores, which write through this XCD's L2,
        // completed before the arrival; the last chunk reads them with
        // device-scope loads issued after its arrival saw every other one.
        const uint64_t at = (uint64_t)row * chunks + chunk;
        __hip_atomic_store(part_sum + at, sum, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(part_small + at, small, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __builtin_amdgcn_s_waitcnt(WAITCNT_VM0);  // the stores have completed
        s_last = atomicAdd(arrive + row, 1u) == chunks - 1 ? 1u : 0u;
    }
    __syncthreads();
    if (!s_last) return;
    // The row's last chunk: every chunk's sum is published. Chunk order, as
    // the certificate's depth (tp_sum_depth) counts it.
    double S = 0.0;
    uint32_t nsmall = 0;
    for (uint32_t c = 0; c < chunks; ++c) {
        const uint64_t at = (uint64_t)row * chunks + c;
        S += __hip_atomic_load(part_sum + at, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        nsmall += __hip_atomic_load(part_small + at, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (threadIdx.x == 0) arrive[row] = 0;  // ready for the next call
    tp_finish(rowp, vocab, chunks, tok, best, S, nsmall, etab, &seq, out_token + row, out_prob + row);
}

}  // namespace rl
