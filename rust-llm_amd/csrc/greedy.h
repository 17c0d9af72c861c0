// The GREEDY path: rows with temperature <= 0 (sample.rs:259-265), which take
// argmax (sample.rs:118-128) of the penalised row (:239-257) and draw nothing.
//
// One launch. Each chunk of a row scans its logits for the largest argmax
// composite (argmax_key, then the lowest id) of the penalised row: the window
// ids that fall in the chunk are bits of an LDS bitmap over its elements, and
// their logits are penalised in registers as they are scanned (the four bits
// of a float4 sit in one word: one LDS read a float4), as the reference
// replaces them in its vector, each id once however often the window repeats
// it. A chunk's best goes to the row's slot by a 64-bit atomic max, and the
// row's last chunk to arrive (a per-row counter) writes the token: kept 1,
// candidate (token, 1.0), no uniform used. Slot and counter are zero between
// calls.
#pragma once
#include "sampler_kernels.h"

namespace rl {

struct GreedyScratch {
    uint64_t *best;    // [slot]: the best composite of the row's finished chunks; zero between calls
    uint32_t *arrive;  // [slot]: chunks of the row finished; zero between calls
};

constexpr uint32_t GREEDY_WIN_PER = 8;  // window ids per thread: windows of up to 2048 ids
static_assert(GREEDY_WIN_PER * FAST_THREADS >= 2048, "a window's ids fit the threads");

// grid (chunks, rows on this path), FAST_THREADS; dynamic LDS: the window
// bitmap (chunk_bitmap_words of the largest chunk, when the call has
// windows).
template <bool VEC>
__global__ __launch_bounds__(FAST_THREADS) void k_greedy(RowIO a, GreedyScratch g) {
    extern __shared__ __align__(16) uint32_t bm[];
    __shared__ uint64_t red[FAST_WAVES];
    __shared__ uint32_t s_last;
    const uint32_t slot = blockIdx.y, chunk = blockIdx.x;
    const uint32_t row = a.rows ? a.rows[slot] : a.row0 + slot;
    const float *rowp = a.logits + (uint64_t)row * a.stride;
    const uint32_t V = a.vocab, tid = threadIdx.x;
    // chunk * n4 < MAX_CHUNKS * 2^19 fits 32 bits (as in k_stream).
    const uint32_t n4 = V / 4;
    const uint32_t q0 = uniform_u32(chunk * n4 / a.chunks), q1 = uniform_u32((chunk + 1) * n4 / a.chunks);
    const uint32_t e0 = 4 * q0, e1 = chunk == a.chunks - 1 ? V : 4 * q1;

    // Loads first, on kernel arguments alone: the row's settings and window
    // length (one vector load), the window's ids (clamped to the call's
    // stride; which of them count is decided once the length is in), then
    // the first tile. A chunk with no float4 loads 16 bytes of its row's
    // settings instead, with no branch around the loads. No window logit is
    // gathered: the penalty is applied to the tile's own registers.
    const uint32_t head_w = row_words(a, row);
    const bool have_win = a.windows && a.wlen && a.wstride > 0;
    const uint32_t *wrow = have_win ? a.windows + (uint64_t)row * a.wstride
                                    : reinterpret_cast<const uint32_t *>(a.settings + row);
    const uint32_t wn = have_win ? (a.wstride < GREEDY_WIN_PER * FAST_THREADS ? a.wstride : GREEDY_WIN_PER * FAST_THREADS)
                                 : 1u;
    uint32_t wid[GREEDY_WIN_PER];
#pragma unroll
    for (uint32_t k = 0; k < GREEDY_WIN_PER; ++k) {
        const uint32_t i = k * FAST_THREADS + tid;
        wid[k] = ((const RL_GLB uint32_t *)wrow)[i < wn ? i : wn - 1];
    }
    constexpr uint32_t STEP = FAST_THREADS * UNROLL;
    f32x4 A[UNROLL], B[UNROLL];
    {
        const bool any = q1 > q0;
        load_tile_clamped<VEC>(A, any ? rowp : (const float *)(a.settings + row), any ? q0 : 0u, any ? q1 : 1u);
    }
    __builtin_amdgcn_sched_barrier(0);
    rl_sampling s;
    uint32_t wl;
    row_head(a, head_w, s, wl);
    const bool pen = penalises(s) && wl > 0;

    // The window ids that fall in this chunk, as bits over its elements.
    if (pen) {
        const uint32_t nwords = (e1 - e0 + 31) / 32;
        for (uint32_t i = tid; i < nwords; i += FAST_THREADS) bm[i] = 0;
        __syncthreads();
#pragma unroll
        for (uint32_t k = 0; k < GREEDY_WIN_PER; ++k) {
            const uint32_t id = wid[k];
            if (k * FAST_THREADS + tid < wl && id >= e0 && id < e1)
                atomicOr(&bm[(id - e0) >> 5], 1u << ((id - e0) & 31));
        }
        __syncthreads();
    }
    auto windowed = [&](uint32_t e) { return ((bm[(e - e0) >> 5] >> ((e - e0) & 31)) & 1u) != 0; };

    // The scan: a lane's elements in ascending id order, so a strictly larger
    // composite is the only update (ties keep the lower id by the composite
    // itself); window ids take their penalised values first.
    uint64_t best = 0;
    auto take = [&](const f32x4 &v, uint32_t f, bool ok) {
        float x[4] = {v.x, v.y, v.z, v.w};
        if (pen && ok) {
            const uint32_t r = 4 * f - e0;
            const uint32_t bits = (bm[r >> 5] >> (r & 31)) & 0xFu;
            if (bits) {
#pragma unroll
                for (uint32_t c = 0; c < 4; ++c)
                    if ((bits >> c) & 1u) x[c] = penalize(x[c], s.repeat_penalty);
            }
        }
#pragma unroll
        for (uint32_t c = 0; c < 4; ++c) {
            const uint64_t cc = ok ? composite(argmax_key(x[c]), 4 * f + c) : 0ull;
            if (cc > best) best = cc;
        }
    };
    if (q1 > q0) {
        for (uint32_t b = q0; b < q1; b += STEP) {
            load_tile_clamped<VEC>(B, rowp, b + STEP, q1);  // past the chunk: clamped, one line a wave
#pragma unroll
            for (uint32_t u = 0; u < UNROLL; ++u) {
                const uint32_t f = b + u * FAST_THREADS + tid;
                take(A[u], f, f < q1);
            }
#pragma unroll
            for (uint32_t u = 0; u < UNROLL; ++u) A[u] = B[u];
        }
    }
    if (chunk == a.chunks - 1) {  // the row's last vocab % 4 elements
        const uint32_t e = 4 * n4 + tid;
        if (e < V) {
            float x = ((const RL_GLB float *)rowp)[e];
            if (pen && windowed(e)) x = penalize(x, s.repeat_penalty);
            const uint64_t cc = composite(argmax_key(x), e);
            if (cc > best) best = cc;
        }
    }
    best = wave_max_u64(best);
    if (lane_id() == 0) red[tid / WAVE] = best;
    __syncthreads();
    if (tid == 0) {
        for (uint32_t w = 1; w < FAST_WAVES; ++w) best = red[w] > best ? red[w] : best;
        if (a.chunks > 1) {
            // Into the row's slot, completed before the arrival; the last
            // chunk then reads the slot with a device-scope load.
            (void)__hip_atomic_fetch_max(g.best + slot, best, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __builtin_amdgcn_s_waitcnt(WAITCNT_VM0);
            s_last = atomicAdd(g.arrive + slot, 1u) == a.chunks - 1 ? 1u : 0u;
        }
    }
    if (a.chunks > 1) {
        __syncthreads();
        if (!s_last) return;
        if (tid == 0) {
            best = __hip_atomic_load(g.best + slot, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            g.best[slot] = 0;  // ready for the next call
            g.arrive[slot] = 0;
        }
    }
    if (tid == 0) write_single(a, row, comp_key(best) == 0 ? 0u : comp_id(best));
}

}  // namespace rl
