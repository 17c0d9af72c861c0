// The sampler's kernels. Two device paths, chosen per row from its settings:
//
//  GREEDY (temperature <= 0): argmax of the penalised row, k_greedy in
//  greedy.h. The stream kernel below still takes such a row as top-k 1 with
//  argmax's keys (w.greedy), which sample_rows no longer sends it: taking
//  that handling out changes the register allocation of the kernel, which
//  then spills (28 bytes a lane of scratch) and runs the 1024-row batch 11 %
//  slower (measured).
//
//  STREAM (1 <= top_k <= 64 with top_k < vocab): one pass
//  over the row in HBM. Each wave keeps the row's best candidates seen so far
//  in LDS under a rising threshold (a workgroup-wide one, shared through an
//  LDS atomic max), so almost every element costs one compare. Penalised
//  window ids are left out of the stream and offered with their penalised
//  values, so the logits are never written. The last wave merges the lists
//  and replays the reference's tail (sample.rs:267-358) on <= 64 candidates,
//  one candidate per lane.
//
//  FULL (top_k == 0, top_k >= vocab, or top_k > 64): the whole candidate list,
//  in full_kernels.h.
#pragma once
#include "rl_device.h"
#include "rl_expf.h"
#include "rl_seqsum.h"

namespace rl {

// s_waitcnt immediate for vmcnt(0) (gfx9 encoding; expcnt and lgkmcnt left at
// their maximum, so only vector memory operations are waited for).
constexpr int WAITCNT_VM0 = 0x0F70;
constexpr uint32_t FAST_THREADS = 256;
constexpr uint32_t FAST_WAVES = FAST_THREADS / WAVE;
constexpr uint32_t KMAX = 64;     // largest top_k the stream path takes (one per lane)
constexpr uint32_t UNROLL = 8;    // float4 loads per thread per tile
// The one-tile instantiation of the stream kernel: the same tile (NT * U
// float4) over twice the waves, two a SIMD, so that each wave's filter,
// bootstrap and sort have half the elements and a second wave to hide their
// latency; and the longest window it marks in its bitmap.
constexpr uint32_t ONE_TILE_THREADS = 512;
constexpr uint32_t ONE_TILE_U = UNROLL * FAST_THREADS / ONE_TILE_THREADS;
constexpr uint32_t ONE_TILE_WIN_MAX = 2048;
constexpr uint32_t MAX_CHUNKS = 32;
constexpr uint32_t FULL_THREADS = 256;
constexpr uint32_t STAGE = 4096;  // elements staged in LDS per sequential block

struct RowIO {
    const float *logits;
    uint64_t stride;
    uint32_t vocab;
    const rl_sampling *settings;  // indexed by row
    const uint32_t *rows;         // this path's rows: rows[slot] = row index; null: row0 + slot
    uint32_t row0;                // the first row when rows is null
    const uint32_t *windows;
    uint32_t wstride;
    const uint32_t *wlen;
    const float *uniforms;
    uint32_t *out_token;
    uint32_t *out_kept;
    uint8_t *out_used;
    uint32_t *out_ids;
    float *out_probs;
    uint64_t cand_stride;
    uint32_t hash_bits;
    uint32_t chunks;
    uint32_t polled;  // a host polls the kept counts of results in host memory
};

struct FastScratch {
    uint64_t *chunk_cands;   // [slot][chunk][KMAX]
    uint32_t *chunk_counts;  // [slot][chunk]
    uint32_t *arrive;        // [slot]: chunks of the row done; zero between calls
};

// The row's window length, at most the call's stride. The load is
// unconditional (from the row's settings when the call has no windows), so
// no branch around it holds up the loads issued after it.
__device__ __forceinline__ uint32_t window_len(const RowIO &a, uint32_t row) {
    const bool have = a.wlen && a.windows;
    const uint32_t l = *(const RL_GLB uint32_t *)(have ? a.wlen + row : (const uint32_t *)(a.settings + row));
    return have ? (l < a.wstride ? l : a.wstride) : 0u;
}

// A row's settings and window length by one vector load: lane i < 10 reads
// dword i of the row's settings, lane 10 its window length (or a settings
// dword when the call has no windows). The values reach every lane through
// readlane (row_head). Scalar loads of the same words are the slow way in at
// kernel start: they miss in the scalar cache, which several CUs share and
// which then serves its misses nearly one at a time; with 1024 workgroups
// starting together they took until about 13 us for most of them, where
// vector loads take one round trip.
static_assert(sizeof(rl_sampling) == 40, "ten dwords of settings");
__device__ __forceinline__ uint32_t row_words(const RowIO &a, uint32_t row) {
    const uint32_t lane = lane_id();
    const bool have = a.wlen && a.windows;
    const uint32_t *set = reinterpret_cast<const uint32_t *>(a.settings + row);
    const uint32_t *p = lane < 10 ? set + lane : have && lane == 10 ? a.wlen + row : set;
    return *(const RL_GLB uint32_t *)p;
}

// The settings and the window length (at most the call's stride) from
// row_words' result.
__device__ __forceinline__ void row_head(const RowIO &a, uint32_t w, rl_sampling &s, uint32_t &wl) {
    s.temperature = __uint_as_float(read_lane_u32(w, 0));
    s.top_p = __uint_as_float(read_lane_u32(w, 1));
    s.min_p = __uint_as_float(read_lane_u32(w, 2));
    s.repeat_penalty = __uint_as_float(read_lane_u32(w, 3));
    s.top_k = (uint64_t)read_lane_u32(w, 4) | ((uint64_t)read_lane_u32(w, 5) << 32);
    s.repeat_last_n = (uint64_t)read_lane_u32(w, 6) | ((uint64_t)read_lane_u32(w, 7) << 32);
    s.seed = (uint64_t)read_lane_u32(w, 8) | ((uint64_t)read_lane_u32(w, 9) << 32);
    const uint32_t l = read_lane_u32(w, 10);
    wl = (a.wlen && a.windows) ? (l < a.wstride ? l : a.wstride) : 0u;
}

// A system-scope store: written through to memory (sc0 sc1). A plain store
// to host memory can stay in this XCD's L2 and reach the host after a later
// one.
template <class T>
__device__ __forceinline__ void store_sys(T *p, T v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// A row's results. When a host polls the kept counts of results in host
// memory (a.polled: the host Sampler's calls), each is a system-scope store
// and the kept count is stored last, once the wave's other stores have
// completed, so that the host sees the row's other outputs when it sees the
// kept count change; other callers wait on the stream and get plain stores.
template <class T>
__device__ __forceinline__ void store_out(const RowIO &a, T *p, T v) {
    if (a.polled)
        store_sys(p, v);
    else
        *p = v;
}

__device__ __forceinline__ void store_kept_last(const RowIO &a, uint32_t row, uint32_t kept, bool writer) {
    if (a.polled) {
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __builtin_amdgcn_s_waitcnt(WAITCNT_VM0);  // this wave's stores have completed
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        if (writer) store_sys(a.out_kept + row, kept);
    } else if (writer) {
        a.out_kept[row] = kept;
    }
}

// A row with one candidate; called by one lane.
__device__ __forceinline__ void write_single(const RowIO &a, uint32_t row, uint32_t tok) {
    store_out(a, a.out_token + row, tok);
    store_out(a, a.out_used + row, (uint8_t)0);
    if (a.out_ids) {
        store_out(a, a.out_ids + (uint64_t)row * a.cand_stride, tok);
        store_out(a, a.out_probs + (uint64_t)row * a.cand_stride, 1.0f);
    }
    store_kept_last(a, row, 1, true);
}

typedef float f32x4 __attribute__((ext_vector_type(4)));

// Row loads are nontemporal: each logit is read once, so they should not
// displace anything from the caches.
template <bool VEC>
__device__ __forceinline__ f32x4 load4(const float *row, uint32_t f) {
    const RL_GLB float *g = (const RL_GLB float *)row;
    if constexpr (VEC) {
        return __builtin_nontemporal_load((const RL_GLB f32x4 *)g + f);
    } else {
        const RL_GLB float *p = g + 4ull * f;
        return f32x4{__builtin_nontemporal_load(p), __builtin_nontemporal_load(p + 1),
                     __builtin_nontemporal_load(p + 2), __builtin_nontemporal_load(p + 3)};
    }
}

// One tile is U float4 per thread, starting at float4 index `base`.
// The same tile with indices at or past `end` clamped to end - 1 (end >= 1):
// every lane loads, so no branch surrounds the loads. A branch around a load
// keeps the compiler from counting the loads in flight, and it then waits for
// all of them, the next tile's included, before the current tile is filtered.
template <bool VEC, uint32_t U = UNROLL, uint32_t NT = FAST_THREADS>
__device__ __forceinline__ void load_tile_clamped(f32x4 *dst, const float *row, uint32_t base, uint32_t end) {
#pragma unroll
    for (uint32_t u = 0; u < U; ++u) {
        const uint32_t f = base + u * NT + threadIdx.x;
        dst[u] = load4<VEC>(row, f < end ? f : end - 1);
    }
}

__device__ __forceinline__ uint64_t read_lane_u64(uint64_t v, uint32_t lane) {
    return ((uint64_t)read_lane_u32((uint32_t)(v >> 32), lane) << 32) | read_lane_u32((uint32_t)v, lane);
}

// ------------------------------------------------- per-wave candidates ---
// A wave of the stream kernel keeps candidates in an LDS buffer. T is a lower
// bound on the row's k-th best composite (this wave's k-th best so far, or
// another wave's, shared through an LDS atomic max): nothing <= T can be among
// the row's k best. `thr` is the value of T's key, a one-compare necessary
// test for composite > T. Candidates are appended without a capacity check;
// the buffer holds KMAX entries plus one half-tile's worth, and compaction
// runs before every half-tile whose passers might not fit. The kernel makes
// no function calls: a call would give every wave a scratch frame, and with
// it a slower launch and spills around the call sites.
constexpr uint32_t SLACK = 48;  // new candidates between compactions
// A tile of U float4 per thread is filtered in two halves (the first the
// larger when U is odd); a wave's buffer holds KMAX candidates, SLACK more,
// and one half-tile's worth.
template <uint32_t U>
struct TileShape {
    static constexpr uint32_t HALF = (U + 1) / 2;                // float4 per thread in the first half
    static constexpr uint32_t HALF_ELEMS = HALF * 4 * WAVE;      // most elements a wave filters per half
    static constexpr uint32_t CBUF = KMAX + SLACK + HALF_ELEMS;  // per-wave candidate buffer
};

struct Stream {
    RL_LDS uint64_t *buf;
    RL_LDS uint64_t *shared_T;
    WindowSet ws;
    uint64_t wtop;  // window_top(ws): candidates above it are not window ids
    uint64_t T;
    float thr;
    uint32_t cnt;
    uint32_t k;
    bool greedy;
    bool pen;
};

// Necessary condition for composite(x) > T, one compare. !(x < thr) lets NaN
// through to the exact test (a NaN sorts first in the total order); in greedy
// mode the starting -FLT_MAX drops -inf, and the exact test drops NaN, which
// argmax never picks.
__device__ __forceinline__ bool prefilter(const Stream &w, float x) { return !(x < w.thr); }

__device__ __forceinline__ void raise_threshold(Stream &w, uint64_t t) {
    t = uniform_u64(t);
    if (t > w.T) {
        w.T = t;
        w.thr = key_value(comp_key(t));
    }
}

__device__ __forceinline__ uint64_t load_shared_T(RL_LDS uint64_t *p) {
    return uniform_u64(__hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP));
}

__device__ __forceinline__ void publish_threshold(RL_LDS uint64_t *p, uint64_t t) {
    if (lane_id() == 0) __hip_atomic_fetch_max(p, t, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// Sorts this wave's candidates, 64 at a time across the wave, keeps the k best
// at buf[0..cnt) and raises the threshold to the k-th. Penalised window ids
// enter the buffer unchecked (a hash lookup per passing element would stall
// the loop on LDS); they are dropped here, so the threshold is the k-th best of
// non-window elements only. Returns the sorted best 64 (lane i holds the i-th).
__device__ __forceinline__ uint64_t compact(Stream &w) {
    const uint32_t lane = lane_id();
    wave_lds_sync();
    uint64_t top = 0;
    uint32_t valid = 0;
    for (uint32_t base = 0; base < w.cnt; base += WAVE) {
        const uint32_t j = base + lane;
        uint64_t v = j < w.cnt ? w.buf[j] : 0ull;
        if (w.pen && v != 0 && v <= w.wtop && window_contains(w.ws, comp_id(v))) v = 0;
        valid += (uint32_t)__popcll(ballot(v != 0));
        top = wave_merge64(top, wave_sort64<false>(v));
    }
    wave_lds_sync();
    const uint32_t n = uniform_u32(valid < w.k ? valid : w.k);
    if (lane < n) w.buf[lane] = top;
    w.cnt = n;
    if (valid >= w.k) {
        raise_threshold(w, read_lane_u64(top, w.k - 1));
        publish_threshold(w.shared_T, w.T);
    }
    raise_threshold(w, load_shared_T(w.shared_T));
    wave_lds_sync();
    return top;
}

// Appends this wave's passing lanes (ballot compaction).
__device__ __forceinline__ void offer(Stream &w, bool pass, uint64_t c) {
    const uint64_t m = ballot(pass);
    if (m == 0) return;
    if (pass) w.buf[w.cnt + lanes_below(m)] = c;
    w.cnt += (uint32_t)__popcll(m);
}

__device__ __forceinline__ uint32_t stream_key(const Stream &w, float x) {
    return w.greedy ? total_key(x + 0.0f) : total_key(x);
}

// A float4 group of the wave: most groups have no lane past the prefilter;
// of the others, usually one or two of the four components do, and only
// those run the exact test (the skip is a scalar test of the prefilter's
// lane mask).
template <bool CHECK>
__device__ __forceinline__ void offer_group(Stream &w, f32x4 v, uint32_t id0, uint32_t nvalid) {
    const float x[4] = {v.x, v.y, v.z, v.w};
    bool pf[4];
    bool any = false;
#pragma unroll
    for (uint32_t c = 0; c < 4; ++c) {
        pf[c] = (!CHECK || c < nvalid) && prefilter(w, x[c]);
        any |= pf[c];
    }
    if (ballot(any) == 0) return;
#pragma unroll
    for (uint32_t c = 0; c < 4; ++c) {
        if (ballot(pf[c]) == 0) continue;
        const uint64_t comp = composite(stream_key(w, x[c]), id0 + c);
        const bool p = pf[c] && comp > w.T && (!w.greedy || x[c] >= -3.40282347e38f);
        offer(w, p, comp);
    }
}

// Filters one tile (U float4 per thread) in two halves, compacting
// before a half whose passers might not fit.
template <bool GUARD, uint32_t U, uint32_t NT>
__device__ __forceinline__ void process_tile(Stream &w, const f32x4 *T, uint32_t base, uint32_t end) {
    constexpr uint32_t HALF = TileShape<U>::HALF;
#pragma unroll
    for (uint32_t h = 0; h < 2; ++h) {
        if (w.cnt >= w.k + SLACK) compact(w);  // then cnt <= k, and k + SLACK + HALF_ELEMS <= CBUF
#pragma unroll
        for (uint32_t u = h * HALF; u < ((h + 1) * HALF < U ? (h + 1) * HALF : U); ++u) {
            const uint32_t f = base + u * NT + threadIdx.x;
            offer_group<GUARD>(w, T[u], 4 * f, (!GUARD || f < end) ? 4u : 0u);
        }
    }
}

// A first threshold from the wave's first tile: each lane's best element
// (window ids excluded), then the k-th best t of those 64 lane maxima. At
// least k distinct elements are >= t, so nothing below t is among the row's k
// best; the threshold is t - 1 because the k elements >= t are not in any
// buffer yet and must still pass the strict test composite > T. Loads at or
// past `end` were clamped (duplicates of the chunk's last element under other
// ids) and are left out; a lane with none contributes nothing, and with fewer
// than k contributing lanes t is 0 (no threshold).
// Returns the sorted lane maxima (lane i: the i-th best).
template <uint32_t U, uint32_t NT>
__device__ __forceinline__ uint64_t bootstrap(Stream &w, const f32x4 *A, uint32_t base, uint32_t end) {
    const uint32_t tid = threadIdx.x;
    uint64_t bound = ~0ull, best = 0;
    for (uint32_t attempt = 0; attempt < 4; ++attempt) {
        best = 0;
#pragma unroll
        for (uint32_t u = 0; u < U; ++u) {
            const float x[4] = {A[u].x, A[u].y, A[u].z, A[u].w};
            const uint32_t f = base + u * NT + tid;
            const uint32_t id0 = 4 * f;
#pragma unroll
            for (uint32_t c = 0; c < 4; ++c) {
                const bool ok = f < end && (!w.greedy || x[c] >= -3.40282347e38f);
                const uint64_t comp = composite(stream_key(w, x[c]), id0 + c);
                if (ok && comp < bound && comp > best) best = comp;
            }
        }
        if (!w.pen || best == 0 || best > w.wtop || !window_contains(w.ws, comp_id(best))) break;
        bound = best;
        best = 0;
    }
    const uint64_t sorted = wave_sort64<true>(best);
    const uint64_t t = read_lane_u64(sorted, w.k - 1);
    raise_threshold(w, t ? t - 1 : 0ull);
    publish_threshold(w.shared_T, w.T);
    return sorted;
}

// The one-tile kernel's bootstrap, on 32-bit keys: each lane's largest key
// over its elements of the tile (the filter's order refines keys by id, so
// every element with a key at or above key t has a composite at or above
// t << 32), and the 64 lane maxima sorted descending across the wave by a
// bitonic network of max and min, half the instructions of one on 64-bit
// composites. Loads at or past `end` (clamped) and, in greedy mode, -inf and
// NaN are left out; a lane with nothing keeps key 0, which no element's
// composite bound uses. Raises the wave's threshold to the k-th lane maximum's
// key (at least k elements are at or above it) and returns the sorted keys.
template <uint32_t U, uint32_t NT>
__device__ __forceinline__ uint32_t bootstrap_keys(Stream &w, const f32x4 *A, uint32_t base, uint32_t end) {
    uint32_t best = 0;
#pragma unroll
    for (uint32_t u = 0; u < U; ++u) {
        const float x[4] = {A[u].x, A[u].y, A[u].z, A[u].w};
        const bool in = base + u * NT + threadIdx.x < end;
#pragma unroll
        for (uint32_t c = 0; c < 4; ++c) {
            const bool ok = in && (!w.greedy || x[c] >= -3.40282347e38f);
            const uint32_t key = stream_key(w, x[c]);
            best = ok && key > best ? key : best;
        }
    }
    const uint32_t sorted = wave_sort_u32_desc(best);
    const uint32_t t = read_lane_u32(sorted, w.k - 1);
    raise_threshold(w, t ? ((uint64_t)t << 32) - 1 : 0ull);
    return sorted;
}

// The workgroups sharing a CU are otherwise served oldest first: the first
// one dispatched finishes its row long before the last, and the CU then
// streams with fewer and fewer waves. Lowering a wave's priority as its row
// progresses (3 up to half the tiles, 2 up to 80 %, 1 up to 95 %, then 0)
// lets the waves that are behind issue first, so the rows on a CU finish
// together. Priority only orders instruction issue; it changes no result.
__device__ __forceinline__ void set_progress_priority(uint32_t done, uint32_t total) {
    if (done * 20 >= total * 19)
        __builtin_amdgcn_s_setprio(0);
    else if (done * 5 >= total * 4)
        __builtin_amdgcn_s_setprio(1);
    else if (done * 2 >= total)
        __builtin_amdgcn_s_setprio(2);
}

// The row's f32::max fold over the penalised logits and its argmax, by one
// wave re-reading the row. Only for a row whose k best are all +NaN, where the
// candidates do not reveal the largest non-NaN value.
__device__ __forceinline__ void rescan_row(const float *rowp, uint32_t vocab, const WindowSet &ws, bool pen,
                                           float penalty, float *out_max, uint32_t *out_tok) {
    const uint32_t lane = lane_id();
    const RL_GLB float *g = (const RL_GLB float *)rowp;
    float mx = -__builtin_inff();
    uint64_t am = 0;
    for (uint32_t e = lane; e < vocab; e += WAVE) {
        float x = g[e];
        if (pen && window_contains(ws, e)) x = penalize(x, penalty);
        mx = fmaxf(mx, x);
        const uint64_t c = composite(argmax_key(x), e);
        am = c > am ? c : am;
    }
    *out_max = uniform_f32(wave_maxnum_f32(mx));
    am = uniform_u64(wave_max_u64(am));
    *out_tok = comp_key(am) == 0 ? 0u : comp_id(am);
}

// By one wave: the row's window ids (window[0..len), those below vocab) into
// an empty set, for rescan_row where the workgroup kept no set of its own.
__device__ __forceinline__ void window_build_wave(const WindowSet &w, const uint32_t *window, uint32_t len,
                                                  uint32_t vocab) {
    for (uint32_t i = lane_id(); i < w.slots; i += WAVE) w.ids[i] = EMPTY_ID;
    wave_lds_sync();
    for (uint32_t i = lane_id(); i < len; i += WAVE) {
        const uint32_t id = window[i];
        if (id < vocab) (void)window_insert(w, id);
    }
    wave_lds_sync();
}

// Binary exponent of a finite nonzero f32 (subnormals count as -126): every
// such value is a multiple of 2^(exponent - 23).
__device__ __forceinline__ int f32_exponent(float p) {
    const int e = (int)((__float_as_uint(p) >> 23) & 0xFFu);
    return e == 0 ? -126 : e - 127;
}

// The row's uniform (0 when the call has none: then no row draws).
__device__ __forceinline__ float row_uniform(const RowIO &a, uint32_t row) {
    return a.uniforms ? a.uniforms[row] : 0.0f;
}

// The reference's tail (sample.rs:259-358) over the row's best nL candidates,
// by one wave: lane j holds candidate j (composite c, 0 past nL), in
// descending order. The sequential f64 and f32 sums are replayed in candidate
// order with readlane, so every lane computes the bits the reference does.
// tab_v (lane_exp_entry) and u (row_uniform) are loaded by the caller ahead
// of the tail, so that it waits for no memory round trip.
// With BUILD_SET, `ws` holds no ids yet: the rare rescan first builds it
// from the row's window (wrow, wl).
template <bool BUILD_SET = false>
__device__ __forceinline__ void finalize_row(const RowIO &a, uint32_t row, const rl_sampling &s, uint32_t k,
                                             uint64_t c, uint32_t nL, const WindowSet &ws, bool pen,
                                             const float *rowp, uint64_t tab_v, float u,
                                             const uint32_t *wrow = nullptr, uint32_t wl = 0) {
    const uint32_t lane = lane_id();
    if (s.temperature <= 0.0f) {  // greedy: argmax (sample.rs:259-265)
        const uint64_t c0 = read_lane_u64(c, 0);
        const uint32_t tok = (nL == 0 || comp_key(c0) == 0) ? 0u : comp_id(c0);
        if (lane == 0) write_single(a, row, tok);
        return;
    }
    const bool in = lane < nL;
    const float v = key_value(comp_key(c));
    const uint32_t id = comp_id(c);
    const bool isnan_v = v != v;
    const uint64_t nonnan = ballot(in && !isnan_v);

    // f32::max fold ignoring NaN, and the no-finite-maximum fallback
    // (sample.rs:270-277).
    float M;
    uint32_t tok_nf = 0;
    if (nonnan == 0) {
        // Negative NaNs sort last, so a -NaN among the best k means the row
        // has no non-NaN value at all; otherwise all k are +NaN.
        const uint64_t negnan = ballot(in && isnan_v && (comp_key(c) & 0x80000000u) == 0);
        if (negnan != 0 || nL < k) {
            M = -__builtin_inff();
        } else {
            if constexpr (BUILD_SET) {
                if (pen) window_build_wave(ws, wrow, wl, a.vocab);
            }
            rescan_row(rowp, a.vocab, ws, pen, s.repeat_penalty, &M, &tok_nf);
        }
    } else {
        const uint32_t f = (uint32_t)__ffsll((long long)nonnan) - 1;
        M = read_lane_f32(v, f);
        // +inf: the lowest id holding it is the first non-NaN candidate.
        tok_nf = read_lane_u32(id, f);
    }
    if (!(M > -__builtin_inff() && M < __builtin_inff())) {
        const uint32_t tok = (M == __builtin_inff()) ? tok_nf : 0u;
        if (lane == 0) write_single(a, row, tok);
        return;
    }

    // exp and the f64 mass (sample.rs:307-311). The argument is never
    // positive (v <= M, T > 0) unless it is NaN (a NaN candidate, or an
    // infinite T): the branch-free non-positive exp runs on every lane (its
    // table is read across lanes), and a NaN gives NaN, as libm's does.
    const float xe = (v - M) / s.temperature;
    const float ee = expf_libm_nonpos_t(xe, LaneExpTable{tab_v});
    const float p = in ? (xe != xe ? xe + xe : ee) : 0.0f;
    // Every nonzero p is a multiple of 2^(e - 23) for its exponent e, and
    // there are at most 64 terms of at most 1, so every partial sum is below
    // 2^7: when the smallest exponent is -23 or more, every f64 partial sum
    // needs at most 53 bits and is exact, and a wave scan (or total) gives the
    // reference's sequential sums bit for bit.
    const int pe = (in && p != 0.0f) ? f32_exponent(p) : (1 << 20);
    const bool exact = wave_min_i32(pe) >= -23;
    uint32_t m = nL;
    if (s.top_p < 1.0f) {  // sample.rs:313-324
        if (exact) {
            const double cum = wave_incl_f64(in ? (double)p : 0.0);
            const double target = (double)s.top_p * uniform_f64(f64_from_bits(read_lane_u64(f64_bits(cum), nL - 1)));
            const uint64_t hit = ballot(in && cum >= target);
            if (hit != 0) m = (uint32_t)__ffsll((unsigned long long)hit);
        } else {
            double sum = 0.0;
            for (uint32_t j = 0; j < nL; ++j) sum += (double)read_lane_f32(p, j);
            const double target = (double)s.top_p * sum;
            double cum = 0.0;
            for (uint32_t j = 0; j < nL; ++j) {
                cum += (double)read_lane_f32(p, j);
                if (cum >= target) {
                    m = j + 1;
                    break;
                }
            }
        }
    }
    bool keep = lane < m;
    uint32_t pos = lane;
    if (s.min_p > 0.0f) {  // stable compaction, sample.rs:326-340
        const bool surv = lane < m && p >= s.min_p;
        const uint64_t sm = ballot(surv);
        const uint32_t w = (uint32_t)__popcll(sm);
        if (w == 0) {
            keep = lane == 0;
            pos = 0;
            m = 1;
        } else {
            keep = surv;
            pos = lanes_below(sm);
            m = w;
        }
    }
    const uint64_t km = ballot(keep);
    double total = 0.0;  // sample.rs:342
    if (exact)
        total = uniform_f64(wave_total_f64(keep ? (double)p : 0.0));
    else
        for (uint64_t mm = km; mm; mm &= mm - 1) total += (double)read_lane_f32(p, (uint32_t)__ffsll((long long)mm) - 1);
    const float inv = (float)(1.0 / total);  // sample.rs:343
    const float q = p * inv;
    float cum = 0.0f;  // the draw, sample.rs:349-358
    uint32_t tok = read_lane_u32(id, 63u - (uint32_t)__clzll((long long)km));
    for (uint64_t mm = km; mm; mm &= mm - 1) {
        const uint32_t j = (uint32_t)__ffsll((long long)mm) - 1;
        cum += read_lane_f32(q, j);
        if (cum > u) {
            tok = read_lane_u32(id, j);
            break;
        }
    }
    if (keep && a.out_ids) {
        store_out(a, a.out_ids + (uint64_t)row * a.cand_stride + pos, id);
        store_out(a, a.out_probs + (uint64_t)row * a.cand_stride + pos, q);
    }
    if (lane == 0) {
        store_out(a, a.out_token + row, tok);
        store_out(a, a.out_used + row, (uint8_t)1);
    }
    store_kept_last(a, row, m, lane == 0);
}

// Merges the window's distinct ids, with their penalised values
// (sample.rs:242-255), into the wave's sorted candidates `top`; returns how
// many were offered. In greedy mode ids whose penalised value argmax could
// never pick (NaN, -inf) are left out. When `top` already holds k candidates,
// `floor` is the k-th of them and ids at or below it are left out too (they
// cannot be among the k best), which usually leaves nothing to sort.
__device__ __forceinline__ uint32_t merge_window(uint64_t &top, const WindowSet &ws, float penalty, bool greedy,
                                                 uint64_t floor) {
    const uint32_t lane = lane_id();
    uint32_t offered = 0;
    for (uint32_t base = 0; base < ws.slots; base += WAVE) {
        const uint32_t i = base + lane;
        const uint32_t id = ws.ids[i];
        uint64_t c = 0;
        if (id != EMPTY_ID) {
            const float x = penalize(ws.vals[i], penalty);
            const uint32_t key = greedy ? argmax_key(x) : total_key(x);
            if (!greedy || key != 0) c = composite(key, id);
            if (c <= floor) c = 0;
        }
        const uint64_t present = ballot(c != 0);
        if (present == 0) continue;
        offered += (uint32_t)__popcll(present);
        top = wave_merge64(top, wave_sort64<false>(c));
    }
    return offered;
}

// A sorted (descending) list of n <= 64 composites as an ascending lane
// vector: lane i holds list[63 - i], zeros where the list is shorter.
__device__ __forceinline__ uint64_t ascending_from(const uint64_t *list, uint32_t n) {
    const uint32_t j = WAVE - 1 - lane_id();
    return j < n ? list[j] : 0ull;
}

// Merges for lists of at most 32 entries (top-k <= 32), two to a wave: a
// vector whose lanes 0-31 and 32-63 hold two independent sequences. half_merge
// takes x with lists A (lanes 0-31) and C (32-63) descending and y with B and
// D ascending, and returns the 32 best of A and B descending in lanes 0-31 and
// of C and D ascending in lanes 32-63 (max(desc, asc) is bitonic and holds
// the 32 best; one 32-lane merge network sorts both halves, five stages
// against the six of a 64-lane merge, for two pairs at once). fold_halves
// then merges the two halves: lanes 0-31 get the 32 best of both, in the
// order DESC (lanes 32-63: the same set in the other order).
__device__ __forceinline__ uint64_t half_merge(uint64_t x, uint64_t y) {
    return bitonic_merge<32, 16, true>(x > y ? x : y);
}
template <bool DESC>
__device__ __forceinline__ uint64_t fold_halves(uint64_t v) {
    const uint64_t o = lane_xor64<32>(v);
    return bitonic_merge<32, 16, DESC>(o > v ? o : v);
}

// The one-tile kernel's finishing chunk when every list holds at most 32
// entries (k <= 32): the row's k best of the chunks' lists by half_merge and
// fold_halves. Each of the first four waves takes the lists j = wave (mod 4)
// in groups of four: a group is two loads a lane (lists 0 and 2 of the group
// descending in x, 1 and 3 ascending in y), one half_merge and one fold;
// the second group's result, folded ascending, merges into the first's.
// Wave 0 then merges the four waves' results the same way. Ends with wave
// 0's finalize_row; the other waves return.
template <uint32_t NW>
__device__ __forceinline__ void finish_top32(const RowIO &a, const FastScratch &sc, uint32_t slot, uint32_t row,
                                             uint32_t k, uint32_t lane, uint32_t wave, uint64_t *part,
                                             uint32_t *s_cnt, const rl_sampling &s, const WindowSet &ws, bool pen,
                                             const float *rowp, uint64_t tab_v, float u_row, const uint32_t *wrow,
                                             uint32_t wl) {
    constexpr uint32_t FW = NW < 4 ? NW : 4;
    constexpr uint32_t GROUPS = (MAX_CHUNKS + 4 * FW - 1) / (4 * FW);
    const uint32_t C = a.chunks;
    const uint64_t *lists = sc.chunk_cands + (uint64_t)slot * C * KMAX;
    const uint32_t *counts = sc.chunk_counts + slot * C;
    const bool merging = wave < FW;
    const uint32_t h = lane >> 5, e = lane & 31u;
    // List i of this wave (i = 4g + pos) is chunk wave + FW * i; lane l loads
    // entry e (x, descending) or 31 - e (y, ascending) of list pos = 2h (x)
    // or 2h + 1 (y). A later group holding one list only (`single`) is
    // loaded ascending into lanes 0-31 instead and merged into the first
    // group's result directly.
    uint64_t x[GROUPS], y[GROUPS];
    uint32_t nx[GROUPS], ny[GROUPS];
    bool single[GROUPS];
#pragma unroll
    for (uint32_t g = 0; g < GROUPS; ++g) {
        const uint32_t jx = wave + FW * (4 * g + 2 * h), jy = jx + FW;
        single[g] = g > 0 && wave + FW * (4 * g + 1) >= C;
        const bool okx = merging && jx < C, oky = merging && jy < C;
        const uint32_t ex = single[g] ? 31u - e : e;
        nx[g] = okx ? __hip_atomic_load(counts + jx, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0u;
        ny[g] = oky ? __hip_atomic_load(counts + jy, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0u;
        x[g] = okx ? __hip_atomic_load(lists + (uint64_t)jx * KMAX + ex, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0ull;
        y[g] = oky ? __hip_atomic_load(lists + (uint64_t)jy * KMAX + (31u - e), __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT)
                   : 0ull;
    }
    uint32_t total = 0;
    uint64_t top = 0;
#pragma unroll
    for (uint32_t g = 0; g < GROUPS; ++g) {
        // Each list's count once: lane 0 holds lists 0 and 1 of the group, lane 32 lists 2 and 3.
        total += read_lane_u32(nx[g] + ny[g], 0) + read_lane_u32(nx[g] + ny[g], 32);
        const uint64_t xv = (single[g] ? 31u - e : e) < nx[g] ? x[g] : 0ull, yv = 31u - e < ny[g] ? y[g] : 0ull;
        if (g == 0) {
            top = fold_halves<true>(half_merge(xv, yv));
        } else if (single[g]) {
            if (merging && wave + FW * 4 * g < C) {
                const uint64_t r = lane < 32 ? xv : 0ull;
                top = bitonic_merge<32, 16, true>(top > r ? top : r);
            }
        } else if (merging && wave + FW * 4 * g < C) {
            const uint64_t r = fold_halves<false>(half_merge(xv, yv));
            top = bitonic_merge<32, 16, true>(top > r ? top : r);
        }
    }
    // The waves' results (lanes 0-31, descending) through LDS; wave 0 merges
    // them as one group: results 0 and 2 descending, 1 and 3 ascending.
    __syncthreads();  // the candidate buffers are free
    if (lane < 32) part[wave * 32 + lane] = top;
    if (lane == 0) s_cnt[wave] = total;
    __syncthreads();
    if (wave != 0) return;
    uint32_t all = 0;
#pragma unroll
    for (uint32_t j = 0; j < FW; ++j) all += s_cnt[j];
    if constexpr (FW == 4) {
        top = fold_halves<true>(half_merge(part[(2 * h) * 32 + e], part[(2 * h + 1) * 32 + (31u - e)]));
    } else {
#pragma unroll
        for (uint32_t j = 1; j < FW; ++j) {
            const uint64_t r = lane < 32 ? part[j * 32 + (31u - lane)] : 0ull;
            top = bitonic_merge<32, 16, true>(top > r ? top : r);
        }
    }
    if (lane == 0) sc.arrive[slot] = 0;  // ready for the next call
    const uint32_t nL = all < k ? all : k;
    if (lane >= nL) top = 0;
    finalize_row<true>(a, row, s, k, top, nL, ws, pen, rowp, tab_v, u_row, wrow, wl);
}

// LDS words of a bitmap over a chunk of at most `elems` elements (one word
// more: a chunk that starts mid-word never reads past it).
__host__ __device__ constexpr uint32_t chunk_bitmap_words(uint32_t elems) { return (elems + 31) / 32 + 1; }

// grid (chunks, rows on this path), NT threads (NT / 64 waves, each with its
// own candidate buffer), U float4 a thread per tile. Dynamic LDS: the window
// set. A row split into chunks is finished by whichever of its chunks
// publishes its list last (a per-row arrival counter), so no second launch.
//
// ONE_TILE: every chunk of the launch holds at most one tile (q1 - q0 <=
// NT * U; the rows of a small call, split over many workgroups). The window
// is then applied where the reference applies it: the chunk marks the window
// ids that fall in it in an LDS bitmap over its elements and penalises those
// logits in its tile's registers before filtering, so its candidates carry
// the penalised values (each id once, however often the window repeats it),
// with no set of the whole window, no gather of window logits and no
// separate merge. Dynamic LDS: that bitmap, then, for the rare rescan of a
// row whose best are all NaN, a set of the window built by one wave.
template <bool VEC, uint32_t U, uint32_t NT, bool ONE_TILE = false>
__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(4))) void k_stream(RowIO a, FastScratch sc) {
    constexpr uint32_t NW = NT / WAVE;
    constexpr uint32_t CBUF = TileShape<U>::CBUF;
    __shared__ uint64_t s_buf[NW * CBUF];
    __shared__ uint64_t s_T;
    __shared__ uint32_t s_cnt[NW];
    __shared__ uint32_t s_tq[NW];  // ONE_TILE: each wave's candidate bound (a key) from the bootstrap
    __shared__ uint32_t s_tn[NW];  // ONE_TILE: lane maxima of the chunk at or above s_tq[j]
    extern __shared__ __align__(16) uint8_t smem[];
    const WindowSet ws = window_set(smem, a.hash_bits);
    const uint32_t slot = blockIdx.y, chunk = blockIdx.x;
    // The common case, every row on this path, needs no lookup before the
    // row's address is known.
    const uint32_t row = a.rows ? a.rows[slot] : a.row0 + slot;
    const float *rowp = a.logits + (uint64_t)row * a.stride;
    const uint32_t V = a.vocab;
    const uint32_t tid = threadIdx.x;
    const uint32_t wave = tid / WAVE;
    const uint32_t lane = lane_id();

    // Loop bounds are wave-uniform; readfirstlane keeps them in SGPRs so the
    // loop control is scalar. chunk * n4 < MAX_CHUNKS * 2^19 fits 32 bits.
    static_assert((uint64_t)MAX_CHUNKS * (1u << 19) < (1ull << 32), "chunk bounds in 32 bits");
    const uint32_t n4 = V / 4;
    const uint32_t q0 = uniform_u32(chunk * n4 / a.chunks);
    const uint32_t q1 = uniform_u32((chunk + 1) * n4 / a.chunks);
    constexpr uint32_t STEP = NT * U;
    const uint32_t nfull = (q1 - q0) / STEP;                    // whole tiles
    const uint32_t ntiles = nfull + ((q1 - q0) % STEP ? 1 : 0);  // plus a partial one

    // Set-up, ordered so that no wait for one load also waits for a tile:
    // the row's settings and window length (one vector load, row_words) and
    // the window ids are loaded first, then the first tile; the ids go into
    // the set, and each id's raw logit is loaded and stored only after the
    // bootstrap has consumed the tile. The id and tile loads are addressed
    // from kernel arguments alone (the id load is clamped to the call's
    // window stride, and which ids count is decided once the settings and
    // length have arrived). A window longer than the workgroup (rare) is
    // built in full after the tile loads, its own loads waiting behind the
    // tile.
    const uint32_t head_w = row_words(a, row);
    const uint32_t *wrow = a.windows + (uint64_t)row * a.wstride;
    const bool have_win = a.windows && a.wlen && a.wstride > 0;
    const uint32_t *idp = have_win ? wrow + (tid < a.wstride ? tid : a.wstride - 1)
                                   : reinterpret_cast<const uint32_t *>(a.settings + row);
    // ONE_TILE loads the window's ids WIN_PER a thread (windows of up to
    // ONE_TILE_WIN_MAX ids; longer ones never reach this kernel), clamped to
    // the call's stride.
    constexpr uint32_t WIN_PER = ONE_TILE ? (ONE_TILE_WIN_MAX + NT - 1) / NT : 1;
    uint32_t wid[WIN_PER];
    if constexpr (ONE_TILE) {
        const uint32_t *wsrc = have_win ? wrow : reinterpret_cast<const uint32_t *>(a.settings + row);
        const uint32_t wn = have_win ? (a.wstride < WIN_PER * NT ? a.wstride : WIN_PER * NT) : 1u;
#pragma unroll
        for (uint32_t j = 0; j < WIN_PER; ++j) {
            const uint32_t i = j * NT + tid;
            wid[j] = ((const RL_GLB uint32_t *)wsrc)[i < wn ? i : wn - 1];
        }
    } else {
        wid[0] = *(const RL_GLB uint32_t *)idp;  // unconditional, see load_tile_clamped
    }
    // The first tile. A row of fewer than 4 logits has no tile; it loads 16
    // bytes of its own settings instead, so that this load needs no branch
    // either.
    f32x4 A[U], B[U];
    {
        const bool any = ntiles > 0;
        load_tile_clamped<VEC, U, NT>(A, any ? rowp : (const float *)(a.settings + row), any ? q0 : 0u, any ? q1 : 1u);
    }
    // The settings and window length are needed from here on (the barrier
    // keeps the wait for them below the tile's loads).
    __builtin_amdgcn_sched_barrier(0);
    rl_sampling s;
    uint32_t wl;
    row_head(a, head_w, s, wl);
    const bool greedy = s.temperature <= 0.0f;
    const uint32_t k = uniform_u32(greedy ? 1u : (uint32_t)s.top_k);
    const bool pen = penalises(s) && wl > 0;
    RL_LDS uint64_t *lT = (RL_LDS uint64_t *)&s_T;
    if (tid == 0) *lT = 0;
    if constexpr (ONE_TILE) {
        if (tid < NW) s_tn[tid] = 0;
    }
    // The chunk's elements [e0, e1): the last chunk also holds the row's
    // last vocab % 4 elements.
    const uint32_t e0 = 4 * q0, e1 = chunk == a.chunks - 1 ? V : 4 * q1;
    RL_LDS uint32_t *bm = (RL_LDS uint32_t *)smem;
    uint32_t my_slot = EMPTY_ID, my_id = EMPTY_ID;
    float my_raw = 0.0f;
    if constexpr (ONE_TILE) {
        if (pen) {
            const uint32_t nwords = (e1 - e0 + 31) / 32;
            for (uint32_t i = tid; i < nwords; i += NT) bm[i] = 0;
        }
        __syncthreads();  // the slots above are set, the bitmap is clear
        if (pen) {
#pragma unroll
            for (uint32_t j = 0; j < WIN_PER; ++j) {
                const uint32_t id = wid[j];
                if (j * NT + tid < wl && id >= e0 && id < e1)
                    (void)__hip_atomic_fetch_or(&bm[(id - e0) >> 5], 1u << ((id - e0) & 31), __ATOMIC_RELAXED,
                                                __HIP_MEMORY_SCOPE_WORKGROUP);
            }
            __syncthreads();
            // The tile's window elements take their penalised values: the
            // four bits of float4 f sit in one word (e0 is a multiple of 4).
#pragma unroll
            for (uint32_t u = 0; u < U; ++u) {
                const uint32_t f = q0 + u * NT + tid;
                const uint32_t r = f < q1 ? f - q0 : 0u;
                const uint32_t bits = f < q1 ? (bm[r >> 3] >> ((r & 7) * 4)) & 0xFu : 0u;
                if (bits) {
                    if (bits & 1u) A[u].x = penalize(A[u].x, s.repeat_penalty);
                    if (bits & 2u) A[u].y = penalize(A[u].y, s.repeat_penalty);
                    if (bits & 4u) A[u].z = penalize(A[u].z, s.repeat_penalty);
                    if (bits & 8u) A[u].w = penalize(A[u].w, s.repeat_penalty);
                }
            }
        }
    } else {
        const bool small_win = pen && wl <= NT;
        if (pen && !small_win)
            window_build(ws, wrow, wl, V, rowp, true);  // ends with a barrier
        else
            window_clear(ws);
        __syncthreads();
        my_id = (small_win && tid < wl) ? wid[0] : EMPTY_ID;
        my_slot = my_id < V ? window_insert(ws, my_id) : EMPTY_ID;
        my_raw = ((const RL_GLB float *)rowp)[my_slot != EMPTY_ID ? my_id : 0u];
        __syncthreads();
    }

    Stream w;
    w.buf = (RL_LDS uint64_t *)s_buf + wave * CBUF;
    w.shared_T = lT;
    w.ws = ws;
    w.wtop = ~0ull;  // the raw logits are not in yet: check every candidate
    w.T = 0;
    w.thr = greedy ? -3.40282347e38f : -__builtin_inff();
    w.cnt = 0;
    w.k = k;
    w.greedy = greedy;
    w.pen = ONE_TILE ? false : pen;  // ONE_TILE: the tile is penalised already

    // Wave priority falls as the row progresses (see set_progress_priority).
    __builtin_amdgcn_s_setprio(3);
    if (ntiles > 0) {
        if constexpr (ONE_TILE) {
            // A bound for the whole chunk: any t with at least k of the
            // chunk's lane maxima (distinct elements) at or above it is at
            // most the chunk's k-th best, so nothing below it is among the
            // chunk's k best. The candidates are each wave's ceil(k / NW)-th
            // lane maximum tq (the least of them always qualifies: every
            // wave has ceil(k / NW) lane maxima at or above it); each wave
            // counts its lane maxima at or above every candidate, and the
            // largest candidate with k in all is the bound. Much tighter
            // than one wave's k-th lane maximum.
            // Lane j < NW handles candidate j: one LDS read of the
            // candidates, one atomic add of this wave's counts, one read of
            // the totals. Keys, as in bootstrap_keys.
            const uint32_t sorted = bootstrap_keys<U, NT>(w, A, q0, q1);
            const uint32_t tq = read_lane_u32(sorted, (k + NW - 1) / NW - 1);
            if (lane == 0) s_tq[wave] = tq;
            __syncthreads();
            const uint32_t cand = lane < NW ? s_tq[lane] : 0u;
            uint32_t cnt = 0;
#pragma unroll
            for (uint32_t j = 0; j < NW; ++j) {
                const uint32_t t = read_lane_u32(cand, j);
                const uint32_t c = (uint32_t)__popcll(ballot(sorted != 0 && sorted >= t));
                cnt = lane == j ? c : cnt;
            }
            if (lane < NW && cnt) (void)__hip_atomic_fetch_add(&s_tn[lane], cnt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            __syncthreads();
            const bool qualifies = lane < NW && s_tn[lane] >= k;
            const uint32_t tc = wave_fold_u32(qualifies ? cand : 0u, [](uint32_t x, uint32_t y) { return x > y ? x : y; });
            raise_threshold(w, tc ? ((uint64_t)tc << 32) - 1 : 0ull);
        } else {
            (void)bootstrap<U, NT>(w, A, q0, q1);
        }
    }
    if (ntiles <= 1) {
        // One tile or none (a chunk of a split row): nothing more to load.
        // The window's raw logits were loaded behind the tile, so they are
        // stored after it is filtered (wtop stays ~0 meanwhile: compaction
        // checks every candidate against the window set); merge_window reads
        // them at the end.
        if (nfull == 1)
            process_tile<false, U, NT>(w, A, q0, q1);
        else if (ntiles == 1)
            process_tile<true, U, NT>(w, A, q0, q1);
        if constexpr (!ONE_TILE) {
            if (my_slot != EMPTY_ID) window_store(ws, my_slot, my_id, my_raw);
            __syncthreads();
            w.wtop = window_top(ws);
        }
    } else if constexpr (!ONE_TILE) {
        // Tile 1 goes out before the window's raw logits are stored, so the
        // store's wait covers the gather alone and the memory pipe stays full.
        load_tile_clamped<VEC, U, NT>(B, rowp, q0 + STEP, q1);
        if (my_slot != EMPTY_ID) window_store(ws, my_slot, my_id, my_raw);
        __syncthreads();
        w.wtop = window_top(ws);
        // Double-buffered: tile t+1 is in flight while tile t is filtered.
        // Loads past the chunk are clamped (they cost one cache line per
        // wave), so the last, partial tile runs through the same loop.
        for (uint32_t t = 0; t < ntiles; t += 2) {
            const uint32_t b0 = q0 + t * STEP, b1 = b0 + STEP;
            if (t < nfull)
                process_tile<false, U, NT>(w, A, b0, q1);
            else
                process_tile<true, U, NT>(w, A, b0, q1);
            load_tile_clamped<VEC, U, NT>(A, rowp, b1 + STEP, q1);
            if (t + 1 < nfull)
                process_tile<false, U, NT>(w, B, b1, q1);
            else if (t + 1 < ntiles)
                process_tile<true, U, NT>(w, B, b1, q1);
            load_tile_clamped<VEC, U, NT>(B, rowp, b1 + 2 * STEP, q1);
            raise_threshold(w, load_shared_T(lT));
            set_progress_priority(t + 2, ntiles);
        }
    }
    __builtin_amdgcn_s_setprio(0);
    // The tail's table entry and uniform, in flight through the row's end.
    const uint64_t tab_v = lane_exp_entry();
    const float u_row = row_uniform(a, row);
    // The row's last vocab % 4 elements.
    if (chunk == a.chunks - 1) {
        if (w.cnt >= w.k + SLACK) compact(w);
        const uint32_t e = 4 * n4 + tid;
        const bool ok = e < V;
        float x = ok ? ((const RL_GLB float *)rowp)[e] : 0.0f;
        if constexpr (ONE_TILE) {
            if (pen && ok && ((bm[(e - e0) >> 5] >> ((e - e0) & 31)) & 1u)) x = penalize(x, s.repeat_penalty);
        }
        offer_group<true>(w, f32x4{x, 0.f, 0.f, 0.f}, e, ok ? 1u : 0u);
    }
    // ONE_TILE: when the waves' buffers hold at most 64 candidates in all
    // (the usual case under the chunk's bound), wave 0 sorts them together
    // once, in place of a sort per wave and a merge per list.
    bool gathered = false;
    if constexpr (ONE_TILE) {
        if (lane == 0) s_cnt[wave] = w.cnt;
        __syncthreads();
        uint32_t all = 0;
#pragma unroll
        for (uint32_t j = 0; j < NW; ++j) all += s_cnt[j];
        gathered = all <= WAVE;
        if (!gathered) {
            compact(w);
            __syncthreads();  // every wave has read the counts
            if (lane == 0) s_cnt[wave] = w.cnt;
            __syncthreads();
        }
    } else {
        compact(w);
        if (lane == 0) s_cnt[wave] = w.cnt;
        __syncthreads();
    }
    __shared__ uint32_t s_last;
    if (wave == 0) {
        const uint64_t *lb = (const uint64_t *)s_buf;
        uint64_t top;
        uint32_t total;
        if (ONE_TILE && gathered) {
            // Lane i takes candidate i: wave j's follow wave j - 1's.
            uint32_t at = 0, base = 0;
#pragma unroll
            for (uint32_t j = 0; j < NW; ++j) {
                const uint32_t c = s_cnt[j];
                if (lane >= base && lane < base + c) at = j * CBUF + (lane - base);
                base += c;
            }
            total = base;
            const uint64_t c = lane < total ? lb[at] : 0ull;
            // Up to 32: a 32-lane network (lanes 32-63 hold zeros).
            top = total <= 32 ? bitonic_sort<32, true>(c) : wave_sort64<true>(c);
        } else {
            // Merge the NW sorted lists: lane i of list j is candidate i of wave j.
            top = lane < s_cnt[0] ? lb[lane] : 0ull;
            total = s_cnt[0];
#pragma unroll
            for (uint32_t j = 1; j < NW; ++j) {
                top = wave_merge64(top, ascending_from(lb + j * CBUF, s_cnt[j]));
                total += s_cnt[j];
            }
        }
        // The window's ids with their penalised values, once per row.
        if (!ONE_TILE && pen && chunk == 0)
            total += merge_window(top, ws, s.repeat_penalty, greedy, total >= k ? read_lane_u64(top, k - 1) : 0ull);
        const uint32_t nL = total < k ? total : k;
        if (lane >= nL) top = 0;
        if (a.chunks == 1) {
            finalize_row<ONE_TILE>(a, row, s, k, top, nL, ws, pen, rowp, tab_v, u_row, wrow, wl);
        } else {
            // Publish this chunk's list; the row's last chunk to arrive finishes
            // it. The list is written with device-scope stores, which write
            // through this XCD's L2, and the arrival waits until they have
            // completed: the list is then visible to every XCD, with no
            // writeback of the whole L2 (what a device-scope fence costs,
            // serialised per XCD).
            uint64_t *dst = sc.chunk_cands + ((uint64_t)slot * a.chunks + chunk) * KMAX;
            if (lane < nL) __hip_atomic_store(dst + lane, top, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (lane == 0)
                __hip_atomic_store(sc.chunk_counts + slot * a.chunks + chunk, nL, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
            __builtin_amdgcn_s_waitcnt(WAITCNT_VM0);  // the stores have completed
            uint32_t old = 0;
            if (lane == 0) old = atomicAdd(&sc.arrive[slot], 1u);
            old = read_lane_u32(old, 0);
            if (lane == 0) s_last = old == a.chunks - 1 ? 1u : 0u;
        }
    }
    if (a.chunks == 1) return;
    __syncthreads();
    if (!s_last) return;
    if constexpr (ONE_TILE) {
        if (k <= 32) {
            finish_top32<NW>(a, sc, slot, row, k, lane, wave, (uint64_t *)s_buf, s_cnt, s, ws, pen, rowp, tab_v, u_row,
                             wrow, wl);
            return;
        }
    }
    // The last chunk of the row: every chunk's list is published. Each of
    // the first FW waves merges the lists j = wave (mod FW), all loaded at
    // once, then wave 0 merges their results and runs the tail (more waves
    // would add more to wave 0's merges than they take off theirs). The
    // lists are read with device-scope loads, which bypass this XCD's L2,
    // issued after the arrival that saw every other chunk's.
    const uint64_t *lists = sc.chunk_cands + (uint64_t)slot * a.chunks * KMAX;
    const uint32_t *counts = sc.chunk_counts + slot * a.chunks;
    constexpr uint32_t FW = NW < 4 ? NW : 4;
    const bool merging = FW == NW || wave < FW;
    // A row is split into at most MAX_CHUNKS.
    constexpr uint32_t PER = (MAX_CHUNKS + FW - 1) / FW;
    uint64_t v[PER];
    uint32_t n[PER];
#pragma unroll
    for (uint32_t i = 0; i < PER; ++i) {
        const uint32_t j = wave + FW * i;
        const bool ok = merging && j < a.chunks;
        n[i] = ok ? __hip_atomic_load(counts + j, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0u;
        v[i] = ok ? __hip_atomic_load(lists + (uint64_t)j * KMAX + (WAVE - 1 - lane), __ATOMIC_RELAXED,
                                      __HIP_MEMORY_SCOPE_AGENT)
                  : 0ull;
    }
    uint64_t top = 0;
    uint32_t total = 0;
#pragma unroll
    for (uint32_t i = 0; i < PER; ++i) {
        if (!merging || wave + FW * i >= a.chunks) break;
        top = wave_merge64(top, WAVE - 1 - lane < n[i] ? v[i] : 0ull);  // lane i: list[63 - i], ascending
        total += n[i];
    }
    uint64_t *part = (uint64_t *)s_buf;
    __syncthreads();  // the candidate buffers are free
    part[wave * WAVE + lane] = top;
    if (lane == 0) s_cnt[wave] = total;
    __syncthreads();
    if (wave != 0) return;
    total = s_cnt[0];
#pragma unroll
    for (uint32_t j = 1; j < FW; ++j) {
        top = wave_merge64(top, part[j * WAVE + (WAVE - 1 - lane)]);
        total += s_cnt[j];
    }
    if (lane == 0) sc.arrive[slot] = 0;  // ready for the next call
    const uint32_t nL = total < k ? total : k;
    if (lane >= nL) top = 0;
    finalize_row<ONE_TILE>(a, row, s, k, top, nL, ws, pen, rowp, tab_v, u_row, wrow, wl);
}

// ------------------------------------------------------------ argmax ---
// grid (chunks, rows): per-chunk best argmax composite.
template <bool VEC>
__global__ __launch_bounds__(FAST_THREADS) void k_argmax_part(const float *logits, uint64_t stride,
                                                              uint32_t vocab, uint32_t chunks,
                                                              uint64_t *part) {
    __shared__ uint64_t red[FAST_WAVES];
    const uint32_t row = blockIdx.y, chunk = blockIdx.x;
    const float *rowp = logits + (uint64_t)row * stride;
    const uint32_t n4 = vocab / 4;
    const uint32_t q0 = (uint32_t)((uint64_t)chunk * n4 / chunks);
    const uint32_t q1 = (uint32_t)((uint64_t)(chunk + 1) * n4 / chunks);
    uint64_t best = 0;
    // Double-buffered tiles of UNROLL float4 per thread; loads past the chunk
    // are clamped and their values skipped.
    constexpr uint32_t STEP = FAST_THREADS * UNROLL;
    if (q1 > q0) {
        f32x4 A[UNROLL], B[UNROLL];
        load_tile_clamped<VEC>(A, rowp, q0, q1);
        for (uint32_t b = q0; b < q1; b += STEP) {
            load_tile_clamped<VEC>(B, rowp, b + STEP, q1);
#pragma unroll
            for (uint32_t u = 0; u < UNROLL; ++u) {
                const uint32_t f = b + u * FAST_THREADS + threadIdx.x;
                const float x[4] = {A[u].x, A[u].y, A[u].z, A[u].w};
#pragma unroll
                for (uint32_t c = 0; c < 4; ++c) {
                    const uint64_t cc = f < q1 ? composite(argmax_key(x[c]), 4 * f + c) : 0ull;
                    best = cc > best ? cc : best;
                }
            }
#pragma unroll
            for (uint32_t u = 0; u < UNROLL; ++u) A[u] = B[u];
        }
    }
    if (chunk == chunks - 1) {
        const uint32_t e = 4 * n4 + threadIdx.x;
        if (e < vocab) {
            const uint64_t cc = composite(argmax_key(rowp[e]), e);
            best = cc > best ? cc : best;
        }
    }
    best = wave_max_u64(best);
    if (lane_id() == 0) red[threadIdx.x / WAVE] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
        for (uint32_t i = 1; i < FAST_WAVES; ++i) best = red[i] > best ? red[i] : best;
        part[(uint64_t)row * chunks + chunk] = best;
    }
}

__global__ void k_argmax_final(const uint64_t *part, uint32_t rows, uint32_t chunks, uint32_t *out) {
    const uint32_t row = blockIdx.x * blockDim.x + threadIdx.x;
    if (row >= rows) return;
    uint64_t best = 0;
    for (uint32_t c = 0; c < chunks; ++c) {
        const uint64_t x = part[(uint64_t)row * chunks + c];
        best = x > best ? x : best;
    }
    out[row] = comp_key(best) == 0 ? 0u : comp_id(best);
}

__global__ void k_expf_range(uint32_t lo_bits, uint64_t count, float *out) {
    __shared__ uint64_t tab[32];
    copy_exp_table((RL_LDS uint64_t *)tab);
    const LdsExpTable etab{(RL_LDS uint64_t *)tab};
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < count) out[i] = expf_libm_t(__uint_as_float(lo_bits + (uint32_t)i), etab);
}

}  // namespace rl
