// The sampler's kernels. Two device paths, chosen per row from its settings:
//
//  STREAM (greedy rows, and 1 <= top_k <= 64 with top_k < vocab): one pass
//  over the row in HBM. Each wave keeps the row's best candidates seen so far
//  in LDS under a rising threshold (a workgroup-wide one, shared through an
//  LDS atomic max), so almost every element costs one compare. Penalised
//  window ids are left out of the stream and offered with their penalised
//  values, so the logits are never written. The last wave merges the lists
//  and replays the reference's tail (sample.rs:267-358) on <= 64 candidates,
//  one candidate per lane.
//
//  FULL (top_k == 0, top_k >= vocab, or top_k > 64): the reference's literal
//  algorithm: total-order keys for the whole row, an LSD radix sort of the
//  row, then the sequential sums and the draw over the sorted row.
#pragma once
#include "rl_device.h"
#include "rl_expf.h"

namespace rl {

constexpr uint32_t FAST_THREADS = 256;
constexpr uint32_t FAST_WAVES = FAST_THREADS / WAVE;
constexpr uint32_t KMAX = 64;     // largest top_k the stream path takes (one per lane)
constexpr uint32_t WBUF = 256;    // per-wave candidate buffer
constexpr uint32_t UNROLL = 8;    // float4 loads per thread per tile
constexpr uint32_t MAX_CHUNKS = 32;
constexpr uint32_t FULL_THREADS = 256;
constexpr uint32_t SORT_THREADS = 1024;
constexpr uint32_t SORT_WAVES = SORT_THREADS / WAVE;
constexpr uint32_t STAGE = 4096;  // elements staged in LDS per sequential block

struct RowIO {
    const float *logits;
    uint64_t stride;
    uint32_t vocab;
    const rl_sampling *settings;  // indexed by row
    const uint32_t *rows;         // this path's rows: rows[slot] = row index
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
};

struct FastScratch {
    uint64_t *chunk_cands;   // [slot][chunk][KMAX]
    uint32_t *chunk_counts;  // [slot][chunk]
};

struct FullScratch {
    uint32_t *keyA, *idA, *keyB, *idB;  // [slot][vocab]
    float *probs;                       // [slot][vocab]
    float *part_max;                    // [slot][chunk]
    uint64_t *part_am;                  // [slot][chunk]
};

__device__ __forceinline__ uint32_t window_len(const RowIO &a, uint32_t row) {
    if (!a.wlen || !a.windows) return 0;
    const uint32_t l = a.wlen[row];
    return l < a.wstride ? l : a.wstride;
}

__device__ __forceinline__ void write_single(const RowIO &a, uint32_t row, uint32_t tok) {
    a.out_token[row] = tok;
    a.out_kept[row] = 1;
    a.out_used[row] = 0;
    if (a.out_ids) {
        a.out_ids[(uint64_t)row * a.cand_stride] = tok;
        a.out_probs[(uint64_t)row * a.cand_stride] = 1.0f;
    }
}

template <bool VEC>
__device__ __forceinline__ float4 load4(const float *row, uint32_t f) {
    if constexpr (VEC) {
        return reinterpret_cast<const float4 *>(row)[f];
    } else {
        const float *p = row + 4ull * f;
        return make_float4(p[0], p[1], p[2], p[3]);
    }
}

// ------------------------------------------------- per-wave candidates ---
struct WaveCands {
    uint64_t *buf;       // LDS, WBUF entries
    uint64_t *shared_T;  // LDS, the workgroup's threshold
    uint64_t T;          // everything kept is > T (a k-th best seen somewhere)
    float thr;           // value of T's key: a cheap necessary test
    uint32_t cnt;
    uint32_t k;
    bool greedy;
};

// Necessary condition for composite(x) > T, one compare: in greedy mode the
// starting -FLT_MAX also drops NaN and -inf, which argmax never picks; in
// sampled mode !(x < thr) lets NaN through to the exact test.
__device__ __forceinline__ bool prefilter(const WaveCands &w, float x) {
    return w.greedy ? (x >= w.thr) : !(x < w.thr);
}

__device__ __forceinline__ void take_threshold(WaveCands &w, uint64_t t) {
    if (t > w.T) {
        w.T = t;
        w.thr = key_value(comp_key(t));
    }
}

__device__ __forceinline__ void refresh(WaveCands &w) {
    const uint64_t s = uniform_u64(__hip_atomic_load((unsigned long long *)w.shared_T, __ATOMIC_RELAXED,
                                                     __HIP_MEMORY_SCOPE_WORKGROUP));
    take_threshold(w, s);
}

// Keeps the wave's k best, sorted, and raises the threshold to the k-th.
__device__ __noinline__ void compact(WaveCands &w) {
    const uint32_t lane = lane_id();
    wave_lds_sync();
    for (uint32_t i = lane; i < WBUF; i += WAVE)
        if (i >= w.cnt) w.buf[i] = 0;
    wave_lds_sync();
    wave_sort_desc(w.buf, WBUF);
    if (w.cnt >= w.k) {
        const uint64_t t = uniform_u64(w.buf[w.k - 1]);
        w.cnt = w.k;
        take_threshold(w, t);
        if (lane == 0) atomicMax((unsigned long long *)w.shared_T, (unsigned long long)w.T);
    }
    refresh(w);
}

// Appends this wave's passing lanes (ballot compaction), compacting first when
// the buffer would overflow.
__device__ __forceinline__ void offer(WaveCands &w, bool pass, uint64_t c) {
    uint64_t m = ballot(pass);
    if (m == 0) return;
    uint32_t n = __popcll(m);
    if (w.cnt + n > WBUF) {
        compact(w);
        pass = pass && (c > w.T);
        m = ballot(pass);
        if (m == 0) return;
        n = __popcll(m);
    }
    if (pass) w.buf[w.cnt + lanes_below(m)] = c;
    w.cnt += n;
}

template <bool CHECK>
__device__ __forceinline__ void offer_group(WaveCands &w, const WindowSet &ws, bool pen, float4 v,
                                            uint32_t id0, uint32_t nvalid) {
    const float x[4] = {v.x, v.y, v.z, v.w};
    bool any = false;
#pragma unroll
    for (uint32_t c = 0; c < 4; ++c) any |= (!CHECK || c < nvalid) && prefilter(w, x[c]);
    if (ballot(any) == 0) return;
#pragma unroll
    for (uint32_t c = 0; c < 4; ++c) {
        bool p = (!CHECK || c < nvalid) && prefilter(w, x[c]);
        uint64_t comp = 0;
        if (p) {
            const uint32_t key = w.greedy ? total_key(x[c] + 0.0f) : total_key(x[c]);
            comp = composite(key, id0 + c);
            p = comp > w.T;
            if (p && pen) p = !window_contains(ws, id0 + c);
        }
        offer(w, p, comp);
    }
}

// k-way merge of sorted lists (one list per lane) by repeated wave max; writes
// the best k to out and returns how many there were.
__device__ __forceinline__ uint32_t merge_heads(const uint64_t *lists, uint32_t list_stride,
                                                const uint32_t *counts, uint32_t nlists, uint32_t k,
                                                uint64_t *out) {
    const uint32_t lane = lane_id();
    const uint32_t cnt = lane < nlists ? counts[lane] : 0u;
    uint32_t pos = 0;
    uint32_t n = 0;
    for (; n < k; ++n) {
        const uint64_t h = pos < cnt ? lists[(uint64_t)lane * list_stride + pos] : 0ull;
        const uint64_t mx = wave_max_u64(h);
        if (mx == 0) break;
        if (pos < cnt && h == mx) ++pos;
        if (lane == 0) out[n] = mx;
    }
    wave_lds_sync();
    return n;
}

// The row's f32::max fold over the penalised logits and its argmax, by one
// wave re-reading the row. Only for a row whose k best are all +NaN, where the
// candidates do not reveal the largest non-NaN value.
__device__ __noinline__ void rescan_row(const float *rowp, uint32_t vocab, const WindowSet &ws,
                                        bool pen, float penalty, float *out_max, uint32_t *out_tok) {
    const uint32_t lane = lane_id();
    float mx = -__builtin_inff();
    uint64_t am = 0;
    for (uint32_t e = lane; e < vocab; e += WAVE) {
        float x = rowp[e];
        if (pen && window_contains(ws, e)) x = penalize(x, penalty);
        mx = fmaxf(mx, x);
        const uint64_t c = composite(argmax_key(x), e);
        am = c > am ? c : am;
    }
    *out_max = uniform_f32(wave_maxnum_f32(mx));
    am = uniform_u64(wave_max_u64(am));
    *out_tok = comp_key(am) == 0 ? 0u : comp_id(am);
}

// The reference's tail (sample.rs:259-358) over the row's best nL candidates
// L (sorted, descending), by one wave: candidate j sits in lane j. The
// sequential f64 and f32 sums are replayed in candidate order with readlane,
// so every lane computes the same bits the reference does.
__device__ __noinline__ void finalize_row(const RowIO &a, uint32_t row, const rl_sampling &s,
                                          uint32_t k, const uint64_t *L, uint32_t nL,
                                          const WindowSet &ws, bool pen, const float *rowp) {
    const uint32_t lane = lane_id();
    if (s.temperature <= 0.0f) {  // greedy: argmax (sample.rs:259-265)
        const uint64_t c0 = nL ? uniform_u64(L[0]) : 0ull;
        const uint32_t tok = (comp_key(c0) == 0) ? 0u : comp_id(c0);
        if (lane == 0) write_single(a, row, tok);
        return;
    }
    const bool in = lane < nL;
    const uint64_t c = in ? L[lane] : 0ull;
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

    // exp and the f64 mass (sample.rs:307-311).
    const float p = in ? expf_libm((v - M) / s.temperature) : 0.0f;
    uint32_t m = nL;
    if (s.top_p < 1.0f) {  // sample.rs:313-324
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
    for (uint64_t mm = km; mm; mm &= mm - 1) total += (double)read_lane_f32(p, (uint32_t)__ffsll((long long)mm) - 1);
    const float inv = (float)(1.0 / total);  // sample.rs:343
    const float q = p * inv;
    const float u = a.uniforms[row];
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
        a.out_ids[(uint64_t)row * a.cand_stride + pos] = id;
        a.out_probs[(uint64_t)row * a.cand_stride + pos] = q;
    }
    if (lane == 0) {
        a.out_token[row] = tok;
        a.out_kept[row] = m;
        a.out_used[row] = 1;
    }
}

// LDS layout of the stream kernel (dynamic shared memory).
struct FastLds {
    uint64_t *wbufs;     // FAST_WAVES * WBUF
    uint64_t *mlist;     // KMAX
    uint64_t *shared_T;  // 1
    uint32_t *wcount;    // FAST_WAVES
    WindowSet ws;
};

__host__ __device__ constexpr size_t fast_lds_bytes(uint32_t hash_bits) {
    return (FAST_WAVES * WBUF + KMAX + 2) * sizeof(uint64_t) + FAST_WAVES * sizeof(uint32_t) +
           ((size_t)1 << hash_bits) * (sizeof(uint32_t) + sizeof(float));
}

__device__ __forceinline__ FastLds fast_lds(uint8_t *smem, uint32_t hash_bits) {
    FastLds l;
    l.wbufs = reinterpret_cast<uint64_t *>(smem);
    l.mlist = l.wbufs + FAST_WAVES * WBUF;
    l.shared_T = l.mlist + KMAX;
    l.wcount = reinterpret_cast<uint32_t *>(l.shared_T + 2);
    l.ws.bits = hash_bits;
    l.ws.slots = 1u << hash_bits;
    l.ws.ids = l.wcount + FAST_WAVES;
    l.ws.vals = reinterpret_cast<float *>(l.ws.ids + l.ws.slots);
    return l;
}

// grid (chunks, rows on this path), FAST_THREADS threads.
template <bool VEC>
__global__ __launch_bounds__(FAST_THREADS) void k_stream(RowIO a, FastScratch sc) {
    extern __shared__ __align__(16) uint8_t smem[];
    FastLds l = fast_lds(smem, a.hash_bits);
    const uint32_t slot = blockIdx.y, chunk = blockIdx.x;
    const uint32_t row = a.rows[slot];
    const rl_sampling s = a.settings[row];
    const bool greedy = s.temperature <= 0.0f;
    const uint32_t k = greedy ? 1u : (uint32_t)s.top_k;
    const uint32_t wl = window_len(a, row);
    const bool pen = penalises(s) && wl > 0;
    const float *rowp = a.logits + (uint64_t)row * a.stride;
    const uint32_t V = a.vocab;
    const uint32_t wave = threadIdx.x / WAVE;
    const uint32_t lane = lane_id();

    if (threadIdx.x == 0) *l.shared_T = 0;
    window_build(l.ws, a.windows + (uint64_t)row * a.wstride, wl, V, rowp, pen);

    WaveCands w;
    w.buf = l.wbufs + wave * WBUF;
    w.shared_T = l.shared_T;
    w.T = 0;
    w.thr = greedy ? -3.40282347e38f : -__builtin_inff();
    w.cnt = 0;
    w.k = k;
    w.greedy = greedy;

    const uint32_t n4 = V / 4;
    const uint32_t q0 = (uint32_t)((uint64_t)chunk * n4 / a.chunks);
    const uint32_t q1 = (uint32_t)((uint64_t)(chunk + 1) * n4 / a.chunks);
    constexpr uint32_t STEP = FAST_THREADS * UNROLL;
    const uint32_t ntiles = (q1 - q0) / STEP;

    float4 A[UNROLL], B[UNROLL];
    if (ntiles > 0) {
#pragma unroll
        for (uint32_t u = 0; u < UNROLL; ++u) A[u] = load4<VEC>(rowp, q0 + u * FAST_THREADS + threadIdx.x);
    }
    for (uint32_t t = 0; t < ntiles; t += 2) {
        const uint32_t b0 = q0 + t * STEP, b1 = b0 + STEP, b2 = b1 + STEP;
        if (t + 1 < ntiles) {
#pragma unroll
            for (uint32_t u = 0; u < UNROLL; ++u) B[u] = load4<VEC>(rowp, b1 + u * FAST_THREADS + threadIdx.x);
        }
#pragma unroll
        for (uint32_t u = 0; u < UNROLL; ++u) {
            const uint32_t f = b0 + u * FAST_THREADS + threadIdx.x;
            offer_group<false>(w, l.ws, pen, A[u], 4 * f, 4);
        }
        if (t + 2 < ntiles) {
#pragma unroll
            for (uint32_t u = 0; u < UNROLL; ++u) A[u] = load4<VEC>(rowp, b2 + u * FAST_THREADS + threadIdx.x);
        }
        if (t + 1 < ntiles) {
#pragma unroll
            for (uint32_t u = 0; u < UNROLL; ++u) {
                const uint32_t f = b1 + u * FAST_THREADS + threadIdx.x;
                offer_group<false>(w, l.ws, pen, B[u], 4 * f, 4);
            }
        }
        refresh(w);
    }
    // The chunk's partial tile, then the row's last vocab % 4 elements.
    const uint32_t rb = q0 + ntiles * STEP;
    for (uint32_t u = 0; u < UNROLL; ++u) {
        const uint32_t f = rb + u * FAST_THREADS + threadIdx.x;
        const bool ok = f < q1;
        const float4 v = ok ? load4<VEC>(rowp, f) : make_float4(0.f, 0.f, 0.f, 0.f);
        offer_group<true>(w, l.ws, pen, v, 4 * f, ok ? 4u : 0u);
    }
    if (chunk == a.chunks - 1) {
        const uint32_t e = 4 * n4 + threadIdx.x;
        const bool ok = e < V;
        const float x = ok ? rowp[e] : 0.0f;
        offer_group<true>(w, l.ws, pen, make_float4(x, 0.f, 0.f, 0.f), e, ok ? 1u : 0u);
    }
    // The window's ids with their penalised values, once per row.
    if (pen && chunk == 0) {
        for (uint32_t base = wave * WAVE; base < l.ws.slots; base += FAST_THREADS) {
            const uint32_t i = base + lane;
            const uint32_t id = i < l.ws.slots ? l.ws.ids[i] : EMPTY_ID;
            bool p = false;
            uint64_t c = 0;
            if (id != EMPTY_ID) {
                const float x = penalize(l.ws.vals[i], s.repeat_penalty);
                const uint32_t key = greedy ? argmax_key(x) : total_key(x);
                c = composite(key, id);
                p = (!greedy || key != 0) && c > w.T;
            }
            offer(w, p, c);
        }
    }
    compact(w);
    if (lane == 0) l.wcount[wave] = w.cnt;
    __syncthreads();
    if (wave != 0) return;
    const uint32_t nL = merge_heads(l.wbufs, WBUF, l.wcount, FAST_WAVES, k, l.mlist);
    if (a.chunks == 1) {
        finalize_row(a, row, s, k, l.mlist, nL, l.ws, pen, rowp);
    } else {
        uint64_t *dst = sc.chunk_cands + ((uint64_t)slot * a.chunks + chunk) * KMAX;
        if (lane < nL) dst[lane] = l.mlist[lane];
        if (lane == 0) sc.chunk_counts[slot * a.chunks + chunk] = nL;
    }
}

// grid (rows on this path), one wave: merges the chunks' lists and finishes.
__global__ __launch_bounds__(WAVE) void k_stream_finalize(RowIO a, FastScratch sc) {
    extern __shared__ __align__(16) uint8_t smem[];
    uint64_t *mlist = reinterpret_cast<uint64_t *>(smem);
    WindowSet ws;
    ws.bits = a.hash_bits;
    ws.slots = 1u << a.hash_bits;
    ws.ids = reinterpret_cast<uint32_t *>(mlist + KMAX);
    ws.vals = reinterpret_cast<float *>(ws.ids + ws.slots);
    const uint32_t slot = blockIdx.x;
    const uint32_t row = a.rows[slot];
    const rl_sampling s = a.settings[row];
    const bool greedy = s.temperature <= 0.0f;
    const uint32_t k = greedy ? 1u : (uint32_t)s.top_k;
    const uint32_t wl = window_len(a, row);
    const bool pen = penalises(s) && wl > 0;
    const float *rowp = a.logits + (uint64_t)row * a.stride;
    window_build(ws, a.windows + (uint64_t)row * a.wstride, wl, a.vocab, rowp, pen);
    const uint32_t nL = merge_heads(sc.chunk_cands + (uint64_t)slot * a.chunks * KMAX, KMAX,
                                    sc.chunk_counts + slot * a.chunks, a.chunks, k, mlist);
    finalize_row(a, row, s, k, mlist, nL, ws, pen, rowp);
}

// ---------------------------------------------------------- FULL path ---
__host__ __device__ constexpr size_t window_lds_bytes(uint32_t hash_bits) {
    return ((size_t)1 << hash_bits) * (sizeof(uint32_t) + sizeof(float));
}

__device__ __forceinline__ uint32_t full_k(const rl_sampling &s, uint32_t V) {
    return s.top_k == 0 ? V : (s.top_k < V ? (uint32_t)s.top_k : V);  // sample.rs:289
}
__device__ __forceinline__ bool identity_order(const rl_sampling &s, uint32_t V) {
    return full_k(s, V) == V && !(s.top_p < 1.0f);  // no select and no sort
}

// grid (chunks, slots), FULL_THREADS: the penalised row as total-order keys in
// id order, plus per-chunk f32::max fold and argmax.
__global__ __launch_bounds__(FULL_THREADS) void k_full_keys(RowIO a, FullScratch f) {
    extern __shared__ __align__(16) uint8_t smem[];
    WindowSet ws;
    ws.bits = a.hash_bits;
    ws.slots = 1u << a.hash_bits;
    ws.ids = reinterpret_cast<uint32_t *>(smem);
    ws.vals = reinterpret_cast<float *>(ws.ids + ws.slots);
    __shared__ float red_max[FULL_THREADS / WAVE];
    __shared__ uint64_t red_am[FULL_THREADS / WAVE];
    const uint32_t slot = blockIdx.y, chunk = blockIdx.x;
    const uint32_t row = a.rows[slot];
    const rl_sampling s = a.settings[row];
    const uint32_t V = a.vocab;
    const uint32_t wl = window_len(a, row);
    const bool pen = penalises(s) && wl > 0;
    const float *rowp = a.logits + (uint64_t)row * a.stride;
    window_build(ws, a.windows + (uint64_t)row * a.wstride, wl, V, rowp, pen);
    const uint32_t e0 = (uint32_t)((uint64_t)chunk * V / a.chunks);
    const uint32_t e1 = (uint32_t)((uint64_t)(chunk + 1) * V / a.chunks);
    uint32_t *keys = f.keyA + (uint64_t)slot * V;
    uint32_t *ids = f.idA + (uint64_t)slot * V;
    float mx = -__builtin_inff();
    uint64_t am = 0;
    for (uint32_t e = e0 + threadIdx.x; e < e1; e += FULL_THREADS) {
        float x = rowp[e];
        if (pen && window_contains(ws, e)) x = penalize(x, s.repeat_penalty);
        keys[e] = total_key(x);
        ids[e] = e;
        mx = fmaxf(mx, x);
        const uint64_t c = composite(argmax_key(x), e);
        am = c > am ? c : am;
    }
    mx = wave_maxnum_f32(mx);
    am = wave_max_u64(am);
    const uint32_t wave = threadIdx.x / WAVE;
    if (lane_id() == 0) {
        red_max[wave] = mx;
        red_am[wave] = am;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (uint32_t i = 1; i < FULL_THREADS / WAVE; ++i) {
            mx = fmaxf(mx, red_max[i]);
            am = red_am[i] > am ? red_am[i] : am;
        }
        f.part_max[slot * a.chunks + chunk] = mx;
        f.part_am[slot * a.chunks + chunk] = am;
    }
}

__device__ __forceinline__ void full_row_max(const RowIO &a, const FullScratch &f, uint32_t slot, float *M,
                                             uint32_t *am_tok) {
    float mx = -__builtin_inff();
    uint64_t am = 0;
    for (uint32_t c = 0; c < a.chunks; ++c) {
        mx = fmaxf(mx, f.part_max[slot * a.chunks + c]);
        const uint64_t x = f.part_am[slot * a.chunks + c];
        am = x > am ? x : am;
    }
    *M = mx;
    *am_tok = comp_key(am) == 0 ? 0u : comp_id(am);
}

// One wave's lanes with the same 8-bit digit (among the lanes where valid).
__device__ __forceinline__ uint64_t match_digit(uint32_t d, bool valid) {
    uint64_t m = ballot(valid);
#pragma unroll
    for (uint32_t b = 0; b < 8; ++b) {
        const bool bit = (d >> b) & 1u;
        const uint64_t bb = ballot(bit);
        m &= bit ? bb : ~bb;
    }
    return m;
}

// grid (slots), SORT_THREADS: stable LSD radix sort of the row's (key, id)
// pairs, descending key, 8 bits a pass; ids were in ascending order, so ties
// keep ascending ids (the order of sample.rs:282-286). Result ends in keyA/idA.
__global__ __launch_bounds__(SORT_THREADS) void k_full_sort(RowIO a, FullScratch f) {
    __shared__ uint32_t hist[256];
    __shared__ uint32_t offs[256];
    __shared__ uint32_t cnt[SORT_WAVES][256];
    __shared__ uint32_t pos[SORT_WAVES][256];
    __shared__ uint32_t skip;
    const uint32_t slot = blockIdx.x;
    const uint32_t row = a.rows[slot];
    const rl_sampling s = a.settings[row];
    const uint32_t V = a.vocab;
    float M;
    uint32_t am_tok;
    full_row_max(a, f, slot, &M, &am_tok);
    if (!(M > -__builtin_inff() && M < __builtin_inff())) return;
    if (identity_order(s, V)) return;
    const uint32_t tid = threadIdx.x, wave = tid / WAVE;
    uint32_t *kin = f.keyA + (uint64_t)slot * V, *iin = f.idA + (uint64_t)slot * V;
    uint32_t *kout = f.keyB + (uint64_t)slot * V, *iout = f.idB + (uint64_t)slot * V;
    for (uint32_t i = tid; i < SORT_WAVES * 256; i += SORT_THREADS) (&cnt[0][0])[i] = 0;
    for (uint32_t shift = 0; shift < 32; shift += 8) {
        if (tid < 256) hist[tid] = 0;
        __syncthreads();
        for (uint32_t base = 0; base < V; base += SORT_THREADS) {
            const uint32_t j = base + tid;
            const bool valid = j < V;
            const uint32_t d = valid ? 255u - ((kin[j] >> shift) & 255u) : 0u;
            const uint64_t peers = match_digit(d, valid);
            if (valid && lanes_below(peers) == 0) atomicAdd(&hist[d], (uint32_t)__popcll(peers));
        }
        __syncthreads();
        if (tid == 0) {
            uint32_t run = 0, sk = 0;
            for (uint32_t d = 0; d < 256; ++d) {
                offs[d] = run;
                if (hist[d] == V) sk = 1;
                run += hist[d];
            }
            skip = sk;
        }
        __syncthreads();
        if (skip) continue;  // every key has this digit: the pass would not move anything
        for (uint32_t base = 0; base < V; base += SORT_THREADS) {
            const uint32_t j = base + tid;
            const bool valid = j < V;
            const uint32_t key = valid ? kin[j] : 0u;
            const uint32_t id = valid ? iin[j] : 0u;
            const uint32_t d = 255u - ((key >> shift) & 255u);
            const uint64_t peers = match_digit(d, valid);
            const uint32_t rank = lanes_below(peers);
            if (valid && rank == 0) cnt[wave][d] = (uint32_t)__popcll(peers);
            __syncthreads();
            if (tid < 256) {
                uint32_t run = offs[tid];
                for (uint32_t w = 0; w < SORT_WAVES; ++w) {
                    const uint32_t c = cnt[w][tid];
                    pos[w][tid] = run;
                    run += c;
                    cnt[w][tid] = 0;
                }
                offs[tid] = run;
            }
            __syncthreads();
            if (valid) {
                const uint32_t dst = pos[wave][d] + rank;
                kout[dst] = key;
                iout[dst] = id;
            }
        }
        __syncthreads();
        uint32_t *t;
        t = kin; kin = kout; kout = t;
        t = iin; iin = iout; iout = t;
    }
    if (kin != f.keyA + (uint64_t)slot * V) {  // an odd number of passes ran
        for (uint32_t j = tid; j < V; j += SORT_THREADS) {
            kout[j] = kin[j];
            iout[j] = iin[j];
        }
    }
}

// grid (slots), FULL_THREADS: the reference's tail over the whole (sorted or
// identity-ordered) candidate list. The sequential sums run on thread 0 over
// blocks staged in LDS; the min-p compaction and the normalisation are
// parallel (both are elementwise and stable).
__global__ __launch_bounds__(FULL_THREADS) void k_full_replay(RowIO a, FullScratch f) {
    __shared__ float stage[STAGE];
    __shared__ uint32_t wave_cnt[FULL_THREADS / WAVE];
    __shared__ uint32_t sh_m, sh_done, sh_total;
    __shared__ float sh_inv;
    __shared__ double sh_target;
    const uint32_t slot = blockIdx.x;
    const uint32_t row = a.rows[slot];
    const rl_sampling s = a.settings[row];
    const uint32_t V = a.vocab;
    const uint32_t tid = threadIdx.x, wave = tid / WAVE, lane = lane_id();
    float M;
    uint32_t am_tok;
    full_row_max(a, f, slot, &M, &am_tok);
    if (!(M > -__builtin_inff() && M < __builtin_inff())) {  // sample.rs:270-277
        if (tid == 0) write_single(a, row, am_tok);
        return;
    }
    const uint32_t k = full_k(s, V);
    uint32_t *keys = f.keyA + (uint64_t)slot * V;
    uint32_t *ids = f.idA + (uint64_t)slot * V;
    float *probs = f.probs + (uint64_t)slot * V;
    for (uint32_t j = tid; j < k; j += FULL_THREADS)
        probs[j] = expf_libm((key_value(keys[j]) - M) / s.temperature);  // sample.rs:309
    if (tid == 0) {
        sh_m = k;
        sh_done = 0;
    }
    __syncthreads();

    if (s.top_p < 1.0f) {  // sample.rs:307-324
        double sum = 0.0;
        for (uint32_t b = 0; b < k; b += STAGE) {
            const uint32_t n = min(STAGE, k - b);
            for (uint32_t i = tid; i < n; i += FULL_THREADS) stage[i] = probs[b + i];
            __syncthreads();
            if (tid == 0)
                for (uint32_t i = 0; i < n; ++i) sum += (double)stage[i];
            __syncthreads();
        }
        if (tid == 0) sh_target = (double)s.top_p * sum;
        __syncthreads();
        const double target = sh_target;
        double cum = 0.0;
        for (uint32_t b = 0; b < k; b += STAGE) {
            const uint32_t n = min(STAGE, k - b);
            for (uint32_t i = tid; i < n; i += FULL_THREADS) stage[i] = probs[b + i];
            __syncthreads();
            if (tid == 0) {
                for (uint32_t i = 0; i < n; ++i) {
                    cum += (double)stage[i];
                    if (cum >= target) {
                        sh_m = b + i + 1;
                        sh_done = 1;
                        break;
                    }
                }
            }
            __syncthreads();
            if (sh_done) break;
        }
    }
    uint32_t m = sh_m;
    if (s.min_p > 0.0f) {  // sample.rs:326-340, a stable in-place compaction
        if (tid == 0) sh_total = 0;
        __syncthreads();
        for (uint32_t b = 0; b < m; b += FULL_THREADS) {
            const uint32_t j = b + tid;
            const bool ok = j < m;
            const float p = ok ? probs[j] : 0.0f;
            const uint32_t id = ok ? ids[j] : 0u;
            const bool surv = ok && p >= s.min_p;
            const uint64_t bm = ballot(surv);
            if (lane == 0) wave_cnt[wave] = (uint32_t)__popcll(bm);
            __syncthreads();
            uint32_t before = sh_total, all = 0;
            for (uint32_t w = 0; w < FULL_THREADS / WAVE; ++w) {
                if (w < wave) before += wave_cnt[w];
                all += wave_cnt[w];
            }
            __syncthreads();
            if (surv) {
                const uint32_t dst = before + lanes_below(bm);
                ids[dst] = id;
                probs[dst] = p;
            }
            if (tid == 0) sh_total += all;
            __syncthreads();
        }
        m = sh_total > 1 ? sh_total : 1u;
    }
    // Normalise: f64 total in order, then f32 multiply (sample.rs:342-347).
    double total = 0.0;
    for (uint32_t b = 0; b < m; b += STAGE) {
        const uint32_t n = min(STAGE, m - b);
        for (uint32_t i = tid; i < n; i += FULL_THREADS) stage[i] = probs[b + i];
        __syncthreads();
        if (tid == 0)
            for (uint32_t i = 0; i < n; ++i) total += (double)stage[i];
        __syncthreads();
    }
    if (tid == 0) sh_inv = (float)(1.0 / total);
    __syncthreads();
    const float inv = sh_inv;
    for (uint32_t j = tid; j < m; j += FULL_THREADS) {
        const float q = probs[j] * inv;
        probs[j] = q;
        if (a.out_ids) {
            a.out_ids[(uint64_t)row * a.cand_stride + j] = ids[j];
            a.out_probs[(uint64_t)row * a.cand_stride + j] = q;
        }
    }
    if (tid == 0) {
        sh_done = 0;
        sh_m = ids[m - 1];  // f32 shortfall: the last candidate (sample.rs:357-358)
    }
    __syncthreads();
    // The draw: f32 running sum against the host's uniform (sample.rs:349-356).
    const float u = a.uniforms[row];
    float cum = 0.0f;
    for (uint32_t b = 0; b < m; b += STAGE) {
        const uint32_t n = min(STAGE, m - b);
        for (uint32_t i = tid; i < n; i += FULL_THREADS) stage[i] = probs[b + i];
        __syncthreads();
        if (tid == 0) {
            for (uint32_t i = 0; i < n; ++i) {
                cum += stage[i];
                if (cum > u) {
                    sh_m = ids[b + i];
                    sh_done = 1;
                    break;
                }
            }
        }
        __syncthreads();
        if (sh_done) break;
    }
    if (tid == 0) {
        a.out_token[row] = sh_m;
        a.out_kept[row] = m;
        a.out_used[row] = 1;
    }
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
    for (uint32_t f = q0 + threadIdx.x; f < q1; f += FAST_THREADS) {
        const float4 v = load4<VEC>(rowp, f);
        const float x[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (uint32_t c = 0; c < 4; ++c) {
            const uint64_t cc = composite(argmax_key(x[c]), 4 * f + c);
            best = cc > best ? cc : best;
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
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < count) out[i] = expf_libm(__uint_as_float(lo_bits + (uint32_t)i));
}

}  // namespace rl
