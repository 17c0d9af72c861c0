// The FULL path's second launch, k_full_rest: one workgroup per row that
// k_full_pass left unfinished. It puts the row's candidates in the reference's
// order (descending penalised logit, ascending id; sample.rs:279-305) with a
// stable LSD radix sort whose passes are chosen by one histogram read, computes
// p = exp((l - max) / T) as the last pass writes each candidate in place
// (:309), takes the mass, the top-p cut, min-p and the normalising total
// (:307-343), draws against the host's uniform (:349-358) and writes the kept
// candidates q = p * (1 / total) (:344-347).
//
// HBM per row: the logits once or twice for the digit histograms, one read of
// the logits for the first pass, 8 bytes read and 8 written per element for
// each further pass (the last writes ids and p, to the candidate outputs when
// the caller asked for them), a read of p for the per-chunk sums, and a read
// and write of the kept prefix for the normalisation (the draw reads up to its
// pick). A row the pass finished exits at once, so a call whose rows all
// finished in the pass costs one empty launch here.
#pragma once
#include "full_kernels.h"

namespace rl {

constexpr uint32_t REST_THREADS = 1024;
constexpr uint32_t REST_WAVES = REST_THREADS / WAVE;
constexpr uint32_t REST_ITEMS = 8;                         // elements per lane per tile of a pass
constexpr uint32_t REST_TILE = REST_THREADS * REST_ITEMS;  // elements per tile
constexpr uint32_t REST_SEG = WAVE * REST_ITEMS;           // a wave's contiguous share of a tile
constexpr uint32_t HIST_ITEMS = 12;                        // loads per thread per histogram step
constexpr uint32_t HIST_STEP = REST_THREADS * HIST_ITEMS;  // elements per histogram step
constexpr uint32_t STAT_CHUNKS = 64;                       // most chunks of the candidate list's sums
constexpr uint32_t STAT_MIN_LOG = 11;                      // chunks of at least 2^11 candidates
constexpr uint32_t HIST_COPIES = 16;                       // histogram copies (lanes with equal lane & 15 share one)
constexpr uint32_t HIST_ROW = 257;                         // a copy's stride: copies of a digit fall in different banks
static_assert(HIST_STEP >= REST_TILE, "the window bitmap covers a tile");

struct RestLds {
    union {
        struct {
            uint32_t k[REST_TILE];  // the tile's keys, reordered by digit
            uint32_t i[REST_TILE];  // and their ids
            double csum[HIST_COPIES][STAT_CHUNKS + 1];  // the last pass's chunk sums of p, a copy per lane group
        } tile;
        uint32_t gh[2][HIST_COPIES * HIST_ROW];  // two digits' histograms, one copy per lane group
        struct {
            float stage[STAGE];
            ChunkLds cr;
        } rep;
    } u;
    uint32_t hist[4][256];           // the row's digit histograms (digits flipped: 255 - d)
    uint32_t offs[256];              // a pass's next output position per digit
    uint32_t cnt[REST_WAVES][256];   // per wave: the tile's count per digit, then its start within the digit's run
    uint64_t peer[REST_WAVES][256];  // per wave: the lanes of one item with each digit (zero between items)
    uint32_t tcount[256], tstart[256];
    uint32_t bm[HIST_STEP / 32];     // window ids in the current step, one bit per element
    uint32_t cls[4];                 // OR and AND of the keys with the top bit clear, then set
    uint64_t exp_tab[32];
    // The f64 sum of p per chunk of the candidate list (2^SH candidates, the
    // last one shorter); and over the whole list the smallest binary exponent
    // of a nonzero p, a NaN or infinite p, the count with p >= min_p, the last
    // index + 1 with p >= min_p and the first with p < min_p.
    double seg_sum[STAT_CHUNKS];
    int st_emin;
    uint32_t st_bad, st_count, st_last_in, st_first_out;
    double red_d[REST_WAVES];
    int64_t red_l[REST_WAVES];
    uint32_t red_u[REST_WAVES];
    uint32_t hcnt[REST_WAVES];       // per wave: the tile's elements with the hot key
    uint32_t run0[257];              // packed passes: where each digit's run of the first pass's output starts
    uint8_t dmap[REST_TILE];         // packed passes: the first pass's digit of each element of the tile
    uint32_t sh_hot_key, sh_hot_count, sh_hot_above;
    uint32_t sh_m, sh_stop, sh_hit, sh_tok;
    double sh_d, sh_hit_sum;
};

// A buffer resource over n 32-bit words at p (raw addressing; gfx9's
// descriptor word 3, 0x00020000: 32-bit data format). Loads at byte offsets
// past 4n return zero and stores there are dropped, so tiles need no clamps;
// each access takes one 32-bit offset register (plus an immediate) instead of
// a 64-bit address.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t words_rsrc(const void *p, uint32_t n) {
    return __builtin_amdgcn_make_buffer_rsrc((void *)p, (short)0, (int)(n * 4u), 0x00020000);
}
// The words [from, from + n) of p, or none when from is past n words.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t tail_rsrc(const uint32_t *p, uint32_t from, uint32_t n) {
    return from < n ? words_rsrc(p + from, n - from) : words_rsrc(p, 0);
}
template <bool NT = false>
__device__ __forceinline__ uint32_t bload(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, byte_off, 0, NT ? 2 : 0);
}
__device__ __forceinline__ void bstore(__amdgpu_buffer_rsrc_t r, uint32_t byte_off, uint32_t v) {
    __builtin_amdgcn_raw_buffer_store_b32(v, r, byte_off, 0, 0);
}

// ------------------------------------------------------ block helpers ---
template <uint32_t NT>
__device__ __forceinline__ uint32_t block_sum_u32(uint32_t v, RL_LDS uint32_t *red) {
    v = wave_sum_u32(v);
    __syncthreads();
    if (lane_id() == 0) red[threadIdx.x / WAVE] = v;
    __syncthreads();
    uint32_t t = 0;
    for (uint32_t w = 0; w < NT / WAVE; ++w) t += red[w];
    return t;
}

template <uint32_t NT>
__device__ __forceinline__ int64_t block_max_i64(int64_t v, RL_LDS int64_t *red) {
    v = (int64_t)wave_fold_u64((uint64_t)v, [](uint64_t a, uint64_t b) { return (int64_t)a > (int64_t)b ? a : b; });
    __syncthreads();
    if (lane_id() == 0) red[threadIdx.x / WAVE] = v;
    __syncthreads();
    int64_t t = red[0];
    for (uint32_t w = 1; w < NT / WAVE; ++w) t = red[w] > t ? red[w] : t;
    return t;
}

// Exclusive prefix of v over the workgroup's threads in thread order; *total
// gets the sum. For doubles it is only used where every partial sum is exact.
template <uint32_t NT, class T>
__device__ __forceinline__ T block_exclusive(T v, RL_LDS T *red, T *total) {
    const uint32_t lane = lane_id(), wave = threadIdx.x / WAVE;
    T incl;
    if constexpr (std::is_same<T, double>::value) {
        incl = wave_incl_f64(v);
    } else {
        static_assert(std::is_same<T, uint32_t>::value, "u32 or f64");
        incl = wave_incl_u32(v);
    }
    __syncthreads();
    if (lane == WAVE - 1) red[wave] = incl;
    __syncthreads();
    T before = 0, all = 0;
    for (uint32_t w = 0; w < NT / WAVE; ++w) {
        if (w < wave) before += red[w];
        all += red[w];
    }
    *total = all;
    return before + incl - v;
}

// Walks src[0..n) in order on thread 0, one LDS-staged block at a time; the
// whole workgroup stages. body(stage, base, count) returns true to stop.
template <uint32_t NT, class Body>
__device__ __forceinline__ void staged_walk(const float *src, uint32_t n, RL_LDS float *stage, RL_LDS uint32_t *stop,
                                            Body body) {
    for (uint32_t b = 0; b < n; b += STAGE) {
        const uint32_t cnt = min(STAGE, n - b);
        for (uint32_t i = threadIdx.x; i < cnt; i += NT) stage[i] = ((const RL_GLB float *)src)[b + i];
        __syncthreads();
        if (threadIdx.x == 0) *stop = body(stage, b, cnt) ? 1u : 0u;
        __syncthreads();
        if (*stop) break;
    }
}

// Where every partial sum of the probabilities is exact: the first j in
// [lo, hi) with base + p[lo] + ... + p[j] >= target, and that sum in *at; or
// hi, with the sum of them all in *at. Any order of addition gives these exact
// sums, so a block scan serves. Whole workgroup.
template <uint32_t NT>
__device__ __forceinline__ uint32_t exact_first_reaching(const float *probs, uint32_t lo, uint32_t hi, double base, double target,
                                         RL_LDS double *red, RL_LDS uint32_t *hit, RL_LDS double *hit_sum,
                                         double *at, const HotRange &hr) {
    for (uint32_t b = lo; b < hi; b += NT * CI) {
        const uint32_t j0 = b + threadIdx.x * CI;
        float pv[CI];
        double mine = 0.0;
#pragma unroll
        for (uint32_t i = 0; i < CI; ++i) {
            uint32_t w = hr.word;
            if (j0 + i < hi && !hr.has(j0 + i)) w = ((const RL_GLB uint32_t *)probs)[j0 + i];
            pv[i] = j0 + i < hi ? __uint_as_float(w) : 0.0f;
            mine += (double)pv[i];
        }
        if (threadIdx.x == 0) *hit = 0xFFFFFFFFu;
        double step_total;
        double c = base + block_exclusive<NT, double>(mine, red, &step_total);
        uint32_t my_hit = 0xFFFFFFFFu;
        double my_sum = 0.0;
#pragma unroll
        for (uint32_t i = 0; i < CI; ++i) {
            if (my_hit == 0xFFFFFFFFu && j0 + i < hi) {
                c += (double)pv[i];
                if (c >= target) {
                    my_hit = j0 + i;
                    my_sum = c;
                }
            }
        }
        if (my_hit != 0xFFFFFFFFu) atomicMin((uint32_t *)hit, my_hit);
        __syncthreads();
        const uint32_t h = *hit;
        if (h != 0xFFFFFFFFu) {
            if (my_hit == h) *hit_sum = my_sum;
            __syncthreads();
            *at = *hit_sum;
            __syncthreads();
            return h;
        }
        base += step_total;
        __syncthreads();
    }
    *at = base;
    return hi;
}

// What a pass needs of its row.
struct RestRow {
    const float *rowp;   // the raw logits
    const uint32_t *win; // the recent-token window
    uint32_t V, k, wl;
    bool pen;
    float penalty, M;
    TempScale tscale;
};

// Window ids in [e0, e0 + n) as bits of L->bm (n <= HIST_STEP). Whole
// workgroup; two barriers.
__device__ __forceinline__ void window_bits(RL_LDS RestLds *L, const RestRow &r, uint32_t e0, uint32_t n) {
    for (uint32_t i = threadIdx.x; i < (n + 31) / 32; i += REST_THREADS) L->bm[i] = 0;
    __syncthreads();
    for (uint32_t i = threadIdx.x; i < r.wl; i += REST_THREADS) {
        const uint32_t id = r.win[i];
        if (id >= e0 && id - e0 < n) atomicOr((uint32_t *)&L->bm[(id - e0) >> 5], 1u << ((id - e0) & 31));
    }
    __syncthreads();
}

// The penalised logit (sample.rs:239-257) of element e0 + off, x its raw
// value, from the bits of the step that starts at e0. An id repeated in the
// window has one bit, so it is penalised once.
__device__ __forceinline__ float penalised(RL_LDS const RestLds *L, const RestRow &r, float x, uint32_t off) {
    return ((L->bm[off >> 5] >> (off & 31)) & 1u) ? penalize(x, r.penalty) : x;
}
// The same with off's word (off >> 5) and bit (off & 31) given.
__device__ __forceinline__ float penalised_at(RL_LDS const RestLds *L, const RestRow &r, float x, uint32_t word,
                                              uint32_t bit) {
    return ((L->bm[word] >> bit) & 1u) ? penalize(x, r.penalty) : x;
}

// The histograms of digits hi and lo (8 bits at 8 * hi and 8 * lo) of the
// penalised row's total-order keys into L->hist[hi] and L->hist[lo]. Each
// lane adds its digits to one of HIST_COPIES copies (lane & 15), so one LDS
// atomic holds at most four lanes on one counter even when most of a row's
// logits are tied, and a copy's row of HIST_ROW counters puts the copies of
// a digit in different banks. The first call (`first`) also puts the OR and
// AND of the keys of each sign into L->cls, and picks a hot key: from the
// first step, the key that the most lanes of one wave-item share with the
// item's first lane, the row's commonest key whenever one key holds a large
// share of the row (any key would do: it only decides which elements skip the
// sort). It counts the keys equal to it and above it into L->sh_hot_count and
// L->sh_hot_above. One read of the logits, HIST_ITEMS loads per thread in
// flight.
__device__ __forceinline__ void rest_histograms(RL_LDS RestLds *L, const RestRow &r, uint32_t hi, uint32_t lo,
                                                bool first) {
    const uint32_t tid = threadIdx.x, lane = lane_id(), wave = tid / WAVE;
    const uint32_t V = r.V;
    constexpr uint32_t GH = HIST_COPIES * HIST_ROW;
    for (uint32_t i = tid; i < 2 * GH; i += REST_THREADS) (&L->u.gh[0][0])[i] = 0;
    if (first && tid < 4) L->cls[tid] = (tid & 1) ? 0xFFFFFFFFu : 0u;
    if (first && tid == 0) {
        L->sh_hot_count = 0;
        L->sh_hot_above = 0;
    }
    __syncthreads();
    uint32_t K = first ? 0u : L->sh_hot_key;
    uint32_t nK = 0, nA = 0;  // this wave's keys equal to K and above it
    RL_LDS uint32_t *h_hi = &L->u.gh[0][(lane & (HIST_COPIES - 1)) * HIST_ROW];
    RL_LDS uint32_t *h_lo = &L->u.gh[1][(lane & (HIST_COPIES - 1)) * HIST_ROW];
    uint32_t or0 = 0u, and0 = 0xFFFFFFFFu, or1 = 0u, and1 = 0xFFFFFFFFu;
    const uint32_t s_hi = 8 * hi, s_lo = 8 * lo;
    // A step gives each wave a contiguous segment, HIST_ITEMS elements a lane
    // 64 apart; the next step's loads are issued before this step's
    // elements are counted.
    const uint32_t wbase = wave * WAVE * HIST_ITEMS + lane;
    const uint32_t hoff = 4 * wbase;  // item i adds 256 i bytes
    const uint32_t *raw = (const uint32_t *)r.rowp;
    uint32_t nx[HIST_ITEMS];
    {
        const auto rs = tail_rsrc(raw, 0, V);
#pragma unroll
        for (uint32_t i = 0; i < HIST_ITEMS; ++i) nx[i] = bload<true>(rs, hoff + 256 * i);
    }
    for (uint32_t b = 0; b < V; b += HIST_STEP) {
        uint32_t x[HIST_ITEMS];
        const auto rs = tail_rsrc(raw, b + HIST_STEP, V);
        // The items' offsets are formed from an opaque copy each step, so they
        // are not all held in registers across the loop.
        uint32_t ho = hoff;
        asm volatile("" : "+v"(ho));
#pragma unroll
        for (uint32_t i = 0; i < HIST_ITEMS; ++i) {
            x[i] = nx[i];
            nx[i] = bload<true>(rs, ho + 256 * i);
        }
        if (r.pen) window_bits(L, r, b, min(HIST_STEP, V - b));
#pragma unroll
        for (uint32_t i = 0; i < HIST_ITEMS; ++i) {
            const float v = r.pen ? penalised_at(L, r, __uint_as_float(x[i]), (wbase >> 5) + 2 * i, wbase & 31u)
                                  : __uint_as_float(x[i]);
            x[i] = total_key(v);
        }
        if (first && b == 0) {
            uint64_t best = 0;  // (lanes << 32) | key
#pragma unroll
            for (uint32_t i = 0; i < HIST_ITEMS; ++i) {
                const uint64_t vm = ballot((int)wbase < (int)V - (int)(i * WAVE));
                if (vm != 0) {
                    const uint32_t k0 = uniform_u32(read_lane_u32(x[i], (uint32_t)__builtin_ctzll(vm)));
                    const uint64_t c = (uint64_t)__popcll(vm & ballot(x[i] == k0));
                    const uint64_t cand = (c << 32) | k0;
                    best = cand > best ? cand : best;
                }
            }
            if (lane == 0) L->red_l[wave] = (int64_t)best;
            __syncthreads();
            uint64_t kb = 0;
            for (uint32_t w = 0; w < REST_WAVES; ++w) kb = (uint64_t)L->red_l[w] > kb ? (uint64_t)L->red_l[w] : kb;
            K = (uint32_t)kb;
            if (tid == 0) L->sh_hot_key = K;
        }
#pragma unroll
        for (uint32_t i = 0; i < HIST_ITEMS; ++i) {
            const bool valid = (int)wbase < (int)(V - b) - (int)(i * WAVE);
            const uint32_t key = x[i];
            if (first) {
                // Keys with the top bit set, then clear (invalid lanes in neither).
                const uint32_t m1 = valid ? 0u - (key >> 31) : 0u;
                const uint32_t m0 = valid ? ~m1 : 0u;
                or1 |= key & m1;
                and1 &= key | ~m1;
                or0 |= key & m0;
                and0 &= key | ~m0;
                const uint64_t vm = ballot(valid);
                nK += (uint32_t)__popcll(vm & ballot(key == K));
                nA += (uint32_t)__popcll(vm & ballot(key > K));
            }
            if (valid) {
                atomicAdd((uint32_t *)&h_hi[255u - ((key >> s_hi) & 255u)], 1u);
                atomicAdd((uint32_t *)&h_lo[255u - ((key >> s_lo) & 255u)], 1u);
            }
        }
        if (r.pen) __syncthreads();  // the bits are rebuilt for the next step
    }
    if (first) {
        if (lane == 0) {
            atomicAdd((uint32_t *)&L->sh_hot_count, nK);
            atomicAdd((uint32_t *)&L->sh_hot_above, nA);
        }
        or0 = wave_fold_u32(or0, [](uint32_t a, uint32_t b) { return a | b; });
        and0 = wave_fold_u32(and0, [](uint32_t a, uint32_t b) { return a & b; });
        or1 = wave_fold_u32(or1, [](uint32_t a, uint32_t b) { return a | b; });
        and1 = wave_fold_u32(and1, [](uint32_t a, uint32_t b) { return a & b; });
        if (lane == 0) {
            atomicOr((uint32_t *)&L->cls[0], or0);
            atomicAnd((uint32_t *)&L->cls[1], and0);
            atomicOr((uint32_t *)&L->cls[2], or1);
            atomicAnd((uint32_t *)&L->cls[3], and1);
        }
    }
    __syncthreads();
    for (uint32_t i = tid; i < 2 * 256; i += REST_THREADS) {
        const uint32_t x = i >> 8, d = i & 255u;
        uint32_t c = 0;
        for (uint32_t g = 0; g < HIST_COPIES; ++g) c += L->u.gh[x][g * HIST_ROW + d];
        L->hist[x ? lo : hi][d] = c;
    }
    __syncthreads();
}

// Exclusive prefix over the 256 digits of src into dst; the first wave, four
// digits a lane.
__device__ __forceinline__ void digit_prefix(RL_LDS const uint32_t *src, RL_LDS uint32_t *dst) {
    const uint32_t lane = lane_id();
    uint32_t v[4], sum = 0;
#pragma unroll
    for (uint32_t q = 0; q < 4; ++q) {
        v[q] = src[4 * lane + q];
        sum += v[q];
    }
    uint32_t run = wave_incl_u32(sum) - sum;
#pragma unroll
    for (uint32_t q = 0; q < 4; ++q) {
        dst[4 * lane + q] = run;
        run += v[q];
    }
}

// A thread's share of the candidate list's statistics (those kept in LDS
// beside the segments): p at index j seen by add.
struct PStats {
    int emin = 1 << 20;
    uint32_t bad = 0, count = 0, last_in = 0, first_out = 0xFFFFFFFFu;
    __device__ __forceinline__ void add(float p, uint32_t j, float min_p) {
        if (!(p <= 3.40282347e38f)) {
            bad = 1;  // NaN or +inf
        } else if (p > 0.0f) {
            emin = min(emin, f32_exponent(p));
        }
        if (p >= min_p) {
            ++count;
            last_in = max(last_in, j + 1);
        } else {
            first_out = min(first_out, j);
        }
    }
    // Folds the wave's shares into L's (lane 0 adds them with LDS atomics,
    // after L's were set by stats_reset and a barrier).
    __device__ __forceinline__ void merge(RL_LDS RestLds *L) {
        emin = (int)wave_fold_u32((uint32_t)emin, [](uint32_t a, uint32_t b) { return (int)a < (int)b ? a : b; });
        bad = wave_fold_u32(bad, [](uint32_t a, uint32_t b) { return a | b; });
        count = wave_sum_u32(count);
        last_in = wave_fold_u32(last_in, [](uint32_t a, uint32_t b) { return a > b ? a : b; });
        first_out = wave_fold_u32(first_out, [](uint32_t a, uint32_t b) { return a < b ? a : b; });
        if (lane_id() == 0) {
            atomicMin((int *)&L->st_emin, emin);
            atomicOr((uint32_t *)&L->st_bad, bad);
            atomicAdd((uint32_t *)&L->st_count, count);
            atomicMax((uint32_t *)&L->st_last_in, last_in);
            atomicMin((uint32_t *)&L->st_first_out, first_out);
        }
    }
};

// The list statistics before any merge (one thread).
__device__ __forceinline__ void stats_reset(RL_LDS RestLds *L) {
    L->st_emin = 1 << 20;
    L->st_bad = 0;
    L->st_count = 0;
    L->st_last_in = 0;
    L->st_first_out = 0xFFFFFFFFu;
}

// Two passes on digits 2 and 3 (keys whose low 16 bits are one value per sign,
// as for logits on a bf16 grid) can pass one word per element between them:
// the first pass writes (key's top byte << 24) | id, and the second takes the
// element's digit 2 from its position (the first pass's output is in runs of
// digit 2, starting at L->run0) and the low 16 bits from its sign.
struct RestPacked {
    uint32_t lo_clear, lo_set;  // the low 16 key bits of keys with the top bit clear, set
    __device__ __forceinline__ uint32_t key(uint32_t d3, uint32_t d2) const {
        return (d3 << 24) | (d2 << 16) | ((d3 & 0x80u) ? lo_set : lo_clear);
    }
};

// The row's hot key K when its elements skip the sort: they are `count` of
// the row, `above` keys are greater, and their p is pK. In the reference's
// order they form one block at [above, above + count), in ascending id.
struct RestHot {
    bool on;
    uint32_t key, count, above;
    float pK;
};

// One stable pass of the sort on digit t (bits 8t..8t+7, descending) over n
// elements: from the raw logits (FROM_LOGITS: keys computed here, ids =
// positions) or from kin/iin, to kout/iout, or (FINAL) the ids to iout and p
// to fp for the first k positions. Each tile gives every wave a contiguous
// segment; a wave ranks its items in order (lanes with the same digit found by
// ballots, the wave's running count per digit in LDS, which they all read and
// then advance by their number), the workgroup reorders the tile by digit in LDS and writes it out in runs, so
// consecutive threads write consecutive addresses. With hot.on, the pass from
// the logits leaves the hot key's elements out of the ranking and writes their
// ids to their block of hid (the final ids) in id order (their p, all pK, are
// not stored: readers of the list take them from a HotRange), and the final
// pass places the keys below the hot key after that block.
template <bool FROM_LOGITS, bool FINAL, bool PACKED = false>
__device__ __forceinline__ void rest_pass(RL_LDS RestLds *L, const RestRow &r, const LdsExpTable &etab, uint32_t t,
                                          uint32_t n, const RestHot &hot, uint32_t *hid,
                                          const uint32_t *kin, const uint32_t *iin, uint32_t *kout, uint32_t *iout,
                                          float *fp, PStats &ps, float min_p, uint32_t SH,
                                          const RestPacked &pk_ = RestPacked{}) {
    const uint32_t tid = threadIdx.x, lane = lane_id(), wave = tid / WAVE;
    const uint32_t V = r.V, shift = 8 * t;
    if (tid < WAVE) digit_prefix(L->hist[t], L->offs);
    __syncthreads();
    if constexpr (PACKED && FROM_LOGITS) {
        // The runs of the output by digit, for the second pass.
        if (tid < 256) L->run0[tid] = L->offs[tid];
        if (tid == 255) L->run0[256] = L->offs[255] + L->hist[t][255];
    }
    uint32_t nk[REST_ITEMS], ni[REST_ITEMS];
    const uint32_t voff = 4 * (wave * REST_SEG + lane);  // item i adds 256 i bytes
    auto fetch = [&](uint32_t tb) {  // tile tb's keys and ids (zeros past the row)
        // The items' offsets come from an opaque copy of voff (one register
        // and immediate offsets, rather than one register per item).
        uint32_t vo = voff;
        asm volatile("" : "+v"(vo));
        if constexpr (FROM_LOGITS) {
            const auto rl = tail_rsrc((const uint32_t *)r.rowp, tb, n);
#pragma unroll
            for (uint32_t i = 0; i < REST_ITEMS; ++i) nk[i] = bload<true>(rl, vo + 256 * i);
        } else if constexpr (PACKED) {
            const auto ri = tail_rsrc(iin, tb, n);
#pragma unroll
            for (uint32_t i = 0; i < REST_ITEMS; ++i) ni[i] = bload(ri, vo + 256 * i);
        } else {
            const auto rk = tail_rsrc(kin, tb, n), ri = tail_rsrc(iin, tb, n);
#pragma unroll
            for (uint32_t i = 0; i < REST_ITEMS; ++i) {
                nk[i] = bload(rk, vo + 256 * i);
                ni[i] = bload(ri, vo + 256 * i);
            }
        }
    };
    // The outputs: past the first k, final writes are dropped (only those are
    // candidates, and the caller's buffers may hold no more).
    const auto rko = words_rsrc(kout, FINAL ? 0u : V);
    const auto rio = words_rsrc(iout, FINAL ? r.k : V);
    const auto rpo = words_rsrc(fp, FINAL ? r.k : 0u);
    const bool hot_out = FROM_LOGITS && hot.on;  // block-uniform
    const auto rhi = words_rsrc(hid, hot_out ? r.k : 0u);
    uint32_t hot_done = 0;  // the hot key's elements in earlier tiles
    fetch(0);
    for (uint32_t tb = 0; tb < n; tb += REST_TILE) {
        const uint32_t e0 = tb + wave * REST_SEG + lane;
        uint32_t tn = min(REST_TILE, n - tb);
        uint32_t kk[REST_ITEMS], ii[REST_ITEMS];
        if constexpr (PACKED && !FROM_LOGITS) {
            // Each element's digit 2 from the run it sits in: the waves
            // write the tile's map run by run, then read it by position.
            // Wave w takes the runs w, w + REST_WAVES, ...; lane q reads the
            // bounds of its q-th run, so all are read at once.
            constexpr uint32_t FR = 256 / REST_WAVES;
            uint32_t rb = 0, re = 0;
            if (lane < FR) {
                rb = L->run0[wave + REST_WAVES * lane];
                re = L->run0[wave + REST_WAVES * lane + 1];
            }
#pragma unroll
            for (uint32_t q = 0; q < FR; ++q) {
                const uint32_t f = wave + REST_WAVES * q;
                const uint32_t lo = max(read_lane_u32(rb, q), tb), hi = min(read_lane_u32(re, q), tb + tn);
                for (uint32_t j = lo + lane; j < hi; j += WAVE) L->dmap[j - tb] = (uint8_t)(255u - f);
            }
            __syncthreads();
#pragma unroll
            for (uint32_t i = 0; i < REST_ITEMS; ++i) {
                const uint32_t w = ni[i];
                kk[i] = pk_.key(w >> 24, L->dmap[wave * REST_SEG + i * WAVE + lane]);
                ii[i] = w & 0x00FFFFFFu;
            }
        } else {
#pragma unroll
            for (uint32_t i = 0; i < REST_ITEMS; ++i) {
                kk[i] = nk[i];
                ii[i] = FROM_LOGITS ? e0 + i * WAVE : ni[i];
            }
        }
        fetch(tb + REST_TILE);
        if constexpr (FROM_LOGITS) {
            if (r.pen) window_bits(L, r, tb, tn);
#pragma unroll
            for (uint32_t i = 0; i < REST_ITEMS; ++i) {
                float v = __uint_as_float(kk[i]);
                if (r.pen) v = penalised(L, r, v, e0 + i * WAVE - tb);
                kk[i] = total_key(v);
            }
        }
        // With the hot key out of the sort, each wave packs its other elements
        // (key and id, in id order) at the start of its share of the tile
        // buffer and its hot ids, in id order, backwards from the share's end,
        // then ranks only the packed items. The buffer is free: the last
        // tile's reads of it ended two barriers ago and this tile's reorder
        // comes after the next two.
        uint32_t packed = 0, wave_hot = 0;  // wave-uniform counts
        RL_LDS uint32_t *pk = &L->u.tile.k[wave * REST_SEG];
        RL_LDS uint32_t *pi = &L->u.tile.i[wave * REST_SEG];
        if (hot_out) {
#pragma unroll
            for (uint32_t i = 0; i < REST_ITEMS; ++i) {
                const bool in = e0 + i * WAVE < n;
                const bool is_hot = in && kk[i] == hot.key;
                const uint64_t km = ballot(in && !is_hot), hm = ballot(is_hot);
                if (in && !is_hot) {
                    const uint32_t at = packed + lanes_below(km);
                    pk[at] = kk[i];
                    pi[at] = ii[i];
                }
                if (is_hot) pk[REST_SEG - 1 - (wave_hot + lanes_below(hm))] = ii[i];
                packed += (uint32_t)__popcll(km);
                wave_hot += (uint32_t)__popcll(hm);
            }
#pragma unroll
            for (uint32_t i = 0; i < REST_ITEMS; ++i) {
                if (i * WAVE < packed) {
                    kk[i] = pk[i * WAVE + lane];
                    ii[i] = pi[i * WAVE + lane];
                }
            }
        }
        // Whether item i takes part in the ranking.
        auto ranked = [&](uint32_t i) { return hot_out ? i * WAVE + lane < packed : e0 + i * WAVE < n; };
        for (uint32_t d = lane; d < 256; d += WAVE) L->cnt[wave][d] = 0;
        // Rank: item i's lanes with digit d follow the wave's earlier items'.
        // The lanes with digit d are found by each setting its bit in the
        // wave's word for d and reading the word back; the wave's LDS
        // accesses run in order, so every lane reads the word after all the
        // item's bits are in and before it is cleared, and every peer reads
        // the wave's count before this item and writes the same count after.
        uint32_t rk[REST_ITEMS];
        const uint64_t my_bit = 1ull << lane;
#pragma unroll
        for (uint32_t i = 0; i < REST_ITEMS; ++i) {
            rk[i] = 0;
            if (hot_out && i * WAVE >= packed) continue;  // wave-uniform
            if (ranked(i)) {
                const uint32_t d = 255u - ((kk[i] >> shift) & 255u);
                RL_LDS uint64_t *w = &L->peer[wave][d];
                __hip_atomic_fetch_or(w, my_bit, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WAVEFRONT);
                const uint64_t peers = __hip_atomic_load(w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WAVEFRONT);
                const uint32_t base = L->cnt[wave][d];
                rk[i] = base + lanes_below(peers);
                __hip_atomic_store(w, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WAVEFRONT);
                L->cnt[wave][d] = base + (uint32_t)__popcll(peers);
            }
        }
        if (hot_out && lane == 0) L->hcnt[wave] = wave_hot;
        __syncthreads();
        if (hot_out) {
            // The hot key's elements of this tile, in id order: the waves'
            // counts give each wave its start; its ids are read back from the
            // end of its share.
            uint32_t at = hot.above + hot_done, all = 0;
            for (uint32_t w = 0; w < REST_WAVES; ++w) {
                const uint32_t c = L->hcnt[w];
                at += w < wave ? c : 0u;
                all += c;
            }
            for (uint32_t h = lane; h < wave_hot; h += WAVE) bstore(rhi, 4 * (at + h), pk[REST_SEG - 1 - h]);
            hot_done += all;
            tn -= all;
        }
        // Per digit: each wave's start within the digit's run of the tile, and
        // the run's length; then the runs' starts.
        if (tid < 256) {
            uint32_t c[REST_WAVES];
#pragma unroll
            for (uint32_t w = 0; w < REST_WAVES; ++w) c[w] = L->cnt[w][tid];
            uint32_t run = 0;
#pragma unroll
            for (uint32_t w = 0; w < REST_WAVES; ++w) {
                L->cnt[w][tid] = run;
                run += c[w];
            }
            L->tcount[tid] = run;
        }
        __syncthreads();
        if (tid < WAVE) digit_prefix(L->tcount, L->tstart);
        __syncthreads();
#pragma unroll
        for (uint32_t i = 0; i < REST_ITEMS; ++i) {
            if (ranked(i)) {
                const uint32_t d = 255u - ((kk[i] >> shift) & 255u);
                const uint32_t at = L->tstart[d] + L->cnt[wave][d] + rk[i];
                L->u.tile.k[at] = kk[i];
                L->u.tile.i[at] = ii[i];
            }
        }
        __syncthreads();
#pragma unroll
        for (uint32_t q = 0; q < REST_ITEMS; ++q) {
            const uint32_t j = q * REST_THREADS + tid;
            if (j < tn) {
                const uint32_t key = L->u.tile.k[j];
                const uint32_t d = 255u - ((key >> shift) & 255u);
                uint32_t dst = L->offs[d] + (j - L->tstart[d]);
                if constexpr (FINAL) {
                    if (hot.on && key < hot.key) dst += hot.count;
                }
                const uint32_t id = L->u.tile.i[j];
                if constexpr (FINAL) {
                    bstore(rio, 4 * dst, id);
                    if (dst < r.k) {
                        // p, and the list's statistics: its chunk's sum (any
                        // order: the sums are used only where they are exact)
                        // and the thread's share of the rest.
                        const float p = expf_libm_t(r.tscale(key_value(key) - r.M), etab);
                        bstore(rpo, 4 * dst, __float_as_uint(p));
                        __hip_atomic_fetch_add(&L->u.tile.csum[lane & (HIST_COPIES - 1)][dst >> SH], (double)p,
                                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
                        ps.add(p, dst, min_p);
                    }
                } else if constexpr (PACKED) {
                    bstore(rio, 4 * dst, (key & 0xFF000000u) | id);
                } else {
                    bstore(rio, 4 * dst, id);
                    bstore(rko, 4 * dst, key);
                }
            }
        }
        __syncthreads();
        if (tid < 256) L->offs[tid] += L->tcount[tid];
        __syncthreads();
    }
}

// The candidates in id order (no sort: top-p off with every id a candidate,
// or every key alike): ids = positions and p, for the first k.
__device__ __forceinline__ void rest_direct(RL_LDS RestLds *L, const RestRow &r, const LdsExpTable &etab, uint32_t *iout, float *fp) {
    const uint32_t lane = lane_id(), wave = threadIdx.x / WAVE;
    const uint32_t V = r.V;
    const uint32_t wbase = wave * WAVE * HIST_ITEMS + lane;
    const uint32_t *raw = (const uint32_t *)r.rowp;
    for (uint32_t b = 0; b < r.k; b += HIST_STEP) {
        uint32_t x[HIST_ITEMS];
        const auto rs = tail_rsrc(raw, b, V);
#pragma unroll
        for (uint32_t i = 0; i < HIST_ITEMS; ++i) x[i] = bload<true>(rs, 4 * (wbase + i * WAVE));
        if (r.pen) window_bits(L, r, b, min(HIST_STEP, V - b));
        const auto ri = tail_rsrc(iout, b, r.k), rp = tail_rsrc((const uint32_t *)fp, b, r.k);
#pragma unroll
        for (uint32_t i = 0; i < HIST_ITEMS; ++i) {
            const uint32_t off = wbase + i * WAVE;
            if (b + off < r.k) {
                const float v = r.pen ? penalised(L, r, __uint_as_float(x[i]), off) : __uint_as_float(x[i]);
                bstore(ri, 4 * off, b + off);
                bstore(rp, 4 * off, __float_as_uint(expf_libm_t(r.tscale(v - r.M), etab)));
            }
        }
        if (r.pen) __syncthreads();
    }
}

// The chunk size of the candidate list's sums for k candidates: a power of
// two, at least 2^STAT_MIN_LOG, and at most STAT_CHUNKS chunks.
__device__ __forceinline__ uint32_t stat_shift(uint32_t k) {
    uint32_t sh = STAT_MIN_LOG;
    while (((uint64_t)k + (1ull << sh) - 1) >> sh > STAT_CHUNKS) ++sh;
    return sh;
}

// grid (slots), REST_THREADS: the rows k_full_pass left (done == 0).
__global__ __launch_bounds__(REST_THREADS) void k_full_rest(RowIO a, FullScratch f) {
    __shared__ RestLds L_;
    RL_LDS RestLds *L = (RL_LDS RestLds *)&L_;
    const uint32_t slot = blockIdx.x;
    const FullRow st = f.row[slot];
    if (st.done) return;
    const uint32_t tid = threadIdx.x, lane = lane_id(), wave = tid / WAVE;
    const uint32_t row = a.rows ? a.rows[slot] : a.row0 + slot;
    const rl_sampling s = a.settings[row];
    const uint32_t V = a.vocab;
    const uint32_t k = full_k(s, V);
    const uint32_t wl = window_len(a, row);
    const RestRow r{a.logits + (uint64_t)row * a.stride,
                    wl > 0 ? a.windows + (uint64_t)row * a.wstride : nullptr,
                    V,
                    k,
                    wl,
                    penalises(s) && wl > 0,
                    s.repeat_penalty,
                    st.M,
                    TempScale(s.temperature)};
    copy_exp_table(L->exp_tab);
    const LdsExpTable etab{L->exp_tab};
    const bool out = a.out_ids != nullptr;
    uint32_t *keyA = f.keyA + (uint64_t)slot * V, *idA = f.idA + (uint64_t)slot * V;
    uint32_t *keyB = f.keyB + (uint64_t)slot * V, *idB = f.idB + (uint64_t)slot * V;
    float *fp = out ? a.out_probs + (uint64_t)row * a.cand_stride : f.probs + (uint64_t)slot * V;
    uint32_t *fid = out ? a.out_ids + (uint64_t)row * a.cand_stride : idA;

    // ---- the candidates in order: fid[0..V), fp[0..k) ----
    if (tid == 0) stats_reset(L);
    for (uint32_t i = tid; i < REST_WAVES * 256; i += REST_THREADS) (&L->peer[0][0])[i] = 0;
    PStats ps;                 // this thread's share of the list's statistics
    bool sorted = false;       // the last sort pass gathered the statistics
    RestHot hot{false, 0u, 0u, 0u, 0.0f};
    // The list's chunks: 2^SH candidates each, CS of them.
    const uint32_t SH = stat_shift(k);
    const uint32_t CS = (uint32_t)(((uint64_t)k + (1ull << SH) - 1) >> SH);
    auto chunk_start = [&](uint32_t c) { return min(c << SH, k); };
    if (identity_order(s, V)) {
        rest_direct(L, r, etab, fid, fp);
    } else {
        // Which passes run: per sign, the OR and the AND of its keys give the
        // bits in which keys of that sign differ. A lower digit's pass is
        // skipped when the digit is the same for all keys of each sign (as
        // for logits on a bf16 grid, whose low 16 key bits follow the sign):
        // keys that agree above it agree on it, so it cannot change the
        // order. The top digit's pass is skipped when it is the same for all.
        rest_histograms(L, r, 3, 2, true);
        const uint32_t c0 = L->cls[0], c1 = L->cls[1], c2 = L->cls[2], c3 = L->cls[3];
        const bool has0 = c1 != 0xFFFFFFFFu, has1 = c2 != 0u;
        const uint32_t vary_sign = (has0 ? (c0 ^ c1) : 0u) | (has1 ? (c2 ^ c3) : 0u);
        const uint32_t all_or = (has0 ? c0 : 0u) | (has1 ? c2 : 0u);
        const uint32_t all_and = (has0 ? c1 : 0xFFFFFFFFu) & (has1 ? c3 : 0xFFFFFFFFu);
        // The digits to sort on, as a bit mask (digit t: bit t), lowest first.
        uint32_t pass_mask = 0;
        for (uint32_t t = 0; t < 3; ++t)
            if (((vary_sign >> (8 * t)) & 255u) != 0) pass_mask |= 1u << t;
        if (((all_or ^ all_and) >> 24) != 0) pass_mask |= 8u;
        uint32_t np = (uint32_t)__builtin_popcount(pass_mask);
        if ((pass_mask & 3u) != 0) rest_histograms(L, r, 1, 0, false);
        if (np == 0) {
            rest_direct(L, r, etab, fid, fp);
        } else {
            // Pass i writes A when i is even, B when odd; the last writes the
            // ids where the candidates go (not into the buffer it reads).
            if (!out) fid = ((np - 1) & 1) ? idB : idA;
            // The hot key's elements skip the sort when they are at least a
            // sixteenth of the row and their block, written by the first pass,
            // stays clear of every later pass's output: always in the caller's
            // buffers, and in idB with two passes (the first writes A, the last
            // reads it).
            hot = RestHot{false, L->sh_hot_key, L->sh_hot_count, L->sh_hot_above, 0.0f};
            hot.on = hot.count >= V / 16 && hot.count < V && (out || np <= 2);
            uint32_t n1 = V;  // the elements of the passes after the first
            if (hot.on) {
                hot.pK = expf_libm_t(r.tscale(key_value(hot.key) - r.M), etab);
                n1 = V - hot.count;
                if (tid < 4 && ((pass_mask >> tid) & 1u)) L->hist[tid][255u - ((hot.key >> (8 * tid)) & 255u)] -= hot.count;
            }
            for (uint32_t i = tid; i < HIST_COPIES * (STAT_CHUNKS + 1); i += REST_THREADS)
                (&L->u.tile.csum[0][0])[i] = 0.0;
            __syncthreads();
            sorted = true;
            const float min_p = s.min_p;
            const uint32_t *kin = nullptr, *iin = nullptr;
            if (pass_mask == 0xCu && V <= 0x01000000u) {
                // Digits 2 and 3 only: the first pass hands the second one
                // word per element (RestPacked).
                const RestPacked pkd{c0 & 0xFFFFu, c2 & 0xFFFFu};
                rest_pass<true, false, true>(L, r, etab, 2, V, hot, fid, nullptr, nullptr, nullptr, idA, nullptr, ps,
                                             min_p, SH, pkd);
                rest_pass<false, true, true>(L, r, etab, 3, n1, hot, nullptr, nullptr, idA, nullptr, fid, fp, ps,
                                             min_p, SH, pkd);
                np = 0;  // done
            }
            uint32_t left = np ? pass_mask : 0u;  // the digits still to sort on
            for (uint32_t i = 0; i < np; ++i) {
                const bool last = i + 1 == np;
                const uint32_t t = (uint32_t)__builtin_ctz(left);
                left &= left - 1u;
                uint32_t *ko = (i & 1) ? keyB : keyA, *io = (i & 1) ? idB : idA;
                if (i == 0 && last)
                    rest_pass<true, true>(L, r, etab, t, V, hot, fid, nullptr, nullptr, nullptr, fid, fp, ps, min_p,
                                          SH);
                else if (i == 0)
                    rest_pass<true, false>(L, r, etab, t, V, hot, fid, nullptr, nullptr, ko, io, nullptr, ps, min_p,
                                           SH);
                else if (last)
                    rest_pass<false, true>(L, r, etab, t, n1, hot, nullptr, kin, iin, nullptr, fid, fp, ps, min_p,
                                           SH);
                else
                    rest_pass<false, false>(L, r, etab, t, n1, hot, nullptr, kin, iin, ko, io, nullptr, ps, min_p,
                                            SH);
                kin = ko;
                iin = io;
            }
        }
    }
    __syncthreads();

    // ---- the candidate list's chunk sums and statistics ----
    if (sorted) {
        // The last pass added each candidate's p to its chunk; the hot key's
        // block adds pK times its overlap with each chunk.
        const uint32_t hot_in = hot.on && hot.above < k ? min(hot.count, k - hot.above) : 0u;
        if (tid == 0 && hot_in > 0) {
            // The hot block's share of the statistics: hot_in equal p.
            const float p = hot.pK;
            if (!(p <= 3.40282347e38f)) {
                ps.bad = 1;
            } else if (p > 0.0f) {
                ps.emin = min(ps.emin, f32_exponent(p));
            }
            if (p >= s.min_p) {
                ps.count += hot_in;
                ps.last_in = max(ps.last_in, hot.above + hot_in);
            } else {
                ps.first_out = min(ps.first_out, hot.above);
            }
        }
        if (tid < CS) {
            double sum = 0.0;
            for (uint32_t g = 0; g < HIST_COPIES; ++g) sum += L->u.tile.csum[g][tid];
            const uint32_t lo = max(chunk_start(tid), hot.above), hi = min(chunk_start(tid + 1), hot.above + hot_in);
            if (hot_in > 0 && lo < hi) sum += (double)(hi - lo) * (double)hot.pK;  // exact where the sums are used
            L->seg_sum[tid] = sum;
        }
    } else {
        // The candidates in id order: one wave a chunk at a time; each lane's
        // share of a chunk (32 consecutive p) in eight 16-byte loads, all in
        // flight together.
        constexpr uint32_t SL = 32;  // consecutive p per lane per step
        typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
        const __amdgpu_buffer_rsrc_t rp = words_rsrc(fp, k);
        for (uint32_t c = wave; c < CS; c += REST_WAVES) {
            const uint32_t j0 = chunk_start(c), j1 = chunk_start(c + 1);
            double sum = 0.0;
            for (uint32_t b = j0; b < j1; b += WAVE * SL) {
                const uint32_t jl = b + lane * SL;
                u32x4 v[SL / 4];
#pragma unroll
                for (uint32_t q = 0; q < SL / 4; ++q)
                    v[q] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rp, 4u * jl + 16u * q, 0, 0));
#pragma unroll
                for (uint32_t q = 0; q < SL / 4; ++q)
#pragma unroll
                    for (uint32_t i = 0; i < 4; ++i) {
                        const uint32_t j = jl + 4 * q + i;
                        if (j < j1) {
                            const float p = __uint_as_float(v[q][i]);
                            sum += (double)p;
                            ps.add(p, j, s.min_p);
                        }
                    }
            }
            sum = wave_total_f64(sum);
            if (lane == 0) L->seg_sum[c] = sum;
        }
    }
    ps.merge(L);
    __syncthreads();

    // ---- the mass, the top-p cut (sample.rs:307-324), min-p (:326-340) and
    // the normalising total (:342-343) ----
    RL_LDS float *stage = L->u.rep.stage;
    RL_LDS uint32_t *stop = &L->sh_stop;
    const uint32_t *fpw = (const uint32_t *)fp;
    const auto as_f32 = [](uint32_t b) { return __uint_as_float(b); };
    RL_LDS ChunkLds *cr = &L->u.rep.cr;
    const bool bad = L->st_bad != 0;
    const int emin = L->st_emin;
    const uint32_t count = L->st_count, last_in = L->st_last_in, first_out = L->st_first_out;
    double tree_mass = 0.0;
    for (uint32_t c = 0; c < CS; ++c) tree_mass += L->seg_sum[c];
    // The candidates with p >= min_p form a prefix of the list.
    const bool surv_prefix = last_in <= first_out;
    // The hot key's block of p (all pK) was not stored: the readers below take
    // it from hr, unless one that reads the list itself runs (a NaN or an
    // infinite p: the staged walks; survivors not a prefix: the min-p
    // compaction), for which it is written out first.
    HotRange hr;
    {
        const uint32_t hot_in = hot.on && hot.above < k ? min(hot.count, k - hot.above) : 0u;
        if (hot_in > 0) {
            if (bad || !surv_prefix) {
                for (uint32_t j = hot.above + tid; j < hot.above + hot_in; j += REST_THREADS) fp[j] = hot.pK;
                __syncthreads();
            } else {
                hr = HotRange{hot.above, hot.above + hot_in, __float_as_uint(hot.pK)};
            }
        }
    }
    // Every partial sum exact: all p are multiples of 2^(emin-23), the mass is
    // below 2^53 of those steps. Then any sum of any of them is exact, so the
    // chunk sums (added in whatever order) are the exact sums too. (The
    // margin keeps a mass rounded below the bound from passing for one that is
    // not.)
    const bool exact = !bad && (emin > 1000 || tree_mass < mul_pow2(1.0 - 0x1p-30, 30 + emin));
    // The exact sum of p[0..n), from the chunk sums and one partial chunk.
    auto exact_prefix = [&](uint32_t n) {
        double b = 0.0;
        uint32_t c = 0;
        while (c < CS && chunk_start(c + 1) <= n) b += L->seg_sum[c++];
        if (c == CS || chunk_start(c) == n) return b;
        double at;
        exact_first_reaching<REST_THREADS>(fp, chunk_start(c), n, b, __builtin_inf(), L->red_d, &L->sh_hit,
                                           &L->sh_hit_sum, &at, hr);
        return at;
    };

    uint32_t m = k;
    bool have_sum_m = false;  // sum_m: the sequential sum of p[0..m)
    double sum_m = 0.0;
    if (s.top_p < 1.0f) {
        double mass = 0.0;
        if (exact) {
            mass = tree_mass;
            const double target = (double)s.top_p * mass;
            // The chunk where the running sum first reaches the target.
            double b = 0.0;
            uint32_t c = 0;
            while (c < CS && !(b + L->seg_sum[c] >= target)) b += L->seg_sum[c++];
            if (c < CS) {
                double at;
                const uint32_t j = exact_first_reaching<REST_THREADS>(fp, chunk_start(c), chunk_start(c + 1), b,
                                                                      target, L->red_d, &L->sh_hit, &L->sh_hit_sum, &at,
                                                                      hr);
                m = j + 1;
                have_sum_m = true;
                sum_m = at;
            } else {
                have_sum_m = true;
                sum_m = mass;
            }
        } else if (!bad) {
            // The mass, then the cut, through one call site of the replay
            // (a target of +inf is never met by a finite sum).
            double tgt = __builtin_inf();
            for (uint32_t job = 0; job < 2; ++job) {
                double at;
                const uint32_t j =
                    chunk_replay<53, REST_THREADS>(fpw, as_f32, k, [tgt](double c) { return c >= tgt; }, cr, &at,
                                                   nullptr, nullptr, hr);
                if (job == 0) {
                    mass = at;
                    tgt = (double)s.top_p * mass;
                } else {
                    have_sum_m = true;
                    if (j < k) {
                        m = j + 1;
                        sum_m = at;
                    } else {
                        sum_m = mass;
                    }
                }
            }
        } else {
            staged_walk<REST_THREADS>(fp, k, stage, stop, [&](RL_LDS float *sv, uint32_t, uint32_t cnt) {
                for (uint32_t i = 0; i < cnt; ++i) mass += (double)sv[i];
                return false;
            });
            if (tid == 0) L->sh_d = mass;
            __syncthreads();
            mass = L->sh_d;
            const double target = (double)s.top_p * mass;
            if (tid == 0) L->sh_m = k;
            __syncthreads();
            double cum = 0.0;
            staged_walk<REST_THREADS>(fp, k, stage, stop, [&](RL_LDS float *sv, uint32_t b, uint32_t cnt) {
                for (uint32_t i = 0; i < cnt; ++i) {
                    cum += (double)sv[i];
                    if (cum >= target) {
                        L->sh_m = b + i + 1;
                        return true;
                    }
                }
                return false;
            });
            __syncthreads();
            m = L->sh_m;
        }
    }
    if (s.min_p > 0.0f) {  // a stable in-place compaction
        uint32_t w;
        if (!bad && surv_prefix) {
            // The survivors are the first `count` of all k candidates (so it
            // is with sorted candidates, where p falls along the order), and
            // min(m, count) of the first m: nothing moves.
            w = min(m, count);
        } else {
            // Survivors anywhere: count them, and compact unless they are
            // already a prefix.
            uint32_t fo = 0xFFFFFFFFu, li = 0, cnt = 0;
            for (uint32_t b = 0; b < m; b += REST_THREADS) {
                const uint32_t j = b + tid;
                if (j < m) {
                    if (((const RL_GLB float *)fp)[j] >= s.min_p) {
                        ++cnt;
                        li = j + 1;
                    } else if (fo == 0xFFFFFFFFu) {
                        fo = j;
                    }
                }
            }
            w = block_sum_u32<REST_THREADS>(cnt, L->red_u);
            const uint32_t lo_out = (uint32_t)-block_max_i64<REST_THREADS>(-(int64_t)fo, L->red_l);
            const uint32_t hi_in = (uint32_t)block_max_i64<REST_THREADS>((int64_t)li, L->red_l);
            if (hi_in > lo_out) {
                uint32_t done = 0;
                for (uint32_t b = 0; b < m; b += REST_THREADS * CI) {
                    const uint32_t j0 = b + tid * CI;
                    float pv[CI];
                    uint32_t iv[CI];
                    uint32_t mine = 0;
#pragma unroll
                    for (uint32_t i = 0; i < CI; ++i) {
                        const bool ok = j0 + i < m;
                        pv[i] = ok ? fp[j0 + i] : 0.0f;
                        iv[i] = ok ? fid[j0 + i] : 0u;
                        mine += (ok && pv[i] >= s.min_p) ? 1u : 0u;
                    }
                    uint32_t step_total;
                    uint32_t dst = done + block_exclusive<REST_THREADS, uint32_t>(mine, L->red_u, &step_total);
#pragma unroll
                    for (uint32_t i = 0; i < CI; ++i) {
                        if (j0 + i < m && pv[i] >= s.min_p) {
                            fid[dst] = iv[i];
                            fp[dst] = pv[i];
                            ++dst;
                        }
                    }
                    done += step_total;
                    __syncthreads();
                }
            }
        }
        if (w != m) have_sum_m = false;
        m = w > 1 ? w : 1u;
    }
    double total = 0.0;
    if (have_sum_m) {
        total = sum_m;  // the same terms in the same order as the top-p pass
    } else if (exact && (surv_prefix || !(s.min_p > 0.0f))) {
        total = exact_prefix(m);  // min-p moved nothing: the chunk sums still apply
    } else if (exact) {
        exact_first_reaching<REST_THREADS>(fp, 0, m, 0.0, __builtin_inf(), L->red_d, &L->sh_hit, &L->sh_hit_sum,
                                           &total, hr);
    } else if (!bad) {
        chunk_replay<53, REST_THREADS>(fpw, as_f32, m, [](double) { return false; }, cr, &total, nullptr, nullptr, hr);
    } else {
        staged_walk<REST_THREADS>(fp, m, stage, stop, [&](RL_LDS float *sv, uint32_t, uint32_t cnt) {
            for (uint32_t i = 0; i < cnt; ++i) total += (double)sv[i];
            return false;
        });
        if (tid == 0) L->sh_d = total;
        __syncthreads();
        total = L->sh_d;
    }
    const float inv = (float)(1.0 / total);
    // q = p * inv is finite for every kept p when every p is and inv is (p <= 1
    // and inv <= 1: the best p is exp(0) = 1, so total >= 1).
    const bool qbad = bad || !(inv <= 3.40282347e38f);

    // ---- the draw: the f32 running sum of q against the uniform
    // (sample.rs:349-356); a shortfall takes the last candidate (:357-358) ----
    const float u = a.uniforms[row];
    uint32_t pick, qdone = 0;  // q is in place for the first qdone candidates
    if (!qbad) {
        // The draw stores q over p for the rounds it stages (when the caller
        // wants the candidates), so the normalisation below reads only the rest.
        double unused;
        const auto qterm = [inv](uint32_t bits) { return __uint_as_float(bits) * inv; };
        const auto over_u = [u](double c) { return c > (double)u; };
        const uint32_t hlo = min(hr.lo, m), hhi = min(hr.hi, m);
        if (hhi > hlo) {
            // The hot key's block of equal terms is crossed in closed form, a
            // step per binade of the sum (equal_run_walk): the replay runs up
            // to the block, and from its end with the sum there. Only the
            // first replay stores q; the normalisation below writes the rest.
            double sb;
            const uint32_t j0 =
                chunk_replay<24, REST_THREADS>(fpw, qterm, hlo, over_u, cr, &sb, out ? (uint32_t *)fp : nullptr, &qdone);
            if (j0 < hlo) {
                pick = j0;
            } else {
                const uint32_t jh = equal_run_walk<24>(sb, __float_as_uint(qterm(hr.word)), hhi - hlo, over_u);
                if (jh < hhi - hlo) {
                    pick = hlo + jh;
                } else {
                    __syncthreads();  // every thread has read the first replay's sum
                    const uint32_t j1 = chunk_replay<24, REST_THREADS>(fpw + hhi, qterm, m - hhi, over_u, cr, &unused,
                                                                       nullptr, nullptr, HotRange(), sb);
                    pick = j1 < m - hhi ? hhi + j1 : m - 1;
                }
            }
        } else {
            const uint32_t j = chunk_replay<24, REST_THREADS>(fpw, qterm, m, over_u, cr, &unused,
                                                              out ? (uint32_t *)fp : nullptr, &qdone, hr);
            pick = j < m ? j : m - 1;
        }
    } else {
        if (tid == 0) L->sh_tok = m - 1;
        __syncthreads();
        float cum = 0.0f;
        staged_walk<REST_THREADS>(fp, m, stage, stop, [&](RL_LDS float *sv, uint32_t b, uint32_t cnt) {
            for (uint32_t i = 0; i < cnt; ++i) {
                cum += sv[i] * inv;
                if (cum > u) {
                    L->sh_tok = b + i;
                    return true;
                }
            }
            return false;
        });
        __syncthreads();
        pick = L->sh_tok;
    }
    __syncthreads();  // every read of p by the draw precedes the writes of q
    if (tid == 0) {
        a.out_token[row] = fid[pick];
        a.out_kept[row] = m;
        a.out_used[row] = 1;
    }
    // ---- the kept candidates: q = p * (1 / total) in place (sample.rs:344-347) ----
    if (out) {
        constexpr uint32_t NU = 8;
        for (uint32_t b = qdone; b < m; b += REST_THREADS * NU) {
            float pv[NU];
#pragma unroll
            for (uint32_t q = 0; q < NU; ++q) {
                const uint32_t j = b + q * REST_THREADS + tid;
                const uint32_t jj = j < m ? j : m - 1;
                uint32_t w = hr.word;
                if (!hr.has(jj)) w = ((const RL_GLB uint32_t *)fp)[jj];
                pv[q] = __uint_as_float(w);
            }
#pragma unroll
            for (uint32_t q = 0; q < NU; ++q) {
                const uint32_t j = b + q * REST_THREADS + tid;
                if (j < m) fp[j] = pv[q] * inv;
            }
        }
    }
}

}  // namespace rl
