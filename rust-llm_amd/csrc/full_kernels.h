// The FULL device path: rows with top_k == 0, top_k >= vocab or top_k > 64
// (sample.rs:279-358 over the whole candidate list). Up to seven launches per
// group of rows, alternating kernels that spread a row over many workgroups
// (the HBM- and ALU-heavy steps) with one workgroup per row (the steps that
// follow the reference's sequential order):
//
//   k_full_keys    (chunks x rows)  total-order keys of the penalised row in id
//                                   order; per chunk the f32::max fold and
//                                   argmax, merged by the row's last chunk to
//                                   finish; rows without a finite maximum
//                                   answered
//   k_full_collect (chunks x rows)  min-p rows: p of every id, chunk sums, the
//                                   survivors (launched when a row may take
//                                   the min-p path)
//   k_full_small   (rows)           min-p rows finished from their survivors,
//                                   or left to the kernels below
//   k_full_sort    (rows)           the row sorted by the reference's order
//                                   unless it keeps id order
//   k_full_probs   (chunks x rows)  p = exp((l - max) / T) in candidate order,
//                                   per-chunk sums, smallest exponent, min-p
//                                   counts
//   k_full_tail    (rows)           mass, top-p cut, min-p, normalising total
//   k_full_finish  (rows, + chunks  the f32 draw over q = p * (1 / total)
//                   x rows)         against the host's uniform, one workgroup
//                                   a row; the other workgroups write the kept
//                                   candidates
//
// The sums are the reference's sequential sums, bit for bit: when every p is a
// multiple of 2^(e_min - 23) and the mass is below 2^(30 + e_min), every partial
// sum is exactly representable, so any order of addition gives the same bits
// and the per-chunk sums serve; otherwise seq_replay (rl_seqsum.h) reproduces
// the sequential rounding in parallel. Rows with a NaN or infinite p (NaN
// logits, a NaN temperature, 1 / total overflowing) are walked in order by one
// thread.
#pragma once
#include "sampler_kernels.h"

namespace rl {

struct FullRow {
    float M;           // the f32::max fold of the penalised row
    uint32_t am_tok;   // argmax of the penalised row
    uint32_t done;     // the row is finished (no finite maximum, or the min-p path)
    uint32_t m;        // candidates kept (after top-p and min-p)
    float inv;         // (1 / total) as f32
    uint32_t qbad;     // a normalised probability may not be finite: the draw walks in order
    uint32_t small;    // the row tries the min-p path first
    uint32_t nsurv;    // min-p survivors collected
    uint32_t overflow; // more survivors than SURV_CAP
    uint32_t ns_key;   // the largest key of an element below min-p (+1; 0 when none)
};

// Survivors the min-p path collects per row (their composites sort in LDS).
constexpr uint32_t SURV_CAP = 4096;
// A row's per-chunk results are read one chunk per lane.
static_assert(MAX_CHUNKS <= WAVE, "a wave holds one lane per chunk");

struct FullScratch {
    uint32_t *keyA, *idA, *keyB, *idB;  // [slot][vocab]
    float *probs;                       // [slot][vocab]
    float *part_max;                    // [slot][chunk] keys pass
    uint64_t *part_am;                  // [slot][chunk]
    double *psum;                       // [slot][chunk] probs pass
    int *pemin;                         // [slot][chunk]
    uint32_t *pcount;                   // [slot][chunk]
    uint32_t *pbad;                     // [slot][chunk]
    uint32_t *plast_in;                 // [slot][chunk] probs pass: last index + 1 with p >= min_p
    uint32_t *pfirst_out;               // [slot][chunk] first index with p < min_p
    uint64_t *surv;                     // [slot][SURV_CAP] min-p survivors (composites)
    FullRow *row;                       // [slot]
    uint32_t *arrive;                   // [slot] keys pass: chunks done; zero between calls
};

constexpr uint32_t UN = 16;                // elements per thread per step of the bulk loops (loads in flight)
constexpr uint32_t REPLAY_THREADS = 512;   // per-row kernels: 8 waves, up to 256 VGPRs each, no spills
constexpr uint32_t REPLAY_WAVES = REPLAY_THREADS / WAVE;
constexpr uint32_t SEQ_ITEMS = 8;          // terms per thread per tile of the sum replay
constexpr uint32_t CI = 8;                 // contiguous elements per thread per step of a scan or compaction

struct NeverStop {
    __device__ bool operator()(double) const { return false; }
};

__device__ __forceinline__ uint32_t full_k(const rl_sampling &s, uint32_t V) {
    return s.top_k == 0 ? V : (s.top_k < V ? (uint32_t)s.top_k : V);  // sample.rs:289
}
__device__ __forceinline__ bool identity_order(const rl_sampling &s, uint32_t V) {
    return full_k(s, V) == V && !(s.top_p < 1.0f);  // no select and no sort
}

// Chunk c of n items split into `chunks`: [chunk_lo(c), chunk_lo(c + 1)).
__device__ __forceinline__ uint32_t chunk_lo(uint32_t n, uint32_t c, uint32_t chunks) {
    return (uint32_t)((uint64_t)n * c / chunks);
}

// Binary exponent of a finite nonzero f32 (subnormals count as -126): every
// such value is a multiple of 2^(exponent - 23).
__device__ __forceinline__ int f32_exponent(float p) {
    const int e = (int)((__float_as_uint(p) >> 23) & 0xFFu);
    return e == 0 ? -126 : e - 127;
}

// The argument (l - max) / t of the reference's p = exp((l - max) / t)
// (sample.rs:309). When t is a power of two with a normal reciprocal, the
// product with that exact reciprocal is the same exact quotient rounded once,
// so it equals the IEEE division bit for bit; the bulk loops then skip the
// division's ten-odd instructions (t = 1 on the zipf and ties rows).
struct TempScale {
    float t, inv;
    bool pow2;
    __device__ explicit TempScale(float t_) : t(t_) {
        const uint32_t b = __float_as_uint(t_);
        const uint32_t e = (b >> 23) & 0xFFu;
        pow2 = (b & 0x807FFFFFu) == 0 && e >= 2 && e <= 252;  // +2^-125 .. +2^125
        inv = pow2 ? __uint_as_float((254u - e) << 23) : 0.0f;
    }
    __device__ float operator()(float d) const { return pow2 ? d * inv : d / t; }
};

// Whether a row tries the min-p path: min-p on, the whole vocabulary as
// candidates (top_k 0 or >= vocab), sampling (not greedy).
__device__ __forceinline__ bool small_eligible(const rl_sampling &s, uint32_t V) {
    return s.min_p > 0.0f && full_k(s, V) == V && s.temperature > 0.0f;
}

// ------------------------------------------------------------- keys ---
// grid (chunks, slots), FULL_THREADS: the penalised row (sample.rs:239-257) as
// total-order keys in id order, and per chunk the f32::max fold (NaN ignored)
// and the argmax composite. A window id's key is its penalised logit's,
// computed from the raw logit, so an id repeated in the window is penalised
// once. Dynamic LDS: a bitmap of the chunk's window ids
// (k_full_keys_lds_bytes). The row's last chunk to finish merges the chunks'
// results (sample.rs:267-277): the row state for the kernels that follow, and
// the answer of a row without a finite maximum (argmax, no draw).
// LDS bytes of k_full_keys's bitmap: one bit per element of the largest chunk.
__host__ __device__ inline size_t k_full_keys_lds_bytes(uint32_t vocab, uint32_t chunks) {
    const uint32_t n4 = vocab / 4;
    const uint32_t most = 4 * ((n4 + chunks - 1) / chunks) + 3;
    return ((size_t)(most + 31) / 32) * 4;
}

template <bool VEC>
__global__ __launch_bounds__(FULL_THREADS) void k_full_keys(RowIO a, FullScratch f) {
    extern __shared__ __align__(16) uint8_t smem[];
    RL_LDS uint32_t *bm = (RL_LDS uint32_t *)smem;  // window ids in this chunk, one bit per element
    __shared__ float red_max[FULL_THREADS / WAVE];
    __shared__ uint64_t red_am[FULL_THREADS / WAVE];
    const uint32_t slot = blockIdx.y, chunk = blockIdx.x;
    const uint32_t row = a.rows[slot];
    const rl_sampling s = a.settings[row];
    const uint32_t V = a.vocab;
    const uint32_t wl = window_len(a, row);
    const bool pen = penalises(s) && wl > 0;
    const float *rowp = a.logits + (uint64_t)row * a.stride;
    const uint32_t n4 = V / 4;
    const uint32_t q0 = chunk_lo(n4, chunk, a.chunks), q1 = chunk_lo(n4, chunk + 1, a.chunks);
    // The chunk's elements [e0, e1) (the last chunk also takes the vocab % 4
    // tail). A bitmap of the window ids among them makes the membership test
    // of four consecutive elements one LDS read, with no probing loop.
    const uint32_t e0 = 4 * q0, e1 = chunk == a.chunks - 1 ? V : 4 * q1;
    const uint32_t nwords = (e1 - e0 + 31) / 32;
    if (pen) {
        for (uint32_t i = threadIdx.x; i < nwords; i += FULL_THREADS) bm[i] = 0;
        __syncthreads();
        const uint32_t *win = a.windows + (uint64_t)row * a.wstride;
        for (uint32_t i = threadIdx.x; i < wl; i += FULL_THREADS) {
            const uint32_t id = win[i];
            if (id >= e0 && id < e1) atomicOr((uint32_t *)&bm[(id - e0) >> 5], 1u << ((id - e0) & 31));
        }
        __syncthreads();
    }
    uint32_t *keys = f.keyA + (uint64_t)slot * V;
    uint32_t *ids = f.idA + (uint64_t)slot * V;
    const bool vstore = ((reinterpret_cast<uintptr_t>(keys) | reinterpret_cast<uintptr_t>(ids)) & 15u) == 0;
    // The ids in id order are written only for a row that keeps that order
    // (no sort); the sort's first pass makes them from positions.
    const bool write_ids = identity_order(s, V);
    float mx = -__builtin_inff();
    uint64_t am = 0;
    auto take = [&](float x, uint32_t id) {
        const uint64_t c = composite(argmax_key(x), id);
        if (x > mx) mx = x;
        if (c > am) am = c;
    };
    // Four 16-byte loads in flight per thread; indices past the chunk are
    // clamped to its last element (a cache hit) and their results dropped.
    constexpr uint32_t KU = 4;
    for (uint32_t q = q0 + threadIdx.x; q < q1; q += FULL_THREADS * KU) {
        f32x4 v[KU];
#pragma unroll
        for (uint32_t u = 0; u < KU; ++u) {
            const uint32_t qq = q + u * FULL_THREADS;
            v[u] = load4<VEC>(rowp, qq < q1 ? qq : q1 - 1);
        }
#pragma unroll
        for (uint32_t u = 0; u < KU; ++u) {
            const uint32_t qq = q + u * FULL_THREADS;
            if (qq >= q1) break;
            float x[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
            if (pen) {  // the four ids' bits share a word: e0 and 4 * qq are multiples of 4
                const uint32_t off = 4 * qq - e0;
                const uint32_t in = (bm[off >> 5] >> (off & 31)) & 15u;
                if (in != 0) {
#pragma unroll
                    for (uint32_t c = 0; c < 4; ++c)
                        if ((in >> c) & 1u) x[c] = penalize(x[c], s.repeat_penalty);
                }
            }
            uint32_t kk[4];
#pragma unroll
            for (uint32_t c = 0; c < 4; ++c) {
                kk[c] = total_key(x[c]);
                take(x[c], 4 * qq + c);
            }
            if (vstore) {
                typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
                *(RL_GLB u32x4 *)(keys + 4 * qq) = u32x4{kk[0], kk[1], kk[2], kk[3]};
                if (write_ids) *(RL_GLB u32x4 *)(ids + 4 * qq) = u32x4{4 * qq, 4 * qq + 1, 4 * qq + 2, 4 * qq + 3};
            } else {
#pragma unroll
                for (uint32_t c = 0; c < 4; ++c) {
                    keys[4 * qq + c] = kk[c];
                    if (write_ids) ids[4 * qq + c] = 4 * qq + c;
                }
            }
        }
    }
    if (chunk == a.chunks - 1) {  // the last vocab % 4 elements
        const uint32_t e = 4 * n4 + threadIdx.x;
        if (e < V) {
            float x = ((const RL_GLB float *)rowp)[e];
            if (pen && ((bm[(e - e0) >> 5] >> ((e - e0) & 31)) & 1u)) x = penalize(x, s.repeat_penalty);
            keys[e] = total_key(x);
            if (write_ids) ids[e] = e;
            take(x, e);
        }
    }
    mx = wave_maxnum_f32(mx);
    am = wave_max_u64(am);
    const uint32_t wave = threadIdx.x / WAVE;
    if (lane_id() == 0) {
        red_max[wave] = mx;
        red_am[wave] = am;
    }
    __syncthreads();
    if (wave != 0) return;
    for (uint32_t i = 1; i < FULL_THREADS / WAVE; ++i) {
        mx = fmaxf(mx, red_max[i]);
        am = red_am[i] > am ? red_am[i] : am;
    }
    // Publish the chunk's result; the row's last chunk to arrive merges them.
    // The results are written with device-scope stores, which write through
    // this XCD's L2, and the arrival waits until they have completed; the
    // merging chunk reads them with device-scope loads after its arrival.
    const uint32_t lane = lane_id();
    if (lane == 0) {
        __hip_atomic_store((uint32_t *)f.part_max + slot * a.chunks + chunk, __float_as_uint(mx), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(f.part_am + slot * a.chunks + chunk, am, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __builtin_amdgcn_s_waitcnt(WAITCNT_VM0);  // the stores have completed
    uint32_t old = 0;
    if (lane == 0) old = atomicAdd(&f.arrive[slot], 1u);
    if (read_lane_u32(old, 0) != a.chunks - 1) return;
    // The last chunk (chunks <= MAX_CHUNKS <= WAVE): lane c reads chunk c.
    const bool ok = lane < a.chunks;
    const uint32_t mbits = ok ? __hip_atomic_load((const uint32_t *)f.part_max + slot * a.chunks + lane,
                                                  __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                              : __float_as_uint(-__builtin_inff());
    const uint64_t cam =
        ok ? __hip_atomic_load(f.part_am + slot * a.chunks + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0ull;
    mx = uniform_f32(wave_maxnum_f32(__uint_as_float(mbits)));
    am = uniform_u64(wave_max_u64(cam));
    if (lane == 0) {
        f.arrive[slot] = 0;  // ready for the next call
        const uint32_t am_tok = comp_key(am) == 0 ? 0u : comp_id(am);
        const bool finite = mx > -__builtin_inff() && mx < __builtin_inff();
        FullRow st{};
        st.M = mx;
        st.am_tok = am_tok;
        st.done = finite ? 0u : 1u;
        st.small = finite && small_eligible(s, V) ? 1u : 0u;
        f.row[slot] = st;
        if (!finite) write_single(a, row, am_tok);  // sample.rs:270-277
    }
}

// ------------------------------------------------------------- sort ---
// One wave's lanes with the same 8-bit digit (among the lanes where valid).
// Per bit: the lane's bit as a 0 / all-ones word, its ballot, and one
// three-input logic operation per mask half (m & ~(ballot ^ own)), so the
// select between a ballot and its complement costs no 64-bit arithmetic.
__device__ __forceinline__ uint64_t match_digit(uint32_t d, bool valid) {
    const uint64_t v = ballot(valid);
    uint32_t lo = (uint32_t)v, hi = (uint32_t)(v >> 32);
#pragma unroll
    for (uint32_t b = 0; b < 8; ++b) {
        const uint32_t own = (uint32_t)((int32_t)(d << (31 - b)) >> 31);  // bit b of d, replicated
        const uint64_t bb = ballot(own != 0u);
        lo &= ~((uint32_t)bb ^ own);
        hi &= ~((uint32_t)(bb >> 32) ^ own);
    }
    return ((uint64_t)hi << 32) | lo;
}

constexpr uint32_t SORT_ITEMS = 10;                         // elements per lane per tile
constexpr uint32_t SORT_UN = 8;                             // loads in flight per thread in the key scans
constexpr uint32_t SORT_TILE = SORT_THREADS * SORT_ITEMS;    // elements per tile
constexpr uint32_t WAVE_SEG = WAVE * SORT_ITEMS;             // a wave's contiguous share of a tile

// grid (slots), SORT_THREADS: a stable LSD radix sort of the row's (key, id)
// pairs by descending key, 8 bits a pass; ids start in ascending order, so
// ties keep ascending ids (the order of sample.rs:282-286). One read decides
// which passes run: a pass is skipped when its digit is the same for every key
// of each sign (as for logits on a bf16 grid, whose low 16 key bits follow the
// sign): keys that agree above such a digit agree on it, so the pass could not
// change the final order. Each tile gives every wave a contiguous segment,
// ranked item by item with wave-local running counts per digit, then
// reordered by digit in LDS and written out in runs. The result ends in
// keyA/idA.
__global__ __launch_bounds__(SORT_THREADS) void k_full_sort(RowIO a, FullScratch f) {
    __shared__ uint32_t hist[4][256];
    __shared__ uint32_t offs[256];
    __shared__ uint32_t cnt[SORT_WAVES][256];
    __shared__ uint32_t pos[SORT_WAVES][256];
    __shared__ uint32_t cls[4];  // OR and AND of the keys with the top bit clear, then set
    __shared__ uint32_t tcount[256], tstart[256];
    // The tile's keys and ids during the passes; before them, each wave's
    // private digit histograms ([wave][digit position][256], the same size).
    __shared__ uint32_t tile_ki[2 * SORT_TILE];
    static_assert(SORT_WAVES * 4 * 256 <= 2 * SORT_TILE, "private histograms fit the tile buffers");
    const uint32_t slot = blockIdx.x;
    if (f.row[slot].done) return;
    const uint32_t row = a.rows[slot];
    const rl_sampling s = a.settings[row];
    const uint32_t V = a.vocab;
    if (identity_order(s, V)) return;
    const uint32_t tid = threadIdx.x, wave = tid / WAVE, lane = lane_id();
    uint32_t *kin = f.keyA + (uint64_t)slot * V, *iin = f.idA + (uint64_t)slot * V;

    // Which passes run: per sign, the OR and the AND of its keys give the bits
    // in which keys of that sign differ (OR ^ AND); over all keys, the bits in
    // which any keys differ.
    if (tid < 4) cls[tid] = (tid & 1) ? 0xFFFFFFFFu : 0u;
    __syncthreads();
    {
        uint32_t or0 = 0u, and0 = 0xFFFFFFFFu, or1 = 0u, and1 = 0xFFFFFFFFu;
        for (uint32_t base = 0; base < V; base += SORT_THREADS * SORT_UN) {
            // Clamped, unconditional loads: a branch around each load would
            // make the loop wait for every load before the first use.
            uint32_t kk[SORT_UN];
#pragma unroll
            for (uint32_t u = 0; u < SORT_UN; ++u) {
                const uint32_t j = base + u * SORT_THREADS + tid;
                kk[u] = ((const RL_GLB uint32_t *)kin)[j < V ? j : V - 1];
            }
#pragma unroll
            for (uint32_t u = 0; u < SORT_UN; ++u) {
                if (base + u * SORT_THREADS + tid < V) {
                    if (kk[u] >> 31) {
                        or1 |= kk[u];
                        and1 &= kk[u];
                    } else {
                        or0 |= kk[u];
                        and0 &= kk[u];
                    }
                }
            }
        }
        for (int m = 32; m >= 1; m >>= 1) {
            or0 |= (uint32_t)__shfl_xor((int)or0, m);
            and0 &= (uint32_t)__shfl_xor((int)and0, m);
            or1 |= (uint32_t)__shfl_xor((int)or1, m);
            and1 &= (uint32_t)__shfl_xor((int)and1, m);
        }
        if (lane == 0) {
            atomicOr(&cls[0], or0);
            atomicAnd(&cls[1], and0);
            atomicOr(&cls[2], or1);
            atomicAnd(&cls[3], and1);
        }
    }
    __syncthreads();
    // An absent sign adds nothing: a key with the top bit clear clears it in
    // the AND of that sign, one with it set sets it in the OR of its sign.
    const bool has0 = cls[1] != 0xFFFFFFFFu, has1 = cls[2] != 0u;
    const uint32_t vary_sign = (has0 ? (cls[0] ^ cls[1]) : 0u) | (has1 ? (cls[2] ^ cls[3]) : 0u);
    const uint32_t all_or = (has0 ? cls[0] : 0u) | (has1 ? cls[2] : 0u);
    const uint32_t all_and = (has0 ? cls[1] : 0xFFFFFFFFu) & (has1 ? cls[3] : 0xFFFFFFFFu);
    // A lower digit's pass is skipped when the digit is the same for all keys
    // of each sign; the top digit's when it is the same for all keys.
    bool need[4];
    for (uint32_t t = 0; t < 3; ++t) need[t] = ((vary_sign >> (8 * t)) & 255u) != 0;
    need[3] = ((all_or ^ all_and) >> 24) != 0;

    // Histograms of the digits that are sorted on (values flipped, 255 - d,
    // for a descending order). Each wave counts into its own histograms, so
    // only lanes of one instruction contend for a counter (many equal keys
    // would otherwise serialise every wave on it); they are summed after.
    RL_LDS uint32_t *ph = (RL_LDS uint32_t *)tile_ki;
    for (uint32_t i = tid; i < SORT_WAVES * 4 * 256; i += SORT_THREADS) ph[i] = 0;
    __syncthreads();
    if (need[0] || need[1] || need[2] || need[3]) {
        uint32_t hot[4] = {256u, 256u, 256u, 256u};  // wave-uniform; 256: none yet
        for (uint32_t base = 0; base < V; base += SORT_THREADS * SORT_UN) {
            uint32_t kk[SORT_UN];
#pragma unroll
            for (uint32_t u = 0; u < SORT_UN; ++u) {
                const uint32_t j = base + u * SORT_THREADS + tid;
                kk[u] = ((const RL_GLB uint32_t *)kin)[j < V ? j : V - 1];
            }
#pragma unroll
            for (uint32_t u = 0; u < SORT_UN; ++u) {
                const bool valid = base + u * SORT_THREADS + tid < V;
#pragma unroll
                for (uint32_t t = 0; t < 4; ++t) {
                    if (!need[t]) continue;
                    const uint32_t d = 255u - ((kk[u] >> (8 * t)) & 255u);
                    // The lanes holding the wave's hot digit add once, through
                    // their first lane; the others one by one.
                    const uint64_t hm = ballot(valid && d == hot[t]);
                    if (hm != 0 && lanes_below(hm) == 0 && ((hm >> lane) & 1ull))
                        atomicAdd(&tile_ki[(wave * 4 + t) * 256 + hot[t]], (uint32_t)__popcll(hm));
                    if (valid && d != hot[t]) atomicAdd(&tile_ki[(wave * 4 + t) * 256 + d], 1u);
                    // The hot digit follows the most frequent one seen: the
                    // first other lane's digit replaces it when it is held by
                    // more lanes of this step.
                    const uint64_t rest = ballot(valid) & ~hm;
                    if (rest != 0) {
                        const uint32_t c = uniform_u32(
                            (uint32_t)__builtin_amdgcn_readlane((int)d, (int)__builtin_ctzll(rest)));
                        if (__popcll(ballot(valid && d == c)) > __popcll(hm)) hot[t] = c;
                    }
                }
            }
        }
    }
    __syncthreads();
    for (uint32_t i = tid; i < 4 * 256; i += SORT_THREADS) {  // i = t * 256 + d
        uint32_t c = 0;
        for (uint32_t w = 0; w < SORT_WAVES; ++w) c += ph[w * 4 * 256 + i];
        (&hist[0][0])[i] = c;
    }
    __syncthreads();

    // The passes. Each tile is ranked per wave (a contiguous segment each),
    // reordered by digit in LDS, and written out in runs, so that consecutive
    // lanes write consecutive addresses.
    uint32_t *kout = f.keyB + (uint64_t)slot * V, *iout = f.idB + (uint64_t)slot * V;
    // k_full_keys leaves the ids unwritten for a row that is sorted: the
    // first pass takes each element's position as its id.
    bool first = true;
    RL_LDS uint32_t *lk = (RL_LDS uint32_t *)tile_ki, *li = (RL_LDS uint32_t *)tile_ki + SORT_TILE;
    for (uint32_t t = 0; t < 4; ++t) {
        if (!need[t]) continue;
        if (tid < WAVE) {  // offs = exclusive prefix of the histogram
            uint32_t v[4], sum = 0;
#pragma unroll
            for (uint32_t q = 0; q < 4; ++q) {
                v[q] = hist[t][4 * tid + q];
                sum += v[q];
            }
            uint32_t incl = sum;
            for (uint32_t d = 1; d < WAVE; d <<= 1) {
                const uint32_t o = (uint32_t)__shfl_up((int)incl, d);
                if (lane >= d) incl += o;
            }
            uint32_t run = incl - sum;
#pragma unroll
            for (uint32_t q = 0; q < 4; ++q) {
                offs[4 * tid + q] = run;
                run += v[q];
            }
        }
        __syncthreads();
        const uint32_t shift = 8 * t;
        // The next tile's keys and ids load while this one is ranked.
        uint32_t nk[SORT_ITEMS], ni[SORT_ITEMS];
#pragma unroll
        for (uint32_t i = 0; i < SORT_ITEMS; ++i) {
            const uint32_t e = wave * WAVE_SEG + lane + i * WAVE;
            nk[i] = ((const RL_GLB uint32_t *)kin)[e < V ? e : V - 1];  // clamped; past V unused
            ni[i] = first ? e : ((const RL_GLB uint32_t *)iin)[e < V ? e : V - 1];
        }
        for (uint32_t tb = 0; tb < V; tb += SORT_TILE) {
            const uint32_t e0 = tb + wave * WAVE_SEG + lane;
            const uint32_t tn = min(SORT_TILE, V - tb);
            uint32_t kk[SORT_ITEMS], ii[SORT_ITEMS], rk[SORT_ITEMS];
#pragma unroll
            for (uint32_t i = 0; i < SORT_ITEMS; ++i) {
                kk[i] = nk[i];
                ii[i] = ni[i];
                const uint32_t e = e0 + SORT_TILE + i * WAVE;
                nk[i] = ((const RL_GLB uint32_t *)kin)[e < V ? e : V - 1];
                ni[i] = first ? e : ((const RL_GLB uint32_t *)iin)[e < V ? e : V - 1];
            }
            for (uint32_t d = lane; d < 256; d += WAVE) cnt[wave][d] = 0;
            wave_lds_sync();
#pragma unroll
            for (uint32_t i = 0; i < SORT_ITEMS; ++i) {
                const bool valid = e0 + i * WAVE < V;
                const uint32_t d = 255u - ((kk[i] >> shift) & 255u);
                const uint64_t peers = match_digit(d, valid);
                const uint32_t before = valid ? cnt[wave][d] : 0u;
                rk[i] = before + lanes_below(peers);
                wave_lds_sync();
                if (valid && lanes_below(peers) == 0) cnt[wave][d] = before + (uint32_t)__popcll(peers);
                wave_lds_sync();
            }
            __syncthreads();
            // Per digit: each wave's start within the digit's run of the tile,
            // and the run's length.
            if (tid < 256) {
                uint32_t run = 0;
                for (uint32_t w = 0; w < SORT_WAVES; ++w) {
                    pos[w][tid] = run;
                    run += cnt[w][tid];
                }
                tcount[tid] = run;
            }
            __syncthreads();
            if (tid < WAVE) {  // tstart = exclusive prefix of the runs' lengths
                uint32_t v[4], sum = 0;
#pragma unroll
                for (uint32_t q = 0; q < 4; ++q) {
                    v[q] = tcount[4 * tid + q];
                    sum += v[q];
                }
                uint32_t incl = sum;
                for (uint32_t d = 1; d < WAVE; d <<= 1) {
                    const uint32_t o = (uint32_t)__shfl_up((int)incl, d);
                    if (lane >= d) incl += o;
                }
                uint32_t run = incl - sum;
#pragma unroll
                for (uint32_t q = 0; q < 4; ++q) {
                    tstart[4 * tid + q] = run;
                    run += v[q];
                }
            }
            __syncthreads();
#pragma unroll
            for (uint32_t i = 0; i < SORT_ITEMS; ++i) {
                if (e0 + i * WAVE < V) {
                    const uint32_t d = 255u - ((kk[i] >> shift) & 255u);
                    const uint32_t at = tstart[d] + pos[wave][d] + rk[i];
                    lk[at] = kk[i];
                    li[at] = ii[i];
                }
            }
            __syncthreads();
            for (uint32_t j = tid; j < tn; j += SORT_THREADS) {
                const uint32_t key = lk[j];
                const uint32_t d = 255u - ((key >> shift) & 255u);
                const uint32_t dst = offs[d] + (j - tstart[d]);
                kout[dst] = key;
                iout[dst] = li[j];
            }
            __syncthreads();
            if (tid < 256) offs[tid] += tcount[tid];
            __syncthreads();
        }
        first = false;
        uint32_t *tmp;
        tmp = kin; kin = kout; kout = tmp;
        tmp = iin; iin = iout; iout = tmp;
    }
    if (kin != f.keyA + (uint64_t)slot * V) {  // an odd number of passes ran
        for (uint32_t j = tid; j < V; j += SORT_THREADS) {
            kout[j] = kin[j];
            iout[j] = iin[j];
        }
    } else if (first) {  // no pass ran (every key alike): the ids in id order
        for (uint32_t j = tid; j < V; j += SORT_THREADS) iin[j] = j;
    }
}

// ----------------------------------------------------------- min-p path ---
// A row with min-p on and the whole vocabulary as candidates keeps only
// candidates with p >= min_p (sample.rs:326-340), usually a few. Those are the
// first candidates of the reference's order (p falls along the order; checked
// below, not assumed), so the row needs only them sorted, plus the mass of the
// whole row for the top-p cut (sample.rs:307-324). The mass's sequential f64
// sum is not computed here: the sum in another order is within a proven
// relative bound of it, and the cut is accepted only when no value in that
// interval could move it. Anything else (too many survivors, a NaN, a cut
// inside the interval) leaves the row to the sorting kernels.

// grid (chunks, slots), FULL_THREADS: for rows on the min-p path, p of every
// id in this chunk (keys in id order), the chunk's f64 sum of p, the
// survivors as composites in the row's list, and the largest key of a
// non-survivor.
__global__ __launch_bounds__(FULL_THREADS) void k_full_collect(RowIO a, FullScratch f) {
    __shared__ uint64_t exp_tab[32];
    __shared__ double red_d[FULL_THREADS / WAVE];
    const uint32_t slot = blockIdx.y, chunk = blockIdx.x;
    const FullRow st = f.row[slot];
    if (st.done || !st.small) return;
    const uint32_t row = a.rows[slot];
    const rl_sampling s = a.settings[row];
    const uint32_t V = a.vocab;
    const uint32_t j0 = chunk_lo(V, chunk, a.chunks), j1 = chunk_lo(V, chunk + 1, a.chunks);
    const uint32_t *keys = f.keyA + (uint64_t)slot * V;
    uint64_t *list = f.surv + (uint64_t)slot * SURV_CAP;
    FullRow *rs = f.row + slot;
    copy_exp_table((RL_LDS uint64_t *)exp_tab);
    const TempScale tscale(s.temperature);
    const LdsExpTable etab{(RL_LDS uint64_t *)exp_tab};
    const uint32_t lane = lane_id();
    double sum = 0.0;
    uint32_t ns_key = 0;  // largest key + 1 of a non-survivor
    bool stop = false;
    // The row's overflow flag loads with a step's keys: the step sees the flag
    // as it was when the step began, which only delays an early stop (an
    // overflowing row's results are not used), and no step waits for it on
    // its own; a wave that overflows the list, or meets a non-finite p, stops
    // at once. (Loading the next step's keys during this one measured no
    // faster: a row that overflows, as a tie-heavy one does, stops after one
    // step and the loads are wasted.)
    for (uint32_t b = j0; b < j1 && !stop; b += FULL_THREADS * UN) {
        uint32_t kk[UN];
#pragma unroll
        for (uint32_t u = 0; u < UN; ++u) {
            const uint32_t j = b + u * FULL_THREADS + threadIdx.x;
            kk[u] = ((const RL_GLB uint32_t *)keys)[j < j1 ? j : j1 - 1];  // clamped: no branch around the load
        }
        const uint32_t overflow_seen = __hip_atomic_load(&rs->overflow, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        // The survivors of all UN steps take their list slots with one
        // atomic per wave (the wave waits for its result).
        uint64_t sm[UN];
        uint32_t wtotal = 0;
        bool nonfinite = false;
#pragma unroll
        for (uint32_t u = 0; u < UN; ++u) {
            const uint32_t j = b + u * FULL_THREADS + threadIdx.x;
            const bool ok = j < j1;
            const float p = ok ? expf_libm_t(tscale(key_value(kk[u]) - st.M), etab) : 0.0f;
            const bool finite = p <= 3.40282347e38f;  // false for NaN
            const bool surv = ok && finite && p >= s.min_p;
            if (ok) sum += (double)p;
            if (ok && finite && !surv) ns_key = max(ns_key, kk[u] + 1u);  // a finite p's key is below 0xFFFFFFFF
            nonfinite |= ok && !finite;
            sm[u] = ballot(surv);
            wtotal += (uint32_t)__popcll(sm[u]);
        }
        if (wtotal != 0) {
            uint32_t base = 0;
            if (lane == 0) base = atomicAdd(&rs->nsurv, wtotal);
            base = uniform_u32(__shfl((int)base, 0));
#pragma unroll
            for (uint32_t u = 0; u < UN; ++u) {
                if ((sm[u] >> lane) & 1ull) {
                    const uint32_t at = base + lanes_below(sm[u]);
                    if (at < SURV_CAP) list[at] = composite(kk[u], b + u * FULL_THREADS + threadIdx.x);
                }
                base += (uint32_t)__popcll(sm[u]);
            }
            if (base > SURV_CAP) {
                if (lane == 0) atomicOr(&rs->overflow, 1u);
                stop = true;  // this wave overflowed the list itself
            }
        }
        if (ballot(nonfinite) != 0) {
            if (lane == 0) atomicOr(&rs->overflow, 1u);
            stop = true;
        }
        stop = stop || uniform_u32(overflow_seen) != 0;
    }
    for (int m = 32; m >= 1; m >>= 1) {
        sum += __shfl_xor(sum, m);
        ns_key = max(ns_key, (uint32_t)__shfl_xor((int)ns_key, m));
    }
    if (lane == 0 && ns_key != 0) atomicMax(&rs->ns_key, ns_key);
    const uint32_t wave = threadIdx.x / WAVE;
    if (lane == 0) red_d[wave] = sum;
    __syncthreads();
    if (threadIdx.x == 0) {
        for (uint32_t w = 1; w < FULL_THREADS / WAVE; ++w) sum += red_d[w];
        f.psum[slot * a.chunks + chunk] = sum;
    }
}

// Sorts n2 (a power of two, <= SURV_CAP) composites in LDS, descending.
__device__ __forceinline__ void lds_bitonic_desc(RL_LDS uint64_t *v, uint32_t n2, uint32_t nt) {
    for (uint32_t size = 2; size <= n2; size <<= 1) {
        for (uint32_t stride = size >> 1; stride > 0; stride >>= 1) {
            for (uint32_t t = threadIdx.x; t < n2 / 2; t += nt) {
                const uint32_t i = 2 * t - (t & (stride - 1)), j = i + stride;
                const bool desc = (i & size) == 0;
                const uint64_t x = v[i], y = v[j];
                if ((x < y) == desc) {
                    v[i] = y;
                    v[j] = x;
                }
            }
            __syncthreads();
        }
    }
}

// k_full_small for a row of at most 64 survivors, on one wave: survivor i in
// lane i after a register bitonic sort, the sequential sums replayed with
// readlane in candidate order (the same f64 and f32 additions, in the same
// order, as the block replay), and no workgroup barrier. Leaves the row to
// the sorting kernels in the same cases as the block path.
__device__ __forceinline__ void small_one_wave(const RowIO &a, const FullScratch &f, uint32_t slot, uint32_t row,
                                               const rl_sampling &s, const FullRow &st, uint32_t c) {
    const uint32_t lane = lane_id();
    const uint32_t V = a.vocab;
    const bool by_id = !(s.top_p < 1.0f);  // top-p off: id order, as in the block path
    const uint64_t *list = f.surv + (uint64_t)slot * SURV_CAP;
    const bool in = lane < c;
    // Every load up front, so that their round trips overlap: the
    // survivors, the chunks' sums (lane ch holds chunk ch's; chunks <= 64)
    // and the uniform.
    uint64_t x = in ? list[lane] : 0ull;
    const double psum_lane = lane < a.chunks ? f.psum[slot * a.chunks + lane] : 0.0;
    const float u = a.uniforms[row];
    if (in && by_id) x = ((uint64_t)(uint32_t)x << 32) | comp_key(x);  // ~id in the high half
    x = wave_sort64<true>(x);
    const uint32_t key = by_id ? (uint32_t)x : comp_key(x);
    const uint32_t id = by_id ? ~(uint32_t)(x >> 32) : comp_id(x);
    const float p = in ? expf_libm((key_value(key) - st.M) / s.temperature) : 0.0f;

    uint32_t kept = c;
    double total = 0.0;
    bool have_total = false;
    if (!by_id) {
        if (st.ns_key != 0 && !(read_lane_u32(key, c - 1) >= st.ns_key)) return;
        if (!(s.top_p > 0.0f)) {
            kept = 1;  // sample.rs:315-323
            total = (double)read_lane_f32(p, 0);
            have_total = true;
        } else {
            // The mass interval of the block path (the same S, summed in the
            // same order, and the same d and bounds).
            double S = 0.0;
            for (uint32_t ch = 0; ch < a.chunks; ++ch)
                S += __longlong_as_double((long long)read_lane_u64((uint64_t)__double_as_longlong(psum_lane), ch));
            const double d = 2.25 * ((double)V + 64.0) * 0x1p-53;
            const double tp = (double)s.top_p;
            const double t_lo = tp * (S * (1.0 - d)) * (1.0 - 0x1p-50);
            const double t_hi = tp * (S * (1.0 + d)) * (1.0 + 0x1p-50);
            // The first partial sums to reach t_lo and t_hi; the cut is
            // certain when they are the same index.
            double cum = 0.0, at = 0.0;
            uint32_t j_lo = c, j_hi = c;
            for (uint32_t j = 0; j < c; ++j) {
                cum += (double)read_lane_f32(p, j);
                if (j_lo == c && cum >= t_lo) {
                    j_lo = j;
                    at = cum;
                }
                if (cum >= t_hi) {
                    j_hi = j;
                    break;
                }
            }
            if (j_lo == c) {
                at = cum;  // no cut among the survivors: their whole sum
            } else {
                if (j_hi != j_lo) return;  // the cut could fall on either side: sort the row
                kept = j_lo + 1;
            }
            total = at;  // the normalising sum, sample.rs:342
            have_total = true;
        }
    }
    if (!have_total)
        for (uint32_t j = 0; j < kept; ++j) total += (double)read_lane_f32(p, j);
    const float inv = (float)(1.0 / total);
    const float q = p * inv;
    if (ballot(lane < kept && !(q <= 3.40282347e38f)) != 0) return;  // the sorting kernels walk it in order
    if (lane < kept && a.out_ids) {
        a.out_ids[(uint64_t)row * a.cand_stride + lane] = id;
        a.out_probs[(uint64_t)row * a.cand_stride + lane] = q;
    }
    float cum = 0.0f;  // the draw, sample.rs:349-358
    uint32_t j = kept - 1;
    for (uint32_t i = 0; i < kept; ++i) {
        cum += read_lane_f32(q, i);
        if (cum > u) {
            j = i;
            break;
        }
    }
    const uint32_t tok = read_lane_u32(id, j);
    if (lane == 0) {
        a.out_token[row] = tok;
        a.out_kept[row] = kept;
        a.out_used[row] = 1;
        f.row[slot].done = 1;
    }
}

// grid (slots), REPLAY_THREADS: finishes a min-p row from its survivors, or
// leaves it (done stays 0) to the sorting kernels.
__global__ __launch_bounds__(REPLAY_THREADS) void k_full_small(RowIO a, FullScratch f) {
    __shared__ uint64_t sv_[SURV_CAP];
    __shared__ float sp_[SURV_CAP];
    __shared__ SeqLds<REPLAY_THREADS> seq;
    __shared__ uint64_t exp_tab[32];
    __shared__ uint32_t sh_bad;
    RL_LDS uint64_t *sv = (RL_LDS uint64_t *)sv_;
    RL_LDS float *sp = (RL_LDS float *)sp_;
    const uint32_t slot = blockIdx.x;
    const FullRow st = f.row[slot];
    if (st.done || !st.small || st.overflow) return;
    const uint32_t c = st.nsurv;
    if (c == 0 || c > SURV_CAP) return;  // no survivor: the reference keeps its first candidate
    const uint32_t row = a.rows[slot];
    const rl_sampling s = a.settings[row];
    const uint32_t V = a.vocab;
    const uint32_t tid = threadIdx.x;
    if (c <= WAVE) {  // one wave, no barrier; the other waves leave
        if (tid < WAVE) small_one_wave(a, f, slot, row, s, st, c);
        return;
    }
    // With top-p off the reference keeps id order (no sort, sample.rs:290-305):
    // the survivors are then sorted by ascending id, stored as
    // (~id << 32 | key) so that the same descending sort serves.
    const bool by_id = !(s.top_p < 1.0f);
    uint32_t n2 = 1;
    while (n2 < c) n2 <<= 1;
    const uint64_t *list = f.surv + (uint64_t)slot * SURV_CAP;
    for (uint32_t i = tid; i < n2; i += REPLAY_THREADS) {
        uint64_t x = 0;
        if (i < c) {
            x = list[i];
            if (by_id) x = ((uint64_t)(uint32_t)x << 32) | comp_key(x);  // ~id in the high half
        }
        sv[i] = x;
    }
    if (tid == 0) sh_bad = 0;
    copy_exp_table((RL_LDS uint64_t *)exp_tab);
    const LdsExpTable etab{(RL_LDS uint64_t *)exp_tab};
    lds_bitonic_desc(sv, n2, REPLAY_THREADS);
    auto key_at = [&](uint32_t i) { return by_id ? (uint32_t)sv[i] : comp_key(sv[i]); };
    auto id_at = [&](uint32_t i) { return by_id ? ~(uint32_t)(sv[i] >> 32) : comp_id(sv[i]); };
    for (uint32_t i = tid; i < c; i += REPLAY_THREADS)
        sp[i] = expf_libm_t((key_value(key_at(i)) - st.M) / s.temperature, etab);
    __syncthreads();
    const auto term = [sp](uint32_t j) { return sp[j]; };

    uint32_t kept = c;
    double total = 0.0;
    bool have_total = false;  // the normalising sum already known from the cut's replay
    if (!by_id) {
        // The survivors must be the first c candidates: every other key is
        // below the smallest survivor key (equal keys have equal p).
        if (st.ns_key != 0 && !(key_at(c - 1) >= st.ns_key)) return;
        if (!(s.top_p > 0.0f)) {
            kept = 1;  // a target <= 0 is met by the first candidate (sample.rs:315-323)
            total = (double)sp[0];
            have_total = true;
        } else {
            // The reference's mass (a sequential f64 sum of all V p's in
            // candidate order) and S (this sum in chunk order) are each
            // within gamma_(V-1) * mass of the exact sum, where
            // gamma_n = n 2^-53 / (1 - n 2^-53); d bounds both, with margin.
            // Each wave loads the chunks' sums at once (lane ch holds chunk
            // ch's) and adds them in chunk order.
            const uint32_t lane = lane_id();
            const double psum_lane = lane < a.chunks ? f.psum[slot * a.chunks + lane] : 0.0;
            double S = 0.0;
            for (uint32_t ch = 0; ch < a.chunks; ++ch)
                S += __longlong_as_double((long long)read_lane_u64((uint64_t)__double_as_longlong(psum_lane), ch));
            const double d = 2.25 * ((double)V + 64.0) * 0x1p-53;
            const double tp = (double)s.top_p;
            const double t_lo = tp * (S * (1.0 - d)) * (1.0 - 0x1p-50);
            const double t_hi = tp * (S * (1.0 + d)) * (1.0 + 0x1p-50);
            double at;
            const uint32_t j_lo =
                seq_replay<53, REPLAY_THREADS, SEQ_ITEMS>(term, c, [t_lo](double v) { return v >= t_lo; }, &seq, &at);
            if (j_lo < c) {
                // Partial sums never decrease and the one before j_lo is below
                // t_lo <= t_hi, so when the sum at j_lo reaches t_hi too, j_lo
                // is also the first index to reach t_hi.
                if (!(at >= t_hi)) {
                    double unused;
                    const uint32_t j_hi = seq_replay<53, REPLAY_THREADS, SEQ_ITEMS>(
                        term, c, [t_hi](double v) { return v >= t_hi; }, &seq, &unused);
                    if (j_hi != j_lo) return;  // the cut could fall on either side: sort the row
                }
                kept = j_lo + 1;
            }
            // The normalising total (sample.rs:342) is the same f64 sum of
            // the same terms in the same order, up to the last kept one: the
            // partial sum the cut's replay stopped at (all c of them when no
            // cut). Min-p removes none of them: every survivor is >= min_p.
            total = at;
            have_total = true;
        }
    }
    // Normalise over the kept candidates (sample.rs:342-347) and draw
    // (:349-358), both in their order.
    if (!have_total) seq_replay<53, REPLAY_THREADS, SEQ_ITEMS>(term, kept, NeverStop{}, &seq, &total);
    const float inv = (float)(1.0 / total);
    for (uint32_t i = tid; i < kept; i += REPLAY_THREADS) {
        const float q = sp[i] * inv;
        if (!(q <= 3.40282347e38f)) sh_bad = 1;
    }
    __syncthreads();
    if (sh_bad) return;  // a non-finite probability: the sorting kernels walk it in order
    for (uint32_t i = tid; i < kept; i += REPLAY_THREADS) {
        const float q = sp[i] * inv;
        sp[i] = q;
        if (a.out_ids) {
            a.out_ids[(uint64_t)row * a.cand_stride + i] = id_at(i);
            a.out_probs[(uint64_t)row * a.cand_stride + i] = q;
        }
    }
    __syncthreads();
    const float u = a.uniforms[row];
    double unused;
    const uint32_t j =
        seq_replay<24, REPLAY_THREADS, SEQ_ITEMS>(term, kept, [u](double v) { return v > (double)u; }, &seq, &unused);
    if (tid == 0) {
        a.out_token[row] = id_at(j < kept ? j : kept - 1);
        a.out_kept[row] = kept;
        a.out_used[row] = 1;
        f.row[slot].done = 1;
    }
}

// ------------------------------------------------------------ probs ---
// grid (chunks, slots), FULL_THREADS: p_j = exp((l_j - max) / T) for the
// candidates of this chunk (sample.rs:309), and per chunk: their f64 sum,
// the smallest binary exponent of a nonzero p, how many are >= min_p, the
// last index of one that is and the first of one that is not, and whether one
// is NaN or infinite.
__global__ __launch_bounds__(FULL_THREADS) void k_full_probs(RowIO a, FullScratch f) {
    __shared__ uint64_t exp_tab[32];
    __shared__ double red_d[FULL_THREADS / WAVE];
    __shared__ int red_e[FULL_THREADS / WAVE];
    __shared__ uint32_t red_c[FULL_THREADS / WAVE], red_b[FULL_THREADS / WAVE];
    __shared__ uint32_t red_li[FULL_THREADS / WAVE], red_fo[FULL_THREADS / WAVE];
    const uint32_t slot = blockIdx.y, chunk = blockIdx.x;
    const FullRow st = f.row[slot];
    if (st.done) return;
    const uint32_t row = a.rows[slot];
    const rl_sampling s = a.settings[row];
    const uint32_t V = a.vocab;
    const uint32_t k = full_k(s, V);
    const uint32_t j0 = chunk_lo(k, chunk, a.chunks), j1 = chunk_lo(k, chunk + 1, a.chunks);
    const uint32_t *keys = f.keyA + (uint64_t)slot * V;
    float *probs = f.probs + (uint64_t)slot * V;
    copy_exp_table((RL_LDS uint64_t *)exp_tab);
    const TempScale tscale(s.temperature);
    const LdsExpTable etab{(RL_LDS uint64_t *)exp_tab};
    double sum = 0.0;
    int emin = 1 << 20;
    uint32_t count = 0, bad = 0, last_in = 0, first_out = 0xFFFFFFFFu;
    // The next step's keys load while this step's exps are computed (clamped
    // loads: no branch around them).
    uint32_t nk[UN];
    if (j0 < j1) {
#pragma unroll
        for (uint32_t u = 0; u < UN; ++u) {
            const uint32_t j = j0 + u * FULL_THREADS + threadIdx.x;
            nk[u] = ((const RL_GLB uint32_t *)keys)[j < j1 ? j : j1 - 1];
        }
    }
    for (uint32_t b = j0; b < j1; b += FULL_THREADS * UN) {
        uint32_t kk[UN];
#pragma unroll
        for (uint32_t u = 0; u < UN; ++u) {
            kk[u] = nk[u];
            const uint32_t j = b + FULL_THREADS * UN + u * FULL_THREADS + threadIdx.x;
            nk[u] = ((const RL_GLB uint32_t *)keys)[j < j1 ? j : j1 - 1];
        }
#pragma unroll
        for (uint32_t u = 0; u < UN; ++u) {
            const uint32_t j = b + u * FULL_THREADS + threadIdx.x;
            if (j < j1) {
                const float p = expf_libm_t(tscale(key_value(kk[u]) - st.M), etab);
                probs[j] = p;
                if (!(p <= 3.40282347e38f)) {
                    bad = 1;  // NaN or +inf
                } else if (p > 0.0f) {
                    emin = min(emin, f32_exponent(p));
                }
                sum += (double)p;
                if (p >= s.min_p) {
                    ++count;
                    last_in = max(last_in, j + 1);
                } else {
                    first_out = min(first_out, j);
                }
            }
        }
    }
    for (int m = 32; m >= 1; m >>= 1) {
        sum += __shfl_xor(sum, m);
        emin = min(emin, __shfl_xor(emin, m));
        count += (uint32_t)__shfl_xor((int)count, m);
        bad |= (uint32_t)__shfl_xor((int)bad, m);
        last_in = max(last_in, (uint32_t)__shfl_xor((int)last_in, m));
        first_out = min(first_out, (uint32_t)__shfl_xor((int)first_out, m));
    }
    const uint32_t wave = threadIdx.x / WAVE;
    if (lane_id() == 0) {
        red_d[wave] = sum;
        red_e[wave] = emin;
        red_c[wave] = count;
        red_b[wave] = bad;
        red_li[wave] = last_in;
        red_fo[wave] = first_out;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (uint32_t w = 1; w < FULL_THREADS / WAVE; ++w) {
            sum += red_d[w];
            emin = min(emin, red_e[w]);
            count += red_c[w];
            bad |= red_b[w];
            last_in = max(last_in, red_li[w]);
            first_out = min(first_out, red_fo[w]);
        }
        const uint32_t i = slot * a.chunks + chunk;
        f.psum[i] = sum;
        f.pemin[i] = emin;
        f.pcount[i] = count;
        f.pbad[i] = bad;
        f.plast_in[i] = last_in;
        f.pfirst_out[i] = first_out;
    }
}

// ------------------------------------------------------------- tail ---

__device__ __forceinline__ uint32_t block_sum_u32(uint32_t v, RL_LDS uint32_t *red) {
    for (int m = 32; m >= 1; m >>= 1) v += (uint32_t)__shfl_xor((int)v, m);
    __syncthreads();
    if (lane_id() == 0) red[threadIdx.x / WAVE] = v;
    __syncthreads();
    uint32_t t = 0;
    for (uint32_t w = 0; w < REPLAY_WAVES; ++w) t += red[w];
    return t;
}

__device__ __forceinline__ int64_t block_max_i64(int64_t v, RL_LDS int64_t *red) {
    for (int m = 32; m >= 1; m >>= 1) {
        const int64_t o = (int64_t)shfl_xor_u64((uint64_t)v, m);
        v = o > v ? o : v;
    }
    __syncthreads();
    if (lane_id() == 0) red[threadIdx.x / WAVE] = v;
    __syncthreads();
    int64_t t = red[0];
    for (uint32_t w = 1; w < REPLAY_WAVES; ++w) t = red[w] > t ? red[w] : t;
    return t;
}

// Exclusive prefix of v over the workgroup's threads in thread order; *total
// gets the sum. For doubles it is only used where every partial sum is exact.
template <class T>
__device__ __forceinline__ T block_exclusive(T v, RL_LDS T *red, T *total) {
    const uint32_t lane = lane_id(), wave = threadIdx.x / WAVE;
    T incl = v;
    for (uint32_t d = 1; d < WAVE; d <<= 1) {
        const T o = __shfl_up(incl, d);
        if (lane >= d) incl += o;
    }
    __syncthreads();
    if (lane == WAVE - 1) red[wave] = incl;
    __syncthreads();
    T before = 0, all = 0;
    for (uint32_t w = 0; w < REPLAY_WAVES; ++w) {
        if (w < wave) before += red[w];
        all += red[w];
    }
    *total = all;
    return before + incl - v;
}

// Walks src[0..n) in order on thread 0, one LDS-staged block at a time; the
// whole workgroup stages. body(stage, base, count) returns true to stop.
template <class Body>
__device__ __forceinline__ void staged_walk(const float *src, uint32_t n, RL_LDS float *stage,
                                            RL_LDS uint32_t *stop, Body body) {
    for (uint32_t b = 0; b < n; b += STAGE) {
        const uint32_t cnt = min(STAGE, n - b);
        for (uint32_t i = threadIdx.x; i < cnt; i += REPLAY_THREADS) stage[i] = ((const RL_GLB float *)src)[b + i];
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
__device__ uint32_t exact_first_reaching(const float *probs, uint32_t lo, uint32_t hi, double base, double target,
                                         RL_LDS double *red, RL_LDS uint32_t *hit, RL_LDS double *hit_sum,
                                         double *at) {
    for (uint32_t b = lo; b < hi; b += REPLAY_THREADS * CI) {
        const uint32_t j0 = b + threadIdx.x * CI;
        float pv[CI];
        double mine = 0.0;
#pragma unroll
        for (uint32_t i = 0; i < CI; ++i) {
            pv[i] = j0 + i < hi ? ((const RL_GLB float *)probs)[j0 + i] : 0.0f;
            mine += (double)pv[i];
        }
        if (threadIdx.x == 0) *hit = 0xFFFFFFFFu;
        double step_total;
        double c = base + block_exclusive<double>(mine, red, &step_total);
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

// grid (slots), REPLAY_THREADS: the mass and the top-p cut (sample.rs:307-324),
// min-p (:326-340) and the normalising total (:342-343). Leaves m and 1/total
// in the row state.
__global__ __launch_bounds__(REPLAY_THREADS) void k_full_tail(RowIO a, FullScratch f) {
    __shared__ float stage_[STAGE];
    __shared__ SeqLds<REPLAY_THREADS> seq;
    __shared__ uint32_t red_u_[REPLAY_WAVES];
    __shared__ int64_t red_l_[REPLAY_WAVES];
    __shared__ double red_d_[REPLAY_WAVES];
    __shared__ uint32_t sh_m_, sh_stop_, sh_hit_;
    __shared__ double sh_d_, sh_hit_sum_;
    __shared__ double chunk_sum_[MAX_CHUNKS];
    RL_LDS double *chunk_sum = (RL_LDS double *)chunk_sum_;
    RL_LDS float *stage = (RL_LDS float *)stage_;
    RL_LDS uint32_t *red_u = (RL_LDS uint32_t *)red_u_;
    RL_LDS int64_t *red_l = (RL_LDS int64_t *)red_l_;
    RL_LDS double *red_d = (RL_LDS double *)red_d_;
    RL_LDS uint32_t *stop = (RL_LDS uint32_t *)&sh_stop_;

    const uint32_t slot = blockIdx.x;
    if (f.row[slot].done) return;
    const uint32_t row = a.rows[slot];
    const rl_sampling s = a.settings[row];
    const uint32_t V = a.vocab;
    const uint32_t tid = threadIdx.x;
    const uint32_t k = full_k(s, V);
    const uint32_t C = a.chunks;
    uint32_t *ids = f.idA + (uint64_t)slot * V;
    float *probs = f.probs + (uint64_t)slot * V;
    const auto term = [probs](uint32_t j) { return ((const RL_GLB float *)probs)[j]; };

    // The chunks' results, in chunk order (C <= MAX_CHUNKS).
    if (tid < C) chunk_sum[tid] = f.psum[slot * C + tid];
    __syncthreads();
    bool bad = false;
    int emin = 1 << 20;
    uint32_t count = 0, last_in = 0, first_out = 0xFFFFFFFFu;
    double tree_mass = 0.0;
    for (uint32_t c = 0; c < C; ++c) {
        const uint32_t i = slot * C + c;
        bad |= f.pbad[i] != 0;
        emin = min(emin, f.pemin[i]);
        count += f.pcount[i];
        last_in = max(last_in, f.plast_in[i]);
        first_out = min(first_out, f.pfirst_out[i]);
        tree_mass += chunk_sum[c];
    }
    // The candidates with p >= min_p form a prefix of the list.
    const bool surv_prefix = last_in <= first_out;
    // Every partial sum exact: all p are multiples of 2^(emin-23), the mass is
    // below 2^53 of those steps. Then the chunk sums are the exact sums too.
    const bool exact = !bad && (emin > 1000 || tree_mass < mul_pow2(1.0, 30 + emin));
    // The exact sum of p[0..n), from the chunk sums and one partial chunk.
    auto exact_prefix = [&](uint32_t n) {
        double b = 0.0;
        uint32_t c = 0;
        while (c < C && chunk_lo(k, c + 1, C) <= n) b += chunk_sum[c++];
        if (c == C || chunk_lo(k, c, C) == n) return b;
        double at;
        exact_first_reaching(probs, chunk_lo(k, c, C), n, b, __builtin_inf(), red_d, (RL_LDS uint32_t *)&sh_hit_, (RL_LDS double *)&sh_hit_sum_, &at);
        return at;
    };

    uint32_t m = k;
    bool have_sum_m = false;  // sum_m: the sequential sum of p[0..m)
    double sum_m = 0.0;
    if (s.top_p < 1.0f) {  // sample.rs:313-324
        double mass = 0.0;
        if (exact) {
            mass = tree_mass;
        } else if (!bad) {
            seq_replay<53, REPLAY_THREADS, SEQ_ITEMS>(term, k, NeverStop{}, &seq, &mass);
        } else {
            staged_walk(probs, k, stage, stop, [&](RL_LDS float *st, uint32_t, uint32_t cnt) {
                for (uint32_t i = 0; i < cnt; ++i) mass += (double)st[i];
                return false;
            });
            if (tid == 0) sh_d_ = mass;
            __syncthreads();
            mass = sh_d_;
        }
        const double target = (double)s.top_p * mass;
        if (exact) {
            // The chunk where the running sum first reaches the target.
            double b = 0.0;
            uint32_t c = 0;
            while (c < C && !(b + chunk_sum[c] >= target)) b += chunk_sum[c++];
            if (c < C) {
                double at;
                const uint32_t j = exact_first_reaching(probs, chunk_lo(k, c, C), chunk_lo(k, c + 1, C), b, target,
                                                        red_d, (RL_LDS uint32_t *)&sh_hit_, (RL_LDS double *)&sh_hit_sum_, &at);
                m = j + 1;
                have_sum_m = true;
                sum_m = at;
            } else {
                have_sum_m = true;
                sum_m = mass;
            }
        } else if (!bad) {
            double at;
            const uint32_t j = seq_replay<53, REPLAY_THREADS, SEQ_ITEMS>(
                term, k, [target](double c) { return c >= target; }, &seq, &at);
            have_sum_m = true;
            if (j < k) {
                m = j + 1;
                sum_m = at;
            } else {
                sum_m = mass;
            }
        } else {
            if (tid == 0) sh_m_ = k;
            __syncthreads();
            double cum = 0.0;
            staged_walk(probs, k, stage, stop, [&](RL_LDS float *st, uint32_t b, uint32_t cnt) {
                for (uint32_t i = 0; i < cnt; ++i) {
                    cum += (double)st[i];
                    if (cum >= target) {
                        sh_m_ = b + i + 1;
                        return true;
                    }
                }
                return false;
            });
            __syncthreads();
            m = sh_m_;
        }
    }
    if (s.min_p > 0.0f) {  // sample.rs:326-340, a stable in-place compaction
        uint32_t w;
        if (!bad && surv_prefix) {
            // The survivors are the first `count` of all k candidates (so it
            // is with sorted candidates, where p falls along the order), and
            // min(m, count) of the first m: nothing moves.
            w = min(m, count);
        } else {
            // Survivors anywhere: count them, and compact unless they are
            // already a prefix.
            uint32_t first_out = 0xFFFFFFFFu, last_in = 0, cnt = 0;
            for (uint32_t b = 0; b < m; b += REPLAY_THREADS) {
                const uint32_t j = b + tid;
                if (j < m) {
                    if (((const RL_GLB float *)probs)[j] >= s.min_p) {
                        ++cnt;
                        last_in = j + 1;
                    } else if (first_out == 0xFFFFFFFFu) {
                        first_out = j;
                    }
                }
            }
            w = block_sum_u32(cnt, red_u);
            const uint32_t lo_out = (uint32_t)-block_max_i64(-(int64_t)first_out, red_l);
            const uint32_t hi_in = (uint32_t)block_max_i64((int64_t)last_in, red_l);
            if (hi_in > lo_out) {
                uint32_t done = 0;
                for (uint32_t b = 0; b < m; b += REPLAY_THREADS * CI) {
                    const uint32_t j0 = b + tid * CI;
                    float pv[CI];
                    uint32_t iv[CI];
                    uint32_t mine = 0;
#pragma unroll
                    for (uint32_t i = 0; i < CI; ++i) {
                        const bool ok = j0 + i < m;
                        pv[i] = ok ? probs[j0 + i] : 0.0f;
                        iv[i] = ok ? ids[j0 + i] : 0u;
                        mine += (ok && pv[i] >= s.min_p) ? 1u : 0u;
                    }
                    uint32_t step_total;
                    uint32_t dst = done + block_exclusive<uint32_t>(mine, red_u, &step_total);
#pragma unroll
                    for (uint32_t i = 0; i < CI; ++i) {
                        if (j0 + i < m && pv[i] >= s.min_p) {
                            ids[dst] = iv[i];
                            probs[dst] = pv[i];
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
    // Normalise: f64 total in order (sample.rs:342-343).
    double total = 0.0;
    if (have_sum_m) {
        total = sum_m;  // the same terms in the same order as the top-p pass
    } else if (exact && (surv_prefix || !(s.min_p > 0.0f))) {
        total = exact_prefix(m);  // min-p moved nothing: the chunk sums still apply
    } else if (exact) {
        exact_first_reaching(probs, 0, m, 0.0, __builtin_inf(), red_d, (RL_LDS uint32_t *)&sh_hit_, (RL_LDS double *)&sh_hit_sum_, &total);
    } else if (!bad) {
        seq_replay<53, REPLAY_THREADS, SEQ_ITEMS>(term, m, NeverStop{}, &seq, &total);
    } else {
        staged_walk(probs, m, stage, stop, [&](RL_LDS float *st, uint32_t, uint32_t cnt) {
            for (uint32_t i = 0; i < cnt; ++i) total += (double)st[i];
            return false;
        });
        if (tid == 0) sh_d_ = total;
        __syncthreads();
        total = sh_d_;
    }
    if (tid == 0) {
        const float inv = (float)(1.0 / total);
        f.row[slot].m = m;
        f.row[slot].inv = inv;
        // q = p * inv is finite for every kept p when every p is and inv is
        // (p <= 1 and inv <= 1: the best p is exp(0) = 1, so total >= 1).
        f.row[slot].qbad = (bad || !(inv <= 3.40282347e38f)) ? 1u : 0u;
    }
}

// ------------------------------------------------------- draw and norm ---
// The kept candidates q = p * (1 / total) (sample.rs:344-347), written to the
// outputs, for chunk `chunk` of slot's m candidates, by the workgroup's
// REPLAY_THREADS threads.
__device__ __forceinline__ void norm_chunk(const RowIO &a, const FullScratch &f, uint32_t slot, uint32_t chunk) {
    constexpr uint32_t NT = REPLAY_THREADS;
    const FullRow st = f.row[slot];
    if (st.done) return;
    const uint32_t row = a.rows[slot];
    const uint32_t V = a.vocab;
    const uint32_t m = st.m;
    const uint32_t j0 = chunk_lo(m, chunk, a.chunks), j1 = chunk_lo(m, chunk + 1, a.chunks);
    const uint32_t *ids = f.idA + (uint64_t)slot * V;
    const float *probs = f.probs + (uint64_t)slot * V;
    constexpr uint32_t NU = UN / 2;  // as many loads in flight per workgroup as UN at FULL_THREADS
    for (uint32_t b = j0; b < j1; b += NT * NU) {
        float pp[NU];
        uint32_t iv[NU];
#pragma unroll
        for (uint32_t u = 0; u < NU; ++u) {
            const uint32_t j = b + u * NT + threadIdx.x;
            const uint32_t jc = j < j1 ? j : j1 - 1;  // clamped: no branch around the loads
            pp[u] = ((const RL_GLB float *)probs)[jc];
            iv[u] = ((const RL_GLB uint32_t *)ids)[jc];
        }
#pragma unroll
        for (uint32_t u = 0; u < NU; ++u) {
            const uint32_t j = b + u * NT + threadIdx.x;
            if (j < j1) {
                a.out_ids[(uint64_t)row * a.cand_stride + j] = iv[u];
                a.out_probs[(uint64_t)row * a.cand_stride + j] = pp[u] * st.inv;
            }
        }
    }
}

// The f32 running sum of q = p * (1 / total) against the host's uniform
// (sample.rs:349-356); a shortfall takes the last candidate (:357-358). The
// whole workgroup, for one slot.
__device__ __forceinline__ void draw_row(const RowIO &a, const FullScratch &f, uint32_t slot, RL_LDS float *stage,
                                         RL_LDS uint32_t *stop, RL_LDS uint32_t *tok_out, SeqLds<REPLAY_THREADS> *seq) {
    const FullRow st = f.row[slot];
    if (st.done) return;
    const uint32_t row = a.rows[slot];
    const uint32_t V = a.vocab;
    const uint32_t m = st.m;
    const uint32_t *ids = f.idA + (uint64_t)slot * V;
    const float *probs = f.probs + (uint64_t)slot * V;
    const float inv = st.inv;
    const float u = a.uniforms[row];
    uint32_t pick;
    if (!st.qbad) {
        double unused;
        const uint32_t j = seq_replay<24, REPLAY_THREADS, SEQ_ITEMS>(
            [probs](uint32_t j) { return ((const RL_GLB uint32_t *)probs)[j]; },
            [inv](uint32_t bits) { return __uint_as_float(bits) * inv; }, m, [u](double c) { return c > (double)u; },
            seq, &unused);
        pick = j < m ? j : m - 1;
    } else {
        if (threadIdx.x == 0) *tok_out = m - 1;
        __syncthreads();
        float cum = 0.0f;
        staged_walk(probs, m, stage, stop, [&](RL_LDS float *sv, uint32_t b, uint32_t cnt) {
            for (uint32_t i = 0; i < cnt; ++i) {
                cum += sv[i] * inv;
                if (cum > u) {
                    *tok_out = b + i;
                    return true;
                }
            }
            return false;
        });
        __syncthreads();
        pick = *tok_out;
    }
    if (threadIdx.x == 0) {
        a.out_token[row] = ids[pick];
        a.out_kept[row] = m;
        a.out_used[row] = 1;
    }
}

// grid (slots + slots * chunks when the candidates are written, else slots),
// REPLAY_THREADS: workgroup x < slots draws slot x's token; the others write
// chunk (x - slots) % chunks of slot (x - slots) / chunks's kept candidates.
// Neither reads what the other writes, so the draws (bound by the replay's
// arithmetic, one workgroup a row) and the writes (bound by HBM) share the
// GPU in one launch.
__global__ __launch_bounds__(REPLAY_THREADS) void k_full_finish(RowIO a, FullScratch f, uint32_t slots) {
    __shared__ float stage_[STAGE];
    __shared__ SeqLds<REPLAY_THREADS> seq;
    __shared__ uint32_t sh_stop_, sh_tok_;
    const uint32_t x = blockIdx.x;
    if (x < slots) {
        draw_row(a, f, x, (RL_LDS float *)stage_, (RL_LDS uint32_t *)&sh_stop_, (RL_LDS uint32_t *)&sh_tok_, &seq);
    } else {
        const uint32_t i = x - slots;
        norm_chunk(a, f, i / a.chunks, i % a.chunks);
    }
}

}  // namespace rl
