// The FULL device path: rows with top_k == 0, top_k >= vocab or top_k > 64
// (sample.rs:279-358 over the whole candidate list). Launches per group of
// rows, alternating kernels that spread a row over many workgroups (the HBM-
// and ALU-heavy steps) with one workgroup per row (the steps that follow the
// reference's sequential order):
//
//   k_full_pass    (chunks x rows)  the one read of every row: the f32::max
//                                   fold; rows without a finite maximum
//                                   answered; min-p rows finished from their
//                                   survivors when the top-p cut is certain
//   k_full_keys    (chunks x rows)  the rows left: total-order keys of the
//                                   penalised row in id order
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
    uint32_t done;     // the row is finished (no finite maximum, or the min-p path)
    uint32_t m;        // candidates kept (after top-p and min-p)
    float inv;         // (1 / total) as f32
    uint32_t qbad;     // a normalised probability may not be finite: the draw walks in order
};

// Candidates the min-p path collects per row (a superset of the survivors).
constexpr uint32_t SURV_CAP = 4096;
// A row's per-chunk results are read one chunk per lane.
static_assert(MAX_CHUNKS <= WAVE, "a wave holds one lane per chunk");

struct FullScratch {
    uint32_t *keyA, *idA, *keyB, *idB;  // [slot][vocab]
    float *probs;                       // [slot][vocab]
    float *part_max;                    // [slot][chunk] k_full_pass: the chunk's maximum
    uint64_t *part_am;                  // [slot][chunk] k_full_pass: candidates listed << 32 | lowest +inf id
    double *psum;                       // [slot][chunk] k_full_pass: its mass; then the probs pass's sum
    int *pemin;                         // [slot][chunk]
    uint32_t *pcount;                   // [slot][chunk]
    uint32_t *pbad;                     // [slot][chunk]
    uint32_t *plast_in;                 // [slot][chunk] probs pass: last index + 1 with p >= min_p
    uint32_t *pfirst_out;               // [slot][chunk] first index with p < min_p
    uint64_t *surv;                     // [slot][SURV_CAP] min-p candidates (composites), a region per chunk
    FullRow *row;                       // [slot]
    uint32_t *arrive;                   // [slot] k_full_pass: chunks done; zero between calls
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
// grid (chunks, slots), FULL_THREADS, after k_full_pass: for the rows it left
// to the sorting kernels, the penalised row (sample.rs:239-257) as
// total-order keys in id order (and the ids, for a row that keeps id order).
// A window id's key is its penalised logit's, computed from the raw logit, so
// an id repeated in the window is penalised once. Dynamic LDS: a bitmap of
// the chunk's window ids (k_full_keys_lds_bytes).
// LDS bytes of the window bitmap: one bit per element of the largest chunk.
__host__ __device__ inline size_t k_full_keys_lds_bytes(uint32_t vocab, uint32_t chunks) {
    const uint32_t n4 = vocab / 4;
    const uint32_t most = 4 * ((n4 + chunks - 1) / chunks) + 3;
    return ((size_t)(most + 31) / 32) * 4;
}

template <bool VEC>
__global__ __launch_bounds__(FULL_THREADS) void k_full_keys(RowIO a, FullScratch f) {
    extern __shared__ __align__(16) uint8_t smem[];
    RL_LDS uint32_t *bm = (RL_LDS uint32_t *)smem;  // window ids in this chunk, one bit per element
    const uint32_t slot = blockIdx.y, chunk = blockIdx.x;
    if (f.row[slot].done) return;
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
            for (uint32_t c = 0; c < 4; ++c) kk[c] = total_key(x[c]);
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
        }
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
// first candidates of the reference's order (p falls along the order; checked,
// not assumed), so the row needs only them sorted, plus the mass of the whole
// row for the top-p cut (sample.rs:307-324). k_full_pass reads the row once:
// per chunk the f32::max fold, the mass relative to the chunk's own maximum
// and a superset of the survivors; the row's last chunk to finish knows the
// true maximum, computes the survivors' p exactly, and accepts the top-p cut
// only when no mass in a proven interval around the reference's could move it.
// Anything else (too many survivors, a NaN, a cut inside the interval) leaves
// the row to the sorting kernels.
//
// The mass interval. The reference's mass is S_ref = sum of p_j in sorted
// order (f64, sequential), p_j = expf(fl(fl(l_j - M) / T)). With y_j =
// (l_j - M) / T exactly, fl rounding twice puts x_j within |y_j| 2^-23 of y_j
// and libm expf is within 0.502 ulp, so p_j = e^(y_j) (1 + e_j) with |e_j| <=
// 2^-23 |y_j| + 2^-24 to first order (plus 2^-149 absolute in the subnormal
// range). The pass computes, relative to a running maximum m <= M that was
// already seen, q_j = exp2_hw(fl(fl(l_j - m) * c2)) with c2 = fl(log2(e) / T)
// rounded once from the f64 quotient: the exponent carries at most 3 roundings
// of 2^-24 relative, so q_j e^((m - M) / T) = e^(y_j) (1 + g_j) with |g_j| <=
// 3 2^-24 |y_j| + H (H bounds the hardware exp2's own error, see HW_EXP2_REL),
// and partial sums are rescaled by f64 factors e^((m_old - m_new) / T) as m
// rises. Splitting at |y| = K: terms with |y_j| <= K are within
// EPS_NEAR relative of each other in the two computations; terms beyond
// differ by at most 2.01 e^(-K) + 2^-124 each (both are below e^(-K) (1 +
// tiny), or flushed subnormals). Summation adds gamma_32 in f32 (each
// thread's terms of one step), a few f64 roundings, and gamma_(V-1) for the
// reference's sequential sum. MASS_REL collects the relative terms.

constexpr uint32_t PASS_U = 10;                          // float4 per thread per step
constexpr uint32_t PASS_STEP = FULL_THREADS * PASS_U;    // float4 per step
constexpr uint32_t FULL_WAVES = FULL_THREADS / WAVE;
constexpr uint32_t FIN_CAP = 1024;                       // survivors the pass finishes itself
constexpr uint32_t PASS_CAND = 1024;                     // candidates a chunk holds in LDS
constexpr uint32_t LIST_OVER = 0xFFFFFFFFu;              // a chunk's candidates did not fit
constexpr double HW_EXP2_REL = 0x1p-21;                  // v_exp_f32 bound assumed (4 ulp; tested <= 1 ulp)
constexpr double MASS_K = 32.0;
constexpr double EPS_NEAR =
    ((0x1p-23 + 3.0 * 0x1p-24) * MASS_K + 1.004 * 0x1p-24 + HW_EXP2_REL) * (1.0 + 0x1p-7);
constexpr double MASS_REL = EPS_NEAR / (1.0 - EPS_NEAR) + 33.0 * 0x1p-24 + 0x1p-40;
constexpr double RESCALE_REL = (0x1p-24 + HW_EXP2_REL) * 1.001;  // one in-loop rescaling factor
// 2.01 e^(-K) + 2^-124 per term (e^-32 = 1.2664165549e-14).
constexpr double MASS_ABS_PER_TERM = 2.01 * 1.2664165549094176e-14 + 0x1p-124;

// Loads of k_full_pass's aligned variant are buffer loads: the resource
// covers the row's n floats (reads past them return zeros, never fault), each
// lane's byte offset is one register and the step's offset is scalar, so no
// per-load 64-bit address stays live across a step. gfx9's descriptor word 3
// (0x00020000: 32-bit data format, raw addressing); nontemporal (aux 2).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t row_rsrc(const float *row, uint32_t n) {
    return __builtin_amdgcn_make_buffer_rsrc((void *)row, (short)0, (int)(n * 4u), 0x00020000);
}
template <bool VEC>
__device__ __forceinline__ f32x4 pass_load(__amdgpu_buffer_rsrc_t r, const float *row, uint32_t f, uint32_t f_lane,
                                           uint32_t end) {
    if constexpr (VEC) {
        // f = f_step + f_lane: the step part (uniform) goes in the scalar offset.
        return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, 16u * f_lane, 16u * (f - f_lane), 2));
    } else {
        return load4<false>(row, f < end ? f : end - 1);
    }
}

// 2^z for z <= 0 as an f64 rescaling factor inside the streaming loop:
// 2^floor(z) exactly (ldexp) times the hardware exp2 of the fraction rounded
// to f32, so the factor is within 2^-24 + HW_EXP2_REL relative (or below
// 2^-1022 where the true value is), with no f64 exp polynomial to keep in
// registers across the loop.
__device__ __forceinline__ double rescale(double z) {
    if (!(z > -1100.0)) return 0.0;
    const double n = __builtin_floor(z);
    return __builtin_ldexp((double)__builtin_amdgcn_exp2f((float)(z - n)), (int)n);
}

// Composite of a survivor in the order its row keeps them: the reference's
// order (descending key, ascending id) when top-p is on; ascending id (stored
// as ~id << 32 | key, so that one descending sort serves) when it is off.
__device__ __forceinline__ uint64_t keep_order(uint64_t c, bool by_id) {
    return by_id ? (((uint64_t)(uint32_t)c << 32) | comp_key(c)) : c;
}
__device__ __forceinline__ uint32_t keep_key(uint64_t x, bool by_id) { return by_id ? (uint32_t)x : comp_key(x); }
__device__ __forceinline__ uint32_t keep_id(uint64_t x, bool by_id) { return by_id ? ~(uint32_t)(x >> 32) : comp_id(x); }

// Sorts n2 (a power of two) composites in LDS, descending, with nt threads.
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

// The row's finish from c <= 64 survivors, on one wave: survivor i in lane i
// (x: its keep_order composite, unsorted), p by libm-exact exp, the top-p cut
// certified against [t_lo, t_hi] (the interval that holds the reference's
// target top_p * mass), the normalising total, q = p * inv and the f32 draw,
// all replayed with readlane in candidate order (the reference's f64 and f32
// additions in its order). Returns false (nothing written) when the cut could
// fall on either side or a q is not finite: the sorting kernels take the row.
__device__ __forceinline__ bool finish_wave(const RowIO &a, uint32_t row, const rl_sampling &s, float M, uint32_t c,
                                            uint64_t x, bool by_id, uint32_t ns_key, double t_lo, double t_hi,
                                            const LdsExpTable &etab) {
    const uint32_t lane = lane_id();
    const bool in = lane < c;
    const float u = a.uniforms[row];
    x = wave_sort64<true>(in ? x : 0ull);
    const uint32_t key = keep_key(x, by_id);
    const uint32_t id = keep_id(x, by_id);
    const float p = in ? expf_libm_t((key_value(key) - M) / s.temperature, etab) : 0.0f;
    uint32_t kept = c;
    double total = 0.0;
    bool have_total = false;
    if (!by_id) {
        // The survivors must be the first c candidates: every other key that
        // could precede them is below the smallest survivor's.
        if (ns_key != 0 && !(read_lane_u32(key, c - 1) >= ns_key)) return false;
        if (!(s.top_p > 0.0f)) {
            kept = 1;  // a target <= 0 is met by the first candidate (sample.rs:315-323)
            total = (double)read_lane_f32(p, 0);
            have_total = true;
        } else {
            // The first partial sums to reach t_lo and t_hi; the cut is
            // certain when they are the same index.
            double at = 0.0;
            uint32_t j_lo = c, j_hi = c;
            // Every p here is a normal f32 >= 2^emin, so a multiple of
            // 2^(emin - 23); with c <= 64 terms <= 1 every partial sum is
            // below 2^7 and needs at most 30 - emin significant bits: when
            // that is <= 53 every f64 partial sum is exact, and an inclusive
            // scan of the wave gives the sequential sums bit for bit.
            const int e = in ? f32_exponent(p) : 1 << 20;
            const int emin = (int)uniform_u32((uint32_t)wave_min_i32(e));
            if (emin >= -23) {
                double cum = in ? (double)p : 0.0;
                for (uint32_t d = 1; d < WAVE; d <<= 1) {
                    const double o = f64_from_bits(shfl_up_u64(f64_bits(cum), (int)d));
                    if (lane >= d) cum += o;
                }
                const uint64_t lo = ballot(in && cum >= t_lo), hi = ballot(in && cum >= t_hi);
                j_lo = lo ? (uint32_t)__ffsll((unsigned long long)lo) - 1u : c;
                j_hi = hi ? (uint32_t)__ffsll((unsigned long long)hi) - 1u : c;
                at = f64_from_bits(read_lane_u64(f64_bits(cum), j_lo == c ? c - 1 : j_lo));
            } else {
                double cum = 0.0;
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
                if (j_lo == c) at = cum;
            }
            if (j_lo != c) {
                if (j_hi != j_lo) return false;
                kept = j_lo + 1;
            }
            total = at;  // the normalising sum, sample.rs:342 (all c when no cut: min-p decides)
            have_total = true;
        }
    }
    if (!have_total)
        for (uint32_t j = 0; j < kept; ++j) total += (double)read_lane_f32(p, j);
    const float inv = (float)(1.0 / total);
    const float q = p * inv;
    if (ballot(lane < kept && !(q <= 3.40282347e38f)) != 0) return false;
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
    }
    return true;
}

// The same finish for 64 < c <= FIN_CAP survivors: sv holds their
// keep_order composites, sorted here by the workgroup (NT threads); sp gets
// their p; one thread then walks them in order exactly as the reference does
// (the f64 cut and total, the f32 draw), and the workgroup writes the kept
// candidates. Every thread returns the same verdict.
template <uint32_t NT>
__device__ __forceinline__ bool finish_block(const RowIO &a, uint32_t row, const rl_sampling &s, float M, uint32_t c,
                                             RL_LDS uint64_t *sv, RL_LDS float *sp, RL_LDS uint32_t *sh,
                                             RL_LDS float *sh_inv, const LdsExpTable &etab, bool by_id,
                                             uint32_t ns_key, double t_lo, double t_hi) {
    const uint32_t tid = threadIdx.x;
    uint32_t n2 = 1;
    while (n2 < c) n2 <<= 1;
    for (uint32_t i = c + tid; i < n2; i += NT) sv[i] = 0;
    __syncthreads();
    lds_bitonic_desc(sv, n2, NT);
    for (uint32_t i = tid; i < c; i += NT) sp[i] = expf_libm_t((key_value(keep_key(sv[i], by_id)) - M) / s.temperature, etab);
    __syncthreads();
    if (tid == 0) {
        // sh[0]: kept (0 when the row is left to the sorting kernels), sh[1]: the drawn index.
        uint32_t kept = c;
        double total = 0.0;
        bool ok = true;
        if (!by_id && ns_key != 0 && !(keep_key(sv[c - 1], false) >= ns_key)) ok = false;
        if (ok && !by_id && !(s.top_p > 0.0f)) {
            kept = 1;  // sample.rs:315-323
            total = (double)sp[0];
        } else if (ok && !by_id) {
            double cum = 0.0;
            uint32_t j_lo = c, j_hi = c;
            for (uint32_t j = 0; j < c; ++j) {
                cum += (double)sp[j];
                if (j_lo == c && cum >= t_lo) {
                    j_lo = j;
                    total = cum;
                }
                if (cum >= t_hi) {
                    j_hi = j;
                    break;
                }
            }
            if (j_lo == c) total = cum;                  // no cut among the survivors
            else if (j_hi != j_lo) ok = false;           // the cut could fall on either side
            else kept = j_lo + 1;
        } else if (ok) {
            for (uint32_t j = 0; j < kept; ++j) total += (double)sp[j];
        }
        float inv = 0.0f;
        uint32_t pick = 0;
        if (ok) {
            inv = (float)(1.0 / total);
            float cum = 0.0f;  // the draw, sample.rs:349-358
            const float u = a.uniforms[row];
            pick = kept - 1;
            for (uint32_t j = 0; j < kept; ++j) {
                const float q = sp[j] * inv;
                if (!(q <= 3.40282347e38f)) ok = false;
                cum += q;
                if (cum > u) {
                    pick = j;
                    break;
                }
            }
            for (uint32_t j = pick + 1; ok && j < kept; ++j)
                if (!(sp[j] * inv <= 3.40282347e38f)) ok = false;
        }
        sh[0] = ok ? kept : 0u;
        sh[1] = pick;
        *sh_inv = inv;
    }
    __syncthreads();
    const uint32_t kept = sh[0];
    if (kept == 0) return false;
    const float inv = *sh_inv;
    if (a.out_ids)
        for (uint32_t i = tid; i < kept; i += NT) {
            a.out_ids[(uint64_t)row * a.cand_stride + i] = keep_id(sv[i], by_id);
            a.out_probs[(uint64_t)row * a.cand_stride + i] = sp[i] * inv;
        }
    if (tid == 0) {
        a.out_token[row] = keep_id(sv[sh[1]], by_id);
        a.out_kept[row] = kept;
        a.out_used[row] = 1;
    }
    return true;
}

// Dynamic LDS of k_full_pass: the chunk's window bitmap while streaming, the
// finisher's survivors (FIN_CAP composites and their p) after.
__host__ __device__ inline size_t k_full_pass_lds_bytes(uint32_t vocab, uint32_t chunks) {
    const size_t fin = (size_t)FIN_CAP * (sizeof(uint64_t) + sizeof(float));
    const size_t bm = k_full_keys_lds_bytes(vocab, chunks);
    return bm > fin ? bm : fin;
}

// grid (chunks, slots), FULL_THREADS: the single read of the full path.
// Every row: the penalised row's f32::max fold per chunk (sample.rs:267-269)
// and the lowest id holding +inf; the row's last chunk to finish answers rows
// without a finite maximum (argmax, no draw, sample.rs:270-277) and leaves the
// maximum in the row state for the sorting kernels. Rows eligible for the
// min-p path also get, per chunk, the mass relative to the chunk's maximum
// and the candidates that could survive min-p (appended to the row's list),
// and the last chunk finishes them when it can (done = 1).
template <bool VEC>
__global__ __launch_bounds__(FULL_THREADS, 4) void k_full_pass(RowIO a, FullScratch f) {
    extern __shared__ __align__(16) uint8_t smem[];
    RL_LDS uint32_t *bm = (RL_LDS uint32_t *)smem;  // window ids in this chunk, one bit per element
    __shared__ float red_m[FULL_WAVES];
    __shared__ double red_s[FULL_WAVES];
    __shared__ uint32_t red_i[FULL_WAVES], red_f[FULL_WAVES];
    __shared__ uint32_t sh_last, sh_count, sh_ns, sh_flag;
    __shared__ uint32_t sh_fin[2];
    __shared__ float sh_inv;
    __shared__ uint64_t exp_tab[32];
    __shared__ uint64_t cbuf[PASS_CAND];  // this chunk's candidates, filtered by its maximum at the end
    __shared__ uint32_t sh_cn, sh_cover;
    __shared__ uint32_t red_cnt[MAX_CHUNKS];   // the finisher: each chunk's listed candidates
    const uint32_t slot = blockIdx.y, chunk = blockIdx.x;
    const uint32_t tid = threadIdx.x, lane = lane_id(), wave = tid / WAVE;
    const uint32_t row = a.rows[slot];
    const rl_sampling s = a.settings[row];
    const uint32_t V = a.vocab;
    const uint32_t C = a.chunks;
    const uint32_t wl = window_len(a, row);
    const bool pen = penalises(s) && wl > 0;
    const float *rowp = a.logits + (uint64_t)row * a.stride;
    const uint32_t n4 = V / 4;
    const uint32_t q0 = chunk_lo(n4, chunk, C), q1 = chunk_lo(n4, chunk + 1, C);
    const uint32_t e0 = 4 * q0, e1 = chunk == C - 1 ? V : 4 * q1;
    const uint32_t nwords = (e1 - e0 + 31) / 32;
    // The window's ids and the exp table load first; then the first step's
    // loads (clamped: no branch around them). Vector loads complete in order,
    // so anything loaded after the step would wait for all of it. The window
    // bitmap and the tables are built while the step is in flight.
    constexpr uint32_t WIN_PER = 8;  // window ids per thread (max_window <= 2048)
    static_assert(WIN_PER * FULL_THREADS >= 2048, "a window's ids fit the threads");
    // Unconditional (clamped) loads: a load under a divergent branch makes
    // the compiler wait for every load in flight, the step's included.
    uint32_t wid[WIN_PER];
    const uint32_t *win = a.windows + (uint64_t)row * a.wstride;
    if (pen) {
#pragma unroll
        for (uint32_t k = 0; k < WIN_PER; ++k) {
            const uint32_t i = k * FULL_THREADS + tid;
            wid[k] = win[i < wl ? i : wl - 1];
        }
    }
    const uint64_t tab = EXP2_32_TAB[tid & 31u];
    const __amdgpu_buffer_rsrc_t rsrc = row_rsrc(rowp, V);
    f32x4 A[PASS_U];
    // Buffer loads need no guard (past the row they return zeros); a uniform
    // branch here would also make the compiler wait for all loads at its end.
    if (VEC || q0 < q1) {
#pragma unroll
        for (uint32_t u = 0; u < PASS_U; ++u) A[u] = pass_load<VEC>(rsrc, rowp, q0 + u * FULL_THREADS + tid, tid, q1);
    }
    if (pen) {
        for (uint32_t i = tid; i < nwords; i += FULL_THREADS) bm[i] = 0;
        __syncthreads();
#pragma unroll
        for (uint32_t k = 0; k < WIN_PER; ++k) {
            const uint32_t id = wid[k];
            if (k * FULL_THREADS + tid < wl && id >= e0 && id < e1)
                atomicOr((uint32_t *)&bm[(id - e0) >> 5], 1u << ((id - e0) & 31));
        }
    }
    if (tid == 0) {
        sh_cn = 0;
        sh_cover = 0;
    }
    if (tid < 32) exp_tab[tid] = tab;  // for the finisher
    __syncthreads();
    const bool eligible = small_eligible(s, V);
    // Workgroup constants, kept in scalar registers.
    const double invT_d = uniform_f64(1.0 / (double)s.temperature);
    const double log2e_T = uniform_f64(1.4426950408889634 * invT_d);
    // Base-2 exponent per unit of (l - m), and the survival test in it: any
    // element below ln(min_p) - 1e-3 (with margin for the roundings of z and
    // of the logarithm) relative to a maximum already seen has p < min_p.
    const float c2 = uniform_f32((float)log2e_T);
    const float zthr = uniform_f32((float)(((double)logf(s.min_p) * (1.0 + 0x1p-18) - 1e-3) * 1.4426950408889634));
    // The mass needs a finite c2 and threshold (T not tiny or huge, min_p > 0).
    bool mass = eligible && c2 < 3.0e38f && c2 > 0.0f && zthr > -3.0e38f;
    uint64_t *list = f.surv + (uint64_t)slot * SURV_CAP;

    float m_run = -__builtin_inff();  // wave-uniform: the wave's maximum so far
    double S = 0.0;                   // per lane: mass relative to m_run
    uint32_t first_inf = 0xFFFFFFFFu;
    bool nan_seen = false;
    // The penalised logit of element e of this chunk, re-read from memory
    // (the candidates' rare path; their row was just read).
    auto value_at = [&](uint32_t e) {
        float v = ((const RL_GLB float *)rowp)[e];
        if (pen && ((bm[(e - e0) >> 5] >> ((e - e0) & 31)) & 1u)) v = penalize(v, s.repeat_penalty);
        return v;
    };
    // Appends this lane's candidates (the set bits i of mb; id_of(i) is the
    // vocabulary id of candidate i) to the chunk's LDS buffer: one LDS atomic
    // per wave, slots by an exclusive scan of the lanes' counts. A full
    // buffer sends the row to the sorting kernels.
    auto append = [&](uint64_t mb, auto id_of) {
        const uint32_t mine = (uint32_t)__popcll(mb);
        uint32_t incl = mine;
        for (uint32_t d = 1; d < WAVE; d <<= 1) {
            const uint32_t o = (uint32_t)__shfl_up((int)incl, d);
            if (lane >= d) incl += o;
        }
        const uint32_t wtotal = (uint32_t)__shfl((int)incl, WAVE - 1);
        uint32_t base = 0;
        if (lane == 0) base = atomicAdd((uint32_t *)&sh_cn, wtotal);
        base = uniform_u32((uint32_t)__shfl((int)base, 0));
        uint32_t at = base + incl - mine;
        while (mb != 0) {
            const uint32_t i = (uint32_t)__ffsll((unsigned long long)mb) - 1u;
            mb &= mb - 1ull;
            const uint32_t e = id_of(i);
            if (at < PASS_CAND) cbuf[at] = composite(total_key(value_at(e)), e);
            ++at;
        }
        if (base + wtotal > PASS_CAND) {
            if (lane == 0) sh_cover = 1;
            mass = false;  // the row leaves the min-p path
        }
    };
    // A step's PASS_U float4 per thread are all in flight at once (a chunk
    // of the 64-row workload is one step); the penalty is applied in place.
    for (uint32_t b = q0; b < q1; b += PASS_STEP) {
        if (b != q0) {
#pragma unroll
            for (uint32_t u = 0; u < PASS_U; ++u) A[u] = pass_load<VEC>(rsrc, rowp, b + u * FULL_THREADS + tid, tid, q1);
        }
        float tmax = -__builtin_inff();
#pragma unroll
        for (uint32_t u = 0; u < PASS_U; ++u) {
            const uint32_t qq = b + u * FULL_THREADS + tid;
            if (pen && qq < q1) {  // the four ids' bits share a word: e0 and 4 * qq are multiples of 4
                const uint32_t off = 4 * qq - e0;
                const uint32_t in = (bm[off >> 5] >> (off & 31)) & 15u;
                if (in != 0) {
#pragma unroll
                    for (uint32_t c = 0; c < 4; ++c)
                        if ((in >> c) & 1u) A[u][c] = penalize(A[u][c], s.repeat_penalty);
                }
            }
            if (qq < q1) tmax = fmaxf(tmax, fmaxf(fmaxf(A[u].x, A[u].y), fmaxf(A[u].z, A[u].w)));
        }
        tmax = uniform_f32(wave_maxnum_f32(tmax));
        if (tmax > m_run) {
            if (tmax == __builtin_inff()) {  // the first +inf of this wave's elements
                uint32_t fi = 0xFFFFFFFFu;
#pragma unroll
                for (uint32_t u = 0; u < PASS_U; ++u) {
                    const uint32_t qq = b + u * FULL_THREADS + tid;
#pragma unroll
                    for (uint32_t c = 0; c < 4; ++c)
                        if (qq < q1 && A[u][c] == __builtin_inff()) fi = min(fi, 4 * qq + c);
                }
                first_inf = min(first_inf, fi);
                mass = false;  // the row has no finite maximum
            } else if (m_run > -__builtin_inff()) {
                S *= rescale(((double)m_run - (double)tmax) * log2e_T);
            }
            m_run = tmax;
        }
        if (mass && m_run > -__builtin_inff()) {
            // The step's terms and the largest z of this lane's elements; a
            // full step needs no per-element bounds test.
            float acc = 0.0f, zmax = -__builtin_inff();
            if (b + PASS_STEP <= q1) {
#pragma unroll
                for (uint32_t u = 0; u < PASS_U; ++u)
#pragma unroll
                    for (uint32_t c = 0; c < 4; ++c) {
                        const float z = (A[u][c] - m_run) * c2;
                        acc += __builtin_amdgcn_exp2f(z);
                        zmax = fmaxf(zmax, z);
                    }
            } else {
#pragma unroll
                for (uint32_t u = 0; u < PASS_U; ++u) {
                    const bool ok = b + u * FULL_THREADS + tid < q1;
#pragma unroll
                    for (uint32_t c = 0; c < 4; ++c) {
                        const float z = (A[u][c] - m_run) * c2;
                        const float q = __builtin_amdgcn_exp2f(z);
                        if (ok) {
                            acc += q;
                            zmax = fmaxf(zmax, z);
                        }
                    }
                }
            }
            S += (double)acc;
            if (ballot(zmax >= zthr) != 0) {  // rare: this wave holds candidates
                uint64_t mb = 0;  // this lane's: bit 4u + c
#pragma unroll
                for (uint32_t u = 0; u < PASS_U; ++u) {
                    const bool ok = b + u * FULL_THREADS + tid < q1;
#pragma unroll
                    for (uint32_t c = 0; c < 4; ++c)
                        if (ok && (A[u][c] - m_run) * c2 >= zthr) mb |= 1ull << (4 * u + c);
                }
                append(mb, [&](uint32_t i) { return 4 * (b + (i >> 2) * FULL_THREADS + tid) + (i & 3u); });
            }
        } else if (eligible && m_run == -__builtin_inff()) {
            // Nothing finite so far: no mass, but a NaN must still send the
            // row to the sorting kernels.
#pragma unroll
            for (uint32_t u = 0; u < PASS_U; ++u)
#pragma unroll
                for (uint32_t c = 0; c < 4; ++c)
                    if (b + u * FULL_THREADS + tid < q1 && A[u][c] != A[u][c]) nan_seen = true;
        }
    }
    if (chunk == C - 1) {  // the last vocab % 4 elements, one per thread (at most 3)
        const uint32_t e = 4 * n4 + tid;
        float xe = -__builtin_inff();
        const bool ok = e < V;
        if (ok) {
            xe = ((const RL_GLB float *)rowp)[e];
            if (pen && ((bm[(e - e0) >> 5] >> ((e - e0) & 31)) & 1u)) xe = penalize(xe, s.repeat_penalty);
        }
        const float tmax = uniform_f32(wave_maxnum_f32(xe));
        if (tmax > m_run) {
            if (tmax == __builtin_inff()) {
                first_inf = min(first_inf, (ok && xe == __builtin_inff()) ? e : 0xFFFFFFFFu);
                mass = false;
            } else if (m_run > -__builtin_inff()) {
                S *= exp(((double)m_run - (double)tmax) * invT_d);
            }
            m_run = tmax;
        }
        if (mass && m_run > -__builtin_inff()) {
            const float z = (xe - m_run) * c2;
            if (ok) S += (double)__builtin_amdgcn_exp2f(z);
            const uint64_t mb = (ok && z >= zthr) ? 1ull : 0ull;
            if (ballot(mb != 0) != 0) append(mb, [&](uint32_t) { return e; });
        } else if (eligible && ok && xe != xe) {
            nan_seen = true;
        }
    }
    // The wave's record: its maximum, its mass relative to it (NaN when a NaN
    // was met), the lowest +inf id.
    S = wave_total_f64(S);
    if (ballot(nan_seen) != 0) S = __builtin_nan("");
    {
        uint32_t fi = first_inf;
        for (int m = 32; m >= 1; m >>= 1) fi = min(fi, (uint32_t)__shfl_xor((int)fi, m));
        first_inf = fi;
    }
    if (lane == 0) {
        red_m[wave] = m_run;
        red_s[wave] = S;
        red_i[wave] = first_inf;
    }
    __syncthreads();
    float Mc = -__builtin_inff();
    for (uint32_t w = 0; w < FULL_WAVES; ++w) Mc = fmaxf(Mc, red_m[w]);
    // The chunk's candidates against its own maximum (still a superset of
    // the row's survivors: M >= Mc), compacted into the chunk's own region of
    // the row's list (SURV_CAP / C entries) with device-scope stores. The
    // count goes with the chunk's record; LIST_OVER marks a region too small.
    const uint32_t region = SURV_CAP / C;
    uint32_t nkeep = 0;
    if (eligible && Mc > -__builtin_inff() && Mc < __builtin_inff() && sh_cover == 0) {
        const uint32_t n = min(sh_cn, PASS_CAND);
        uint32_t mine = 0;  // this wave's kept candidates, its slice of the buffer
        const uint32_t per = (n + FULL_WAVES - 1) / FULL_WAVES;
        const uint32_t lo = min(n, wave * per), hi = min(n, lo + per);
        for (uint32_t b = lo; b < hi; b += WAVE) {
            const uint32_t i = b + lane;
            const uint64_t cc = i < hi ? cbuf[i] : 0ull;
            mine += (uint32_t)__popcll(ballot(i < hi && (key_value(comp_key(cc)) - Mc) * c2 >= zthr));
        }
        if (lane == 0) red_f[wave] = mine;
        __syncthreads();
        uint32_t at = 0;
        for (uint32_t w = 0; w < FULL_WAVES; ++w) {
            if (w < wave) at += red_f[w];
            nkeep += red_f[w];
        }
        if (nkeep <= region) {
            uint64_t *dst = list + chunk * region;
            for (uint32_t b = lo; b < hi; b += WAVE) {
                const uint32_t i = b + lane;
                const uint64_t cc = i < hi ? cbuf[i] : 0ull;
                const bool keep = i < hi && (key_value(comp_key(cc)) - Mc) * c2 >= zthr;
                const uint64_t mk = ballot(keep);
                if (keep) __hip_atomic_store(dst + at + lanes_below(mk), cc, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                at += (uint32_t)__popcll(mk);
            }
        } else {
            nkeep = LIST_OVER;
        }
    } else if (sh_cover != 0) {
        nkeep = LIST_OVER;
    }
    if (wave == 0) {
        uint32_t fi = 0xFFFFFFFFu;
        for (uint32_t w = 0; w < FULL_WAVES; ++w) fi = min(fi, red_i[w]);
        double Sc = 0.0;
        if (Mc > -__builtin_inff() && Mc < __builtin_inff())
            for (uint32_t w = 0; w < FULL_WAVES; ++w)
                if (red_m[w] > -__builtin_inff()) Sc += red_s[w] * exp(((double)red_m[w] - (double)Mc) * invT_d);
        for (uint32_t w = 0; w < FULL_WAVES; ++w)
            if (red_s[w] != red_s[w]) Sc = __builtin_nan("");
        // Publish the chunk's record with device-scope stores (they write
        // through this XCD's L2); the arrival waits until every store of this
        // workgroup's waves has completed, the list entries included.
        if (lane == 0) {
            const uint32_t i = slot * C + chunk;
            __hip_atomic_store((uint32_t *)f.part_max + i, __float_as_uint(Mc), __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store((uint64_t *)f.psum + i, (uint64_t)__double_as_longlong(Sc), __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(f.part_am + i, ((uint64_t)nkeep << 32) | fi, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    __builtin_amdgcn_s_waitcnt(WAITCNT_VM0);  // this wave's stores have completed
    __syncthreads();                          // and every other wave's
    if (tid == 0) sh_last = atomicAdd(&f.arrive[slot], 1u) == C - 1 ? 1u : 0u;
    __syncthreads();
    if (!sh_last) return;

    // ---- the row's last chunk: every chunk's record, then the row ----
    // The first K = SPEC * FULL_THREADS / C entries of every chunk's region
    // load now, before the counts are known (thread t takes entries
    // t % (K / SPEC) + j K / SPEC of chunk t / (K / SPEC)): most chunks list
    // fewer than K, so their entries need no second round trip.
    constexpr uint32_t SPEC = 4;
    const uint32_t region_c = SURV_CAP / C, KT = FULL_THREADS / C, K = SPEC * KT;
    const uint32_t sch = tid / KT, sidx = tid % KT;
    uint64_t spec[SPEC];
#pragma unroll
    for (uint32_t j = 0; j < SPEC; ++j)
        spec[j] = (eligible && sch < C) ? __hip_atomic_load(list + sch * region_c + sidx + j * KT, __ATOMIC_RELAXED,
                                                            __HIP_MEMORY_SCOPE_AGENT)
                                        : 0ull;
    const bool okc = lane < C;  // C <= MAX_CHUNKS <= WAVE: lane c holds chunk c
    const float Mr = okc ? __uint_as_float(__hip_atomic_load((const uint32_t *)f.part_max + slot * C + lane,
                                                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT))
                         : -__builtin_inff();
    const double Sc = okc ? __longlong_as_double((long long)__hip_atomic_load(
                                (const uint64_t *)f.psum + slot * C + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT))
                          : 0.0;
    const uint64_t rec = okc ? __hip_atomic_load(f.part_am + slot * C + lane, __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT)
                             : ((uint64_t)0 << 32) | 0xFFFFFFFFu;
    uint32_t fi = (uint32_t)rec;
    const uint32_t nc = (uint32_t)(rec >> 32);  // chunk lane's listed candidates, or LIST_OVER
    const bool lover = ballot(nc == LIST_OVER) != 0;
    // How many candidates all chunks listed.
    uint32_t incl = nc == LIST_OVER ? 0u : nc;
    for (uint32_t d = 1; d < WAVE; d <<= 1) {
        const uint32_t o = (uint32_t)__shfl_up((int)incl, d);
        if (lane >= d) incl += o;
    }
    const uint32_t nlist = uniform_u32((uint32_t)__shfl((int)incl, WAVE - 1));
    if (wave == 0 && okc) red_cnt[lane] = nc == LIST_OVER ? 0u : nc;
    const float M = uniform_f32(wave_maxnum_f32(Mr));
    for (int m = 32; m >= 1; m >>= 1) fi = min(fi, (uint32_t)__shfl_xor((int)fi, m));
    if (tid == 0) f.arrive[slot] = 0;  // ready for the next call
    const bool finite = M > -__builtin_inff() && M < __builtin_inff();
    if (!finite || !eligible) {
        if (tid == 0) {
            FullRow st{};
            st.M = M;
            st.done = finite ? 0u : 1u;
            f.row[slot] = st;
            // sample.rs:270-277: argmax, no draw; the first +inf, or 0 when
            // nothing is above -inf.
            if (!finite) write_single(a, row, M == __builtin_inff() ? uniform_u32(fi) : 0u);
        }
        return;
    }
    // The mass interval (identical on every wave).
    const double term = (okc && Mr > -__builtin_inff()) ? Sc * exp(((double)Mr - (double)M) * invT_d) : 0.0;
    const double Smid = wave_total_f64(term);
    bool ok_row = Smid == Smid && !lover && nlist > 0 && c2 < 3.0e38f && c2 > 0.0f && zthr > -3.0e38f;
    // The survivors: every listed candidate's exact p (sample.rs:309), kept
    // when p >= min_p (sample.rs:333); the largest key of one that is not.
    RL_LDS uint64_t *sv = (RL_LDS uint64_t *)smem;
    RL_LDS float *sp = (RL_LDS float *)(smem + FIN_CAP * sizeof(uint64_t));
    const bool by_id = !(s.top_p < 1.0f);
    if (tid == 0) {
        sh_count = 0;
        sh_ns = 0;
    }
    __syncthreads();  // red_cnt, sh_count and sh_ns are set
    const LdsExpTable etab{(RL_LDS uint64_t *)exp_tab};
    const TempScale tscale(s.temperature);
    if (ok_row) {
        uint32_t ns = 0;
        auto take = [&](uint64_t c) {
            const uint32_t key = comp_key(c);
            const float p = expf_libm_t(tscale(key_value(key) - M), etab);
            if (p >= s.min_p) {
                const uint32_t at = atomicAdd((uint32_t *)&sh_count, 1u);
                if (at < FIN_CAP) sv[at] = keep_order(c, by_id);
            } else {
                ns = max(ns, key + 1u);  // a finite p's key is below 0xFFFFFFFF
            }
        };
#pragma unroll
        for (uint32_t j = 0; j < SPEC; ++j)
            if (sch < C && sidx + j * KT < red_cnt[sch]) take(spec[j]);
        // The entries at K and beyond of chunks that listed more, all loads
        // of one pass in flight together (entry i of them belongs to the last
        // chunk whose count of extras before it is <= i).
        uint32_t extra = 0;
        for (uint32_t ch = 0; ch < C; ++ch) extra += red_cnt[ch] > K ? red_cnt[ch] - K : 0u;
        for (uint32_t i = tid; i < extra; i += FULL_THREADS) {
            uint32_t ch = 0, before = 0, acc = 0;
            for (uint32_t k = 0; k < C; ++k) {
                const uint32_t e = red_cnt[k] > K ? red_cnt[k] - K : 0u;
                if (acc <= i && e != 0) {
                    ch = k;
                    before = acc;
                }
                acc += e;
            }
            take(__hip_atomic_load(list + ch * region_c + K + (i - before), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
        }
        for (int m = 32; m >= 1; m >>= 1) ns = max(ns, (uint32_t)__shfl_xor((int)ns, m));
        if (lane == 0 && ns != 0) atomicMax((uint32_t *)&sh_ns, ns);
    }
    __syncthreads();
    const uint32_t c = sh_count, ns_key = sh_ns;
    ok_row = ok_row && c > 0 && c <= FIN_CAP;
    // t_lo <= top_p * S_ref <= t_hi, with the reference's target rounding.
    // Each step after a chunk's first can rescale the terms before it once
    // more (RESCALE_REL each); the absolute terms cover the far terms and
    // factors below 2^-1022.
    const uint32_t steps = (chunk_lo(V / 4, 1, C) + PASS_STEP) / PASS_STEP;  // the largest chunk's steps, or more
    const double rel = MASS_REL + (double)steps * RESCALE_REL;
    const double abs_err = MASS_ABS_PER_TERM * (double)V + (double)V * 0x1p-1000;
    const double gam = ((double)V + 64.0) * 0x1p-53;
    const double S_lo = (Smid * (1.0 - rel) - abs_err) * (1.0 - gam);
    const double S_hi = (Smid * (1.0 + rel) + abs_err) * (1.0 + gam);
    const double tp = (double)s.top_p;
    const double t_lo = tp * S_lo * (1.0 - 0x1p-48);
    const double t_hi = tp * S_hi * (1.0 + 0x1p-48);
    bool fin = false;
    if (ok_row && c <= WAVE) {
        if (wave == 0) {
            const uint64_t xw = lane < c ? sv[lane] : 0ull;
            fin = finish_wave(a, row, s, M, c, xw, by_id, ns_key, t_lo, t_hi, etab);
            if (lane == 0) sh_flag = fin ? 1u : 0u;
        }
        __syncthreads();
        fin = sh_flag != 0;
    } else if (ok_row) {
        fin = finish_block<FULL_THREADS>(a, row, s, M, c, sv, sp, (RL_LDS uint32_t *)sh_fin, (RL_LDS float *)&sh_inv,
                                         etab, by_id, ns_key, t_lo, t_hi);
    }
    if (tid == 0) {
        FullRow st{};
        st.M = M;
        st.done = fin ? 1u : 0u;
        f.row[slot] = st;
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
