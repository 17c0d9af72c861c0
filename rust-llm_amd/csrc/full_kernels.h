// The FULL device path: rows with top_k == 0, top_k >= vocab or top_k > 64
// (sample.rs:279-358 over the whole candidate list). Two launches per group
// of rows:
//
//   k_full_pass  (chunks x rows)  the one read of every row: the f32::max
//                                 fold; rows without a finite maximum
//                                 answered; min-p rows finished from their
//                                 survivors when the top-p cut is certain
//   k_full_rest  (rows)           the rows left, one workgroup each
//                                 (full_rest.h): the candidates sorted, p, the
//                                 cut, min-p, the total, the draw and the kept
//                                 candidates
//
// The sums are the reference's sequential sums, bit for bit: when every p is a
// multiple of 2^(e_min - 23) and the mass is below 2^(30 + e_min), every partial
// sum is exactly representable, so any order of addition gives the same bits
// and per-chunk sums serve; otherwise seq_replay (rl_seqsum.h) reproduces the
// sequential rounding in parallel. Rows with a NaN or infinite p (NaN logits,
// a NaN temperature, 1 / total overflowing) are walked in order by one thread.
#pragma once
#include "minp_bound.h"
#include "sampler_kernels.h"

namespace rl {

struct FullRow {
    float M;           // the f32::max fold of the penalised row
    uint32_t done;     // the row is finished (no finite maximum, or the min-p path)
};

// Candidates the min-p path collects per row (a superset of the survivors).
constexpr uint32_t SURV_CAP = 4096;
// A row's per-chunk results are read one chunk per lane.
static_assert(MAX_CHUNKS <= WAVE, "a wave holds one lane per chunk");

struct FullScratch {
    uint32_t *keyA, *idA, *keyB, *idB;  // [slot][vocab] k_full_rest: the sort's passes
    float *probs;                       // [slot][vocab] k_full_rest: p when the candidates are not returned
    float *part_max;                    // [slot][chunk] k_full_pass: the chunk's maximum
    uint64_t *part_am;                  // [slot][chunk] k_full_pass: candidates listed << 32 | lowest +inf id
    double *psum;                       // [slot][chunk] k_full_pass: its mass
    uint64_t *surv;                     // [slot][SURV_CAP] min-p candidates (composites), a region per chunk
    FullRow *row;                       // [slot]
    uint32_t *arrive;                   // [slot] k_full_pass: chunks done; zero between calls
};

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
// Callers split a row's float4 (n <= 2^19, the vocabulary being at most 2^21)
// into at most MAX_CHUNKS, so n * c fits 32 bits.
static_assert((uint64_t)MAX_CHUNKS * (1u << 19) < (1ull << 32), "chunk bounds in 32 bits");
__device__ __forceinline__ uint32_t chunk_lo(uint32_t n, uint32_t c, uint32_t chunks) {
    return n * c / chunks;
}

// The argument (l - max) / t of the reference's p = exp((l - max) / t)
// (sample.rs:309). When t is a power of two with a normal reciprocal, the
// product with that exact reciprocal is the same exact quotient rounded once,
// so it equals the IEEE division bit for bit; the bulk loops then skip the
// division's ten-odd instructions (t = 1 on the zipf and ties rows).
struct TempScale {
    float t, inv;
    bool pow2;
    __device__ __forceinline__ explicit TempScale(float t_) : t(t_) {
        const uint32_t b = __float_as_uint(t_);
        const uint32_t e = (b >> 23) & 0xFFu;
        pow2 = (b & 0x807FFFFFu) == 0 && e >= 2 && e <= 252;  // +2^-125 .. +2^125
        inv = pow2 ? __uint_as_float((254u - e) << 23) : 0.0f;
    }
    __device__ __forceinline__ float operator()(float d) const { return pow2 ? d * inv : d / t; }
};

// Whether a row tries the min-p path: min-p on, the whole vocabulary as
// candidates (top_k 0 or >= vocab), sampling (not greedy).
__device__ __forceinline__ bool small_eligible(const rl_sampling &s, uint32_t V) {
    return s.min_p > 0.0f && full_k(s, V) == V && s.temperature > 0.0f;
}

// LDS bytes of a chunk's window bitmap: one bit per element of the largest
// chunk.
__host__ __device__ inline size_t chunk_bitmap_bytes(uint32_t vocab, uint32_t chunks) {
    const uint32_t n4 = vocab / 4;
    const uint32_t most = 4 * ((n4 + chunks - 1) / chunks) + 3;
    return ((size_t)(most + 31) / 32) * 4;
}

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
// the row to k_full_rest.
//
// The mass interval that certifies the top-p cut, and the constants it rests
// on, are in minp_bound.h (shared with a host-built test of the bound).

using minp::PASS_U;
using minp::PASS_STEP;
static_assert(minp::PASS_THREADS == FULL_THREADS, "the certificate's step shape is k_full_pass's");
constexpr uint32_t FULL_WAVES = FULL_THREADS / WAVE;
constexpr uint32_t FIN_CAP = 1024;                       // survivors the pass finishes itself
constexpr uint32_t PASS_CAND = 1024;                     // candidates a chunk holds in LDS
constexpr uint32_t LIST_OVER = 0xFFFFFFFFu;              // a chunk's candidates did not fit

// Loads of k_full_pass's aligned variant are buffer loads through a resource
// that starts at the step and ends at the chunk's end: float4 f of the step
// is at byte offset 16 f (a lane's register plus nothing else, so no 64-bit
// address stays live across a step), and a load past the chunk returns zeros
// without a memory access. gfx9's descriptor word 3 (0x00020000: 32-bit data
// format, raw addressing); nontemporal (aux 2).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t step_rsrc(const float *row, uint32_t b4, uint32_t end4) {
    return __builtin_amdgcn_make_buffer_rsrc((void *)(row + 4 * (uint64_t)b4), (short)0,
                                             (int)(b4 < end4 ? 16u * (end4 - b4) : 0u), 0x00020000);
}
// Float4 f of the chunk that ends at float4 end, from the step at float4 b4
// (VEC: through r = step_rsrc(row, b4, end)).
template <bool VEC>
__device__ __forceinline__ f32x4 pass_load(__amdgpu_buffer_rsrc_t r, const float *row, uint32_t f, uint32_t b4,
                                           uint32_t end) {
    if constexpr (VEC) {
        return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, 16u * (f - b4), 0, 2));
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
// fall on either side or a q is not finite: k_full_rest takes the row.
__device__ __forceinline__ bool finish_wave(const RowIO &a, uint32_t row, const rl_sampling &s, float M, uint32_t c,
                                            uint64_t x, bool by_id, uint32_t ns_key, double t_lo, double t_hi,
                                            const LdsExpTable &etab) {
    const uint32_t lane = lane_id();
    const bool in = lane < c;
    const float u = a.uniforms[row];
    // Up to 32 survivors: a 32-lane network (lanes 32-63 hold zeros).
    x = c <= 32 ? bitonic_sort<32, true>(in ? x : 0ull) : wave_sort64<true>(in ? x : 0ull);
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
                const double cum = wave_incl_f64(in ? (double)p : 0.0);
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
        // sh[0]: kept (0 when the row is left to k_full_rest), sh[1]: the drawn index.
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
    const size_t bm = chunk_bitmap_bytes(vocab, chunks);
    return bm > fin ? bm : fin;
}

// grid (chunks, slots), FULL_THREADS: the single read of the full path.
// Every row: the penalised row's f32::max fold per chunk (sample.rs:267-269)
// and the lowest id holding +inf; the row's last chunk to finish answers rows
// without a finite maximum (argmax, no draw, sample.rs:270-277) and leaves the
// maximum in the row state for k_full_rest. Rows eligible for the
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
    const uint32_t row = a.rows ? a.rows[slot] : a.row0 + slot;
    const uint32_t V = a.vocab;
    const uint32_t C = a.chunks;
    const float *rowp = a.logits + (uint64_t)row * a.stride;
    const uint32_t n4 = V / 4;
    const uint32_t q0 = chunk_lo(n4, chunk, C), q1 = chunk_lo(n4, chunk + 1, C);
    const uint32_t e0 = 4 * q0, e1 = chunk == C - 1 ? V : 4 * q1;
    const uint32_t nwords = (e1 - e0 + 31) / 32;
    // The row's settings and window length (one vector load, row_words), the
    // window's ids and the exp table load first; then the first step's loads
    // (clamped: no branch around them). Vector loads complete in order, so
    // anything loaded after the step would wait for all of it. The window
    // bitmap and the tables are built while the step is in flight. The id
    // loads are clamped to the call's window stride, so they wait for neither
    // the row's settings nor its window length (which ids count is decided
    // when the bitmap is built).
    const uint32_t head_w = row_words(a, row);
    constexpr uint32_t WIN_PER = 8;  // window ids per thread (max_window <= 2048)
    static_assert(WIN_PER * FULL_THREADS >= 2048, "a window's ids fit the threads");
    // Unconditional (clamped) loads: a load under a divergent branch makes
    // the compiler wait for every load in flight, the step's included.
    uint32_t wid[WIN_PER];
    {
        const bool have_win = a.windows && a.wlen && a.wstride > 0;  // kernel arguments only
        // With no windows the loads read the row's settings (never used).
        const uint32_t *win = have_win ? a.windows + (uint64_t)row * a.wstride
                                       : reinterpret_cast<const uint32_t *>(a.settings + row);
        const uint32_t wn = !have_win ? 1u : a.wstride < WIN_PER * FULL_THREADS ? a.wstride : WIN_PER * FULL_THREADS;
#pragma unroll
        for (uint32_t k = 0; k < WIN_PER; ++k) {
            const uint32_t i = k * FULL_THREADS + tid;
            wid[k] = ((const RL_GLB uint32_t *)win)[i < wn ? i : wn - 1];
        }
    }
    const uint64_t tab = EXP2_32_TAB[tid & 31u];
    f32x4 A[PASS_U];
    // Buffer loads need no guard (past the row they return zeros); a uniform
    // branch here would also make the compiler wait for all loads at its end.
    if (VEC || q0 < q1) {
        const __amdgpu_buffer_rsrc_t rs = step_rsrc(rowp, q0, q1);
#pragma unroll
        for (uint32_t u = 0; u < PASS_U; ++u) A[u] = pass_load<VEC>(rs, rowp, q0 + u * FULL_THREADS + tid, q0, q1);
    }
    // The row's settings and window length, needed from here on (the
    // barrier keeps the wait for them below the step's loads).
    __builtin_amdgcn_sched_barrier(0);
    rl_sampling s;
    uint32_t wl;
    row_head(a, head_w, s, wl);
    const bool pen = penalises(s) && wl > 0;
    // Which of this thread's ids fall in the chunk, worked out outside the
    // branch below so that the compiler keeps their loads ahead of the step's.
    uint32_t in_chunk = 0;
#pragma unroll
    for (uint32_t k = 0; k < WIN_PER; ++k)
        if (k * FULL_THREADS + tid < wl && wid[k] >= e0 && wid[k] < e1) in_chunk |= 1u << k;
    if (pen) {
        for (uint32_t i = tid; i < nwords; i += FULL_THREADS) bm[i] = 0;
        __syncthreads();
#pragma unroll
        for (uint32_t k = 0; k < WIN_PER; ++k) {
            const uint32_t id = wid[k];
            if ((in_chunk >> k) & 1u) atomicOr((uint32_t *)&bm[(id - e0) >> 5], 1u << ((id - e0) & 31));
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
    // buffer sends the row to k_full_rest.
    auto append = [&](uint64_t mb, auto id_of) {
        const uint32_t mine = (uint32_t)__popcll(mb);
        const uint32_t incl = wave_incl_u32(mine);
        const uint32_t wtotal = (uint32_t)__builtin_amdgcn_readlane((int)incl, WAVE - 1);
        uint32_t base = 0;
        if (lane == 0) base = atomicAdd((uint32_t *)&sh_cn, wtotal);
        base = (uint32_t)__builtin_amdgcn_readlane((int)base, 0);
        if (base + wtotal > PASS_CAND) {
            // The buffer is full: the row leaves the min-p path, and nothing
            // more is listed (or re-read) for it.
            if (lane == 0) sh_cover = 1;
            mass = false;
            return;
        }
        uint32_t at = base + incl - mine;
        while (mb != 0) {
            const uint32_t i = (uint32_t)__ffsll((unsigned long long)mb) - 1u;
            mb &= mb - 1ull;
            const uint32_t e = id_of(i);
            cbuf[at++] = composite(total_key(value_at(e)), e);
        }
    };
    // A step's PASS_U float4 per thread are all in flight at once (a chunk
    // of the 64-row workload is one step); the penalty is applied in place.
    for (uint32_t b = q0; b < q1; b += PASS_STEP) {
        if (b != q0) {
            const __amdgpu_buffer_rsrc_t rs = step_rsrc(rowp, b, q1);
#pragma unroll
            for (uint32_t u = 0; u < PASS_U; ++u) A[u] = pass_load<VEC>(rs, rowp, b + u * FULL_THREADS + tid, b, q1);
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
            // row to k_full_rest.
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
        fi = wave_fold_u32(fi, [](uint32_t a, uint32_t b) { return a < b ? a : b; });
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
    const uint32_t incl = wave_incl_u32(nc == LIST_OVER ? 0u : nc);
    const uint32_t nlist = (uint32_t)__builtin_amdgcn_readlane((int)incl, WAVE - 1);
    if (wave == 0 && okc) red_cnt[lane] = nc == LIST_OVER ? 0u : nc;
    const float M = uniform_f32(wave_maxnum_f32(Mr));
    fi = wave_fold_u32(fi, [](uint32_t a, uint32_t b) { return a < b ? a : b; });
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
        ns = wave_fold_u32(ns, [](uint32_t a, uint32_t b) { return a > b ? a : b; });
        if (lane == 0 && ns != 0) atomicMax((uint32_t *)&sh_ns, ns);
    }
    __syncthreads();
    const uint32_t c = sh_count, ns_key = sh_ns;
    ok_row = ok_row && c > 0 && c <= FIN_CAP;
    // t_lo <= top_p * S_ref <= t_hi (minp_bound.h).
    double t_lo, t_hi;
    minp::target_interval(Smid, V, C, s.top_p, &t_lo, &t_hi);
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

}  // namespace rl
