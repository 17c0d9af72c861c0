// Device-side helpers shared by the sampler kernels: the reference's orders as
// integer keys, wave primitives for wave64, and the recent-token window set.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "rl_sampler.h"

namespace rl {

constexpr uint32_t WAVE = 64;
constexpr uint32_t EMPTY_ID = 0xFFFFFFFFu;

// Address-space-qualified pointers: LDS accesses compile to ds_* and HBM
// accesses to global_* instructions. Generic (flat) accesses would be counted
// against both the LDS and the memory wait counters, so an LDS access in the
// streaming loop would wait for every load in flight.
#define RL_LDS __attribute__((address_space(3)))
#define RL_GLB __attribute__((address_space(1)))

// ---------------------------------------------------------------- orders --
// f32::total_cmp (used by the selection and sort, sample.rs:282-286) as an
// unsigned key: a larger key is later in the total order. -NaN < -inf < ... <
// -0 < +0 < ... < +inf < +NaN.
__device__ __forceinline__ uint32_t total_key(float v) {
    const uint32_t b = __float_as_uint(v);
    return b ^ ((uint32_t)((int32_t)b >> 31) | 0x80000000u);
}

__device__ __forceinline__ float key_value(uint32_t k) {
    const uint32_t b = (k & 0x80000000u) ? (k ^ 0x80000000u) : ~k;
    return __uint_as_float(b);
}

// Descending logit then ascending id, as one u64 that is larger for the
// candidate that comes first. Composite 0 is never a real candidate (it would
// need id 0xFFFFFFFF), so it pads buffers.
__device__ __forceinline__ uint64_t composite(uint32_t key, uint32_t id) {
    return ((uint64_t)key << 32) | (uint32_t)~id;
}
__device__ __forceinline__ uint32_t comp_key(uint64_t c) { return (uint32_t)(c >> 32); }
__device__ __forceinline__ uint32_t comp_id(uint64_t c) { return ~(uint32_t)c; }

// argmax's order (sample.rs:118-128): IEEE '>' from a start of -inf, so NaN
// and -inf never win and -0 ties +0. As a key: 0 for NaN and -inf (they lose
// to everything, and a row of only those returns id 0), else the total-order
// key of v + 0.0 (which maps -0 to +0).
__device__ __forceinline__ uint32_t argmax_key(float v) {
    return (v > -__builtin_inff()) ? total_key(v + 0.0f) : 0u;
}

// sample.rs:249-253: a positive logit is divided by the penalty, anything
// else (including -0 and NaN) multiplied.
__device__ __forceinline__ float penalize(float v, float p) { return v > 0.0f ? v / p : v * p; }

__device__ __forceinline__ bool penalises(const rl_sampling &s) {
    return s.repeat_penalty != 1.0f && s.repeat_last_n > 0;  // sample.rs:82-84
}

// ---------------------------------------------------------- wave helpers --
__device__ __forceinline__ uint32_t lane_id() { return __lane_id(); }

__device__ __forceinline__ uint64_t ballot(bool p) { return __ballot(p); }

__device__ __forceinline__ uint32_t lanes_below(uint64_t mask) {
    return __builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32),
                                     __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
}

__device__ __forceinline__ uint32_t uniform_u32(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_readfirstlane((int)v);
}
__device__ __forceinline__ uint64_t uniform_u64(uint64_t v) {
    const uint32_t lo = uniform_u32((uint32_t)v);
    const uint32_t hi = uniform_u32((uint32_t)(v >> 32));
    return ((uint64_t)hi << 32) | lo;
}
__device__ __forceinline__ float uniform_f32(float v) { return __uint_as_float(uniform_u32(__float_as_uint(v))); }
__device__ __forceinline__ double uniform_f64(double v) {
    return __longlong_as_double((long long)uniform_u64((uint64_t)__double_as_longlong(v)));
}

__device__ __forceinline__ uint32_t read_lane_u32(uint32_t v, uint32_t lane) {
    return (uint32_t)__builtin_amdgcn_readlane((int)v, (int)lane);
}
__device__ __forceinline__ float read_lane_f32(float v, uint32_t lane) {
    return __uint_as_float(read_lane_u32(__float_as_uint(v), lane));
}

// Lane exchange: lane i receives v from lane i ^ S, using DPP row operations
// for S <= 8 and the gfx950 permlane swaps for 16 and 32 (VALU ops, no LDS
// round trip). Lane layouts as measured on gfx950: quad_perm [1,0,3,2] and
// [2,3,0,1] are xor 1 and xor 2; row_shl:4 / row_shr:4 read lane i+4 / i-4
// within a row of 16; row_ror:8 reads lane i^8; permlane16_swap(v, v) returns
// {rows 0,0,2,2; rows 1,1,3,3} and permlane32_swap(v, v) {low, low; high,
// high} halves.
template <uint32_t S>
__device__ __forceinline__ uint32_t lane_xor(uint32_t v) {
    if constexpr (S == 1) {
        return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, false);
    } else if constexpr (S == 2) {
        return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xF, 0xF, false);
    } else if constexpr (S == 4) {
        const uint32_t up = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x104, 0xF, 0xF, false);
        const uint32_t dn = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x114, 0xF, 0xF, false);
        return (lane_id() & 4) ? dn : up;
    } else if constexpr (S == 8) {
        return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x128, 0xF, 0xF, false);
    } else if constexpr (S == 16) {
        const auto p = __builtin_amdgcn_permlane16_swap(v, v, false, false);
        return (lane_id() & 16) ? p[0] : p[1];
    } else {
        static_assert(S == 32, "lane_xor stride");
        const auto p = __builtin_amdgcn_permlane32_swap(v, v, false, false);
        return (lane_id() & 32) ? p[0] : p[1];
    }
}

template <uint32_t S>
__device__ __forceinline__ uint64_t lane_xor64(uint64_t v) {
    return ((uint64_t)lane_xor<S>((uint32_t)(v >> 32)) << 32) | lane_xor<S>((uint32_t)v);
}

// v combined by op with the values of the lanes i ^ 32, i ^ 16, ..., i ^ 1 in
// turn (every lane gets the result; the same order as a shuffle butterfly
// from 32 down).
template <class Op>
__device__ __forceinline__ uint32_t wave_fold_u32(uint32_t v, Op op) {
    v = op(v, lane_xor<32>(v));
    v = op(v, lane_xor<16>(v));
    v = op(v, lane_xor<8>(v));
    v = op(v, lane_xor<4>(v));
    v = op(v, lane_xor<2>(v));
    v = op(v, lane_xor<1>(v));
    return v;
}
template <class Op>
__device__ __forceinline__ uint64_t wave_fold_u64(uint64_t v, Op op) {
    v = op(v, lane_xor64<32>(v));
    v = op(v, lane_xor64<16>(v));
    v = op(v, lane_xor64<8>(v));
    v = op(v, lane_xor64<4>(v));
    v = op(v, lane_xor64<2>(v));
    v = op(v, lane_xor64<1>(v));
    return v;
}

// The wave's maximum of v in every lane (butterfly over the lane exchanges;
// fmaxf ignores a NaN operand, as f32::max does).
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
    uint64_t o;
    o = lane_xor64<32>(v), v = o > v ? o : v;
    o = lane_xor64<16>(v), v = o > v ? o : v;
    o = lane_xor64<8>(v), v = o > v ? o : v;
    o = lane_xor64<4>(v), v = o > v ? o : v;
    o = lane_xor64<2>(v), v = o > v ? o : v;
    o = lane_xor64<1>(v), v = o > v ? o : v;
    return v;
}
__device__ __forceinline__ float wave_maxnum_f32(float v) {
    v = fmaxf(v, __uint_as_float(lane_xor<32>(__float_as_uint(v))));
    v = fmaxf(v, __uint_as_float(lane_xor<16>(__float_as_uint(v))));
    v = fmaxf(v, __uint_as_float(lane_xor<8>(__float_as_uint(v))));
    v = fmaxf(v, __uint_as_float(lane_xor<4>(__float_as_uint(v))));
    v = fmaxf(v, __uint_as_float(lane_xor<2>(__float_as_uint(v))));
    v = fmaxf(v, __uint_as_float(lane_xor<1>(__float_as_uint(v))));
    return v;
}

// The wave's total of v in every lane (butterfly over the lane exchanges).
__device__ __forceinline__ uint32_t wave_sum_u32(uint32_t v) {
    v += lane_xor<1>(v);
    v += lane_xor<2>(v);
    v += lane_xor<4>(v);
    v += lane_xor<8>(v);
    v += lane_xor<16>(v);
    v += lane_xor<32>(v);
    return v;
}

// Inclusive scan of v over the wave with DPP (VALU operations, no LDS round
// trip): within each row of 16 lanes the values 1, 2, 4 and 8 lanes back
// (row_shr), then rows 1 and 3 add the last lane of rows 0 and 2
// (row_bcast:15) and rows 2 and 3 add lane 31 (row_bcast:31); a lane a shift
// reads from outside its row, or a row the mask leaves out, adds 0.
__device__ __forceinline__ uint32_t wave_incl_u32(uint32_t v) {
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x111, 0xF, 0xF, false);  // row_shr:1
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x112, 0xF, 0xF, false);  // row_shr:2
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x114, 0xF, 0xF, false);  // row_shr:4
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x118, 0xF, 0xF, false);  // row_shr:8
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x142, 0xA, 0xF, false);  // row_bcast:15
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x143, 0xC, 0xF, false);  // row_bcast:31
    return v;
}

// One compare-exchange stage of a bitonic network across the wave: lanes i
// and i^STRIDE, blocks of SIZE lanes alternately descending and ascending
// (the final SIZE = 64 block runs in the direction DESC).
template <uint32_t SIZE, uint32_t STRIDE, bool DESC>
__device__ __forceinline__ uint64_t bitonic_stage(uint64_t v) {
    const uint32_t lane = lane_id();
    const uint64_t o = lane_xor64<STRIDE>(v);
    const bool lower = (lane & STRIDE) == 0;
    const bool block_desc = ((lane & SIZE) == 0) == DESC;
    const bool keep_max = lower == block_desc;
    const bool o_big = o > v;
    return (keep_max == o_big) ? o : v;
}

// The same network on 32-bit values, whose compare-exchange is one max and
// one min: sorts one u32 per lane descending across the wave.
template <uint32_t SIZE, uint32_t STRIDE>
__device__ __forceinline__ uint32_t bitonic_merge_u32(uint32_t v) {
    const uint32_t lane = lane_id();
    const uint32_t o = lane_xor<STRIDE>(v);
    const bool lower = (lane & STRIDE) == 0;
    const bool block_desc = (lane & SIZE) == 0 || SIZE == WAVE;
    const uint32_t hi = v > o ? v : o, lo = v > o ? o : v;
    v = lower == block_desc ? hi : lo;
    if constexpr (STRIDE > 1) v = bitonic_merge_u32<SIZE, STRIDE / 2>(v);
    return v;
}
template <uint32_t SIZE>
__device__ __forceinline__ uint32_t bitonic_sort_u32(uint32_t v) {
    if constexpr (SIZE > 2) v = bitonic_sort_u32<SIZE / 2>(v);
    return bitonic_merge_u32<SIZE, SIZE / 2>(v);
}
__device__ __forceinline__ uint32_t wave_sort_u32_desc(uint32_t v) { return bitonic_sort_u32<WAVE>(v); }

template <uint32_t SIZE, uint32_t STRIDE, bool DESC>
__device__ __forceinline__ uint64_t bitonic_merge(uint64_t v) {
    v = bitonic_stage<SIZE, STRIDE, DESC>(v);
    if constexpr (STRIDE > 1) v = bitonic_merge<SIZE, STRIDE / 2, DESC>(v);
    return v;
}

template <uint32_t SIZE, bool DESC>
__device__ __forceinline__ uint64_t bitonic_sort(uint64_t v) {
    if constexpr (SIZE > 2) v = bitonic_sort<SIZE / 2, DESC>(v);
    return bitonic_merge<SIZE, SIZE / 2, DESC>(v);
}

// Sorts one u64 per lane across the wave: lane i ends with the i-th largest
// (DESC) or the i-th smallest.
template <bool DESC>
__device__ __forceinline__ uint64_t wave_sort64(uint64_t v) {
    return bitonic_sort<WAVE, DESC>(v);
}

// The 64 largest of a (descending across lanes) and b (ascending),
// descending: max(a_i, b_i) is a bitonic sequence holding the top 64, which a
// half-cleaner cascade sorts.
__device__ __forceinline__ uint64_t wave_merge64(uint64_t a_desc, uint64_t b_asc) {
    return bitonic_merge<WAVE, WAVE / 2, true>(a_desc > b_asc ? a_desc : b_asc);
}

// Orders this wave's LDS accesses: everything written before is visible to
// every lane of the wave after.
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// ------------------------------------------------------ the window set ---
// The recent-token window as an open-addressed set in LDS, built once per
// workgroup: slot ids (EMPTY_ID when free) and the raw logit of each id, so the
// penalised value can be formed without writing the logits. Inserting an id
// twice keeps one slot, which is the reference's once-per-distinct-id rule
// (sample.rs:242-247); ids >= vocab are skipped (sample.rs:248).
//
// `top` holds the largest raw composite of any id in the set, under both the
// total-order key and argmax's key: a candidate whose composite is above it
// cannot be a window id, so the lookup is skipped for it. Once a stream's
// threshold has passed the window's raw values, no lookup happens at all.
struct WindowSet {
    RL_LDS uint32_t *ids;
    RL_LDS float *vals;
    RL_LDS uint64_t *top;
    uint32_t bits;  // log2(slots)
    uint32_t slots;
};

// LDS bytes of a set with 2^bits slots: ids, raw values, then `top`.
__host__ __device__ constexpr size_t window_lds_bytes(uint32_t hash_bits) {
    return ((size_t)1 << hash_bits) * (sizeof(uint32_t) + sizeof(float)) + sizeof(uint64_t);
}

__device__ __forceinline__ WindowSet window_set(void *lds_base, uint32_t bits) {
    WindowSet w;
    w.bits = bits;
    w.slots = 1u << bits;
    w.ids = (RL_LDS uint32_t *)lds_base;
    w.vals = (RL_LDS float *)(w.ids + w.slots);
    w.top = (RL_LDS uint64_t *)(w.vals + w.slots);  // slots >= 64, so 8-byte aligned
    return w;
}

// The largest raw composite of the set's ids (0 for an empty set); valid after
// window_build.
__device__ __forceinline__ uint64_t window_top(const WindowSet &w) { return uniform_u64(*w.top); }

__device__ __forceinline__ uint32_t window_hash(uint32_t id, uint32_t bits) {
    return (id * 0x9E3779B1u) >> (32u - bits);
}

__device__ __forceinline__ bool window_contains(const WindowSet &w, uint32_t id) {
    uint32_t s = window_hash(id, w.bits);
    for (;;) {
        const uint32_t v = w.ids[s];
        if (v == id) return true;
        if (v == EMPTY_ID) return false;
        s = (s + 1) & (w.slots - 1);
    }
}

// Empties the set (no barrier).
__device__ __forceinline__ void window_clear(const WindowSet &w) {
    for (uint32_t i = threadIdx.x; i < w.slots; i += blockDim.x) w.ids[i] = EMPTY_ID;
    if (threadIdx.x == 0) *w.top = 0;
}

// Inserts id (< vocab); returns the slot when this call inserted it, EMPTY_ID
// when the id was already there.
__device__ __forceinline__ uint32_t window_insert(const WindowSet &w, uint32_t id) {
    uint32_t s = window_hash(id, w.bits);
    for (;;) {
        const uint32_t old = atomicCAS((uint32_t *)&w.ids[s], EMPTY_ID, id);
        if (old == EMPTY_ID) return s;
        if (old == id) return EMPTY_ID;
        s = (s + 1) & (w.slots - 1);
    }
}

// Records the raw logit x of the id inserted at `slot`.
__device__ __forceinline__ void window_store(const WindowSet &w, uint32_t slot, uint32_t id, float x) {
    w.vals[slot] = x;
    const uint32_t k0 = total_key(x), k1 = total_key(x + 0.0f);
    __hip_atomic_fetch_max(w.top, composite(k0 > k1 ? k0 : k1, id), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// Whole-workgroup: clears the set, inserts window[0..len), and gathers each
// distinct id's raw logit from `row`. Ends with a barrier.
__device__ __forceinline__ void window_build(const WindowSet &w, const uint32_t *window, uint32_t len,
                                             uint32_t vocab, const float *row, bool active) {
    window_clear(w);
    __syncthreads();
    if (active) {
        for (uint32_t i = threadIdx.x; i < len; i += blockDim.x) {
            const uint32_t id = window[i];
            if (id >= vocab) continue;
            const uint32_t slot = window_insert(w, id);
            if (slot != EMPTY_ID) window_store(w, slot, id, ((const RL_GLB float *)row)[id]);
        }
    }
    __syncthreads();
}

}  // namespace rl
