// Exact replay of a sequential floating-point sum of non-negative f32 terms,
// computed in parallel.
//
// The reference accumulates in a fixed order: the probability mass and the
// top-p cumulative sum in f64 (sample.rs:307-324), the normalising total in
// f64 (:342) and the draw's cumulative sum in f32 (:349-356). Each partial sum
// is rounded to the precision P of its type (53 or 24 bits), so a different
// order or a tree reduction gives different bits. This header reproduces the
// sequential bits without a sequential loop.
//
// While the running sum s stays inside one binade [2^E, 2^(E+1)), every value
// it takes is a multiple of u = 2^(E-P+1), and adding a term x rounds to that
// grid: s + x -> s + u * rnd(x / u). rnd rounds to nearest; only an exact tie
// (x / u = q + 1/2) depends on s, through the parity of s / u (ties go to the
// even significand), and a tie always leaves the significand even. So within a
// segment each term is a map  parity -> (increment, new parity),  maps compose
// associatively, and a parallel scan of them gives every partial sum exactly.
// A term whose exact sum leaves the binade (s + x >= 2^(E+1)) is added with
// the hardware's own IEEE addition, which starts a new segment; there are at
// most as many segments as binades the sum passes through.
//
// The core (grid, term maps, composition) is plain C++ usable on the host,
// where a test checks it against sequential loops; the workgroup-wide replay
// is device code.
#pragma once
#include <stdint.h>
#include <string.h>

#if defined(__HIPCC__)
#define RL_HD __host__ __device__
#else
#define RL_HD
#endif

namespace rl {

// Increments are saturated here: far above any segment's capacity (< 2^54).
constexpr uint64_t SEQ_SAT = 1ull << 60;

RL_HD inline uint64_t sat_add(uint64_t a, uint64_t b) {
    const uint64_t c = a + b;  // a, b <= SEQ_SAT, so no wrap-around
    return c > SEQ_SAT ? SEQ_SAT : c;
}

RL_HD inline uint64_t f64_bits(double d) {
    uint64_t b;
    memcpy(&b, &d, 8);
    return b;
}

RL_HD inline double f64_from_bits(uint64_t b) {
    double d;
    memcpy(&d, &b, 8);
    return d;
}

// v * 2^e for |e| <= 1022: one multiplication by a power of two, exact while
// the result stays a normal double (true for every use here).
RL_HD inline double mul_pow2(double v, int e) { return v * f64_from_bits((uint64_t)(1023 + e) << 52); }

// n * 2^e, exact for n < 2^53.
RL_HD inline double scaled(uint64_t n, int e) { return mul_pow2((double)n, e); }

// The segment the running sum s (> 0, a P-bit value) is in: values are
// multiples of 2^uexp, s = n * 2^uexp, and the segment lasts while the
// significand stays below lim.
struct SumSeg {
    int uexp;
    uint64_t n;
    uint64_t lim;
};

template <int P>
RL_HD inline SumSeg seg_of(double s) {
    SumSeg g;
    const int E = (int)((f64_bits(s) >> 52) & 0x7FF) - 1023;  // s is a normal double here
    if (P == 24 && E < -126) {
        // An f32 subnormal sum: the grid is 2^-149 up to the smallest normal.
        g.uexp = -149;
        g.lim = 1ull << 23;
    } else {
        g.uexp = E - (P - 1);
        g.lim = 1ull << P;
    }
    g.n = (uint64_t)mul_pow2(s, -g.uexp);
    return g;
}

// The term map: from parity 0 (1) the term adds i0 (i1) grid steps and leaves
// parity p0 (p1).
struct TermMap {
    uint64_t i0, i1;
    uint32_t p0, p1;
};

RL_HD inline TermMap map_identity() { return TermMap{0, 0, 0, 1}; }

// The map of adding the f32 term with bits xb (finite, >= 0) on the grid
// 2^uexp.
RL_HD inline TermMap map_of(uint32_t xb, int uexp) {
    uint32_t m = xb & 0x7FFFFFu;
    const int ex = (int)((xb >> 23) & 0xFFu);
    int lsb = -149;  // x = m * 2^lsb
    if (ex != 0) {
        m |= 0x800000u;
        lsb = ex - 150;
    }
    if (m == 0) return map_identity();
    const int sh = lsb - uexp;
    if (sh >= 0) {  // a multiple of the grid step: added exactly
        const uint64_t n = sh > 36 ? SEQ_SAT : ((uint64_t)m << sh);
        const uint32_t b = (uint32_t)(n & 1);
        return TermMap{n, n, b, b ^ 1u};
    }
    const int d = -sh;
    if (d >= 25) return map_identity();  // below half a step: no effect
    const uint64_t q = m >> d;
    const uint32_t rem = m & ((1u << d) - 1u), half = 1u << (d - 1);
    if (rem != half) {
        const uint64_t n = q + (rem > half ? 1u : 0u);
        const uint32_t b = (uint32_t)(n & 1);
        return TermMap{n, n, b, b ^ 1u};
    }
    // An exact tie: round to the even significand, which leaves parity 0.
    return TermMap{q + (q & 1), q + ((q + 1) & 1), 0u, 0u};
}

// The grid steps the term adds when it is not an exact tie; *tie is set when
// it is one (its increment then depends on the parity of the sum).
RL_HD inline uint64_t inc_of(uint32_t xb, int uexp, bool *tie) {
    uint32_t m = xb & 0x7FFFFFu;
    const int ex = (int)((xb >> 23) & 0xFFu);
    int lsb = -149;
    if (ex != 0) {
        m |= 0x800000u;
        lsb = ex - 150;
    }
    *tie = false;
    const int sh = lsb - uexp;
    if (sh >= 0) return sh > 36 ? SEQ_SAT : ((uint64_t)m << sh);
    const int d = -sh;
    if (d >= 25) return 0;
    const uint32_t rem = m & ((1u << d) - 1u), half = 1u << (d - 1);
    *tie = m != 0 && rem == half;
    return (uint64_t)(m >> d) + (rem > half ? 1u : 0u);
}

// a, then b.
RL_HD inline TermMap map_then(const TermMap &a, const TermMap &b) {
    TermMap c;
    c.i0 = sat_add(a.i0, a.p0 ? b.i1 : b.i0);
    c.p0 = a.p0 ? b.p1 : b.p0;
    c.i1 = sat_add(a.i1, a.p1 ? b.i1 : b.i0);
    c.p1 = a.p1 ? b.p1 : b.p0;
    return c;
}

RL_HD inline uint64_t map_inc(const TermMap &t, uint32_t parity) { return parity ? t.i1 : t.i0; }
RL_HD inline uint32_t map_parity(const TermMap &t, uint32_t parity) { return parity ? t.p1 : t.p0; }

// One IEEE addition in precision P of a P-bit value and an f32 term.
template <int P>
RL_HD inline double add_p(double s, float x) {
    if (P == 24) return (double)((float)s + x);
    return s + (double)x;
}

#if defined(__HIPCC__)
// ------------------------------------------------------------- device ---
// LDS a workgroup of NT threads needs for seq_replay.
template <uint32_t NT>
struct SeqLds {
    TermMap wave_map[NT / 64];
    uint64_t wave_sum[NT / 64];
    uint32_t wave_tie[NT / 64];
    uint32_t cross, hit, nonzero;
    double s_new;
};

__device__ __forceinline__ uint64_t shfl_u64(uint64_t v, int src) {
    return ((uint64_t)(uint32_t)__shfl((int)(uint32_t)(v >> 32), src) << 32) | (uint32_t)__shfl((int)(uint32_t)v, src);
}
__device__ __forceinline__ uint64_t shfl_up_u64(uint64_t v, int d) {
    return ((uint64_t)(uint32_t)__shfl_up((int)(uint32_t)(v >> 32), d) << 32) |
           (uint32_t)__shfl_up((int)(uint32_t)v, d);
}
__device__ __forceinline__ uint64_t shfl_xor_sat_sum(uint64_t v) {
    for (int m = 32; m >= 1; m >>= 1) {
        const uint64_t o = ((uint64_t)(uint32_t)__shfl_xor((int)(uint32_t)(v >> 32), m) << 32) |
                           (uint32_t)__shfl_xor((int)(uint32_t)v, m);
        v = sat_add(v, o);
    }
    return v;
}

__device__ __forceinline__ TermMap shfl_up_map(const TermMap &v, int d) {
    TermMap o;
    o.i0 = shfl_up_u64(v.i0, d);
    o.i1 = shfl_up_u64(v.i1, d);
    o.p0 = (uint32_t)__shfl_up((int)v.p0, d);
    o.p1 = (uint32_t)__shfl_up((int)v.p1, d);
    return o;
}

// Inclusive scans across the wave: lane i gets lanes 0..i combined in order.
__device__ __forceinline__ TermMap wave_scan_map(TermMap v) {
    const uint32_t lane = __lane_id();
    for (int d = 1; d < 64; d <<= 1) {
        const TermMap o = shfl_up_map(v, d);
        if (lane >= (uint32_t)d) v = map_then(o, v);
    }
    return v;
}
__device__ __forceinline__ uint64_t wave_scan_sum(uint64_t v) {
    const uint32_t lane = __lane_id();
    for (int d = 1; d < 64; d <<= 1) {
        const uint64_t o = shfl_up_u64(v, d);
        if (lane >= (uint32_t)d) v = sat_add(o, v);
    }
    return v;
}

// Replays s = fl_P(s + x_j) for j = 0, 1, ... over the n terms
// x_j = term(fetch(j)) (finite, >= 0), in order, with the whole workgroup (NT
// threads, ITEMS consecutive terms per thread per tile). fetch(j) returns the
// raw 32 bits a term is made from and term turns them into the f32 term, so
// the next tile's fetches stay in flight while the current tile is reduced
// (a term computed at fetch time would wait for its load there). Returns the first j whose partial sum satisfies
// pred (a predicate that stays true once true as the sum grows), or n; when
// it returns n, *sum is the sequential sum of all n terms, and otherwise the
// partial sum at the returned index. Every thread of the workgroup must call
// it with the same arguments; it contains barriers.
//
// Tiles are aligned to NT * ITEMS terms and the next tile is loaded while the
// current one is reduced. When the sum leaves its segment inside a tile, the
// rest of the tile is processed again from registers under the new segment.
// Per pass over a tile: when no remaining term of the tile is an exact rounding
// tie, every term's increment is independent of the sum, so a block reduction
// tells whether the sum leaves its segment or meets pred inside the tile, and
// only then is a block scan needed to find where. A tile holding a tie goes
// through the parity-carrying term maps instead.
template <int P, uint32_t NT, uint32_t ITEMS, class Fetch, class Term, class Pred>
__device__ __forceinline__ uint32_t seq_replay(Fetch fetch, Term term, uint32_t n, Pred pred, SeqLds<NT> *L, double *sum) {
    constexpr uint32_t TILE = NT * ITEMS;
    constexpr uint32_t NW = NT / 64;
    const uint32_t tid = threadIdx.x, lane = __lane_id(), wave = tid / 64;
    double s = 0.0;
    bool zero = true;
    SumSeg g{0, 0, 0};
    uint32_t pos = 0;  // the next term to add
    uint32_t cur = 0xFFFFFFFFu, nxt = 0xFFFFFFFFu;  // bases of the tiles in xb and nb
    uint32_t xb[ITEMS], nb[ITEMS];  // terms of the current tile, raw bits of the next
    if (n > 0 && pred(0.0)) {
        // A predicate that +0 already meets is met by the first term's sum.
        *sum = add_p<P>(0.0, term(fetch(0)));
        return 0;
    }
    while (pos < n) {
        const uint32_t base = pos / TILE * TILE;
        const uint32_t j0 = base + tid * ITEMS;
        if (base != cur) {
            if (base == nxt) {
#pragma unroll
                for (uint32_t i = 0; i < ITEMS; ++i) xb[i] = j0 + i < n ? __float_as_uint(term(nb[i])) : 0u;
            } else {
#pragma unroll
                for (uint32_t i = 0; i < ITEMS; ++i) xb[i] = j0 + i < n ? __float_as_uint(term(fetch(j0 + i))) : 0u;
            }
            cur = base;
            nxt = base + TILE;
#pragma unroll
            for (uint32_t i = 0; i < ITEMS; ++i) {
                const uint32_t j = nxt + tid * ITEMS + i;
                nb[i] = fetch(j < n ? j : n - 1);  // clamped: no branch around the load
            }
        }
        // This tile's terms from pos on (the others count as +0).
        uint32_t xv[ITEMS];
#pragma unroll
        for (uint32_t i = 0; i < ITEMS; ++i) xv[i] = j0 + i >= pos ? xb[i] : 0u;
        if (zero) {
            // The sum stays +0 up to the first nonzero term.
            if (tid == 0) L->nonzero = 0xFFFFFFFFu;
            __syncthreads();
            uint32_t my_nz = 0xFFFFFFFFu, x_nz = 0;
#pragma unroll
            for (uint32_t i = 0; i < ITEMS; ++i) {
                if (my_nz == 0xFFFFFFFFu && (xv[i] & 0x7FFFFFFFu) != 0) {
                    my_nz = j0 + i;
                    x_nz = xv[i];
                }
            }
            if (my_nz != 0xFFFFFFFFu) atomicMin(&L->nonzero, my_nz);
            __syncthreads();
            const uint32_t jz = L->nonzero;
            __syncthreads();
            if (jz == 0xFFFFFFFFu) {
                pos = base + TILE;
                continue;
            }
            if (my_nz == jz) L->s_new = (double)__uint_as_float(x_nz);
            __syncthreads();
            s = L->s_new;
            __syncthreads();
            zero = false;
            if (pred(s)) {
                *sum = s;
                return jz;
            }
            g = seg_of<P>(s);
            pos = jz + 1;
            continue;
        }
        const uint32_t par0 = (uint32_t)(g.n & 1);
        const uint64_t room = g.lim - g.n;
        uint64_t mine = 0;
        bool tie = false;
#pragma unroll
        for (uint32_t i = 0; i < ITEMS; ++i) {
            bool t;
            mine = sat_add(mine, inc_of(xv[i], g.uexp, &t));
            tie |= t;
        }
        const uint64_t wsum = shfl_xor_sat_sum(mine);
        const bool wtie = __ballot(tie) != 0;
        if (lane == 0) {
            L->wave_sum[wave] = wsum;
            L->wave_tie[wave] = wtie ? 1u : 0u;
        }
        if (tid == 0) {
            L->cross = 0xFFFFFFFFu;
            L->hit = 0xFFFFFFFFu;
        }
        __syncthreads();
        uint64_t total = 0;
        uint32_t anytie = 0;
        for (uint32_t w = 0; w < NW; ++w) {
            total = sat_add(total, L->wave_sum[w]);
            anytie |= L->wave_tie[w];
        }
        if (!anytie && total < room && !pred(scaled(g.n + total, g.uexp))) {
            // Nothing happens in the rest of this tile.
            g.n += total;
            s = scaled(g.n, g.uexp);
            pos = base + TILE;
            __syncthreads();
            continue;
        }
        // Something happens here: the exclusive prefix of this thread's terms.
        uint64_t I;
        uint32_t par;
        if (!anytie) {
            const uint64_t incl = wave_scan_sum(mine);
            __syncthreads();
            if (lane == 63) L->wave_sum[wave] = incl;
            __syncthreads();
            uint64_t before = 0;
            for (uint32_t w = 0; w < wave; ++w) before = sat_add(before, L->wave_sum[w]);
            uint64_t prev = shfl_up_u64(incl, 1);
            if (lane == 0) prev = 0;
            I = sat_add(before, prev);
            par = 0;  // unused without ties
        } else {
            TermMap agg = map_identity();
#pragma unroll
            for (uint32_t i = 0; i < ITEMS; ++i) agg = map_then(agg, map_of(xv[i], g.uexp));
            const TermMap incl = wave_scan_map(agg);
            if (lane == 63) L->wave_map[wave] = incl;
            __syncthreads();
            TermMap before = map_identity(), all = map_identity();
            for (uint32_t w = 0; w < NW; ++w) {
                if (w < wave) before = map_then(before, L->wave_map[w]);
                all = map_then(all, L->wave_map[w]);
            }
            total = map_inc(all, par0);  // the increment of the rest of the tile, ties included
            TermMap prev = shfl_up_map(incl, 1);
            if (lane == 0) prev = map_identity();
            const TermMap excl = map_then(before, prev);
            I = map_inc(excl, par0);
            par = map_parity(excl, par0);
        }
        uint32_t my_cross = 0xFFFFFFFFu, my_hit = 0xFFFFFFFFu, x_cross = 0;
        uint64_t I_cross = 0, I_hit = 0;
#pragma unroll
        for (uint32_t i = 0; i < ITEMS; ++i) {
            const uint32_t j = j0 + i;
            if (j >= n || my_cross != 0xFFFFFFFFu || my_hit != 0xFFFFFFFFu) break;
            if (j < pos) continue;
            uint64_t step;
            if (!anytie) {
                bool t;
                step = inc_of(xv[i], g.uexp, &t);
            } else {
                const TermMap e = map_of(xv[i], g.uexp);
                step = map_inc(e, par);
                par = map_parity(e, par);
            }
            const uint64_t In = sat_add(I, step);
            if (In >= room) {  // this term's sum leaves the segment
                my_cross = j;
                I_cross = I;
                x_cross = xv[i];
            } else if (pred(scaled(g.n + In, g.uexp))) {
                my_hit = j;
                I_hit = In;
            } else {
                I = In;
            }
        }
        if (my_cross != 0xFFFFFFFFu) atomicMin(&L->cross, my_cross);
        if (my_hit != 0xFFFFFFFFu) atomicMin(&L->hit, my_hit);
        __syncthreads();
        const uint32_t cross = L->cross, hit = L->hit;
        if (hit < cross) {
            if (my_hit == hit) L->s_new = scaled(g.n + I_hit, g.uexp);
            __syncthreads();
            *sum = L->s_new;
            __syncthreads();
            return hit;
        }
        if (cross != 0xFFFFFFFFu) {
            if (my_cross == cross) L->s_new = add_p<P>(scaled(g.n + I_cross, g.uexp), __uint_as_float(x_cross));
            __syncthreads();
            s = L->s_new;
            __syncthreads();
            if (pred(s)) {
                *sum = s;
                return cross;
            }
            g = seg_of<P>(s);
            pos = cross + 1;  // the rest of this tile is redone from registers
            continue;
        }
        // Only a tie tile can get here without an event.
        g.n += total;
        s = scaled(g.n, g.uexp);
        pos = base + TILE;
        __syncthreads();
    }
    *sum = s;
    return n;
}
// The same over terms that need no transformation: load(j) is the f32 term.
template <int P, uint32_t NT, uint32_t ITEMS, class Load, class Pred>
__device__ __forceinline__ uint32_t seq_replay(Load load, uint32_t n, Pred pred, SeqLds<NT> *L, double *sum) {
    return seq_replay<P, NT, ITEMS>([load](uint32_t j) { return __float_as_uint(load(j)); },
                                    [](uint32_t bits) { return __uint_as_float(bits); }, n, pred, L, sum);
}
#endif  // __HIPCC__

}  // namespace rl
