// Exact replay of a sequential floating-point sum of non-negative f32 terms,
// computed in parallel.
//
// The reference accumulates in a fixed order: the probability mass and the
// top-p cumulative sum in f64 (sample.rs:307-324), the normalising total in
// f64 (:342) and the draw's cumulative sum in f32 (:349-356); top_probability
// sums in f64 (forward.rs:1678). Each partial sum is rounded to the precision
// P of its type (53 or 24 bits), so a different order or a tree reduction
// gives different bits. This header reproduces the sequential bits without a
// sequential loop.
//
// While the running sum s stays inside one binade [2^E, 2^(E+1)), every value
// it takes is a multiple of u = 2^(E-P+1), and adding a term x rounds to that
// grid: s + x -> s + u * rnd(x / u). rnd rounds to nearest; only an exact tie
// (x / u = q + 1/2) depends on s, through the parity of s / u (ties go to the
// even significand), and a tie always leaves the significand even. So within a
// segment each term is a map  parity -> (increment, new parity),  and maps
// compose associatively. A term whose exact sum leaves the binade
// (s + x >= 2^(E+1)) is added with the hardware's own IEEE addition, which
// starts a new segment.
//
// Because a tie fixes the parity, a run of terms needs no general map: it adds
// `base` steps plus, at its first tie, one step that depends on the parity
// entering the run, and leaves a parity that is fixed once the run holds a
// tie (StepRun). Across the 64 lanes of a wave, the parity entering each lane
// follows from two ballots: the lanes holding a tie and the lanes leaving an
// odd parity (parity_in).
//
// A stretch of terms in which no addition can round needs no segments at all:
// when s and every term are multiples of the grid of a binade that lies above
// the stretch's end sum, every partial sum is exactly representable, the
// sequential sum is the exact sum, and any summation order (an f64 tree)
// computes it exactly, however many binades the sum crosses on the way.
//
// The core (grid, term maps, runs, parities) is plain C++ usable on the host,
// where a test checks it against sequential loops; the workgroup-wide replay
// is device code.
#pragma once
#include <stdint.h>
#include <string.h>

#if defined(__HIPCC__)
#include <type_traits>

#include "rl_device.h"
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

// The same segment with the step count and its limit held as f64 values:
// integers below 2^54, exact, so that sums of step counts below the room stay
// exact with no 64-bit integer conversions (which the device does in software).
struct SumSegF {
    int uexp;
    double n;
    double lim;
};

template <int P>
RL_HD inline SumSegF segf_of(double s) {
    SumSegF g;
    const int E = (int)((f64_bits(s) >> 52) & 0x7FF) - 1023;  // s is a normal double here
    if (P == 24 && E < -126) {
        g.uexp = -149;
        g.lim = 0x1p23;
    } else {
        g.uexp = E - (P - 1);
        g.lim = P == 24 ? 0x1p24 : 0x1p53;
    }
    g.n = mul_pow2(s, -g.uexp);
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

RL_HD inline uint32_t popc64(uint64_t v) { return (uint32_t)__builtin_popcountll(v); }

// Grid steps are counted in f64: every count below 2^53 is exact, and a term
// is turned into its steps with exact operations (a scaling by a power of
// two, floor, a subtraction). A term's steps are capped at STEP_CAP (above any
// segment's room, at most 2^53), and so is a run's total; a sum that reaches
// 2^53 is no longer exact, but it stays at or above the room, so it still
// reads as leaving the segment, and only sums below the room are used as
// exact values.
constexpr double STEP_CAP = 0x1p54;

RL_HD inline float f32_from_bits(uint32_t b) {
    float f;
    memcpy(&f, &b, 4);
    return f;
}

// The parity (0 or 1) of an integer-valued v below 2^53.
RL_HD inline uint32_t parity_of(double v) { return v - 2.0 * __builtin_floor(v * 0.5) != 0.0 ? 1u : 0u; }

// The steps of the f32 term x (finite, >= 0) on the grid whose step is
// 1 / scale (scale a power of two): x * scale rounded to nearest, an exact tie
// (*tie set) rounded down.
RL_HD inline double step_of(float x, double scale, bool *tie) {
    const double y = (double)x * scale;
    const double fl = __builtin_floor(y);
    const double fr = y - fl;
    *tie = fr == 0.5;
    const double q = fr > 0.5 ? fl + 1.0 : fl;
    return q < STEP_CAP ? q : STEP_CAP;
}

// A run of consecutive terms on the grid of one segment, as a function of the
// parity p entering it: it adds base + (tie ? (p ^ c) & 1 : 0) steps. A tie
// leaves the significand even, so after the run's first tie the parity is
// known: it is that of base - mark, mark being base just after the last tie.
struct StepRun {
    double base, mark;
    uint32_t tie, c;
};

RL_HD inline StepRun run_identity() { return StepRun{0.0, 0.0, 0, 0}; }

// Appends the f32 term with bits xb on the grid with step 1 / scale.
RL_HD inline void run_add(StepRun &r, uint32_t xb, double scale) {
    bool t;
    const double q = step_of(f32_from_bits(xb), scale, &t);
    if (!t) {
        r.base += q;
    } else if (!r.tie) {
        // The parity before this tie is p ^ parity(base); the tie rounds up
        // iff that plus q is odd.
        r.tie = 1;
        r.c = parity_of(r.base) ^ parity_of(q);
        r.base += q;
        r.mark = r.base;
    } else {
        r.base += q + (double)(parity_of(r.base - r.mark) ^ parity_of(q));
        r.mark = r.base;
    }
}

// The run's par: the parity it leaves, relative to the entering one without a
// tie (p ^ par) and absolute with one.
RL_HD inline uint32_t run_par(const StepRun &r) { return r.tie ? parity_of(r.base - r.mark) : parity_of(r.base); }

// Runs 0, 1, ... in order: T has bit i set when run i holds a tie, O when run
// i's run_par is 1. The parity entering run i (0 <= i <= 64; 64 means after the
// last run) is p0 ^ k when *dep is set (p0 enters run 0), and k otherwise.
RL_HD inline uint32_t parity_in(uint64_t T, uint64_t O, uint32_t i, uint32_t *dep) {
    const uint64_t below = i ? (~0ull >> (64 - i)) : 0ull;
    const uint64_t tb = T & below;
    if (tb == 0) {
        *dep = 1;
        return popc64(O & below) & 1u;
    }
    *dep = 0;
    const uint32_t t = 63u - (uint32_t)__builtin_clzll(tb);  // the last run with a tie before i
    const uint64_t after = below & ~((2ull << t) - 1ull);     // runs t+1 .. i-1, none with a tie
    return (uint32_t)((O >> t) & 1u) ^ (popc64(O & after) & 1u);
}

// The exponent of the lowest set bit of a nonzero finite f32 term's value.
RL_HD inline int low_bit_exp(uint32_t xb) {
    uint32_t m = xb & 0x7FFFFFu;
    const int ex = (int)((xb >> 23) & 0xFFu);
    if (ex != 0) return ex - 150 + __builtin_ctz(m | 0x800000u);
    return -149 + __builtin_ctz(m);
}

// The grid exponent of precision-P values in the binade of `up` (> 0, normal):
// the finest grid on which every P-bit value below 2^(E+1) lies, E = the
// binade of up.
template <int P>
RL_HD inline int grid_exp_of(double up) {
    const int E = (int)((f64_bits(up) >> 52) & 0x7FF) - 1023;
    const int gx = E - (P - 1);
    return (P == 24 && gx < -149) ? -149 : gx;
}

// Whether the segment's sum g.n * 2^g.uexp (n > 0) is a multiple of 2^gx.
RL_HD inline bool seg_multiple(const SumSeg &g, int gx) {
    return g.uexp >= gx || (int)__builtin_ctzll(g.n) >= gx - g.uexp;
}

// Adds `count` equal terms x (bits xb: finite, >= 0) in order to the running
// sum s (a P-bit value >= 0, pred(s) false), one segment of the sum at a time.
// On the grid of s's segment the first term adds map_inc(t, parity) steps and
// every later one t.i0: a term that is not an exact tie adds the same steps
// from either parity, and a tie leaves the significand even. So the partial
// sums inside the segment are n + first + (j - 1) * rest for the j-th term, up
// to the term whose sum would reach the segment's end, which is added with the
// IEEE addition and starts the next segment. pred must be monotone in the
// partial sum. Returns the index of the first term whose partial sum meets
// pred, with that sum in s, or count, with the sum of all of them in s. The
// cost is a step per segment the sum crosses (and a bisection where pred is
// met), whatever count is.
template <int P, class Pred>
RL_HD inline uint32_t equal_run_walk(double &s, uint32_t xb, uint32_t count, Pred pred) {
    if (xb == 0u) return count;  // +0 adds nothing
    const float x = f32_from_bits(xb);
    uint32_t done = 0;
    while (done < count) {
        if (!(s > 0.0)) {  // from +0 the first term is the sum
            s = add_p<P>(s, x);
            if (pred(s)) return done;
            ++done;
            continue;
        }
        const SumSeg g = seg_of<P>(s);
        const TermMap t = map_of(xb, g.uexp);
        const uint64_t first = map_inc(t, (uint32_t)(g.n & 1u)), rest = t.i0;
        const uint64_t left = count - done;
        // K: the terms whose sums stay below the segment's end (at most left).
        uint64_t K;
        if (g.n + first >= g.lim) {
            K = 0;
        } else if (rest == 0) {
            K = left;
        } else {
            const uint64_t a = g.lim - g.n - first;  // the first j with sum >= lim is 1 + ceil(a / rest)
            const uint64_t jl = 1 + (a + rest - 1) / rest;
            K = jl - 1 < left ? jl - 1 : left;
        }
        if (K > 0) {
            auto sum_at = [&](uint64_t j) { return scaled(g.n + first + (j - 1) * rest, g.uexp); };
            if (pred(sum_at(K))) {
                uint64_t lo = 1, hi = K;  // the first j in [1, K] meeting pred
                while (lo < hi) {
                    const uint64_t mid = lo + (hi - lo) / 2;
                    if (pred(sum_at(mid)))
                        hi = mid;
                    else
                        lo = mid + 1;
                }
                s = sum_at(lo);
                return done + (uint32_t)(lo - 1);
            }
            s = sum_at(K);
            done += (uint32_t)K;
            if (done == count) return count;
        }
        s = add_p<P>(s, x);  // this term's sum leaves the segment
        if (pred(s)) return done;
        ++done;
    }
    return count;
}

#if defined(__HIPCC__)
// ------------------------------------------------------------- device ---
// LDS a workgroup of NT threads needs for seq_replay. The per-wave records
// alternate between two sets from one pass to the next, so that a pass needs
// one barrier: a wave writes a set only after every wave has passed the
// barrier behind which the set was last read.
template <uint32_t NT>
struct SeqLds {
    double wave_base[2][NT / 64];    // steps, every tie resolved but the wave's first (capped)
    double wave_fsum[2][NT / 64];    // f64 sum of the wave's terms
    uint32_t wave_bits[2][NT / 64];  // bit 0: a tie; bit 1: the first tie's constant; bit 2: par
    int32_t wave_low[2][NT / 64];    // lowest bit exponent of the wave's nonzero terms
    uint32_t cross, hit, nonzero;
    double s_new;
};

// Butterfly totals across the wave with DPP and permlane exchanges (VALU
// operations, no LDS round trip); every lane gets the same total (the f64
// additions are commutative, so both lanes of a pair compute the same sum).
template <uint32_t S>
__device__ __forceinline__ double lane_xor_f64(double v) {
    return f64_from_bits(lane_xor64<S>(f64_bits(v)));
}
__device__ __forceinline__ double wave_total_f64(double v) {
    v += lane_xor_f64<1>(v);
    v += lane_xor_f64<2>(v);
    v += lane_xor_f64<4>(v);
    v += lane_xor_f64<8>(v);
    v += lane_xor_f64<16>(v);
    v += lane_xor_f64<32>(v);
    return v;
}
__device__ __forceinline__ int wave_min_i32(int v) {
    v = min(v, (int)lane_xor<1>((uint32_t)v));
    v = min(v, (int)lane_xor<2>((uint32_t)v));
    v = min(v, (int)lane_xor<4>((uint32_t)v));
    v = min(v, (int)lane_xor<8>((uint32_t)v));
    v = min(v, (int)lane_xor<16>((uint32_t)v));
    v = min(v, (int)lane_xor<32>((uint32_t)v));
    return v;
}

// Scans across the wave with DPP (VALU operations, no LDS round trip). The
// inclusive scan adds within each row of 16 lanes the values 1, 2, 4 and 8
// lanes back (row_shr), then rows 1 and 3 add the last lane of rows 0 and 2
// (row_bcast:15) and rows 2 and 3 add lane 31 (row_bcast:31); a lane a shift
// reads from outside its row, or a row the mask leaves out, adds +0. The
// exclusive scan shifts the wave by one lane first (wave_shr:1; lane 0 gets
// +0), so the sum for lane i never includes lane i's own value, which may be
// far larger (a capped step count): the sums of the lanes before an event
// stay exact. Both add integers (or values whose every partial sum is
// exact), so the order of the additions does not change the result.
template <int CTRL, int ROWS>
__device__ __forceinline__ double dpp_f64(double v) {
    const uint64_t b = f64_bits(v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)b, CTRL, ROWS, 0xF, false);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(b >> 32), CTRL, ROWS, 0xF, false);
    return f64_from_bits(((uint64_t)hi << 32) | lo);
}
__device__ __forceinline__ double wave_incl_f64(double v) {
    v += dpp_f64<0x111, 0xF>(v);  // row_shr:1
    v += dpp_f64<0x112, 0xF>(v);  // row_shr:2
    v += dpp_f64<0x114, 0xF>(v);  // row_shr:4
    v += dpp_f64<0x118, 0xF>(v);  // row_shr:8
    v += dpp_f64<0x142, 0xA>(v);  // row_bcast:15 into rows 1 and 3
    v += dpp_f64<0x143, 0xC>(v);  // row_bcast:31 into rows 2 and 3
    return v;
}
__device__ __forceinline__ double wave_excl_f64(double v) { return wave_incl_f64(dpp_f64<0x138, 0xF>(v)); }

// The workgroup's barrier, or (WAVE_ONLY) the wave's own LDS sync.
template <bool WAVE_ONLY>
__device__ __forceinline__ void replay_sync() {
    if constexpr (WAVE_ONLY) {
        wave_lds_sync();
    } else {
        __syncthreads();
    }
}

// Replays s = fl_P(s + x_j) for j = 0, 1, ... from s = s0 (a P-bit value >= 0;
// seq_replay starts from +0) over the n terms
// x_j = term(fetch(j)) (finite, >= 0), in order, with the whole workgroup (NT
// threads, ITEMS consecutive terms per thread per tile). fetch(j) returns the
// raw 32 bits a term is made from and term turns them into the f32 term, so
// the next tile's fetches stay in flight while the current tile is reduced
// (a term computed at fetch time would wait for its load there). Returns the
// first j whose partial sum satisfies pred (a predicate that stays true once
// true as the sum grows), or n; when it returns n, *sum is the sequential sum
// of all n terms, and otherwise the partial sum at the returned index. Every
// thread of the workgroup must call it with the same arguments; it contains
// barriers. With WAVE_ONLY (NT = 64) one wave runs it by itself: its syncs are
// the wave's own, and the other waves of the workgroup take no part.
//
// Tiles are aligned to NT * ITEMS terms and the next tile is loaded while the
// current one is reduced. A pass over (the rest of) a tile reduces, per wave,
// the terms' f64 sum, their lowest bit and their steps on the current
// segment's grid with the ties resolved (StepRun, parity_in), and the waves'
// records are combined in order behind one barrier. If no addition in the
// tile can round, the sum moves to the exact end sum, across binades; else if
// the steps stay in the segment and pred stays false, the sum moves by them.
// Otherwise a scan locates the event: the first term whose sum meets pred, or
// leaves the segment (added with the IEEE addition; the rest of the tile is
// then processed again from registers under the new segment).
template <int P, uint32_t NT, uint32_t ITEMS, bool WAVE_ONLY, class Fetch, class Term, class Pred>
__device__ __forceinline__ uint32_t seq_replay_from(Fetch fetch, Term term, uint32_t n, Pred pred, double s0,
                                                    SeqLds<NT> *L, double *sum) {
    static_assert(!WAVE_ONLY || NT == 64, "a wave-only replay is one wave");
    constexpr uint32_t TILE = NT * ITEMS;
    constexpr uint32_t NW = NT / 64;
    const uint32_t tid = WAVE_ONLY ? __lane_id() : threadIdx.x, lane = __lane_id(), wave = tid / 64;
    double s = s0;
    bool zero = !(s0 > 0.0);
    SumSeg g = zero ? SumSeg{0, 0, 0} : seg_of<P>(s0);
    uint32_t pos = 0;  // the next term to add
    uint32_t set = 0;  // the LDS record set this pass writes
    // Whether passes still test for a tile without rounding: once a tile
    // fails the test, later ones (a larger sum, a coarser grid) almost never
    // pass it, and its data (an f64 sum and a lowest bit per term) is skipped.
    bool try_exact = true;
    uint32_t cur = 0xFFFFFFFFu, nxt = 0xFFFFFFFFu;  // bases of the tiles in xb and nb
    uint32_t xb[ITEMS], nb[ITEMS];  // terms of the current tile, raw bits of the next
    if (n > 0 && pred(s0)) {
        // A predicate that the start already meets is met by the first term's
        // sum (the sum only grows).
        *sum = add_p<P>(s0, term(fetch(0)));
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
            replay_sync<WAVE_ONLY>();
            uint32_t my_nz = 0xFFFFFFFFu, x_nz = 0;
#pragma unroll
            for (uint32_t i = 0; i < ITEMS; ++i) {
                if (my_nz == 0xFFFFFFFFu && (xv[i] & 0x7FFFFFFFu) != 0) {
                    my_nz = j0 + i;
                    x_nz = xv[i];
                }
            }
            if (my_nz != 0xFFFFFFFFu) atomicMin(&L->nonzero, my_nz);
            replay_sync<WAVE_ONLY>();
            const uint32_t jz = L->nonzero;
            replay_sync<WAVE_ONLY>();
            if (jz == 0xFFFFFFFFu) {
                pos = base + TILE;
                continue;
            }
            if (my_nz == jz) L->s_new = (double)__uint_as_float(x_nz);
            replay_sync<WAVE_ONLY>();
            s = L->s_new;
            replay_sync<WAVE_ONLY>();
            zero = false;
            if (pred(s)) {
                *sum = s;
                return jz;
            }
            g = seg_of<P>(s);
            pos = jz + 1;
            continue;
        }
        // This thread's terms: a run on the segment's grid, their f64 sum and
        // their lowest bit.
        const double scale = mul_pow2(1.0, -g.uexp);  // steps per unit
        StepRun r = run_identity();
        double fs = 0.0;
        int low = 0x7FFFFFFF;
#pragma unroll
        for (uint32_t i = 0; i < ITEMS; ++i) run_add(r, xv[i], scale);
        if (try_exact) {
#pragma unroll
            for (uint32_t i = 0; i < ITEMS; ++i) {
                fs += (double)__uint_as_float(xv[i]);
                if (xv[i] & 0x7FFFFFFFu) low = min(low, low_bit_exp(xv[i]));
            }
        }
        r.base = r.base < STEP_CAP ? r.base : STEP_CAP;
        const uint64_t T = __ballot(r.tie != 0), O = __ballot(run_par(r) != 0);
        uint32_t dep;
        const uint32_t k = parity_in(T, O, lane, &dep);
        // The wave's steps with every tie resolved but its first, whose step
        // depends on the parity entering the wave.
        const double wb = wave_total_f64(r.base + ((r.tie && !dep) ? (double)((k ^ r.c) & 1u) : 0.0));
        double wf = 0.0;
        int wl = (int)0x80000000u;  // fails the test below
        if (try_exact) {
            wf = wave_total_f64(fs);
            wl = wave_min_i32(low);
        }
        uint32_t bits;
        if (T != 0) {
            const uint32_t ft = (uint32_t)__builtin_ctzll(T);
            const uint32_t cf = (uint32_t)__builtin_amdgcn_readlane((int)r.c, (int)ft);
            uint32_t d0, d1;
            const uint32_t kf = parity_in(T, O, ft, &d0);
            const uint32_t po = parity_in(T, O, 64, &d1);
            bits = 1u | (((kf ^ cf) & 1u) << 1) | (po << 2);
        } else {
            bits = (popc64(O) & 1u) << 2;
        }
        if (lane == 0) {
            L->wave_base[set][wave] = wb < STEP_CAP ? wb : STEP_CAP;
            L->wave_fsum[set][wave] = wf;
            L->wave_bits[set][wave] = bits;
            L->wave_low[set][wave] = wl;
        }
        if (tid == 0) {
            L->cross = 0xFFFFFFFFu;
            L->hit = 0xFFFFFFFFu;
        }
        replay_sync<WAVE_ONLY>();
        // The waves in order, from the segment's parity: the tile's steps, the
        // parity entering this wave and the steps and f64 sum before it. Lane
        // w reads wave w's record; the combination reads those lanes into
        // scalar registers.
        const uint32_t rl = lane < NW ? lane : 0u;
        const uint64_t rbase = f64_bits(L->wave_base[set][rl]);
        const uint32_t rbits = L->wave_bits[set][rl];
        uint64_t rfsum = 0;
        int rlow = 0x7FFFFFFF;
        if (try_exact) {
            rfsum = f64_bits(L->wave_fsum[set][rl]);
            rlow = L->wave_low[set][rl];
        }
        uint32_t p = (uint32_t)(g.n & 1u), pw = 0;
        double tot = 0.0, tot_before = 0.0;
        double fsum = 0.0, f_before = 0.0;
        int lowest = 0x7FFFFFFF;
#pragma unroll 2
        for (uint32_t w = 0; w < NW; ++w) {
            if (w == wave) {
                tot_before = tot;
                pw = p;
                f_before = fsum;
            }
            const uint32_t b = (uint32_t)__builtin_amdgcn_readlane((int)rbits, (int)w);
            const double bw = f64_from_bits(((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(rbase >> 32), (int)w) << 32) |
                                            (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)rbase, (int)w));
            tot += bw + ((b & 1u) ? (double)((p ^ (b >> 1)) & 1u) : 0.0);
            p = (b & 1u) ? ((b >> 2) & 1u) : (p ^ ((b >> 2) & 1u));
            if (try_exact) {
                fsum += f64_from_bits(((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(rfsum >> 32), (int)w) << 32) |
                                      (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)rfsum, (int)w));
                lowest = min(lowest, __builtin_amdgcn_readlane(rlow, (int)w));
            }
        }
        set ^= 1u;
        // No addition in the rest of the tile rounds when s and every term are
        // multiples of the grid of a binade above the end sum (the f64 sum
        // est is within far less than 2^-30 of the exact one, and exact when
        // this holds: every subset sum is then representable).
        const double est = s + fsum;
        const int gx = grid_exp_of<P>(est * (1.0 + 0x1p-30));
        if (try_exact && lowest >= gx && seg_multiple(g, gx)) {
            if (!pred(est)) {
                s = est;
                g = seg_of<P>(s);
                pos = base + TILE;
                continue;
            }
            // Every partial sum is exact: the first that meets pred.
            double run = (s + f_before) + wave_excl_f64(fs);
            uint32_t my_hit = 0xFFFFFFFFu;
            double v_hit = 0.0;
#pragma unroll
            for (uint32_t i = 0; i < ITEMS; ++i) {
                const uint32_t j = j0 + i;
                if (j >= n || my_hit != 0xFFFFFFFFu) break;
                if (j < pos) continue;
                run += (double)__uint_as_float(xv[i]);
                if (pred(run)) {
                    my_hit = j;
                    v_hit = run;
                }
            }
            if (my_hit != 0xFFFFFFFFu) atomicMin(&L->hit, my_hit);
            replay_sync<WAVE_ONLY>();
            const uint32_t hit = L->hit;
            if (my_hit == hit) L->s_new = v_hit;
            replay_sync<WAVE_ONLY>();
            *sum = L->s_new;
            replay_sync<WAVE_ONLY>();
            return hit;
        }
        try_exact = false;
        const double room = (double)(g.lim - g.n);
        if (tot < room && !pred(scaled(g.n + (uint64_t)tot, g.uexp))) {
            // Nothing happens in the rest of this tile.
            g.n += (uint64_t)tot;
            s = scaled(g.n, g.uexp);
            pos = base + TILE;
            continue;
        }
        // Something happens here: the parity entering this thread's terms and
        // the steps before them, then its terms one by one.
        // The steps before this thread's terms are exact: they stay below the
        // room for every thread up to the event's.
        const uint32_t pl = dep ? (pw ^ k) : k;
        const double mine = r.base + (r.tie ? (double)((pl ^ r.c) & 1u) : 0.0);
        double I = tot_before + wave_excl_f64(mine);
        uint32_t par = pl;
        uint32_t my_cross = 0xFFFFFFFFu, my_hit = 0xFFFFFFFFu, x_cross = 0;
        double I_cross = 0.0, I_hit = 0.0;
#pragma unroll
        for (uint32_t i = 0; i < ITEMS; ++i) {
            const uint32_t j = j0 + i;
            if (j >= n || my_cross != 0xFFFFFFFFu || my_hit != 0xFFFFFFFFu) break;
            if (j < pos) continue;
            bool t;
            const double q = step_of(__uint_as_float(xv[i]), scale, &t);
            const uint32_t pq = parity_of(q);
            const double step = t ? q + (double)(par ^ pq) : q;
            par = t ? 0u : (par ^ pq);
            const double In = I + step;
            if (In >= room) {  // this term's sum leaves the segment
                my_cross = j;
                I_cross = I;
                x_cross = xv[i];
            } else if (pred(scaled(g.n + (uint64_t)In, g.uexp))) {
                my_hit = j;
                I_hit = In;
            } else {
                I = In;
            }
        }
        if (my_cross != 0xFFFFFFFFu) atomicMin(&L->cross, my_cross);
        if (my_hit != 0xFFFFFFFFu) atomicMin(&L->hit, my_hit);
        replay_sync<WAVE_ONLY>();
        const uint32_t cross = L->cross, hit = L->hit;
        if (hit < cross) {
            if (my_hit == hit) L->s_new = scaled(g.n + (uint64_t)I_hit, g.uexp);
            replay_sync<WAVE_ONLY>();
            *sum = L->s_new;
            replay_sync<WAVE_ONLY>();
            return hit;
        }
        if (cross == 0xFFFFFFFFu) {
            // Not reached: a step total at or past the room, or pred met at
            // the end, has its event in this tile. Kept so that every path
            // moves pos forward.
            g.n += (uint64_t)(tot < room ? tot : 0.0);
            s = scaled(g.n, g.uexp);
            pos = base + TILE;
            continue;
        }
        if (my_cross == cross) L->s_new = add_p<P>(scaled(g.n + (uint64_t)I_cross, g.uexp), __uint_as_float(x_cross));
        replay_sync<WAVE_ONLY>();
        s = L->s_new;
        replay_sync<WAVE_ONLY>();
        if (pred(s)) {
            *sum = s;
            return cross;
        }
        g = seg_of<P>(s);
        pos = cross + 1;  // the rest of this tile is redone from registers
    }
    *sum = s;
    return n;
}
template <int P, uint32_t NT, uint32_t ITEMS, class Fetch, class Term, class Pred>
__device__ __forceinline__ uint32_t seq_replay(Fetch fetch, Term term, uint32_t n, Pred pred, SeqLds<NT> *L, double *sum) {
    return seq_replay_from<P, NT, ITEMS, false>(fetch, term, n, pred, 0.0, L, sum);
}
// The same over terms that need no transformation: load(j) is the f32 term.
template <int P, uint32_t NT, uint32_t ITEMS, class Load, class Pred>
__device__ __forceinline__ uint32_t seq_replay(Load load, uint32_t n, Pred pred, SeqLds<NT> *L, double *sum) {
    return seq_replay<P, NT, ITEMS>([load](uint32_t j) { return __float_as_uint(load(j)); },
                                    [](uint32_t bits) { return __uint_as_float(bits); }, n, pred, L, sum);
}

// ------------------------------------------------------ chunked replay ---
// The same replay for long sums with a workgroup of 1024 threads, in rounds
// of CR_ROUND chunks of CR_CH terms, with two roles that run side by side.
// Waves 1 .. 15 (the workers) stage the rounds: each thread loads its
// CR_ITEMS consecutive terms of a round three rounds ahead, each half wave
// takes a chunk and computes its f64 sum, from which every chunk's start is
// predicted, and then counts its chunk's steps on the grid of the binade its
// start is predicted in, ties resolved but the first (the record seq_replay
// keeps per wave). Wave 0 chains the records of round r in order from the
// exact running sum while the workers prepare round r + 1 (one barrier per
// round): a record applies when the sum is on its grid, and the chunk then
// has no event if its end stays in the binade and fails pred (the partial
// sums only grow); any other chunk (the first nonzero term, a binade left,
// pred met, a start off the predicted grid) is added by wave 0 alone from
// LDS (wave_walk, seq_walk). The start of round r + 1 is predicted from the
// exact start of round r plus round r's f64 chunk sums; the f32 or f64
// running sum differs from that by its roundings, far less than a binade, so
// only a start within that distance of a binade's end misses its grid. A
// long sum thus costs a wave pass per binade crossing, hidden behind the
// staging of the next round where it is shorter, plus a barrier per round.
constexpr uint32_t CR_ITEMS = 8;               // consecutive terms per lane
constexpr uint32_t CR_CH = 32 * CR_ITEMS;      // terms per chunk (half a wave's)
constexpr uint32_t CR_WORKERS = 15;            // the waves that stage (all but wave 0)
constexpr uint32_t CR_ROUND = 2 * CR_WORKERS;  // chunks per round: two a worker wave
constexpr uint32_t CR_TERMS = CR_ROUND * CR_CH;

struct ChunkLds {
    __attribute__((aligned(16))) uint32_t terms[2][CR_TERMS];  // rounds r and r + 1 (by r & 1)
    double fsum[3][CR_ROUND];   // f64 sum of each chunk's terms, rounds r .. r + 2 (by r % 3)
    double base[2][CR_ROUND];   // its steps, every tie resolved but the first (capped)
    uint32_t bits[2][CR_ROUND]; // bit 0: a tie; bit 1: the first tie's constant; bit 2: par
    int32_t uexp[2][CR_ROUND];  // the grid its steps count; INT32_MIN: no record
    double s[2];                // the running sum at the start of round r (by r & 1)
    uint32_t hit[2];            // the first index meeting pred, or n, as of that start
};
// Sum of v over the 32 lanes of this half wave (every lane gets it).
__device__ __forceinline__ double half_total_f64(double v) {
    v += lane_xor_f64<1>(v);
    v += lane_xor_f64<2>(v);
    v += lane_xor_f64<4>(v);
    v += lane_xor_f64<8>(v);
    v += lane_xor_f64<16>(v);
    return v;
}

__device__ __forceinline__ double read_lane_f64(double v, uint32_t l) {
    const uint64_t b = f64_bits(v);
    return f64_from_bits(((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(b >> 32), (int)l) << 32) |
                         (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)b, (int)l));
}

// One wave adds the len (<= 64 * WK) terms t[0..len) to the running sum s
// (a P-bit value >= 0) in order, every lane the same: lane l holds terms
// l * WK .. l * WK + WK - 1. Per event (the sum leaving its binade, or pred
// becoming true) one pass: every lane counts its terms' steps on the
// segment's grid with the ties resolved (StepRun, parity_in), an exclusive
// scan gives each lane's start, a ballot finds the first lane whose terms
// hold the event, and that lane's terms are stepped through one by one (the
// term that leaves the binade is added with the IEEE addition, and the
// terms after it are counted again on the new grid). Returns the index of
// the first term whose partial sum meets pred, with that sum in s, or len
// with the total in s.
template <int P, uint32_t WK, class Pred>
__device__ __forceinline__ uint32_t wave_walk(RL_LDS const uint32_t *t, uint32_t len, Pred pred, double &s) {
    const uint32_t lane = __lane_id();
    uint32_t x[WK];
#pragma unroll
    for (uint32_t i = 0; i < WK; ++i) x[i] = lane * WK + i < len ? t[lane * WK + i] : 0u;
    uint32_t pos = 0;  // the next term to add
    for (;;) {
        if (!(s > 0.0)) {
            // The sum stays +0 up to the first nonzero term, which it then equals.
            uint32_t jz = 0xFFFFFFFFu;
#pragma unroll
            for (uint32_t i = 0; i < WK; ++i)
                if (jz == 0xFFFFFFFFu && lane * WK + i >= pos && (x[i] & 0x7FFFFFFFu) != 0) jz = lane * WK + i;
            const uint64_t nz = __ballot(jz != 0xFFFFFFFFu);
            if (nz == 0) return len;
            const uint32_t l = (uint32_t)__builtin_ctzll(nz);
            const uint32_t j = (uint32_t)__builtin_amdgcn_readlane((int)jz, (int)l);
            uint32_t xb = 0;
#pragma unroll
            for (uint32_t i = 0; i < WK; ++i)
                if (j - l * WK == i) xb = (uint32_t)__builtin_amdgcn_readlane((int)x[i], (int)l);
            s = (double)__uint_as_float(xb);
            if (pred(s)) return j;
            pos = j + 1;
            continue;
        }
        const SumSegF g = segf_of<P>(s);
        const double scale = mul_pow2(1.0, -g.uexp);
        StepRun r = run_identity();
#pragma unroll
        for (uint32_t i = 0; i < WK; ++i) run_add(r, lane * WK + i >= pos ? x[i] : 0u, scale);
        r.base = r.base < STEP_CAP ? r.base : STEP_CAP;
        const uint64_t T = __ballot(r.tie != 0), O = __ballot(run_par(r) != 0);
        uint32_t dep;
        const uint32_t k = parity_in(T, O, lane, &dep);
        const uint32_t pl = dep ? (parity_of(g.n) ^ k) : k;  // the parity entering this lane's terms
        const double mine = r.base + (r.tie ? (double)((pl ^ r.c) & 1u) : 0.0);
        const double before = wave_excl_f64(mine);  // exact below the room, where it is used
        const double room = g.lim - g.n;
        const double upto = before + mine;
        const bool ev = !(upto < room) || pred(mul_pow2(g.n + upto, g.uexp));
        const uint64_t evm = __ballot(ev);
        if (evm == 0) {
            s = mul_pow2(g.n + read_lane_f64(upto, 63), g.uexp);
            return len;
        }
        // The first lane holding an event steps through its terms.
        const uint32_t l = (uint32_t)__builtin_ctzll(evm);
        double nn = g.n + read_lane_f64(before, l);  // exact: below the room
        uint32_t par = parity_of(nn);
        bool crossed = false;
#pragma unroll
        for (uint32_t i = 0; i < WK; ++i) {
            const uint32_t j = l * WK + i;
            if (crossed || j < pos || j >= len) continue;
            const uint32_t xb = (uint32_t)__builtin_amdgcn_readlane((int)x[i], (int)l);
            bool tie;
            const double q = step_of(__uint_as_float(xb), scale, &tie);
            const uint32_t pq = parity_of(q);
            const double step = tie ? q + (double)(par ^ pq) : q;
            if (nn + step >= g.lim) {
                // This term leaves the binade: the IEEE addition, then a new
                // segment from the next term.
                s = add_p<P>(mul_pow2(nn, g.uexp), __uint_as_float(xb));
                if (pred(s)) return j;
                pos = j + 1;
                crossed = true;
                continue;
            }
            nn += step;
            par = tie ? 0u : (par ^ pq);
            if (pred(mul_pow2(nn, g.uexp))) {
                s = mul_pow2(nn, g.uexp);
                return j;
            }
        }
        if (!crossed) {  // not reached: the lane's event is in its terms
            s = mul_pow2(nn, g.uexp);
            pos = (l + 1) * WK;
        }
    }
}

// The same as wave_walk, one term after another (every lane alike), in
// blocks of SW_BLOCK terms: the next block's 16-byte LDS reads are issued
// before this block's additions, and pred is tested on a block's last sum
// first (the partial sums only grow, so a block whose last sum fails pred
// holds no hit). f32 sums run in f32 registers (the same IEEE additions,
// with no conversions on the dependency chain). t must be 16-byte aligned;
// the words past len up to the next multiple of SW_BLOCK are read and
// ignored. For a chunk whose sum leaves several binades this is cheaper than
// a wave pass per binade.
constexpr uint32_t SW_BLOCK = 16;

template <int P, class Pred>
__device__ __forceinline__ uint32_t seq_walk(RL_LDS const uint32_t *t, uint32_t len, Pred pred, double &s) {
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    typedef typename std::conditional<P == 24, float, double>::type acc_t;
    u32x4 nq[SW_BLOCK / 4];
#pragma unroll
    for (uint32_t q = 0; q < SW_BLOCK / 4; ++q) nq[q] = *(RL_LDS const u32x4 *)&t[4 * q];
    acc_t run = (acc_t)s;  // s is a P-bit value: exact
    for (uint32_t j = 0; j < len; j += SW_BLOCK) {
        float x[SW_BLOCK];
#pragma unroll
        for (uint32_t q = 0; q < SW_BLOCK / 4; ++q)
#pragma unroll
            for (uint32_t i = 0; i < 4; ++i) x[4 * q + i] = j + 4 * q + i < len ? __uint_as_float(nq[q][i]) : 0.0f;
        if (j + SW_BLOCK < len) {
#pragma unroll
            for (uint32_t q = 0; q < SW_BLOCK / 4; ++q) nq[q] = *(RL_LDS const u32x4 *)&t[j + SW_BLOCK + 4 * q];
        }
        acc_t a[SW_BLOCK];
        a[0] = run + (acc_t)x[0];
#pragma unroll
        for (uint32_t i = 1; i < SW_BLOCK; ++i) a[i] = a[i - 1] + (acc_t)x[i];
        if (pred((double)a[SW_BLOCK - 1])) {
#pragma unroll
            for (uint32_t i = 0; i < SW_BLOCK; ++i)
                if (pred((double)a[i])) {
                    s = (double)a[i];
                    return j + i;
                }
        }
        run = a[SW_BLOCK - 1];
    }
    s = (double)run;
    return len;
}

// A range of a term array whose words are all one value that is not stored
// there: readers take `word` for j in [lo, hi) (an empty range by default).
struct HotRange {
    uint32_t lo = 0, hi = 0, word = 0;
    __device__ __forceinline__ bool has(uint32_t j) const { return j - lo < hi - lo; }
    __device__ __forceinline__ uint32_t fix(uint32_t j, uint32_t w) const { return has(j) ? word : w; }
};

// Returns as seq_replay does, for the terms x_j = term(src[j]) (raw 32-bit
// words; src[j] read as hr.word for j in hr), j < n, added to the running sum
// s0 (a P-bit value >= 0; +0 by default); every thread of the workgroup
// (1024) calls it. With wb, the
// terms of every round it stages are also stored to wb[j] (wb may be src: a
// round's words are read two rounds before they are written), and *staged
// gets how many: a prefix of [0, n).
template <int P, uint32_t NT, class Term, class Pred>
__device__ __forceinline__ uint32_t chunk_replay(const uint32_t *src, Term term, uint32_t n, Pred pred,
                                                 RL_LDS ChunkLds *L, double *sum, uint32_t *wb = nullptr,
                                                 uint32_t *staged = nullptr, const HotRange &hr_in = HotRange(),
                                                 double s0 = 0.0) {
    static_assert(NT / 64 - 1 == CR_WORKERS, "wave 0 chains, the other waves stage two chunks each");
    // The range cut at n: the words past n are zeros.
    HotRange hr = hr_in;
    hr.hi = min(hr.hi, n);
    hr.lo = min(hr.lo, hr.hi);
    const uint32_t tid = threadIdx.x, lane = __lane_id(), wave = tid / 64;
    const bool worker = wave != 0;
    const uint32_t wt = tid - 64;  // a worker's thread index
    const uint32_t half = lane >> 5, hl = lane & 31u, my = 2 * (wave - 1) + half;  // a worker half wave's chunk
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc((void *)src, (short)0, (int)(n * 4u), 0x00020000);
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    // A worker's CR_ITEMS raw words of round r (zeros past n: they add
    // nothing).
    u32x4 xr[CR_ITEMS / 4];
    auto fetch_round = [&](uint32_t r) {
        // A thread whose words all lie in hr loads none.
        const uint32_t j0 = r * CR_TERMS + wt * CR_ITEMS;
        if (hr.has(j0) && hr.has(j0 + CR_ITEMS - 1)) {
#pragma unroll
            for (uint32_t q = 0; q < CR_ITEMS / 4; ++q) xr[q] = u32x4{0u, 0u, 0u, 0u};
        } else {
#pragma unroll
            for (uint32_t q = 0; q < CR_ITEMS / 4; ++q)
                xr[q] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, 4u * j0 + 16u * q, 0, 0));
        }
    };
    const uint32_t rounds = (uint32_t)(((uint64_t)n + CR_TERMS - 1) / CR_TERMS);
    const uint32_t chunks = (uint32_t)(((uint64_t)n + CR_CH - 1) / CR_CH);
    const __amdgpu_buffer_rsrc_t rw =
        __builtin_amdgcn_make_buffer_rsrc((void *)wb, (short)0, wb ? (int)(n * 4u) : 0, 0x00020000);
    if (staged) *staged = 0;
    if (n > 0 && pred(s0)) {
        // A predicate that s0 already meets is met by the first term's sum.
        *sum = add_p<P>(s0, term(hr.fix(0, __builtin_amdgcn_raw_buffer_load_b32(rs, 0, 0, 0))));
        return 0;
    }
    if (rounds == 0) {
        *sum = s0;
        return n;
    }
    // A worker's terms of the round it stages, and their f64 chunk sum.
    uint32_t x[CR_ITEMS];
    auto stage = [&](uint32_t r) {
        double fs = 0.0;
#pragma unroll
        for (uint32_t q = 0; q < CR_ITEMS / 4; ++q)
#pragma unroll
            for (uint32_t i = 0; i < 4; ++i) {
                x[4 * q + i] = __float_as_uint(term(hr.fix(r * CR_TERMS + wt * CR_ITEMS + 4 * q + i, xr[q][i])));
                fs += (double)__uint_as_float(x[4 * q + i]);
            }
        fs = half_total_f64(fs);
        if (hl == 0) L->fsum[r % 3][my] = fs;
    };
    // Round r's terms into LDS (and wb), and each chunk's record on the grid
    // of its start predicted from s_round, the round's predicted start.
    auto prepare = [&](uint32_t r, double s_round) {
        const uint32_t b = r & 1u;
#pragma unroll
        for (uint32_t q = 0; q < CR_ITEMS / 4; ++q)
            *(RL_LDS u32x4 *)&L->terms[b][wt * CR_ITEMS + 4 * q] = u32x4{x[4 * q], x[4 * q + 1], x[4 * q + 2], x[4 * q + 3]};
        if (wb) {
#pragma unroll
            for (uint32_t q = 0; q < CR_ITEMS / 4; ++q)
                __builtin_amdgcn_raw_buffer_store_b128(u32x4{x[4 * q], x[4 * q + 1], x[4 * q + 2], x[4 * q + 3]}, rw,
                                                       4u * (r * CR_TERMS + wt * CR_ITEMS) + 16u * q, 0, 0);
        }
        const double pre = wave_excl_f64(lane < CR_ROUND ? L->fsum[r % 3][lane] : 0.0);
        const uint32_t c0 = (uint32_t)__builtin_amdgcn_readfirstlane((int)(my - half));  // the wave's first chunk
        const double start = s_round + (half ? read_lane_f64(pre, c0 + 1) : read_lane_f64(pre, c0));
        const bool rec = start > 0.0;
        const int32_t ux = rec ? seg_of<P>(start).uexp : INT32_MIN;
        const double scale = rec ? mul_pow2(1.0, -ux) : 1.0;
        StepRun rr = run_identity();
#pragma unroll
        for (uint32_t i = 0; i < CR_ITEMS; ++i) run_add(rr, x[i], scale);
        rr.base = rr.base < STEP_CAP ? rr.base : STEP_CAP;
        const uint64_t Tw = __ballot(rr.tie != 0), Ow = __ballot(run_par(rr) != 0);
        const uint64_t T = half ? (Tw >> 32) : (Tw & 0xFFFFFFFFull);
        const uint64_t O = half ? (Ow >> 32) : (Ow & 0xFFFFFFFFull);
        uint32_t dep;
        const uint32_t k = parity_in(T, O, hl, &dep);
        const double wsum = half_total_f64(rr.base + ((rr.tie && !dep) ? (double)((k ^ rr.c) & 1u) : 0.0));
        uint32_t bits;
        const uint32_t ft = T != 0 ? (uint32_t)__builtin_ctzll(T) : 0u;
        // The first tie's constant, from the lane holding it in each half.
        const uint32_t T0 = (uint32_t)Tw, T1 = (uint32_t)(Tw >> 32);
        const uint32_t c_lo = (uint32_t)__builtin_amdgcn_readlane((int)rr.c, T0 ? (int)__builtin_ctz(T0) : 0);
        const uint32_t c_hi = (uint32_t)__builtin_amdgcn_readlane((int)rr.c, T1 ? 32 + (int)__builtin_ctz(T1) : 32);
        const uint32_t cf = half ? c_hi : c_lo;
        if (T != 0) {
            uint32_t d0, d1;
            const uint32_t kf = parity_in(T, O, ft, &d0);
            const uint32_t po = parity_in(T, O, 32, &d1);
            bits = 1u | (((kf ^ cf) & 1u) << 1) | (po << 2);
        } else {
            bits = (popc64(O) & 1u) << 2;
        }
        if (hl == 0) {
            L->uexp[b][my] = ux;
            L->base[b][my] = wsum < STEP_CAP ? wsum : STEP_CAP;
            L->bits[b][my] = bits;
        }
    };
    // Round 0 and the sums of round 1 before the first chain.
    if (worker) {
        fetch_round(0);
        stage(0);
        if (rounds > 1) fetch_round(1);
    }
    if (tid == 0) {
        L->s[0] = s0;
        L->hit[0] = n;
    }
    __syncthreads();
    if (worker) {
        prepare(0, s0);
        if (rounds > 1) {
            stage(1);
            if (rounds > 2) fetch_round(2);
        }
    }
    __syncthreads();
    uint32_t r = 0, hit = n;
    while (true) {
        if (!worker) {
            // The chain of round r; lane c holds chunk c's record. From the
            // current chunk on, the chunks on the sum's grid without a tie add
            // their steps (a scan); the first one whose end leaves the binade
            // or meets pred, or whose record does not apply, stops the run, and
            // is added by wave_walk or seq_walk (or by its record, when only a
            // tie stopped it).
            __builtin_amdgcn_s_setprio(2);  // the round's critical path
            const uint32_t b = r & 1u;
            double s = L->s[b];
            const uint32_t nr = min(CR_ROUND, chunks - r * CR_ROUND);
            const bool lr = lane < nr;
            const int32_t rux = lr ? L->uexp[b][lane] : INT32_MIN;
            const uint32_t rbits = lr ? L->bits[b][lane] : 0u;
            const double rbase = lr ? L->base[b][lane] : 0.0;
            uint32_t c = 0;
            while (c < nr) {
                if (s > 0.0) {
                    const SumSegF g = segf_of<P>(s);
                    const double room = g.lim - g.n;
                    const bool ok = lane >= c && lr && rux == g.uexp && !(rbits & 1u);
                    const double incl = wave_incl_f64(ok ? rbase : 0.0);
                    const bool good = ok && incl < room && !pred(mul_pow2(g.n + incl, g.uexp));
                    const uint64_t stopm = __ballot(lane >= c && lr && !good);
                    const uint32_t f = stopm ? (uint32_t)__builtin_ctzll(stopm) : nr;
                    if (f > c) {
                        s = mul_pow2(g.n + read_lane_f64(incl, f - 1), g.uexp);
                        c = f;
                        continue;
                    }
                    if (__builtin_amdgcn_readlane(rux, (int)c) == g.uexp) {
                        // Only a tie stopped it: the record with the parity.
                        const uint32_t bb = (uint32_t)__builtin_amdgcn_readlane((int)rbits, (int)c);
                        const double inc = read_lane_f64(rbase, c) +
                                           ((bb & 1u) ? (double)((parity_of(g.n) ^ (bb >> 1)) & 1u) : 0.0);
                        if (inc < room) {
                            const double e = mul_pow2(g.n + inc, g.uexp);
                            if (!pred(e)) {
                                s = e;
                                ++c;
                                continue;
                            }
                        }
                    }
                }
                const uint32_t start_j = (r * CR_ROUND + c) * CR_CH;
                const uint32_t len = min(CR_CH, n - start_j);
                // A chunk that at least quadruples the sum (or starts it) leaves
                // two binades or more: term by term; else by wave passes.
                const double cf = L->fsum[r % 3][c];
                const uint32_t j = (!(s > 0.0) || cf >= 3.0 * s)
                                       ? seq_walk<P>(&L->terms[b][c * CR_CH], len, pred, s)
                                       : wave_walk<P, CR_CH / 64>(&L->terms[b][c * CR_CH], len, pred, s);
                if (j < len) {
                    hit = start_j + j;
                    break;
                }
                ++c;
            }
            __builtin_amdgcn_s_setprio(0);
            if (lane == 0) {
                L->s[b ^ 1u] = s;
                L->hit[b ^ 1u] = hit;
            }
        } else if (r + 1 < rounds) {
            // Round r + 1 from round r's exact start and its chunk sums; then
            // the sums of round r + 2 and the loads of round r + 3.
            const double tot = wave_total_f64(lane < CR_ROUND ? L->fsum[r % 3][lane] : 0.0);
            prepare(r + 1, L->s[r & 1u] + tot);
            if (r + 2 < rounds) {
                stage(r + 2);
                if (r + 3 < rounds) fetch_round(r + 3);
            }
        }
        __syncthreads();
        ++r;
        hit = L->hit[r & 1u];
        if (hit != n || r == rounds) break;
    }
    // Rounds 0 .. r were stored to wb (those below rounds).
    if (staged) *staged = (uint32_t)min((uint64_t)n, (uint64_t)(r + 1) * CR_TERMS);
    *sum = L->s[r & 1u];
    return hit;
}
#endif  // __HIPCC__

}  // namespace rl
