// Checks the exact parallel replay of sequential sums (rust-llm_amd/csrc/
// rl_seqsum.h) against plain sequential loops, on the host.
//
// For each case: an array of non-negative f32 terms; the plain loop
// s = fl_P(s + x_j) (P = 24: f32, P = 53: f64) gives every partial sum. The
// replay walks the same array in tiles of `tile` terms the way the device
// does: per tile, the exact path when no addition in it can round (the sum
// moves to the exact end sum, across binades), else the composition of the
// term maps of the current segment, the first term whose partial sum leaves
// the segment (added with the IEEE addition instead), and the first term whose
// partial sum meets a monotone predicate. Both the final sums and the
// predicate indices must agree, bit for bit, for every threshold tried. It
// also checks that the device's per-thread runs and ballot parities compose
// to the same steps and parities as the term maps, and that the term maps
// compose associatively.
//
// Output: one line "ok <cases>" or the first mismatch; exit status 0 on
// success.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>
#include <algorithm>

#include "rl_seqsum.h"

using namespace rl;

static uint64_t rs = 0x9E3779B97F4A7C15ull;
static uint64_t rnd() {
    rs += 0x9E3779B97F4A7C15ull;
    uint64_t z = rs;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
static double unit() { return (double)(rnd() >> 11) * 0x1.0p-53; }
static uint32_t fbits(float f) {
    uint32_t b;
    memcpy(&b, &f, 4);
    return b;
}
static float from_bits(uint32_t b) {
    float f;
    memcpy(&f, &b, 4);
    return f;
}

// Plain sequential sums: partial[j] = sum after adding x[j].
template <int P>
static void plain(const std::vector<float> &x, std::vector<double> &partial) {
    partial.resize(x.size());
    if (P == 24) {
        float s = 0.0f;
        for (size_t j = 0; j < x.size(); ++j) {
            s = s + x[j];
            partial[j] = s;
        }
    } else {
        double s = 0.0;
        for (size_t j = 0; j < x.size(); ++j) {
            s = s + (double)x[j];
            partial[j] = s;
        }
    }
}

static int failures = 0;
static long exact_tiles = 0;

// The device algorithm, run serially: returns the first j whose partial sum
// is >= thr (or > thr when strict), or n; *sum gets the partial sum there, or
// the final sum when none.
template <int P>
static uint32_t replay(const std::vector<float> &x, uint32_t tile, double thr, bool strict, bool use_pred,
                       double *sum) {
    auto pred = [&](double s) { return use_pred && (strict ? s > thr : s >= thr); };
    const uint32_t n = (uint32_t)x.size();
    double s = 0.0;
    bool zero = true;
    SumSeg g{0, 0, 0};
    uint32_t pos = 0;
    if (n > 0 && pred(0.0)) {
        *sum = add_p<P>(0.0, x[0]);
        return 0;
    }
    while (pos < n) {
        // Tiles aligned to `tile`; terms below pos count as +0.
        const uint32_t base = pos / tile * tile;
        const uint32_t end = base + tile < n ? base + tile : n;
        auto term = [&](uint32_t j) { return j >= pos ? fbits(x[j]) : 0u; };
        if (zero) {
            uint32_t jz = n;
            for (uint32_t j = base; j < end; ++j)
                if ((term(j) & 0x7FFFFFFFu) != 0) {
                    jz = j;
                    break;
                }
            if (jz == n) {
                pos = base + tile;
                continue;
            }
            s = x[jz];
            zero = false;
            if (pred(s)) {
                *sum = s;
                return jz;
            }
            g = seg_of<P>(s);
            pos = jz + 1;
            continue;
        }
        // As on the device: when s and every term left in the tile are
        // multiples of the grid of a binade above the end sum, no addition
        // rounds, and the f64 sum is the exact sum.
        {
            double fsum = 0.0;
            int lowest = 0x7FFFFFFF;
            for (uint32_t j = base; j < end; ++j) {
                fsum += (double)from_bits(term(j));
                if (term(j) & 0x7FFFFFFFu) lowest = std::min(lowest, low_bit_exp(term(j)));
            }
            const double est = s + fsum;
            const int gx = grid_exp_of<P>(est * (1.0 + 0x1p-30));
            if (lowest >= gx && seg_multiple(g, gx)) {
                ++exact_tiles;
                if (!pred(est)) {
                    s = est;
                    g = seg_of<P>(s);
                    pos = base + tile;
                    continue;
                }
                double run = s;
                for (uint32_t j = pos; j < end; ++j) {
                    run += (double)x[j];
                    if (pred(run)) {
                        *sum = run;
                        return j;
                    }
                }
                printf("FAIL exact tile: pred met at the end but not on the way\n");
                ++failures;
                return n;
            }
        }
        const uint32_t par0 = (uint32_t)(g.n & 1);
        const uint64_t room = g.lim - g.n;
        // The segment's steps: a tile without an exact tie uses the plain
        // increments, a tile with one the parity-carrying maps (the device's
        // runs and parities compose to the same, check_runs).
        bool anytie = false;
        for (uint32_t j = base; j < end; ++j) {
            bool t;
            inc_of(term(j), g.uexp, &t);
            anytie |= t;
        }
        TermMap acc = map_identity();
        uint64_t plain_acc = 0;
        uint32_t cross = n, hit = n;
        uint64_t before = 0;
        for (uint32_t j = base; j < end; ++j) {
            uint64_t I;
            TermMap nx{};
            if (anytie) {
                nx = map_then(acc, map_of(term(j), g.uexp));
                I = map_inc(nx, par0);
            } else {
                bool t;
                I = sat_add(plain_acc, inc_of(term(j), g.uexp, &t));
            }
            if (I >= room) {
                cross = j;
                before = anytie ? map_inc(acc, par0) : plain_acc;
                break;
            }
            if (j >= pos && pred(scaled(g.n + I, g.uexp))) {
                hit = j;
                *sum = scaled(g.n + I, g.uexp);
                break;
            }
            if (anytie)
                acc = nx;
            else
                plain_acc = I;
        }
        if (hit < n) return hit;
        if (cross < n) {
            s = add_p<P>(scaled(g.n + before, g.uexp), x[cross]);
            if (pred(s)) {
                *sum = s;
                return cross;
            }
            g = seg_of<P>(s);
            pos = cross + 1;
            continue;
        }
        g.n += anytie ? map_inc(acc, par0) : plain_acc;
        s = scaled(g.n, g.uexp);
        pos = base + tile;
    }
    *sum = s;
    return n;
}

template <int P>
static void check(const std::vector<float> &x, const char *what, uint32_t tile) {
    std::vector<double> partial;
    plain<P>(x, partial);
    const uint32_t n = (uint32_t)x.size();
    double sum = -1.0;
    const uint32_t none = replay<P>(x, tile, 0.0, false, false, &sum);
    const double want = n ? partial[n - 1] : 0.0;
    if (none != n || memcmp(&sum, &want, 8) != 0) {
        if (failures++ < 5)
            printf("FAIL P=%d %s n=%u tile=%u: sum %.17g want %.17g\n", P, what, n, tile, sum, want);
        return;
    }
    // Thresholds: every partial sum, and values just around some of them.
    for (int t = 0; t < 26 && n; ++t) {
        const uint32_t j = (uint32_t)(rnd() % n);
        double thr = partial[j];
        const int wiggle = (int)(rnd() % 3) - 1;
        if (wiggle) thr = std::nextafter(thr, wiggle > 0 ? INFINITY : -INFINITY);
        if (t == 24) thr = 0.0;   // a target of 0 (top_p = 0): met by the first term
        if (t == 25) thr = -1.0;
        for (int strict = 0; strict < 2; ++strict) {
            uint32_t w = n;
            for (uint32_t i = 0; i < n; ++i)
                if (strict ? partial[i] > thr : partial[i] >= thr) {
                    w = i;
                    break;
                }
            double at = -1.0;
            const uint32_t got = replay<P>(x, tile, thr, strict, true, &at);
            if (got != w || (got < n && memcmp(&at, &partial[got], 8) != 0)) {
                if (failures++ < 5)
                    printf("FAIL P=%d %s n=%u tile=%u thr=%.17g strict=%d: index %u want %u\n", P, what, n, tile,
                           thr, strict, got, w);
                return;
            }
        }
    }
}

// Random term maps compose associatively.
static void check_assoc() {
    for (int t = 0; t < 200000; ++t) {
        TermMap m[3];
        for (auto &v : m) {
            const int uexp = -60 + (int)(rnd() % 40);
            v = map_of((uint32_t)(rnd() & 0x7FFFFFFFu) % 0x7F800000u, uexp);
        }
        const TermMap a = map_then(map_then(m[0], m[1]), m[2]);
        const TermMap b = map_then(m[0], map_then(m[1], m[2]));
        if (a.i0 != b.i0 || a.i1 != b.i1 || a.p0 != b.p0 || a.p1 != b.p1) {
            if (failures++ < 5) printf("FAIL associativity\n");
            return;
        }
    }
}

// The workgroup's step arithmetic (StepRun per thread, parity_in across the
// 64 lanes of a wave from the tie and odd-parity masks, the waves' records
// combined in order) against the composition of the term maps: the tile's
// total steps and final parity, and every thread's entering parity and steps
// before it, from both starting parities. Terms are drawn tie-heavy on a
// random grid.
static void check_runs() {
    for (int rep = 0; rep < 3000; ++rep) {
        const int uexp = -60 + (int)(rnd() % 30);
        const uint32_t items = 1 + (uint32_t)(rnd() % 8), nw = 1 + (uint32_t)(rnd() % 4);
        const uint32_t tie_pct = (uint32_t)(rnd() % 101);
        const uint32_t n = items * 64 * nw;
        std::vector<uint32_t> x(n);
        for (uint32_t i = 0; i < n; ++i) {
            const uint64_t q = rnd() % 1024;
            const uint32_t kind = (uint32_t)(rnd() % 100);
            float v;
            if (kind < tie_pct)
                v = ldexpf((float)(2 * q + 1), uexp - 1);  // an exact tie on the grid
            else if (kind % 4 == 0)
                v = 0.0f;
            else if (kind % 4 == 1)
                v = ldexpf((float)q, uexp);  // a multiple of the step
            else
                v = ldexpf((float)(rnd() % (1u << 20)), uexp - 10);  // anything in between
            x[i] = fbits(v);
        }
        for (uint32_t p0 = 0; p0 < 2; ++p0) {
            // Per thread and per wave, as the device computes them.
            std::vector<StepRun> run(64 * nw);
            std::vector<uint32_t> k(64 * nw), dep(64 * nw);
            std::vector<double> wbase(nw);
            std::vector<uint32_t> wbits(nw);
            for (uint32_t w = 0; w < nw; ++w) {
                uint64_t T = 0, O = 0;
                for (uint32_t l = 0; l < 64; ++l) {
                    StepRun r = run_identity();
                    for (uint32_t i = 0; i < items; ++i) run_add(r, x[((w * 64 + l) * items) + i], ldexp(1.0, -uexp));
                    run[w * 64 + l] = r;
                    if (r.tie) T |= 1ull << l;
                    if (run_par(r)) O |= 1ull << l;
                }
                double wb = 0.0;
                for (uint32_t l = 0; l < 64; ++l) {
                    const StepRun &r = run[w * 64 + l];
                    k[w * 64 + l] = parity_in(T, O, l, &dep[w * 64 + l]);
                    wb += r.base + ((r.tie && !dep[w * 64 + l]) ? (double)((k[w * 64 + l] ^ r.c) & 1u) : 0.0);
                }
                uint32_t bits;
                if (T) {
                    const uint32_t ft = (uint32_t)__builtin_ctzll(T);
                    uint32_t d0, d1;
                    const uint32_t kf = parity_in(T, O, ft, &d0);
                    const uint32_t po = parity_in(T, O, 64, &d1);
                    bits = 1u | (((kf ^ run[w * 64 + ft].c) & 1u) << 1) | (po << 2);
                } else {
                    bits = (popc64(O) & 1u) << 2;
                }
                wbase[w] = wb;
                wbits[w] = bits;
            }
            uint32_t p = p0;
            double tot = 0.0;
            std::vector<double> before(nw);
            std::vector<uint32_t> pin(nw);
            for (uint32_t w = 0; w < nw; ++w) {
                before[w] = tot;
                pin[w] = p;
                const uint32_t b = wbits[w];
                tot += wbase[w] + ((b & 1u) ? (double)((p ^ (b >> 1)) & 1u) : 0.0);
                p = (b & 1u) ? ((b >> 2) & 1u) : (p ^ ((b >> 2) & 1u));
            }
            // The maps, term by term.
            TermMap acc = map_identity();
            for (uint32_t w = 0; w < nw; ++w) {
                double I = before[w];
                for (uint32_t l = 0; l < 64; ++l) {
                    const uint32_t t = w * 64 + l;
                    const uint32_t pl = dep[t] ? (pin[w] ^ k[t]) : k[t];
                    if ((double)map_inc(acc, p0) != I || map_parity(acc, p0) != pl) {
                        if (failures++ < 5)
                            printf("FAIL runs: thread %u of %u, items %u, p0 %u: steps %llu/%llu parity %u/%u\n", t,
                                   64 * nw, items, p0, (unsigned long long)I,
                                   (unsigned long long)map_inc(acc, p0), pl, map_parity(acc, p0));
                        return;
                    }
                    I += run[t].base + (run[t].tie ? (double)((pl ^ run[t].c) & 1u) : 0.0);
                    for (uint32_t i = 0; i < items; ++i) acc = map_then(acc, map_of(x[t * items + i], uexp));
                }
            }
            if ((double)map_inc(acc, p0) != tot || map_parity(acc, p0) != p) {
                if (failures++ < 5) printf("FAIL runs: tile total, items %u, p0 %u\n", items, p0);
                return;
            }
        }
    }
}

// equal_run_walk (a run of equal terms crossed a segment at a time) against
// the plain loop from the same start: the sum after the run, and the first
// index meeting `partial > thr` and `partial >= thr` for thresholds at, just
// below and just above partial sums, 0 and past the end. Terms are drawn as
// exact ties on the start's grid, multiples of it, zeros, subnormals, terms
// far below half a step, and terms larger than the start.
template <int P>
static void check_equal_runs(int &cases) {
    for (int rep = 0; rep < 3000; ++rep) {
        double s0 = 0.0;
        const int sk = (int)(rnd() % 6);
        if (sk == 1) s0 = (double)from_bits(1u + (uint32_t)(rnd() % 0x7FFFFFu));      // subnormal f32
        if (sk >= 2) s0 = (double)(float)ldexp(unit() + 0.5, -(int)(rnd() % 40));
        if (P == 53 && sk == 5) s0 = ldexp(1.0 + unit(), -(int)(rnd() % 40));        // a full f64
        float x;
        const int xk = (int)(rnd() % 8);
        const int gx = s0 > 0.0 ? seg_of<P>(s0).uexp : -149;
        switch (xk) {
        case 0: x = (float)ldexp((double)(2 * (rnd() % 64) + 1), gx - 1); break;     // an exact tie
        case 1: x = (float)ldexp((double)(rnd() % 4096), gx); break;                 // a multiple of the step
        case 2: x = 0.0f; break;
        case 3: x = from_bits(1u + (uint32_t)(rnd() % 0x7FFFFFu)); break;            // subnormal
        case 4: x = (float)ldexp(unit(), gx - 3); break;                             // below half a step
        case 5: x = (float)(s0 * (1.0 + 4.0 * unit()) + 1e-30); break;               // larger than the start
        default: x = (float)ldexp(unit() + 0.5, -(int)(rnd() % 30) - 4); break;
        }
        if (!(x >= 0.0f) || !std::isfinite(x)) x = 0.0f;
        if (P == 24) s0 = (double)(float)s0;
        const uint32_t n = 1 + (uint32_t)(rnd() % (rep % 10 == 0 ? 300000 : 3000));
        std::vector<double> partial(n);
        if (P == 24) {
            float a = (float)s0;
            for (uint32_t i = 0; i < n; ++i) partial[i] = a = a + x;
        } else {
            double a = s0;
            for (uint32_t i = 0; i < n; ++i) partial[i] = a = a + (double)x;
        }
        double sum = s0;
        const uint32_t all = equal_run_walk<P>(sum, fbits(x), n, [](double) { return false; });
        if (all != n || memcmp(&sum, &partial[n - 1], 8) != 0) {
            if (failures++ < 5)
                printf("FAIL equal run P=%d s0=%.17g x=%a n=%u: sum %.17g want %.17g\n", P, s0, (double)x, n, sum,
                       partial[n - 1]);
            return;
        }
        for (int t = 0; t < 12; ++t) {
            const uint32_t j = (uint32_t)(rnd() % n);
            double thr = partial[j];
            const int wiggle = (int)(rnd() % 3) - 1;
            if (wiggle) thr = std::nextafter(thr, wiggle > 0 ? INFINITY : -INFINITY);
            if (t == 10) thr = partial[n - 1] * 2.0 + 1.0;  // never met
            if (t == 11) thr = s0;                           // met by the first term that moves the sum
            if (thr < s0 || (thr == s0 && false)) continue;
            for (int strict = 0; strict < 2; ++strict) {
                if (!strict && !(s0 < thr)) continue;  // pred must be false at the start
                uint32_t w = n;
                for (uint32_t i = 0; i < n; ++i)
                    if (strict ? partial[i] > thr : partial[i] >= thr) {
                        w = i;
                        break;
                    }
                double at = s0;
                const uint32_t got = equal_run_walk<P>(
                    at, fbits(x), n, [thr, strict](double c) { return strict ? c > thr : c >= thr; });
                const double want_at = w < n ? partial[w] : partial[n - 1];
                if (got != w || memcmp(&at, &want_at, 8) != 0) {
                    if (failures++ < 5)
                        printf("FAIL equal run P=%d s0=%.17g x=%a n=%u thr=%.17g strict=%d: index %u want %u\n", P,
                               s0, (double)x, n, thr, strict, got, w);
                    return;
                }
            }
        }
        ++cases;
    }
}

template <int P>
static void run_all(int &cases) {
    const uint32_t tiles[] = {1, 7, 64, 2048};
    for (int rep = 0; rep < 60; ++rep) {
        const uint32_t n = 1 + (uint32_t)(rnd() % (rep < 30 ? 300 : 5000));
        std::vector<float> x(n);
        const int kind = rep % 10;
        for (uint32_t i = 0; i < n; ++i) {
            float v = 0.0f;
            switch (kind) {
            case 0: v = (float)unit(); break;                                   // uniform [0, 1)
            case 1: v = expf((float)(-40.0 * unit())); break;                   // wide range
            case 2: v = (float)(1.0 + unit() * 1e-3); break;                    // narrow, exact sums
            case 3: v = from_bits((uint32_t)(rnd() % 0x00800000u)); break;      // subnormals
            case 4: v = (rnd() & 3) ? 0.0f : (float)unit(); break;              // many zeros
            case 5: v = (rnd() & 1) ? 0.75f : 1.0f / 3.0f; break;               // ties of few values
            case 6: v = ldexpf(1.0f + (float)(rnd() % 8) / 8.0f, -(int)(rnd() % 60)); break;  // short significands
            case 7: v = from_bits(0x3F800000u + (uint32_t)(rnd() % 4)); break;  // ~1, many exact ties
            case 8: v = expf((float)(-100.0 * unit())); break;                  // very wide
            default: v = (float)(unit() * unit() * unit()); break;
            }
            x[i] = v;
        }
        if (rep % 3 == 0) std::sort(x.begin(), x.end(), [](float a, float b) { return a > b; });
        for (uint32_t t : tiles) {
            check<P>(x, "random", t);
            ++cases;
        }
    }
    // Constant runs that cross many binades: every add of the same value.
    for (int rep = 0; rep < 20; ++rep) {
        const float v = ldexpf((float)(1 + rnd() % 255), -(int)(rnd() % 20) - 8);
        std::vector<float> x(3000, v);
        for (uint32_t t : tiles) {
            check<P>(x, "constant", t);
            ++cases;
        }
    }
}

int main() {
    int cases = 0;
    check_assoc();
    check_runs();
    run_all<24>(cases);
    run_all<53>(cases);
    check_equal_runs<24>(cases);
    check_equal_runs<53>(cases);
    if (failures) {
        printf("%d failures\n", failures);
        return 1;
    }
    if (exact_tiles == 0) {
        printf("FAIL no tile took the exact path\n");
        return 1;
    }
    printf("ok %d\n", cases);
    return 0;
}
