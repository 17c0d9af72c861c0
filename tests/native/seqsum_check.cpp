// Checks the exact parallel replay of sequential sums (rust-llm_amd/csrc/
// rl_seqsum.h) against plain sequential loops, on the host.
//
// For each case: an array of non-negative f32 terms; the plain loop
// s = fl_P(s + x_j) (P = 24: f32, P = 53: f64) gives every partial sum. The
// replay walks the same array in tiles of `tile` terms the way the device
// does: per tile, the composition of the term maps of the current segment,
// the first term whose partial sum leaves the segment (added with the IEEE
// addition instead), and the first term whose partial sum meets a monotone
// predicate. Both the final sums and the predicate indices must agree, bit for
// bit, for every threshold tried.
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
        const uint32_t par0 = (uint32_t)(g.n & 1);
        const uint64_t room = g.lim - g.n;
        // As on the device: a tile without an exact tie uses the plain
        // increments, a tile with one the parity-carrying maps.
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

static int failures = 0;

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
    run_all<24>(cases);
    run_all<53>(cases);
    if (failures) {
        printf("%d failures\n", failures);
        return 1;
    }
    printf("ok %d\n", cases);
    return 0;
}
