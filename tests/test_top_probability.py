"""top_probability (crates/rust-llm/src/forward.rs:1671-1680): the oracle
pinned on the CPU, and the device's rl_top_probability_rows against it.

The reference returns the argmax (IEEE '>' from -inf, lowest id on a tie) and
(1 / sum) as f32, where sum is the f64 sum, in id order, of exp(v - best)
(f32 subtraction, libm expf). The pins: results fixed by the mathematics
(n equal logits give 1/n; one finite logit among -inf gives 1; two logits a, b
give 1 / (1 + e^(b-a)) in exact f64 terms), the NaN cases of the reference's
arithmetic, a sum long enough that f32 accumulation would be visibly wrong,
and a step-by-step recomputation (Python float additions of libm expf
values) on random rows. The device's certificate (an interval around its own
f64 sum that holds the sequential sum) is pinned against exact sums (fsum):
its bound on the sequential sum's error holds on rows built so that every
addition rounds the same way, and on random rows.
"""
import math

import numpy as np
import pytest

import oracle as O
import rl_sampler as R

INF = float("inf")
NAN = float("nan")


def f32(x):
    return np.float32(x)


def test_equal_logits_give_one_over_n():
    for n, v in ((1, 0.0), (2, 3.5), (7, -2.0), (1000, 1.25), (151936, -0.5)):
        tok, p = O.top_probability(np.full(n, v, np.float32))
        assert tok == 0
        assert p == f32(1.0 / n), (n, p)


def test_sum_is_accumulated_in_f64():
    # 2^24 + 2 equal terms: an f32 running sum would stop at 2^24.
    n = (1 << 24) + 2
    tok, p = O.top_probability(np.zeros(n, np.float32))
    assert p == f32(1.0 / n) and p != f32(1.0 / (1 << 24))


def test_one_finite_logit_among_minus_infinity():
    x = np.full(1000, -np.inf, np.float32)
    x[417] = 3.0
    assert O.top_probability(x) == (417, f32(1.0))


def test_two_logits_closed_form():
    rng = np.random.default_rng(2)
    for _ in range(200):
        a, b = rng.normal(0, 4, 2).astype(np.float32)
        tok, p = O.top_probability(np.array([a, b], np.float32))
        hi, lo = (a, b) if a >= b else (b, a)
        assert tok == (0 if a >= b else 1)
        other = float(O.libm_expf(f32(lo - hi)))
        first_then_second = (1.0 + other) if tok == 0 else (other + 1.0)
        assert p == f32(1.0 / first_then_second)


def test_ties_take_the_first_and_nan_never_wins():
    assert O.top_probability(np.array([1, 3, 3, 2], np.float32))[0] == 1
    assert O.top_probability(np.array([np.nan, 1.0], np.float32))[0] == 1
    assert O.top_probability(np.array([-0.0, 0.0], np.float32)) == (0, f32(0.5))


@pytest.mark.parametrize("row, tok", [
    ([-INF, -INF, -INF], 0),   # best stays -inf: -inf - -inf is NaN
    ([NAN, NAN], 0),           # nothing beats -inf
    ([1.0, NAN, 2.0], 2),      # a NaN term
    ([1.0, INF, 2.0, INF], 1),  # +inf - +inf is NaN
])
def test_nan_cases(row, tok):
    t, p = O.top_probability(np.array(row, np.float32))
    assert t == tok and np.isnan(p)


def test_step_by_step_recomputation():
    rng = np.random.default_rng(5)
    for n, scale in ((1, 1.0), (17, 3.0), (1000, 2.0), (5000, 10.0), (3000, 0.01)):
        x = rng.normal(0, scale, n).astype(np.float32)
        best, bv = 0, -math.inf
        for i, v in enumerate(x):
            if v > bv:
                best, bv = i, v
        s = -0.0
        for v in x:
            s += float(O.libm_expf(f32(f32(v) - f32(bv))))
        assert O.top_probability(x) == (best, f32(1.0 / s)), n


def seq_error_bound(terms):
    """The device certificate's bound on the sequential sum's distance from the
    exact sum (rust-llm_amd/csrc/top_probability.h): terms <= 1 with one term
    exactly 1, E the binade of the sum, (small + 200) * 2^(E-53), small the
    nonzero terms below 2^-26; None for E > 3."""
    t = np.asarray(terms, np.float32)
    S = math.fsum(t.astype(np.float64)) * (1.0 + 1e-12)
    E = math.frexp(S)[1] - 1
    if E > 3:
        return None
    small = int(np.count_nonzero((t > 0) & (t < 2.0 ** -26)))
    return (small + 200) * 2.0 ** (E - 53)


def test_sequential_sum_error_bound_holds_where_the_rounding_errors_add_up():
    # 1 followed by k halves of the f64 grid at 1: every addition is an exact
    # tie and rounds to the even significand, 1.0, so the error grows by
    # 2^-53 a step; the same with the grid at 2, 4 and 8. A bound that
    # counted too few terms (a threshold too low, a wrong binade) fails here.
    # The terms (1 + 2^-23) * 2^(E-30), just below 2^(E-29), also tie at
    # every step (their lowest bit is half the grid): the largest terms that
    # can round.
    for E, lead in ((0, [1.0]), (1, [1.0, 1.0]), (2, [1.0] * 4), (3, [1.0] * 8)):
        for k, x in ((300, 2.0 ** (E - 53)), (5000, 2.0 ** (E - 53)), (40000, 2.0 ** (E - 53)),
                     (3000, (1.0 + 2.0 ** -23) * 2.0 ** (E - 30))):
            terms = np.array(lead + [x] * k, np.float32)
            seq = 0.0
            for x in terms:
                seq += float(x)
            exact = math.fsum(terms.astype(np.float64))
            err = abs(seq - exact) + math.ulp(exact)
            assert err >= k * 2.0 ** (E - 53) * 0.99, (E, k)  # the errors do add up
            assert err <= seq_error_bound(terms), (E, k)


def test_sequential_sum_error_bound_on_random_rows():
    g = np.random.default_rng(31)
    for rep in range(60):
        n = int(g.integers(1000, 30000))
        kind = rep % 4
        if kind == 0:
            x = np.exp(-np.abs(g.standard_normal(n) * 12.0)).astype(np.float32)   # peaked
        elif kind == 1:
            x = np.exp(-g.uniform(0.0, 60.0, n)).astype(np.float32)                # many tiny terms
        elif kind == 2:
            x = (g.uniform(0.5, 1.0, n) * 2.0 ** g.integers(-40, -20, n)).astype(np.float32)
        else:
            x = np.where(g.random(n) < 0.5, 0.0, np.exp(-g.uniform(20.0, 40.0, n))).astype(np.float32)
        x[int(g.integers(0, n))] = 1.0
        bound = seq_error_bound(x)
        if bound is None:
            continue
        seq = float(np.cumsum(x.astype(np.float64))[-1])
        exact = math.fsum(x.astype(np.float64))
        assert abs(seq - exact) + math.ulp(exact) <= bound, rep


# ------------------------------------------------------------------ GPU --
def gpu_top_probability(device, x):
    import torch
    rows, V = x.shape
    ctx = R.DeviceSampler(rows, V, max_window=0)
    tok = torch.empty(rows, dtype=torch.int32, device=device)
    prob = torch.empty(rows, dtype=torch.float32, device=device)
    ctx.top_probability_rows(torch.from_numpy(np.ascontiguousarray(x)).to(device), rows, V, tok, prob)
    torch.cuda.synchronize()
    return tok.cpu().numpy().view(np.uint32), prob.cpu().numpy()


def assert_same(got, want, label):
    gt, gp = got
    wt, wp = want
    assert np.array_equal(gt, wt), "%s: tokens differ at %s" % (label, np.nonzero(gt != wt)[0][:8])
    both_nan = np.isnan(gp) & np.isnan(wp)
    bad = np.nonzero((gp.view(np.uint32) != wp.view(np.uint32)) & ~both_nan)[0]
    assert bad.size == 0, "%s: probabilities differ at rows %s: %s vs %s" % (label, bad[:8], gp[bad[:8]],
                                                                              wp[bad[:8]])


@pytest.mark.gpu
@pytest.mark.parametrize("rows, V, scale", [(1, 248320, 2.0), (9, 151936, 2.5), (64, 4099, 5.0), (300, 1000, 1.0),
                                            (1100, 257, 3.0), (4, 3, 1.0), (290, 248320, 2.0)])
def test_rows_match_the_oracle(device, rows, V, scale):
    rng = np.random.default_rng(rows * 7 + V)
    x = rng.normal(0, scale, (rows, V)).astype(np.float32)
    x[0, rng.integers(0, V)] = 9.0
    assert_same(gpu_top_probability(device, x), O.top_probability_rows(x), "V=%d" % V)


@pytest.mark.gpu
@pytest.mark.parametrize("V", [5000, 151936])
def test_special_rows(device, V):
    # At 5000 a row is one chunk; at 151936 it is split, and a NaN row is
    # written by its first chunk while the others finish through the last.
    rng = np.random.default_rng(3)
    x = rng.normal(0, 1, (10, V)).astype(np.float32)
    x[0, :] = -np.inf
    x[1, :] = np.nan
    x[2, 77] = np.nan
    x[3, 5] = np.inf
    x[4, :] = 2.0                      # all equal: 1/V
    x[5, :] = -np.inf
    x[5, 4321] = 0.5                   # a single finite value: 1
    x[6, ::2] = -0.0
    x[6, 1::2] = 0.0
    x[7, :] = 1e-30
    x[7, 9] = 3.4e38                   # terms underflow to 0: exactly 1
    x[8, :] = rng.choice(np.array([0.0, -1.0, -2.0], np.float32), V)
    assert_same(gpu_top_probability(device, x), O.top_probability_rows(x), "special rows")


@pytest.mark.gpu
def test_rows_whose_probability_sits_on_an_f32_rounding_boundary(device):
    # Sums 1 + x + ... + x whose reciprocal lies within 1e-11 (relative) of a midpoint
    # between two f32 values: the certificate cannot decide them, so the
    # device replays the sequential sum; the result must still be exact.
    V = 60000
    rows = []
    for x_logit in (-0.75, -1.5, -3.0, -0.3):
        x = float(O.libm_expf(f32(x_logit)))
        s = 1.0  # the reference's sequential sum: 1, then k terms x
        for k in range(1, V):
            s += x
            r = 1.0 / s
            lo = np.float32(r)
            nb = np.nextafter(lo, np.float32(np.inf if np.float64(lo) < r else -np.inf))
            mid = (np.float64(lo) + np.float64(nb)) / 2.0
            if abs(r - mid) < 1e-11 * r:
                row = np.full(V, -np.inf, np.float32)
                row[0] = 0.0
                row[1:k + 1] = x_logit
                rows.append(row)
                break
    assert len(rows) >= 2, "no boundary case found"
    x = np.stack(rows)
    assert_same(gpu_top_probability(device, x), O.top_probability_rows(x), "boundary rows")
