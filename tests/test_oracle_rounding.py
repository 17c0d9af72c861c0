"""Pins of the oracle's sequential arithmetic (sample.rs:307-358), on the CPU.

The naive f64 reference of the reference's tests pins the kept sets only to
1e-5; the exact bits of the mass, the top-p cut, the normalising total, the
f32 normalisation and the f32 draw are pinned here. Each case is checked
against a step-by-step walk of the reference's text written with explicit
precisions (Python floats for the f64 sums, numpy float32 for the f32 steps,
libm expf for `.exp()`), and each case is built so that one plausible mistake
in that arithmetic changes the outcome: a variant of the walk with the mistake
planted is shown to disagree with the oracle on it.

The mistakes: an f32 mass accumulator (sum and cut), `cum > target` for
`cum >= target` in the cut, `cum >= u` for `cum > u` in the draw, the
normalising factor kept in f64 instead of `(1/total) as f32`, and an f32
normalising total.
"""
import numpy as np
import pytest

import oracle as O

f32 = np.float32


def walk(logits, temperature, top_k, top_p, min_p, u, *, mass32=False, cut_gt=False, draw_ge=False,
         inv64=False, total32=False):
    """Sampler::pick for one row with no penalty, step by step as the
    reference's text reads (sample.rs:267-358); keyword flags plant one
    mistake each. Returns (token, kept ids, kept probabilities)."""
    l = np.asarray(logits, np.float32)
    n = l.size
    mx = f32(np.nanmax(l))
    assert np.isfinite(mx) and not np.isnan(l).any()
    # Descending value, ascending id on ties (sample.rs:282-286): for finite
    # values without NaN the total order is the numeric one.
    order = sorted(range(n), key=lambda i: (-float(l[i]), i))
    k = n if top_k == 0 else min(top_k, n)
    assert top_p < 1.0 or k == n, "the select_nth order is not restated here"
    cand = order[:k] if top_p < 1.0 else list(range(n))
    T = f32(temperature)
    probs = [f32(O.libm_expf(f32(f32(l[i] - mx) / T))) for i in cand]
    total_mass = f32(0) if mass32 else 0.0
    for p in probs:
        total_mass = f32(total_mass + p) if mass32 else total_mass + float(p)
    m = k
    if top_p < 1.0:
        target = f32(f32(top_p) * total_mass) if mass32 else float(f32(top_p)) * total_mass
        cum = f32(0) if mass32 else 0.0
        for j, p in enumerate(probs):
            cum = f32(cum + p) if mass32 else cum + float(p)
            if (cum > target) if cut_gt else (cum >= target):
                m = j + 1
                break
    if min_p > 0.0:
        keep = [(c, p) for c, p in zip(cand[:m], probs[:m]) if p >= f32(min_p)]
        if keep:
            cand = [c for c, _ in keep] + cand[m:]
            probs = [p for _, p in keep] + probs[m:]
        m = max(len(keep), 1)
    total = f32(0) if total32 else 0.0
    for p in probs[:m]:
        total = f32(total + p) if total32 else total + float(p)
    if inv64:
        q = [f32(float(p) * (1.0 / float(total))) for p in probs[:m]]
    else:
        inv = f32(1.0 / float(total))
        q = [f32(p * inv) for p in probs[:m]]
    cum = f32(0)
    token = cand[m - 1]
    for j, p in enumerate(q):
        cum = f32(cum + p)
        if (cum >= u) if draw_ge else (cum > u):
            token = cand[j]
            break
    return token, np.array(cand[:m], np.uint32), np.array(q, np.float32)


def oracle_pick(logits, temperature, top_k, top_p, min_p, u):
    s = O.sampling(temperature=temperature, top_k=top_k, top_p=top_p, min_p=min_p, repeat_penalty=1.0,
                   repeat_last_n=0, seed=0)
    r = O.pick_rows(np.asarray(logits, np.float32), s, uniforms=np.array([u], np.float32))
    k = int(r["kept"][0])
    return int(r["token"][0]), r["ids"][0, :k].copy(), r["probs"][0, :k].copy()


def same(a, b):
    return a[0] == b[0] and np.array_equal(a[1], b[1]) and np.array_equal(a[2].view(np.uint32),
                                                                           b[2].view(np.uint32))


def check(case, mistake):
    """The oracle equals the text; the planted mistake does not."""
    want = walk(*case)
    got = oracle_pick(*case)
    assert same(got, want), "oracle %s != text %s" % (got, want)
    planted = walk(*case, **{mistake: True})
    assert not same(planted, want), "the case does not tell %s apart" % mistake
    return want, planted


def test_the_top_p_cut_is_cum_at_or_above_the_target():
    # Eight tied maxima: every p is exp(0) = 1, the mass is 8 and the target
    # 0.5 * 8 = 4 is reached exactly at the fourth candidate.
    case = (np.ones(8, np.float32), 1.0, 0, 0.5, 0.0, f32(0.99))
    want, planted = check(case, "cut_gt")
    assert len(want[1]) == 4 and len(planted[1]) == 5


def test_the_draw_is_the_first_cum_above_the_uniform():
    # Four tied candidates, each normalised to exactly 0.25: the running sum
    # meets u = 0.5 exactly at the second, and `>` walks on to the third.
    case = (np.array([3.0, 3.0, 3.0, 3.0, -50.0], np.float32), 1.0, 0, 0.9, 0.0, f32(0.5))
    want, planted = check(case, "draw_ge")
    assert want[0] == 2 and planted[0] == 1


def f64_and_f32_prefix_sums(probs):
    c64, c32 = [], []
    a, b = 0.0, f32(0)
    for p in probs:
        a += float(p)
        b = f32(b + p)
        c64.append(a)
        c32.append(float(b))
    return np.array(c64), np.array(c32)


def test_the_mass_and_the_cut_are_summed_in_f64():
    # A hot row of 4000 candidates: f32 running sums drift from the f64 ones.
    # top_p is chosen so that the f64 target falls strictly between the f64
    # and the f32 partial sums at the step where they differ most, so an f32
    # accumulator cuts at another index.
    l = O.test_logits(4000, 17, 3.0)
    T = 4.0
    mx = f32(l.max())
    order = sorted(range(l.size), key=lambda i: (-float(l[i]), i))
    probs = [f32(O.libm_expf(f32(f32(l[i] - mx) / f32(T)))) for i in order]
    c64, c32 = f64_and_f32_prefix_sums(probs)
    mass64 = c64[-1]
    found = None
    for j in np.argsort(-np.abs(c64 - c32))[:200]:
        lo, hi = sorted((c64[j], c32[j]))
        for cand_p in (f32((lo + hi) / 2 / mass64), np.nextafter(f32(lo / mass64), f32(1)),
                       np.nextafter(f32(hi / mass64), f32(0))):
            t = float(f32(cand_p)) * mass64
            if lo < t < hi and 0 < float(cand_p) < 1:
                found = float(cand_p)
                break
        if found is not None:
            break
    assert found is not None, "no f32 top_p separates the f64 and f32 partial sums"
    case = (l, T, 0, found, 0.0, f32(0.4))
    want, planted = check(case, "mass32")
    assert len(want[1]) != len(planted[1])


@pytest.mark.parametrize("mistake", ["inv64", "total32"])
def test_the_normalisation_is_f32_times_the_f32_reciprocal_of_an_f64_total(mistake):
    # Rows with many kept candidates: the planted normalisation changes at
    # least one probability's bits on some row.
    told = False
    for seed in range(1, 30):
        l = O.test_logits(1500, seed, 2.5)
        case = (l, 1.7, 0, 0.97, 0.0, f32(0.3))
        want = walk(*case)
        got = oracle_pick(*case)
        assert same(got, want), "seed %d: oracle != text" % seed
        if not same(walk(*case, **{mistake: True}), want):
            told = True
    assert told, "no row tells %s apart" % mistake


def test_min_p_compacts_in_place_before_the_total():
    # min-p with top-p: survivors keep their order, the total is over them only.
    for seed in (3, 4, 5):
        l = O.test_logits(3000, seed, 4.0)
        case = (l, 0.9, 0, 0.95, 0.05, f32(0.61))
        assert same(oracle_pick(*case), walk(*case)), seed
    # min-p without top-p keeps id order (no sort, sample.rs:303).
    l = O.test_logits(600, 8, 3.0)
    case = (l, 1.0, 0, 1.0, 0.2, f32(0.5))
    tok, ids, probs = oracle_pick(*case)
    assert np.all(np.diff(ids.astype(np.int64)) > 0)
    assert same((tok, ids, probs), walk(*case))


def test_random_rows_follow_the_text_bit_for_bit():
    g = np.random.default_rng(11)
    for i in range(40):
        n = int(g.integers(2, 3000))
        l = O.test_logits(n, 100 + i, float(g.choice([0.5, 3.0, 20.0])))
        T = float(g.choice([0.3, 0.6, 1.0, 2.0]))
        top_p = float(g.choice([0.0, 0.5, 0.9, 0.95, 0.999]))
        min_p = float(g.choice([0.0, 0.0, 0.02, 0.3]))
        u = f32(g.random())
        case = (l, T, 0, top_p, min_p, u)
        assert same(oracle_pick(*case), walk(*case)), (i, n, T, top_p, min_p, u)
