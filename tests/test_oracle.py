"""Pins the oracle (the C restatement of crates/rust-llm/src/sample.rs) before
anything is compared against it: published RNG vectors, the reference's own
known-answer tests, and independent checks that a plausible mistake (a
dropped term, a wrong index or sign, a reversed order) would fail."""
import math
import struct

import numpy as np
import pytest

import oracle as O

S = O.sampling


# ------------------------------------------------------------------ Rng ---
def test_splitmix64_published_vectors():
    # SplitMix64 (Steele, Lea, Flood 2014), the seeding of sample.rs:373-385.
    assert O.splitmix64_stream(0, 4) == [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4,
                                         0x06C45D188009454F, 0xF88BB8A8724C81EC]
    assert O.splitmix64_stream(1234567, 5) == [6457827717110365317, 3203168211198807973, 9817491932198370423,
                                               4593380528125082431, 16408922859458223821]


def test_xoshiro256pp_published_vector():
    # The reference implementation's sequence from the state {1, 2, 3, 4}
    # (sample.rs:387-398 restates the same step).
    r = O.OracleRng(state=(1, 2, 3, 4))
    assert [r.next_u64() for _ in range(10)] == [
        41943041, 58720359, 3588806011781223, 3591011842654386, 9228616714210784205,
        9973669472204895162, 14011001112246962877, 12406186145184390807, 15849039046786891736,
        10450023813501588000]


def test_seeding_is_splitmix_into_the_state():
    r = O.OracleRng(0)
    assert r.state() == tuple(O.splitmix64_stream(0, 4))


def test_next_f32_is_the_top_24_bits():  # sample.rs:401-403
    a, b = O.OracleRng(99), O.OracleRng(99)
    for _ in range(1000):
        u = a.next_u64()
        f = b.next_f32()
        assert f * (1 << 24) == (u >> 40)
        assert 0.0 <= f < 1.0


def test_the_generator_stays_in_the_unit_interval_and_covers_it():  # sample.rs:417-429
    r = O.OracleRng(7)
    buckets = [0] * 8
    for _ in range(80_000):
        v = r.next_f32()
        assert 0.0 <= v < 1.0
        buckets[int(v * 8.0)] += 1
    assert all(n > 8_000 for n in buckets), buckets


def test_the_same_seed_gives_the_same_stream():  # sample.rs:431-437
    one = [O.OracleRng(42).next_u64() for _ in range(8)]
    again = [O.OracleRng(42).next_u64() for _ in range(8)]
    assert one == again
    assert one[0] != O.OracleRng(43).next_u64()


# --------------------------------------------------------------- argmax ---
def py_argmax(values):
    """Textbook first-strict-maximum scan from -inf (NaN never compares)."""
    best, best_v = 0, -math.inf
    for i, v in enumerate(values):
        if v > best_v:
            best, best_v = i, v
    return best


def test_argmax_known_answers():  # sample.rs:410-415, tests/sample.rs:244-252
    assert O.argmax([1.0, 3.0, 3.0, 2.0]) == 1
    assert O.argmax([-5.0]) == 0
    assert O.argmax([-np.inf, -np.inf]) == 0
    ties = np.full(64, -1.0, np.float32)
    ties[7] = ties[40] = 5.0
    assert O.argmax(ties) == 7
    assert O.argmax(np.full(64, -np.inf, np.float32)) == 0


def test_argmax_against_brute_force_with_special_values():
    rng = np.random.default_rng(5)
    specials = np.array([np.nan, -np.nan, np.inf, -np.inf, 0.0, -0.0], np.float32)
    for trial in range(300):
        n = int(rng.integers(1, 40))
        x = rng.choice(np.array([-1.0, 0.0, 1.0, 2.0], np.float32), n)
        mask = rng.random(n) < 0.3
        x[mask] = rng.choice(specials, int(mask.sum()))
        assert O.argmax(x) == py_argmax(x.tolist()), x


# ------------------------------------------------------- total order ---
def total_key(v):
    """f32::total_cmp's key, from the IEEE bit pattern (independent of the C)."""
    b = struct.unpack("<i", struct.pack("<f", v))[0]
    return b ^ ((b >> 31) & 0x7FFFFFFF)


def test_selection_and_order_against_brute_force():
    """Kept set and order of every top-k (top_p < 1 needs the order): a sort by
    (total order descending, id ascending) written independently."""
    rng = np.random.default_rng(11)
    for trial in range(200):
        n = int(rng.integers(2, 60))
        # few distinct values so ties are everywhere; a few specials
        x = rng.choice(np.array([-2.0, -0.0, 0.0, 1.0, 1.5, 3.0], np.float32), n)
        k = int(rng.integers(1, n + 1))
        # p = 0.9999 keeps (almost) everything but requires the sorted order
        set_ = S(1.0, k, 0.9999, 0.0, 1.0, 0, 1)
        res = O.pick_rows(x, set_, uniforms=[0.5])
        kept = int(res["kept"][0])
        order = sorted(range(n), key=lambda i: (-total_key(float(x[i])), i))[:k]
        assert res["ids"][0, :kept].tolist() == order[:kept], (x, k)


# ----------------------------------------------------- the pipeline ---
CASES = [  # tests/sample.rs:129-209
    ("temperature only", S(0.7, 0, 1.0, 0.0, 1.0, 0, 1)),
    ("a cold temperature", S(0.05, 0, 1.0)),
    ("a hot temperature", S(4.0, 0, 1.0)),
    ("top-k only", S(1.0, 17, 1.0, 0.0, 1.0, 0, 2)),
    ("top-p only", S(1.0, 0, 0.6, 0.0, 1.0, 0, 3)),
    ("min-p only", S(1.0, 0, 1.0, 0.3, 1.0, 0, 4)),
    ("the defaults", S()),
    ("everything at once", S(0.8, 40, 0.9, 0.02, 1.3, 16, 5)),
]


def same_candidates(what, ids, probs, wid, wp):
    """tests/sample.rs:102-123."""
    a, b = np.argsort(ids, kind="stable"), np.argsort(wid, kind="stable")
    assert np.array_equal(ids[a], wid[b]), what
    d = np.abs(probs[a].astype(np.float64) - wp[b])
    assert np.all(d <= 1e-5 * np.maximum(wp[b], 1e-6)), (what, d.max())


@pytest.mark.parametrize("what,set_", CASES, ids=[c[0] for c in CASES])
def test_the_pipeline_matches_a_naive_reference(what, set_):
    recent = [3, 11, 400, 11, 7, 1999, 0, 3]
    for seed in (1, 2, 3):
        for spread in (0.5, 4.0, 30.0):
            l = O.test_logits(2048, seed, spread)
            s = O.OracleSampler(l.size, set_)
            for t in recent:
                s.remember(t)
            token = s.sample(l)
            ids, probs = s.candidates()
            wid, wp = O.naive(l, set_, recent)
            label = "%s, logit seed %d, spread %s" % (what, seed, spread)
            same_candidates(label, ids, probs, wid, wp)
            assert token in set(wid.tolist()), label
            # the kept probabilities are normalised
            assert abs(float(np.sum(probs.astype(np.float64))) - 1.0) < 1e-5, label


def test_the_window_keeps_the_most_recent_tokens():  # sample.rs:439-460
    s = O.OracleSampler(5, S(0.0, 0, 1.0, 0.0, 2.0, 3, 0))
    for t in (0, 1, 2, 3):
        s.remember(t)
    logits = np.array([1.0, 0.0, 0.0, 1.5, 0.0], np.float32)
    assert s.sample(logits) == 0
    s.reset()
    assert s.sample(logits) == 3


def test_temperature_zero_is_argmax():  # tests/sample.rs:234-261
    for seed in (1, 9, 77):
        l = O.test_logits(4096, seed, 6.0)
        assert O.OracleSampler(l.size, O.Sampling(**O.GREEDY)).sample(l) == O.argmax(l)
    dead = np.full(64, -np.inf, np.float32)
    s = O.OracleSampler(64, S(temperature=0.8))
    assert s.sample(dead) == 0
    assert s.rng_state() == O.OracleRng(0).state(), "a row with no finite maximum draws nothing"


def test_a_penalty_of_one_changes_nothing():  # tests/sample.rs:316-329
    l = O.test_logits(1024, 5, 3.0)
    s = O.OracleSampler(l.size, S(0.0, 0, 1.0, 0.0, 1.0, 64, 0))
    for t in range(64):
        s.remember(t)
    assert s.sample(l) == O.argmax(l)


def test_the_same_seed_gives_the_same_tokens():  # tests/sample.rs:331-348
    l = O.test_logits(4096, 12, 2.0)

    def run(seed):
        s = O.OracleSampler(l.size, S(seed=seed))
        return [s.sample(l) for _ in range(32)]

    a = run(7)
    assert a == run(7)
    assert a != run(8)


def test_the_edges_of_every_parameter():  # tests/sample.rs:350-412
    l = O.test_logits(1024, 21, 3.0)
    base = dict(temperature=1.0, top_k=0, top_p=1.0, min_p=0.0, repeat_penalty=1.0, repeat_last_n=0, seed=99)
    top = O.argmax(l)
    for what, kw, want in [
        ("top_k 1", dict(base, top_k=1), 1),
        ("top_k at the vocabulary", dict(base, top_k=l.size), l.size),
        ("top_k past the vocabulary", dict(base, top_k=l.size * 3), l.size),
        ("top_p 0", dict(base, top_p=0.0), 1),
        ("min_p 1", dict(base, min_p=1.0), 1),
    ]:
        s = O.OracleSampler(l.size, S(**kw))
        token = s.sample(l)
        ids, probs = s.candidates()
        assert ids.size == want, what
        wid, wp = O.naive(l, S(**kw))
        same_candidates(what, ids, probs, wid, wp)
        if want == 1:
            assert token == top and probs[0] == 1.0, what
    for kw in (dict(base, top_p=1.0), dict(base, min_p=0.0)):
        s = O.OracleSampler(l.size, S(**kw))
        s.sample(l)
        ids, _ = s.candidates()
        assert ids.size == l.size
        # no truncation and no order needed: the identity order (sample.rs:290-292)
        assert np.array_equal(ids, np.arange(l.size, dtype=np.uint32))


def test_the_repetition_penalty_moves_both_signs_towards_zero():  # tests/sample.rs:416-460
    l = np.array([2.0, -2.0, 1.0, -1.0, 0.0], np.float32)
    s = O.OracleSampler(l.size, S(1.0, 0, 1.0, 0.0, 2.0, 4, 1))
    for t in (0, 1):
        s.remember(t)
    s.sample(l)
    p = dict(zip(*[a.tolist() for a in s.candidates()]))
    assert abs(p[0] - p[2]) < 1e-6
    assert p[1] < p[3]
    for a, b in ((2, 4), (4, 3)):
        assert abs(p[a] / p[b] - math.exp(1.0)) < 1e-5


def test_the_draw_follows_the_reported_probabilities():  # tests/sample.rs:462-504
    l = O.test_logits(512, 31, 1.0)
    s = O.OracleSampler(l.size, S(1.0, 8, 1.0, 0.0, 1.0, 0, 4))
    s.sample(l)
    want = dict(zip(*[a.tolist() for a in s.candidates()]))
    draws = 50_000
    counts = {}
    for _ in range(draws):
        t = s.sample(l)
        counts[t] = counts.get(t, 0) + 1
    for id_, p in want.items():
        got = counts.get(id_, 0) / draws
        assert abs(got - p) < 4 * math.sqrt(p * (1 - p) / draws) + 0.003
    assert set(counts) <= set(want)


def test_the_largest_unnormalised_probability_is_exactly_one():
    """min-p's threshold is min_p itself because exp(0) == 1 (sample.rs:326-328):
    with min_p = 1 only candidates whose logit equals the maximum survive."""
    l = np.array([0.5, 2.0, 2.0, 1.999999, -1.0], np.float32)
    res = O.pick_rows(l, S(1.0, 0, 1.0, 1.0, 1.0, 0, 0), uniforms=[0.75])
    assert sorted(res["ids"][0, :res["kept"][0]].tolist()) == [1, 2]
    assert res["probs"][0, 0] == np.float32(0.5) and res["probs"][0, 1] == np.float32(0.5)


def test_a_window_id_past_the_vocabulary_is_ignored():  # sample.rs:248
    l = np.array([1.0, 0.5, 0.25], np.float32)
    res = O.pick_rows(l, S(0.0, 0, 1.0, 0.0, 4.0, 2, 0), windows=np.array([[7, 0]], np.uint32), wlen=[2])
    assert res["token"][0] == 1  # 1.0 / 4 = 0.25 < 0.5
    res = O.pick_rows(l, S(0.0, 0, 1.0, 0.0, 4.0, 2, 0), windows=np.array([[7, 9]], np.uint32), wlen=[2])
    assert res["token"][0] == 0


def test_the_draw_stops_at_the_first_cumulative_sum_above_u():  # sample.rs:349-358
    l = np.log(np.array([0.5, 0.3, 0.2], np.float32)).astype(np.float32)
    set_ = S(1.0, 0, 0.9999, 0.0, 1.0, 0, 0)
    res = O.pick_rows(np.tile(l, (4, 1)), set_, uniforms=np.array([0.0, 0.49, 0.51, 0.99999994], np.float32))
    assert res["token"].tolist()[:3] == [0, 0, 1]
    q = res["probs"][0, :3]
    # every uniform below the f32 running sum picks within the list
    assert res["token"][3] in (1, 2)
    assert q[0] > q[1] > q[2]
