"""The reference's own sampler tests (crates/rust-llm/src/sample.rs:406-461,
crates/rust-llm/tests/sample.rs, crates/rust-llm/tests/sample_allocations.rs),
run against the GPU sampler through the host Sampler API, and checked both the
way the reference checks them and bit-for-bit against the oracle.
"""
import numpy as np
import pytest

import oracle as O
import rl_sampler as R
from conftest import as_oracle_settings

pytestmark = pytest.mark.gpu
S = R.sampling


def same_candidates(what, got, want):
    """tests/sample.rs:102-123: same surviving set, probabilities to 1e-5."""
    ids, probs = got
    wid, wp = want
    order = np.argsort(ids, kind="stable")
    worder = np.argsort(wid, kind="stable")
    assert np.array_equal(ids[order], wid[worder]), "%s: the surviving candidates differ" % what
    mine = probs[order].astype(np.float64)
    theirs = wp[worder]
    d = np.abs(mine - theirs)
    assert np.all(d <= 1e-5 * np.maximum(theirs, 1e-6)), "%s: probabilities differ by %g" % (what, d.max())


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


@pytest.mark.parametrize("what,set_", CASES, ids=[c[0] for c in CASES])
def test_the_pipeline_matches_a_naive_reference(device, what, set_):
    recent = [3, 11, 400, 11, 7, 1999, 0, 3]
    for seed in (1, 2, 3):
        for spread in (0.5, 4.0, 30.0):
            l = O.test_logits(2048, seed, spread)
            s = R.HostSampler(l.size, set_)
            o = O.OracleSampler(l.size, as_oracle_settings(set_))
            for t in recent:
                s.remember(t)
                o.remember(t)
            token = s.sample(l)
            label = "%s, logit seed %d, spread %s" % (what, seed, spread)
            want = O.naive(l, as_oracle_settings(set_), recent)
            got = s.candidates()
            same_candidates(label, got, want)
            assert token in set(want[0].tolist()), "%s: drew %d, not a candidate" % (label, token)
            # and bit-for-bit against the restated pipeline
            assert token == o.sample(l), label
            oi, op = o.candidates()
            assert np.array_equal(got[0], oi) and np.array_equal(got[1].view(np.uint32), op.view(np.uint32)), label
            assert s.rng_state() == o.rng_state(), label


def test_temperature_zero_is_argmax(device):  # tests/sample.rs:234-261
    for seed in (1, 9, 77):
        l = O.test_logits(4096, seed, 6.0)
        s = R.HostSampler.greedy(l.size)
        assert s.sample(l) == O.argmax(l), "logit seed %d" % seed
    ties = np.full(64, -1.0, np.float32)
    ties[7] = 5.0
    ties[40] = 5.0
    assert R.HostSampler.greedy(64).sample(ties) == 7
    dead = np.full(64, -np.inf, np.float32)
    assert R.HostSampler.greedy(64).sample(dead) == 0
    s = R.HostSampler(64, S(temperature=0.8))
    assert s.sample(dead) == 0, "a drawing sampler on all -inf"
    assert s.rng_state() == R.RngStream(0).state(), "no draw on a row with no finite maximum"


def test_argmax_takes_the_first_of_a_tie(device):  # sample.rs:410-415
    assert R.host_argmax(np.array([1.0, 3.0, 3.0, 2.0], np.float32)) == 1
    assert R.host_argmax(np.array([-5.0], np.float32)) == 0
    assert R.host_argmax(np.array([-np.inf, -np.inf], np.float32)) == 0


ORDER_BASE = dict(temperature=1.0, top_k=20, top_p=1.0, min_p=0.0, repeat_penalty=1.0, repeat_last_n=0, seed=1)


@pytest.mark.xfail(strict=True, reason=(
    "known deviation: with top_p >= 1 and 0 < top_k < vocab the reference leaves its candidates in the "
    "order Rust's select_nth_unstable_by produces (sample.rs:294); that order cannot be reproduced here "
    "(Rust's core library is not available), so the device returns them in descending order; same kept "
    "set and probabilities, but the draw walks another order"))
def test_with_top_p_off_the_candidates_are_not_sorted(device):  # tests/sample.rs:286-294
    l = O.test_logits(1024, 44, 3.0)
    off = R.HostSampler(l.size, S(**ORDER_BASE))
    off.sample(l)
    values = l[off.candidates()[0]]
    assert values.size == 20
    assert np.any(values[:-1] < values[1:]), "with top-p off the candidates came back in descending order"


def test_the_candidates_are_ordered_where_the_order_is_used(device):  # tests/sample.rs:272-312
    l = O.test_logits(1024, 44, 3.0)
    base = ORDER_BASE
    off = R.HostSampler(l.size, S(**base))
    off.sample(l)
    assert off.candidates()[0].size == 20
    on = R.HostSampler(l.size, S(**dict(base, top_p=0.999)))
    on.sample(l)
    ids, probs = on.candidates()
    values = l[ids]
    assert np.all(values[:-1] >= values[1:]), "top-p cut a prefix of an unordered candidate set"
    assert np.all(probs[:-1] >= probs[1:])


def test_a_penalty_of_one_changes_nothing(device):  # tests/sample.rs:316-329
    l = O.test_logits(1024, 5, 3.0)
    s = R.HostSampler(l.size, R.greedy_sampling(repeat_penalty=1.0, repeat_last_n=64))
    for t in range(64):
        s.remember(t)
    assert s.sample(l) == O.argmax(l)


def test_the_same_seed_gives_the_same_tokens(device):  # tests/sample.rs:331-348
    l = O.test_logits(4096, 12, 2.0)

    def run(seed):
        s = R.HostSampler(l.size, S(seed=seed))
        return [s.sample(l) for _ in range(32)]

    a = run(7)
    assert a == run(7), "the same seed gave a different sequence"
    assert a != run(8), "two seeds gave the same 32 tokens"
    o = O.OracleSampler(l.size, O.sampling(seed=7))
    assert a == [o.sample(l) for _ in range(32)], "the sequence differs from the oracle's"


def test_the_edges_of_every_parameter(device):  # tests/sample.rs:350-412
    l = O.test_logits(1024, 21, 3.0)
    base = dict(temperature=1.0, top_k=0, top_p=1.0, min_p=0.0, repeat_penalty=1.0, repeat_last_n=0, seed=99)
    top = O.argmax(l)
    edges = [
        ("top_k 1", dict(base, top_k=1), 1),
        ("top_k at the vocabulary", dict(base, top_k=l.size), l.size),
        ("top_k past the vocabulary", dict(base, top_k=l.size * 3), l.size),
        ("top_p 0", dict(base, top_p=0.0), 1),
        ("min_p 1", dict(base, min_p=1.0), 1),
    ]
    for what, kw, want in edges:
        s = R.HostSampler(l.size, S(**kw))
        token = s.sample(l)
        ids, probs = s.candidates()
        assert ids.size == want, "%s: kept %d candidates" % (what, ids.size)
        same_candidates(what, (ids, probs), O.naive(l, O.sampling(**kw)))
        if want == 1:
            assert token == top, "%s: a single candidate has to be the argmax" % what
            assert probs[0] == 1.0, "%s: a single candidate carries all the mass" % what
    for what, kw in (("top_p 1", dict(base, top_p=1.0)), ("min_p 0", dict(base, min_p=0.0))):
        s = R.HostSampler(l.size, S(**kw))
        s.sample(l)
        assert s.candidates()[0].size == l.size, "%s cut something" % what


def test_the_repetition_penalty_moves_both_signs_towards_zero(device):  # tests/sample.rs:416-460
    l = np.array([2.0, -2.0, 1.0, -1.0, 0.0], np.float32)
    s = R.HostSampler(l.size, S(1.0, 0, 1.0, 0.0, 2.0, 4, 1))
    for t in (0, 1):
        s.remember(t)
    s.sample(l)
    ids, probs = s.candidates()
    p = dict(zip(ids.tolist(), probs.tolist()))
    assert abs(p[0] - p[2]) < 1e-6, "a penalised +2 should land on an untouched +1"
    assert p[1] < p[3], "a penalised -2 should sit below an untouched -1"
    for a, b in ((2, 4), (4, 3)):
        assert abs(p[a] / p[b] - np.exp(np.float32(1.0))) < 1e-5


def test_the_window_keeps_the_most_recent_tokens(device):  # sample.rs:439-460
    s = R.HostSampler(5, R.greedy_sampling(repeat_penalty=2.0, repeat_last_n=3))
    for t in (0, 1, 2, 3):
        s.remember(t)
    logits = np.array([1.0, 0.0, 0.0, 1.5, 0.0], np.float32)
    assert s.sample(logits) == 0
    s.reset()
    assert s.sample(logits) == 3


def test_the_draw_follows_the_reported_probabilities(device):  # tests/sample.rs:462-504
    import torch
    l = O.test_logits(512, 31, 1.0)
    set_ = S(1.0, 8, 1.0, 0.0, 1.0, 0, 4)
    s = R.HostSampler(l.size, set_)
    s.sample(l)
    want = dict(zip(*[a.tolist() for a in s.candidates()]))
    # 50 000 draws in one batched call: the same row, one uniform each from the
    # stream the sampler would walk (every row draws).
    draws = 50_000
    rng = R.RngStream(4)
    rng.next_f32()  # the first call above consumed one
    uniforms = np.array([rng.next_f32() for _ in range(draws)], np.float32)
    ctx = R.DeviceSampler(draws, l.size, max_window=1)
    rows = torch.from_numpy(np.tile(l, (draws, 1))).to(device)
    res = R.sample_batch(ctx, rows, [set_] * draws, uniforms=torch.from_numpy(uniforms).to(device),
                         with_candidates=False)
    counts = np.bincount(res.token, minlength=l.size)
    for id_, p in want.items():
        got = counts[id_] / draws
        se = np.sqrt(p * (1 - p) / draws)
        assert abs(got - p) < 4 * se + 0.003, "token %d drawn %.4f, reported %.4f" % (id_, got, p)
    assert set(np.nonzero(counts)[0].tolist()) <= set(want), "drew a token that is not a candidate"
    # and the same 50 000 picks as the oracle walking its own Sampler
    o = O.OracleSampler(l.size, as_oracle_settings(set_))
    o.sample(l)
    seq = np.array([o.sample(l) for _ in range(2000)], np.uint32)
    assert np.array_equal(seq, res.token[:2000])


def test_sampling_allocates_nothing_per_token(device):  # tests/sample_allocations.rs:75-136
    import torch
    vocab = 248_320
    l = O.alloc_test_logits(vocab, 3)
    dl = torch.from_numpy(l).to(device)
    cases = [
        ("greedy", R.greedy_sampling()),
        ("the defaults", S()),
        ("top-k off", S(1.0, 0, 0.9, 0.05, 1.2, 64, 1)),
        ("every stage on", S(0.8, 40, 0.9, 0.05, 1.1, 64, 2)),
    ]
    for what, set_ in cases:
        s = R.HostSampler(vocab, set_)
        for t in range(set_.repeat_last_n):
            s.remember(t // 2)
        for _ in range(2):
            s.sample(dl)
        torch.cuda.synchronize()
        free0 = torch.cuda.mem_get_info()[0]
        for _ in range(8):
            s.sample(dl)
        torch.cuda.synchronize()
        free1 = torch.cuda.mem_get_info()[0]
        assert free1 == free0, "%s: device memory changed by %d bytes over 8 calls" % (what, free0 - free1)
