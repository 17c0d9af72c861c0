"""The host Sampler (the reference's Sampler API over the device ABI) against
the oracle's Sampler: multi-step sequences, the speculative-verify walk of
crates/rust-llm/src/generate.rs:389-451, and batched serving."""
import numpy as np
import pytest

import oracle as O
import rl_sampler as R
import workloads as W
from conftest import as_oracle_settings

pytestmark = pytest.mark.gpu


def test_a_long_sequence_matches_the_oracle(device):
    """Many sample calls on changing logits with the ring filling, wrapping
    and being reset, as a generation loop drives it (generate.rs:343-367)."""
    rng = np.random.default_rng(1)
    V = 20000
    for set_ in (R.sampling(0.8, 40, 0.9, 0.02, 1.3, 16, 5), R.greedy_sampling(repeat_penalty=1.5, repeat_last_n=8),
                 R.sampling(1.0, 0, 0.95, 0.05, 1.1, 32, 7)):
        s = R.HostSampler(V, set_)
        o = O.OracleSampler(V, as_oracle_settings(set_))
        prompt = rng.integers(0, V, 40)
        for t in prompt:
            s.remember(int(t))
            o.remember(int(t))
        for step in range(60):
            l = rng.normal(0, 2.0, V).astype(np.float32)
            l[rng.integers(0, V, 5)] = 9.0
            if step == 30:
                s.reset()
                o.reset()
            a, b = s.sample(l), o.sample(l)
            assert a == b, (set_, step)
            gi, gp = s.candidates()
            oi, op = o.candidates()
            assert np.array_equal(gi, oi) and np.array_equal(gp.view(np.uint32), op.view(np.uint32)), (set_, step)
            assert s.rng_state() == o.rng_state(), (set_, step)


def oracle_walk(o, rows, drafts):
    """generate.rs:412-429: row i is consumed only while picks equal drafts."""
    picks = []
    for i in range(rows.shape[0]):
        t = o.sample(rows[i])
        picks.append(t)
        if i < len(drafts) and t != drafts[i]:
            break
    return picks


def host_walk(s, d_rows, drafts):
    picks = s.verify(d_rows, drafts)
    committed = []
    for i in range(len(picks)):
        t = s.commit_verified(i)
        committed.append(t)
        if i < len(drafts) and t != drafts[i]:
            break
    return committed


@pytest.mark.parametrize("greedy", [False, True])
def test_the_verify_walk_matches_sequential_sampling(device, greedy):
    import torch
    wl = W.WORKLOADS["verify_greedy" if greedy else "verify"]
    rows, _, _ = wl.generate()
    set_ = wl.settings(0)
    history = wl.history()
    # The "right" drafter offers what sequential sampling will pick, so every
    # row is consumed; the "wrong" one never matches (tests/speculate.rs:205-300).
    probe = O.OracleSampler(wl.vocab, as_oracle_settings(set_))
    for t in history:
        probe.remember(int(t))
    right = [probe.sample(rows[i]) for i in range(rows.shape[0] - 1)]
    d_rows = torch.from_numpy(rows).to(device)
    for drafter, drafts in (("right", right), ("wrong", [(t + 1) % wl.vocab for t in right])):
        o = O.OracleSampler(wl.vocab, as_oracle_settings(set_))
        s = R.HostSampler(wl.vocab, set_, max_rows=rows.shape[0])
        for t in history:
            o.remember(int(t))
            s.remember(int(t))
        want = oracle_walk(o, rows, drafts)
        got = host_walk(s, d_rows, drafts)
        assert got == want, drafter
        assert s.rng_state() == o.rng_state(), drafter
        gi, gp = s.candidates()
        oi, op = o.candidates()
        assert np.array_equal(gi, oi) and np.array_equal(gp, op), drafter
        if drafter == "right":
            assert len(got) == rows.shape[0]


def test_a_verify_row_without_a_finite_maximum_shifts_the_stream(device):
    """Row 2 has no finite maximum, so it draws nothing (sample.rs:270-277) and
    the rows after it take the uniforms one place earlier."""
    import torch
    V = 5000
    rng = np.random.default_rng(2)
    rows = rng.normal(0, 2, (6, V)).astype(np.float32)
    rows[2, :] = -np.inf
    set_ = R.sampling(0.7, 20, 0.95, 0.0, 1.2, 16, 99)
    probe = O.OracleSampler(V, as_oracle_settings(set_))
    right = [probe.sample(rows[i]) for i in range(5)]
    o = O.OracleSampler(V, as_oracle_settings(set_))
    s = R.HostSampler(V, set_, max_rows=6)
    got = host_walk(s, torch.from_numpy(rows).to(device), right)
    want = oracle_walk(o, rows, right)
    assert got == want and len(got) == 6
    assert s.rng_state() == o.rng_state()


def test_batched_serving_matches_separate_samplers(device):
    import torch
    rng = np.random.default_rng(3)
    V = 30000
    sets = [R.sampling(0.6, 20, 0.95, 0.0, 1.0, 64, 10 + i) for i in range(6)] + \
           [R.sampling(1.0, 0, 0.9, 0.05, 1.2, 16, 20), R.greedy_sampling(repeat_penalty=1.3, repeat_last_n=8)]
    host = [R.HostSampler(V, s_, max_rows=len(sets)) for s_ in sets]
    oracles = [O.OracleSampler(V, as_oracle_settings(s_)) for s_ in sets]
    for step in range(5):
        logits = rng.normal(0, 2.5, (len(sets), V)).astype(np.float32)
        got = R.host_sample_batch(host, torch.from_numpy(logits).to(device))
        want = [o.sample(logits[i]) for i, o in enumerate(oracles)]
        assert got.tolist() == want, step
        for h, o in zip(host, oracles):
            assert h.rng_state() == o.rng_state()
            gi, _ = h.candidates()
            oi, _ = o.candidates()
            assert np.array_equal(gi, oi)


def test_a_vocabulary_mismatch_is_an_error_not_a_panic(device):
    s = R.HostSampler(100, R.sampling())
    with pytest.raises(R.SamplerError) as e:
        s.sample(np.zeros(99, np.float32))
    assert e.value.code == R.RL_ERR_VOCAB


def test_committing_past_a_rejected_draft_is_refused(device):
    """Row r of a verify assumed drafts[0..r) were accepted; once the committed
    token of row r-1 differs from drafts[r-1] the generation loop stops
    (generate.rs:412-429), and committing row r is an argument error that
    changes nothing."""
    import torch
    V = 4000
    rows = np.random.default_rng(4).normal(0, 2, (4, V)).astype(np.float32)
    set_ = R.sampling(0.7, 20, 0.95, 0.0, 1.2, 16, 5)
    s = R.HostSampler(V, set_, max_rows=4)
    d_rows = torch.from_numpy(rows).to(device)
    # Nothing is committed by a verify, so a second one picks row 0 the same
    # way: a draft one past that pick is rejected.
    first_pick = int(s.verify(d_rows, [0, 0, 0])[0])
    wrong = (first_pick + 1) % V
    picks = s.verify(d_rows, [wrong, wrong, wrong])
    assert picks[0] == first_pick
    assert s.commit_verified(0) == first_pick != wrong
    state = s.rng_state()
    ids, probs = s.candidates()
    with pytest.raises(R.SamplerError) as e:
        s.commit_verified(1)
    assert e.value.code == R.RL_ERR_ARGUMENT
    assert s.rng_state() == state
    gi, gp = s.candidates()
    assert np.array_equal(gi, ids) and np.array_equal(gp, probs)
