"""The five synthetic workloads: deterministic per row, shaped as specified,
with uniforms from the reference's Rng and the adversarial tie block placed
across the top-p boundary."""
import numpy as np
import pytest

import oracle as O
import rl_sampler as R
import workloads as W
from conftest import as_oracle_settings


def test_rows_are_deterministic_and_independent_of_the_slice():
    for name in ("single", "zipf", "spikes", "verify", "ties"):
        wl = W.WORKLOADS[name]
        a, wa, la = wl.generate(0, min(3, wl.rows))
        if wl.rows > 1:
            b, wb, lb = wl.generate(1, min(2, wl.rows - 1))
            assert np.array_equal(a[1:1 + b.shape[0]], b), name
            assert np.array_equal(wa[1:1 + b.shape[0]], wb), name
        c, _, _ = wl.generate(0, 1, threads=1)
        assert np.array_equal(a[0], c[0]), name


def test_the_single_row_has_eight_spikes_at_twelve():
    l, _, _ = W.WORKLOADS["single"].generate()
    assert l.shape == (1, W.V1)
    assert int(np.sum(l[0] == 12.0)) == 8
    assert abs(float(np.std(l[0][l[0] != 12.0])) - 2.5) < 0.05


def test_the_spike_rows():
    l, w, n = W.WORKLOADS["spikes"].generate(0, 4)
    assert l.shape == (4, W.V2)
    for r in range(4):
        high = l[r][l[r] >= 8.0]  # the 16 spikes plus N(0, 2^2)'s own tail past 4 sigma
        assert 16 <= high.size <= 16 + 30 and high.max() < 14.0
    assert w.shape == (4, 64) and np.all(w < W.V2) and np.all(n == 64)


def test_the_tie_rows():
    l, _, _ = W.WORKLOADS["ties"].generate(0, 2)
    for r in range(2):
        row = l[r]
        assert int(np.sum(row == np.float32(-0.0234375))) >= (W.V1 * 2) // 5
        bits = row.view(np.uint32)
        assert np.all(bits & 0xFFFF == 0), "every value lies on the bf16 grid"


def test_the_tie_block_straddles_the_top_p_boundary():
    wl = W.WORKLOADS["ties"]
    l, w, n = wl.generate(0, 2)
    sets = [as_oracle_settings(s) for s in wl.settings_list(0, 2)]
    res = O.pick_rows(l, sets, w, n, wl.uniforms(0, 2))
    for r in range(2):
        row = l[r]
        order = np.lexsort((np.arange(row.size), -row.astype(np.float64)))
        tie_pos = np.nonzero(row[order] == np.float32(-0.0234375))[0]
        kept = int(res["kept"][r])
        assert tie_pos[0] < kept - 1 < tie_pos[-1], "the cut falls inside the tie block"
        # and the survivors of the block are its lowest ids
        kept_ids = set(res["ids"][r, :kept].tolist())
        block = order[tie_pos]
        inside = [i for i in block if i in kept_ids]
        assert inside == sorted(block.tolist())[:len(inside)]


def test_verify_windows_are_history_plus_drafts():
    wl = W.WORKLOADS["verify"]
    _, w, _ = wl.generate()
    hist, drafts = wl.history(), wl.drafts()
    seq = np.concatenate([hist, drafts])
    for i in range(wl.rows):
        assert np.array_equal(w[i], seq[i:i + 64]), i


def test_uniforms_come_from_the_reference_rng():
    wl = W.WORKLOADS["spikes"]
    u = wl.uniforms(5, 3)
    assert list(u) == [O.OracleRng(3000 + 5 + i).next_f32() for i in range(3)]
    v = W.WORKLOADS["verify"].uniforms()
    r = O.OracleRng(4000)
    assert list(v) == [r.next_f32() for _ in range(9)]


def test_algorithmic_bytes_of_the_bench_workload():
    # logits once, 64-id windows, uniforms, token + kept, and the kept
    # (id, prob) pairs: 20 per row on the bench workload
    assert W.WORKLOADS["spikes"].algorithmic_bytes(kept_total=1024 * 20) == 1_017_556_992
    # a top-k 0 row counts what it keeps, not the vocabulary
    zipf = W.WORKLOADS["zipf"]
    assert zipf.algorithmic_bytes(kept_total=700) == 64 * (151936 * 4 + 64 * 4 + 12) + 700 * 8
