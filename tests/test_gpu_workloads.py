"""The five workload shapes on the GPU against the oracle, at full size.

Bar: token ids, kept counts, the used-uniform flags and the kept candidate ids
(in order) bit-exact; normalised probabilities within 1e-6 relative (and, as
the device replays the reference's arithmetic, expected bit-exact too).
"""
import numpy as np
import pytest

import oracle as O
import rl_sampler as R
import workloads as W
from conftest import as_oracle_settings

pytestmark = pytest.mark.gpu

PROB_RTOL = 1e-6  # the stated tolerance for normalised probabilities


def gpu_run(device, wl, logits, windows, wlen, uniforms, settings, ctx=None):
    import torch
    rows, V = logits.shape
    ctx = ctx or R.DeviceSampler(rows, V, max_window=W.WINDOW)
    L = torch.from_numpy(logits).to(device)
    Wt = torch.from_numpy(windows.view(np.int32)).to(device)
    WL = torch.from_numpy(wlen.view(np.int32)).to(device)
    U = torch.from_numpy(uniforms).to(device)
    return ctx, R.sample_batch(ctx, L, settings, windows=Wt, window_len=WL, uniforms=U)


def oracle_run(logits, windows, wlen, uniforms, settings, cand_cap):
    return O.pick_rows(logits, [as_oracle_settings(s) for s in settings], windows, wlen, uniforms,
                       cand_cap=cand_cap)


def assert_same(name, got, want, rows):
    bad_tok = np.nonzero(got.token[:rows] != want["token"][:rows])[0]
    assert bad_tok.size == 0, "%s: token differs at rows %s: gpu %s oracle %s" % (
        name, bad_tok[:8], got.token[bad_tok[:8]], want["token"][bad_tok[:8]])
    assert np.array_equal(got.kept[:rows], want["kept"][:rows]), "%s: kept counts differ" % name
    assert np.array_equal(got.used[:rows], want["used"][:rows]), "%s: used-uniform flags differ" % name
    for r in range(rows):
        k = int(want["kept"][r])
        gi, gp = got.ids[r, :k], got.probs[r, :k]
        wi, wp = want["ids"][r, :k], want["probs"][r, :k]
        assert np.array_equal(gi, wi), "%s row %d: kept candidate ids differ" % (name, r)
        rel = np.abs(gp.astype(np.float64) - wp) / np.maximum(np.abs(wp.astype(np.float64)), 1e-30)
        assert rel.max(initial=0.0) <= PROB_RTOL, "%s row %d: probability off by %g relative" % (name, r, rel.max())
        assert np.array_equal(gp.view(np.uint32), wp.view(np.uint32)), \
            "%s row %d: probabilities within 1e-6 but not bit-identical" % (name, r)


@pytest.mark.parametrize("name", ["single", "single_greedy", "verify", "verify_greedy", "spikes", "zipf", "ties"])
def test_workload_matches_oracle(device, name):
    wl = W.WORKLOADS[name]
    print("workload %s: %s" % (name, wl.description), flush=True)
    logits, windows, wlen = wl.generate()
    settings = wl.settings_list()
    uniforms = wl.uniforms()
    ctx, got = gpu_run(device, wl, logits, windows, wlen, uniforms, settings)
    want = oracle_run(logits, windows, wlen, uniforms, settings, got.ids.shape[1])
    assert_same(name, got, want, wl.rows)
    # The logits were never written and the context's counters return to
    # zero: a second call on the same context gives the same answers (the
    # kept prefix of each row; the rest of the candidate buffers is not
    # written).
    _, again = gpu_run(device, wl, logits, windows, wlen, uniforms, settings, ctx=ctx)
    assert_same(name + " (second call)", again, want, wl.rows)
    print("workload %s: %d rows bit-exact, kept %s.." % (name, wl.rows, got.kept[:4]), flush=True)
