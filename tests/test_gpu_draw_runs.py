"""The full path's draw across a row's block of equal terms, against the oracle.

When one key holds a sixteenth of a row or more, its candidates form one block
of equal q in the sorted list, and the f32 draw (sample.rs:349-358) crosses
that block in closed form, a step per binade of the running sum, between two
replays of the terms before and after it. These tests put the uniform at the
running sum's values around every place where that hand-over happens: at the
block's first and last terms, the partial sums just below and above them,
inside the block, right after it, at the list's end (a sum that never passes
u takes the last candidate) and at 0. The running sums come from the oracle's
own kept probabilities, added in order in f32 (numpy's add.accumulate is
sequential). Each uniform gets its own copy of the row, so one call covers
them all; tokens, kept counts and candidates must match bit for bit."""
import numpy as np
import pytest

import oracle as O
import rl_sampler as R
from conftest import as_oracle_settings
from test_gpu_edges import assert_match, run_both

pytestmark = pytest.mark.gpu


def block_rows(rng, V):
    """Rows whose commonest key (a tenth to three quarters of the ids) sits
    in the middle or at the bottom of the order, over bf16-grid and full-f32
    neighbours."""
    rows, hots = [], []
    for fill, hot in (("bf16", -0.0234375), ("f32", 0.3), ("f32", -7.0), ("bf16", 0.0625)):
        for share in (0.1, 0.4, 0.75):
            if fill == "bf16":
                x = (rng.normal(0, 0.01, V).astype(np.float32).view(np.uint32) & 0xFFFF0000).view(np.float32)
            else:
                x = rng.normal(0, 1.0, V).astype(np.float32)
            x[rng.random(V) < share] = np.float32(hot)
            rows.append(x)
            hots.append(np.float32(hot))
    return rows, hots


def uniforms_around_the_block(ids, probs, row, hot):
    """Uniforms at and next to the f32 running sums where the draw hands over
    between the replays and the block."""
    k = ids.size
    cum = np.add.accumulate(probs[:k].astype(np.float32), dtype=np.float32)
    inb = np.flatnonzero(row[ids[:k]] == hot)
    us = [0.0, float(np.nextafter(np.float32(1.0), np.float32(0.0))), float(cum[-1])]
    if inb.size:
        lo, hi = int(inb[0]), int(inb[-1]) + 1
        for j in (lo - 2, lo - 1, lo, lo + 1, (lo + hi) // 2, hi - 2, hi - 1, hi, hi + 1, hi + 7, k - 2):
            if 0 <= j < k:
                c = np.float32(cum[j])
                us += [float(c), float(np.nextafter(c, np.float32(0.0))), float(np.nextafter(c, np.float32(2.0)))]
    return [u for u in us if 0.0 <= u < 1.0]


@pytest.mark.parametrize("top_p", [0.999, 0.8])
def test_the_draw_across_a_block_of_equal_terms(device, top_p):
    rng = np.random.default_rng(int(top_p * 1000))
    V = 20011
    base, hots = block_rows(rng, V)
    settings0 = [R.sampling(1.0, 0, top_p, 0.0, 1.0, 0, r) for r in range(len(base))]
    logits0 = np.stack(base)
    zeros = np.zeros((len(base), 1), np.uint32)
    first = O.pick_rows(logits0, [as_oracle_settings(s) for s in settings0], zeros,
                        np.zeros(len(base), np.uint32), np.full(len(base), 0.5, np.float32), cand_cap=V)
    rows, settings, uniforms, which = [], [], [], []
    for r, row in enumerate(base):
        k = int(first["kept"][r])
        for u in uniforms_around_the_block(first["ids"][r][:k], first["probs"][r][:k], row, hots[r]):
            rows.append(row)
            settings.append(settings0[r])
            uniforms.append(u)
            which.append(r)
    logits = np.stack(rows)
    n = logits.shape[0]
    windows = np.zeros((n, 1), np.uint32)
    wlen = np.zeros(n, np.uint32)
    uniforms = np.array(uniforms, np.float32)
    print("draw across equal terms: top_p %g, %d rows of %d" % (top_p, n, V), flush=True)
    got, want = run_both(device, logits, settings, windows, wlen, uniforms)
    assert_match("equal-term block, top_p %g" % top_p, got, want, settings)
    # The uniforms reach every side of the block: some pick inside it, some
    # before and some after it.
    inside = sum(1 for i in range(n) if logits[i][want["token"][i]] == hots[which[i]])
    assert 0 < inside < n
