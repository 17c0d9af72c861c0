"""The greedy path (temperature <= 0: argmax of the penalised row,
sample.rs:259-265 and :118-128) on the GPU, against the oracle.

k_greedy leaves the row's window ids out of its scan and adds their
penalised values once; these rows put the decision exactly there: the raw
maximum on a window id that the penalty pushes below another element, a
penalty below 1 that lifts a window id above the rest, a window id's
penalised value tied with a plain element (the lower id wins), ids repeated
in the window and ids past the vocabulary, rows whose only finite value is a
window id, NaN and infinite rows, -0 against +0. Each row is run split over
chunks (one row, 19 chunks) and unsplit (1100 rows, one chunk each), with the
candidates written and without. Results must match bit for bit."""
import numpy as np
import pytest

import oracle as O
import rl_sampler as R
from conftest import as_oracle_settings

pytestmark = pytest.mark.gpu


def greedy_rows(rng, V, W):
    rows, wins, sets = [], [], []

    def add(x, win, penalty):
        w = np.full(W, V + 3, np.uint32)  # ids past the vocabulary pad the window
        w[:len(win)] = win
        rows.append(x.astype(np.float32))
        wins.append(w)
        sets.append(R.greedy_sampling(repeat_penalty=penalty, repeat_last_n=W))

    base = lambda: rng.normal(0.0, 1.0, V)  # below 6 everywhere
    # The raw maximum is a window id; the penalty sends it below the runner-up.
    x = base(); x[777] = 20.0; x[5000] = 12.0
    add(x, [777, 3, 777], 2.0)
    # A penalty below 1 lifts a window id (positive: divided) above the rest.
    x = base(); x[12345] = 9.0; x[99] = 10.0
    add(x, [12345, 12345, V + 1], 0.5)
    # A negative window logit multiplied by a penalty below 1 rises toward 0.
    x = np.full(V, -5.0); x[4242] = -3.0; x[V - 1] = -2.5
    add(x, [4242], 0.25)
    # The window id's penalised value ties a plain element: the lower id wins.
    x = base(); x[300] = 16.0; x[150] = 8.0; x[V - 2] = 8.0
    add(x, [300], 2.0)
    x = base(); x[V - 3] = 16.0; x[150] = 8.0
    add(x, [V - 3], 2.0)
    # The only finite value sits on a window id; everything else -inf.
    x = np.full(V, -np.inf); x[60000] = 1.5
    add(x, [60000, 7], 3.0)
    # All -inf: token 0.
    add(np.full(V, -np.inf), [0, 1, 2], 2.0)
    # NaN everywhere but two values; NaN on window ids too.
    x = np.full(V, np.nan); x[10] = -1.0; x[20] = -1.0
    add(x, [10, 11, 12], 1.5)
    # +inf on a window id stays +inf (inf / p), the first +inf wins.
    x = base(); x[500] = np.inf; x[900] = np.inf
    add(x, [900, 500], 2.0)
    # -0 against +0 as the maximum (equal for argmax: the lower id).
    x = np.full(V, -1.0); x[40] = -0.0; x[30] = 0.0
    add(x, [30], 2.0)
    # No penalty (1.0): the window is ignored.
    x = base(); x[777] = 20.0
    add(x, [777], 1.0)
    # Windows over the row's last vocab % 4 elements and the chunk edges.
    for at in (V - 1, V - 2, 8191, 8192, 7996):
        x = base(); x[at] = 15.0; x[(at + 3) % V] = 14.0
        add(x, [at], 1.5)
    return np.stack(rows), np.stack(wins), sets


@pytest.mark.parametrize("V", [151936, 100003])
@pytest.mark.parametrize("candidates", [True, False])
def test_greedy_rows_match_the_oracle(device, V, candidates):
    import torch
    rng = np.random.default_rng(V + candidates)
    W = 64
    logits, windows, settings = greedy_rows(rng, V, W)
    n = logits.shape[0]
    wlen = np.full(n, W, np.uint32)
    uniforms = np.zeros(n, np.float32)
    want = O.pick_rows(logits, [as_oracle_settings(s) for s in settings], windows, wlen, uniforms, cand_cap=1)
    for reps in (1, 1100 // n + 1):  # one chunk-split row at a time, then many rows of one chunk each
        rows = n if reps == 1 else n * reps
        lg = np.tile(logits, (reps, 1))
        wn = np.tile(windows, (reps, 1))
        st = settings * reps
        batches = [[r] for r in range(n)] if reps == 1 else [list(range(rows))]
        for idx in batches:
            m = len(idx)
            print("greedy: V=%d rows=%d candidates=%s" % (V, m, candidates), flush=True)
            ctx = R.DeviceSampler(m, V, max_window=W)
            ctx.configure([st[i] for i in idx])
            tok = torch.empty(m, dtype=torch.int32, device=device)
            kept = torch.empty_like(tok)
            used = torch.empty(m, dtype=torch.uint8, device=device)
            ids = torch.empty((m, 1), dtype=torch.int32, device=device) if candidates else None
            probs = torch.empty((m, 1), dtype=torch.float32, device=device) if candidates else None
            ctx.sample_rows(torch.from_numpy(np.ascontiguousarray(lg[idx]).reshape(-1)).to(device), m, V, tok, kept,
                            used, windows=torch.from_numpy(np.ascontiguousarray(wn[idx]).view(np.int32)).to(device),
                            window_stride=W, window_len=torch.from_numpy(np.full(m, W, np.int32)).to(device),
                            uniforms=torch.zeros(m, dtype=torch.float32, device=device), out_ids=ids,
                            out_probs=probs, cand_stride=1 if candidates else 0)
            torch.cuda.synchronize()
            t = tok.cpu().numpy().view(np.uint32)
            for j, i in enumerate(idx):
                r = i % n
                assert t[j] == want["token"][r], (V, r, t[j], want["token"][r])
            assert (kept.cpu().numpy() == 1).all()
            assert (used.cpu().numpy() == 0).all()
            if candidates:
                assert np.array_equal(ids.cpu().numpy().view(np.uint32)[:, 0], t)
                assert (probs.cpu().numpy()[:, 0] == 1.0).all()
