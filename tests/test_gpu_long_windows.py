"""Repetition-penalty windows of 65 ids up to longer than the vocabulary on the
GPU, against the oracle.

The reference penalises each distinct id of recent[..filled] once
(sample.rs:239-257), whatever the window's length. These tests run windows
longer than the stream kernel's one-id-per-thread set-up (256), longer than a
wave, and at the context's largest (2048), on every device path:
  - the stream path (top-k 20 and 64, top-k 1, greedy), whose window set is
    built before the first tile once the window passes 256 ids;
  - the full path's sort (top-k 0, top-p on), whose passes mark window ids per
    step from the whole window;
  - the full path's min-p rows, whose pass loads up to 2048 window ids, eight a
    thread.
Rows carry spikes on window ids (so the penalty decides the kept set), ids
past the vocabulary, repeats, and ids in the row's last vocab % 4 elements.
Windows are given with the context's stride (2048) and with a stride equal to
the window (the stream kernel sizes its set from the call's stride). Windows
past 2048 ids (2049, 3000, 4096, 6000, and 12 000 over a vocabulary of 5003)
run on a penalised copy of the rows, on both paths and through the host's
verify walk.
Results must match bit for bit."""
import numpy as np
import pytest

import oracle as O
import rl_sampler as R
from conftest import as_oracle_settings

pytestmark = pytest.mark.gpu

MAX_WINDOW = 2048


def long_window_settings(wl):
    return [
        R.sampling(0.6, 20, 0.95, 0.0, 1.3, wl, 1),          # stream, top-k 20
        R.greedy_sampling(repeat_penalty=1.3, repeat_last_n=wl),
        R.sampling(1.0, 0, 0.95, 0.0, 1.2, wl, 3),           # full path, sorted
        R.sampling(1.0, 0, 0.9, 0.05, 1.5, wl, 4),           # full path, min-p
        R.sampling(0.8, 64, 0.9, 0.0, 0.7, wl, 5),           # stream, top-k 64, penalty < 1
        R.sampling(1.0, 0, 0.99, 0.02, 0.8, wl, 6),          # min-p, penalty < 1
        R.sampling(0.6, 1, 0.95, 0.0, 2.0, wl, 7),           # stream, top-k 1
        R.greedy_sampling(repeat_penalty=0.5, repeat_last_n=wl),
    ]


def window_rows(rng, rows, V, wl):
    """Windows of wl ids (ids past the vocabulary, repeats, tail ids) and
    logits N(0, 2^2) with spikes, most of them on window ids."""
    win = rng.integers(0, V + 8, (rows, wl)).astype(np.uint32)
    if wl > 7:
        win[:, 5::7] = win[:, : len(range(5, wl, 7))]  # repeats of earlier ids
    win[:, 2] = V - 1
    win[:, 3] = V - 1 - (V % 4 if V % 4 else 4)
    logits = rng.normal(0.0, 2.0, (rows, V)).astype(np.float32)
    for r in range(rows):
        inside = np.unique(win[r][win[r] < V])
        hot = rng.choice(inside, min(16, inside.size), replace=False)
        logits[r, hot] = rng.uniform(6.0, 12.0, hot.size).astype(np.float32)
        logits[r, rng.choice(V, 8, replace=False)] = rng.uniform(6.0, 12.0, 8).astype(np.float32)
        logits[r, V - 1] = 11.0
    return logits, win


def run_case(device, logits, settings, windows, wlen, uniforms, stride_mode, max_window=MAX_WINDOW):
    import torch
    rows, V = logits.shape
    wl = windows.shape[1]
    wstride = max_window if stride_mode == "max" else wl
    wbuf = np.zeros((rows, wstride), np.uint32)
    wbuf[:, :wl] = windows
    ctx = R.DeviceSampler(rows, V, max_window=max_window)
    ctx.configure(settings)
    cs = ctx.required_cand_stride()
    tok = torch.empty(rows, dtype=torch.int32, device=device)
    kept = torch.empty_like(tok)
    used = torch.empty(rows, dtype=torch.uint8, device=device)
    ids = torch.empty((rows, cs), dtype=torch.int32, device=device)
    probs = torch.empty((rows, cs), dtype=torch.float32, device=device)
    ctx.sample_rows(torch.from_numpy(logits.reshape(-1)).to(device), rows, V, tok, kept, used,
                    windows=torch.from_numpy(wbuf.view(np.int32)).to(device), window_stride=wstride,
                    window_len=torch.from_numpy(wlen.view(np.int32)).to(device),
                    uniforms=torch.from_numpy(uniforms).to(device), out_ids=ids, out_probs=probs, cand_stride=cs)
    torch.cuda.synchronize()
    got = dict(token=tok.cpu().numpy().view(np.uint32), kept=kept.cpu().numpy().view(np.uint32),
               used=used.cpu().numpy(), ids=ids.cpu().numpy().view(np.uint32), probs=probs.cpu().numpy())
    want = O.pick_rows(logits, [as_oracle_settings(s) for s in settings], windows, wlen, uniforms, cand_cap=cs)
    return got, want


def assert_rows_match(label, got, want, settings):
    for r in range(got["token"].size):
        where = "%s row %d (%r)" % (label, r, settings[r])
        assert got["token"][r] == want["token"][r], where
        assert got["kept"][r] == want["kept"][r], where
        assert got["used"][r] == want["used"][r], where
        k = int(want["kept"][r])
        assert np.array_equal(got["ids"][r, :k], want["ids"][r, :k]), where
        assert np.array_equal(got["probs"][r, :k].view(np.uint32), want["probs"][r, :k].view(np.uint32)), where


@pytest.mark.parametrize("V", [151936, 100003])
@pytest.mark.parametrize("wl", [65, 256, 257, 1024, 2048])
def test_long_windows_match_the_oracle(device, V, wl):
    rng = np.random.default_rng(V + 7 * wl)
    settings = long_window_settings(wl)
    rows = len(settings)
    logits, windows = window_rows(rng, rows, V, wl)
    wlen = np.full(rows, wl, np.uint32)
    wlen[6] = wl // 2  # a shorter window beside the long ones
    uniforms = rng.random(rows).astype(np.float32)
    # The penalty must decide something: some row's token or kept set differs
    # from the same row without it.
    plain = O.pick_rows(logits, [as_oracle_settings(s) for s in settings], windows, np.zeros(rows, np.uint32),
                        uniforms, cand_cap=V)
    for stride_mode in ("max", "exact"):
        print("long windows: V=%d wl=%d stride=%s" % (V, wl, stride_mode), flush=True)
        got, want = run_case(device, logits, settings, windows, wlen, uniforms, stride_mode)
        assert_rows_match("V=%d wl=%d stride=%s" % (V, wl, stride_mode), got, want, settings)
    assert any(plain["token"][r] != want["token"][r] or plain["kept"][r] != want["kept"][r] for r in range(rows))


def test_a_long_window_on_one_row_and_on_many(device):
    # One row (the stream kernel splits it into chunks and merges the window
    # once, in chunk 0's list) and 300 rows (four chunks a row), windows of
    # 2048 ids, stride 2048.
    V = 151936
    for rows in (1, 300):
        rng = np.random.default_rng(rows)
        base = long_window_settings(2048)
        settings = [base[r % len(base)] for r in range(rows)]
        logits, windows = window_rows(rng, rows, V, 2048)
        wlen = np.full(rows, 2048, np.uint32)
        wlen[::5] = rng.integers(0, 2049, wlen[::5].size)
        uniforms = rng.random(rows).astype(np.float32)
        print("long windows: %d rows" % rows, flush=True)
        got, want = run_case(device, logits, settings, windows, wlen, uniforms, "max")
        assert_rows_match("%d rows" % rows, got, want, settings)


@pytest.mark.parametrize("V", [151936, 100003])
@pytest.mark.parametrize("wl", [2049, 6000])
def test_windows_longer_than_the_on_chip_set(device, V, wl):
    """Windows past 2048 ids run on a penalised copy of the rows (the copy
    takes float4 loads for V = 151936 and single floats for the odd 100003),
    with the window's stride equal to it and inside a context made for 8192."""
    rng = np.random.default_rng(V + 11 * wl)
    settings = long_window_settings(wl)
    rows = len(settings)
    logits, windows = window_rows(rng, rows, V, wl)
    wlen = np.full(rows, wl, np.uint32)
    wlen[6] = wl // 2
    wlen[1] = 0  # a penalising row with an empty window: no penalty
    uniforms = rng.random(rows).astype(np.float32)
    plain = O.pick_rows(logits, [as_oracle_settings(s) for s in settings], windows, np.zeros(rows, np.uint32),
                        uniforms, cand_cap=V)
    for stride_mode, mw in (("exact", wl), ("max", 8192)):
        print("windows past the set: V=%d wl=%d stride=%s max_window=%d" % (V, wl, stride_mode, mw), flush=True)
        got, want = run_case(device, logits, settings, windows, wlen, uniforms, stride_mode, max_window=mw)
        assert_rows_match("V=%d wl=%d stride=%s" % (V, wl, stride_mode), got, want, settings)
    assert any(plain["token"][r] != want["token"][r] or plain["kept"][r] != want["kept"][r] for r in range(rows))


def test_a_window_longer_than_the_vocabulary(device):
    """A ring longer than the vocabulary (sample.rs:166 takes any length):
    12 000 ids over V = 5003, so every id repeats and most of the vocabulary
    is penalised, ids past V among them."""
    V, wl = 5003, 12000
    rng = np.random.default_rng(12000)
    settings = long_window_settings(wl)
    rows = len(settings)
    logits, windows = window_rows(rng, rows, V, wl)
    wlen = np.full(rows, wl, np.uint32)
    wlen[3] = 4000
    uniforms = rng.random(rows).astype(np.float32)
    got, want = run_case(device, logits, settings, windows, wlen, uniforms, "exact", max_window=wl)
    assert_rows_match("V=%d wl=%d" % (V, wl), got, want, settings)


def test_a_window_past_the_set_on_many_rows(device):
    """160 rows with 3000-id windows: the copy kernels' grid walks the rows."""
    V = 151936
    rows = 160
    rng = np.random.default_rng(300)
    base = long_window_settings(3000)
    settings = [base[r % len(base)] for r in range(rows)]
    logits, windows = window_rows(rng, rows, V, 3000)
    wlen = np.full(rows, 3000, np.uint32)
    wlen[::5] = rng.integers(0, 3001, wlen[::5].size)
    uniforms = rng.random(rows).astype(np.float32)
    print("windows past the set: %d rows" % rows, flush=True)
    got, want = run_case(device, logits, settings, windows, wlen, uniforms, "max", max_window=4096)
    assert_rows_match("%d rows" % rows, got, want, settings)


def oracle_walk(o, rows, drafts):
    picks = []
    for i in range(rows.shape[0]):
        t = o.sample(rows[i])
        picks.append(t)
        if i < len(drafts) and t != drafts[i]:
            break
    return picks


@pytest.mark.parametrize("last_n", [300, 2048, 4096])
@pytest.mark.parametrize("kind", ["top_k", "min_p", "greedy"])
def test_the_verify_walk_with_a_long_window(device, kind, last_n):
    """generate.rs:389-451 with a ring of 300 or 2048 ids, wrapped by a long
    history: nine rows, row i's window the ring after drafts 0..i-1, spikes on
    ring ids so that the penalty decides the picks."""
    import torch
    V = 151936
    rng = np.random.default_rng(last_n + len(kind))
    set_ = {"top_k": R.sampling(0.6, 20, 0.95, 0.0, 1.3, last_n, 11),
            "min_p": R.sampling(1.0, 0, 0.9, 0.05, 1.2, last_n, 12),
            "greedy": R.greedy_sampling(repeat_penalty=1.3, repeat_last_n=last_n)}[kind]
    history = rng.integers(0, V, last_n + 700).astype(np.uint32)
    history[::9] = history[0]
    rows = rng.normal(0.0, 2.0, (9, V)).astype(np.float32)
    recent = history[-last_n:]
    for i in range(9):
        hot = rng.choice(recent, 12, replace=False)
        rows[i, hot] = rng.uniform(7.0, 12.0, hot.size).astype(np.float32)
        rows[i, rng.choice(V, 6, replace=False)] = rng.uniform(7.0, 12.0, 6).astype(np.float32)
    probe = O.OracleSampler(V, as_oracle_settings(set_))
    for t in history:
        probe.remember(int(t))
    right = [probe.sample(rows[i]) for i in range(8)]
    d_rows = torch.from_numpy(rows).to(device)
    for drafter, drafts in (("right", right), ("wrong", [(t + 1) % V for t in right])):
        print("verify walk: %s last_n=%d drafter=%s" % (kind, last_n, drafter), flush=True)
        o = O.OracleSampler(V, as_oracle_settings(set_))
        s = R.HostSampler(V, set_, max_rows=9)
        for t in history:
            o.remember(int(t))
            s.remember(int(t))
        want = oracle_walk(o, rows, drafts)
        picks = s.verify(d_rows, drafts)
        got = []
        for i in range(len(picks)):
            t = s.commit_verified(i)
            got.append(t)
            if i < len(drafts) and t != drafts[i]:
                break
        assert got == want, (kind, last_n, drafter)
        assert s.rng_state() == o.rng_state()
        gi, gp = s.candidates()
        oi, op = o.candidates()
        assert np.array_equal(gi, oi) and np.array_equal(gp.view(np.uint32), op.view(np.uint32))
        # and one more token through the single-row call, window full
        l = rows[-1].copy()
        l[recent[:5]] = 13.0
        assert s.sample(l) == o.sample(l)
        gi, gp = s.candidates()
        oi, op = o.candidates()
        assert np.array_equal(gi, oi) and np.array_equal(gp.view(np.uint32), op.view(np.uint32))
