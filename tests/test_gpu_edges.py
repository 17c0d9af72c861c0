"""Randomized differential tests of the GPU sampler against the oracle.

Every row gets its own random settings (both device paths in one call), its
own window (with repeats and ids past the vocabulary) and uniform; rows carry
ties, signed zeros and special values. Results must match bit for bit (a NaN
probability matches a NaN)."""
import numpy as np
import pytest

import oracle as O
import rl_sampler as R
from conftest import as_oracle_settings

pytestmark = pytest.mark.gpu

TEMPS = [0.0, 0.05, 0.6, 1.0, 4.0]
TOPP = [0.0, 0.5, 0.9, 0.999, 1.0]
MINP = [0.0, 0.02, 0.3, 1.0]
PEN = [1.0, 0.5, 1.3, 2.0]
LASTN = [0, 4, 64]


def random_settings(rng, V):
    topk = [0, 1, 2, 5, 20, 63, 64, 65, max(V - 1, 1), V, 3 * V]
    return R.sampling(float(rng.choice(TEMPS)), int(rng.choice(topk)), float(rng.choice(TOPP)),
                      float(rng.choice(MINP)), float(rng.choice(PEN)), int(rng.choice(LASTN)),
                      int(rng.integers(0, 1 << 30)))


def random_rows(rng, rows, V, kind):
    if kind == "normal":
        x = rng.normal(0.0, 3.0, (rows, V)).astype(np.float32)
    elif kind == "ties":
        x = rng.choice(np.array([-1.5, -0.0, 0.0, 0.25, 2.0, 2.0], np.float32), (rows, V))
    elif kind == "spikes":
        x = rng.normal(0.0, 2.0, (rows, V)).astype(np.float32)
        for r in range(rows):
            x[r, rng.choice(V, min(V, 16), replace=False)] = rng.uniform(8, 14, min(V, 16))
    else:
        raise ValueError(kind)
    return x


def inject_specials(rng, x, frac):
    specials = np.array([np.nan, -np.nan, np.inf, -np.inf, 0.0, -0.0, 3.4e38, -3.4e38], np.float32)
    m = rng.random(x.shape) < frac
    x[m] = rng.choice(specials, int(m.sum()))
    return x


def run_both(device, logits, settings, windows, wlen, uniforms, stride=None):
    import torch
    rows, V = logits.shape
    stride = stride or V
    buf = np.zeros((rows, stride), np.float32)
    buf[:, :V] = logits
    # a row stride that is not a multiple of 4 floats exercises the unaligned loads
    flat = torch.from_numpy(buf.reshape(-1)).to(device)
    ctx = R.DeviceSampler(rows, V, max_window=windows.shape[1])
    ctx.configure(settings)
    cs = ctx.required_cand_stride()
    tok = torch.empty(rows, dtype=torch.int32, device=device)
    kept = torch.empty_like(tok)
    used = torch.empty(rows, dtype=torch.uint8, device=device)
    ids = torch.empty((rows, cs), dtype=torch.int32, device=device)
    probs = torch.empty((rows, cs), dtype=torch.float32, device=device)
    ctx.sample_rows(flat, rows, stride, tok, kept, used,
                    windows=torch.from_numpy(windows.view(np.int32)).to(device), window_stride=windows.shape[1],
                    window_len=torch.from_numpy(wlen.view(np.int32)).to(device),
                    uniforms=torch.from_numpy(uniforms).to(device), out_ids=ids, out_probs=probs,
                    cand_stride=cs)
    torch.cuda.synchronize()
    got = dict(token=tok.cpu().numpy().view(np.uint32), kept=kept.cpu().numpy().view(np.uint32),
               used=used.cpu().numpy(), ids=ids.cpu().numpy().view(np.uint32), probs=probs.cpu().numpy())
    want = O.pick_rows(logits, [as_oracle_settings(s) for s in settings], windows, wlen, uniforms, cand_cap=cs)
    return got, want


def assert_match(label, got, want, settings):
    for r in range(got["token"].size):
        where = "%s row %d (%r)" % (label, r, settings[r])
        assert got["token"][r] == want["token"][r], where
        assert got["kept"][r] == want["kept"][r], where
        assert got["used"][r] == want["used"][r], where
        k = int(want["kept"][r])
        assert np.array_equal(got["ids"][r, :k], want["ids"][r, :k]), where
        gp, wp = got["probs"][r, :k], want["probs"][r, :k]
        both_nan = np.isnan(gp) & np.isnan(wp)
        assert np.array_equal(gp.view(np.uint32)[~both_nan], wp.view(np.uint32)[~both_nan]), where


def make_case(rng, rows, V, kind, special=0.0, wl=16):
    logits = random_rows(rng, rows, V, kind)
    if special:
        logits = inject_specials(rng, logits, special)
    settings = [random_settings(rng, V) for _ in range(rows)]
    windows = rng.integers(0, V + 8, (rows, wl)).astype(np.uint32)  # some ids past the vocabulary
    windows[:, 1::3] = windows[:, 0:1]  # repeats
    wlen = np.array([min(int(s.repeat_last_n), wl) if s.repeat_last_n else 0 for s in settings], np.uint32)
    uniforms = rng.random(rows).astype(np.float32)
    return logits, settings, windows, wlen, uniforms


@pytest.mark.parametrize("V,rows,kind,special", [
    (1003, 64, "normal", 0.0),
    (2048, 64, "ties", 0.0),
    (2048, 48, "ties", 0.05),
    (4099, 32, "spikes", 0.002),
    (5, 40, "normal", 0.1),
    (151936, 3, "spikes", 0.0),
    (151936, 2, "normal", 0.0005),
])
def test_random_rows_match_the_oracle(device, V, rows, kind, special):
    rng = np.random.default_rng(V * 1000 + rows)
    logits, settings, windows, wlen, uniforms = make_case(rng, rows, V, kind, special)
    print("case V=%d rows=%d kind=%s special=%g" % (V, rows, kind, special), flush=True)
    got, want = run_both(device, logits, settings, windows, wlen, uniforms)
    assert_match("V=%d %s" % (V, kind), got, want, settings)


def test_unaligned_row_stride(device):
    rng = np.random.default_rng(7)
    logits, settings, windows, wlen, uniforms = make_case(rng, 16, 4099, "spikes", 0.001)
    got, want = run_both(device, logits, settings, windows, wlen, uniforms, stride=4099 + 3)
    assert_match("stride 4102", got, want, settings)


def test_rows_with_many_nans_and_infinities(device):
    rng = np.random.default_rng(3)
    V = 3000
    logits = rng.normal(0, 1, (12, V)).astype(np.float32)
    logits[0, :40] = np.nan                      # >= k positive NaNs: the rescan path
    logits[1, :] = -np.inf                        # nothing finite
    logits[2, :] = np.nan                         # nothing but NaN
    logits[3, 100] = np.inf                       # +inf wins everything
    logits[3, 200] = np.inf
    logits[4, :] = -np.nan
    logits[5, ::2] = -np.inf
    logits[6, :25] = np.nan
    logits[6, 30] = np.inf
    logits[7, 5] = np.nan
    logits[8, :] = 0.0
    logits[8, 17] = -0.0
    logits[9, :] = -0.0
    logits[9, 11] = 0.0
    logits[10, :64] = np.nan
    logits[11, :] = 1.0
    settings = []
    for r in range(12):
        for s in (R.sampling(0.7, 20, 0.9, 0.0, 1.3, 8, r), R.greedy_sampling(repeat_penalty=1.3, repeat_last_n=8)):
            settings.append(s)
    logits = np.repeat(logits, 2, axis=0)
    rows = logits.shape[0]
    windows = rng.integers(0, V, (rows, 8)).astype(np.uint32)
    wlen = np.full(rows, 8, np.uint32)
    uniforms = rng.random(rows).astype(np.float32)
    got, want = run_both(device, logits, settings, windows, wlen, uniforms)
    assert_match("special rows", got, want, settings)


def test_argmax_rows_match_the_oracle(device):
    import torch
    rng = np.random.default_rng(9)
    V = 70001
    x = inject_specials(rng, random_rows(rng, 33, V, "ties"), 0.001)
    x[0, :] = -np.inf
    x[1, :] = np.nan
    ctx = R.DeviceSampler(33, V, max_window=0)
    out = torch.empty(33, dtype=torch.int32, device=device)
    ctx.argmax_rows(torch.from_numpy(x).to(device), 33, V, out)
    torch.cuda.synchronize()
    assert out.cpu().numpy().tolist() == [O.argmax(x[r]) for r in range(33)]


def test_errors_are_status_codes(device):
    import torch
    ctx = R.DeviceSampler(4, 100, max_window=8)
    l = torch.zeros((4, 100), device=device)
    o = torch.empty(4, dtype=torch.int32, device=device)
    u8 = torch.empty(4, dtype=torch.uint8, device=device)
    with pytest.raises(R.SamplerError) as e:
        ctx.sample_rows(l, 4, 100, o, o, u8)
    assert e.value.code == R.RL_ERR_NOT_CONFIGURED
    ctx.configure([R.greedy_sampling()] * 4)
    with pytest.raises(R.SamplerError) as e:
        ctx.sample_rows(l, 4, 100, o, o, u8, vocab=99)
    assert e.value.code == R.RL_ERR_VOCAB  # where the reference panics (sample.rs:222-226)
    with pytest.raises(R.SamplerError) as e:
        ctx.sample_rows(l, 5, 100, o, o, u8)
    assert e.value.code == R.RL_ERR_CAPACITY
    with pytest.raises(R.SamplerError) as e:
        ctx.sample_rows(l, 4, 100, o, o, u8, windows=o, window_stride=9, window_len=o)
    assert e.value.code == R.RL_ERR_CAPACITY
    kept = torch.empty(4, dtype=torch.int32, device=device)
    l[:, 37] = 1.0
    ctx.sample_rows(l, 4, 100, o, kept, u8)  # and a good call still works
    torch.cuda.synchronize()
    assert o.cpu().tolist() == [37, 37, 37, 37]
    assert kept.cpu().tolist() == [1, 1, 1, 1]


def test_full_path_rows_of_equal_keys(device):
    # Rows whose keys agree in every digit the sort would rank on (a constant
    # row, all -0.0), or in all but the sign bit (a mix of +0.0 and -0.0), sent
    # down the full path (top-k 0): the kept candidates are the ties in
    # ascending id order (sample.rs:282-286), whatever passes the sort skips.
    V, rows = 3000, 8
    rng = np.random.default_rng(77)
    logits = np.empty((rows, V), np.float32)
    logits[0] = 1.25
    logits[1] = -3.0
    logits[2] = -0.0
    logits[3] = rng.choice(np.array([0.0, -0.0], np.float32), V)
    logits[4] = 7.5
    logits[5] = -np.inf
    logits[6] = 0.5
    logits[7] = rng.choice(np.array([0.0, -0.0], np.float32), V)
    topp = [0.5, 0.9, 0.999, 0.3, 0.01, 0.9, 1.0, 0.75]
    settings = [R.sampling(1.0 if r % 2 else 0.6, 0, topp[r], 0.0, 1.0, 0, r) for r in range(rows)]
    windows = np.zeros((rows, 1), np.uint32)
    wlen = np.zeros(rows, np.uint32)
    uniforms = rng.random(rows).astype(np.float32)
    got, want = run_both(device, logits, settings, windows, wlen, uniforms)
    assert_match("equal keys", got, want, settings)
    for r in (0, 1, 2, 4):
        k = int(want["kept"][r])
        assert np.array_equal(want["ids"][r, :k], np.arange(k, dtype=np.uint32)), r


def test_full_path_rows_with_nans_and_infinities(device):
    # The rows of the special-rows test on the full path (top-k 0): NaN and
    # infinite p leave the draw to walk q = p * (1 / total) in order, and the
    # kept candidates are written beside the draw in the same launch.
    rng = np.random.default_rng(4)
    V = 3000
    logits = rng.normal(0, 1, (10, V)).astype(np.float32)
    logits[0, :40] = np.nan
    logits[1, :] = -np.inf
    logits[2, :] = np.nan
    logits[3, 100] = np.inf
    logits[4, :25] = np.nan
    logits[4, 30] = np.inf
    logits[5, 5] = np.nan
    logits[6, :] = 0.0
    logits[7, ::3] = -np.inf
    logits[8, 7] = 3.4e38
    logits[9, :] = 1.0
    settings = []
    for r in range(10):
        settings += [R.sampling(1.0, 0, 0.9, 0.0, 1.3, 8, r), R.sampling(3.0, 0, 1.0, 0.0, 1.0, 0, r),
                     R.sampling(1e-30, 0, 0.95, 0.05, 1.0, 0, r), R.sampling(0.5, 0, 0.99, 0.02, 1.2, 8, r)]
    logits = np.repeat(logits, 4, axis=0)
    rows = logits.shape[0]
    windows = rng.integers(0, V, (rows, 8)).astype(np.uint32)
    wlen = np.full(rows, 8, np.uint32)
    uniforms = rng.random(rows).astype(np.float32)
    got, want = run_both(device, logits, settings, windows, wlen, uniforms)
    assert_match("full-path special rows", got, want, settings)


def hot_key_rows(rng, V):
    # Rows where one value holds a tenth to three quarters of the ids (at the
    # top, in the middle or at the bottom of the order) beside other values
    # that leave the sort one, two or four digit passes: values apart only in
    # their top byte, bf16-grid values, and f32 values with full mantissas.
    rows, names = [], []
    for fill in ("top-byte", "bf16", "f32"):
        for where in ("max", "mid", "min"):
            for share in (0.1, 0.4, 0.75):
                if fill == "top-byte":
                    x = rng.choice(np.array([0.5, 2.0, 8.0, 32.0, -2.0, -8.0], np.float32), V)
                    hot = {"max": 128.0, "mid": 2.0, "min": -32.0}[where]
                elif fill == "bf16":
                    x = (rng.normal(0, 0.01, V).astype(np.float32).view(np.uint32) & 0xFFFF0000).view(np.float32)
                    hot = {"max": 0.0625, "mid": -0.0234375, "min": -0.125}[where]
                else:
                    x = rng.normal(0, 1.0, V).astype(np.float32)
                    hot = {"max": 6.5, "mid": 0.3, "min": -7.0}[where]
                x[rng.random(V) < share] = np.float32(hot)
                rows.append(x)
                names.append("%s/%s/%.2f" % (fill, where, share))
    # Special hot values: NaN and +inf make p NaN or infinite (the list's own
    # walks run), -inf gives p = 0, and -0.0 ties +0.0's neighbours.
    for hot, share in ((np.nan, 0.3), (np.inf, 0.2), (-np.inf, 0.5), (-0.0, 0.4)):
        x = rng.normal(0, 1.0, V).astype(np.float32)
        x[rng.random(V) < share] = np.float32(hot)
        rows.append(x)
        names.append("f32/special %r/%.2f" % (hot, share))
    return np.stack(rows), names


@pytest.mark.parametrize("candidates", [True, False])
def test_full_path_rows_with_a_dominant_key(device, candidates):
    # The sort leaves a row's commonest key out of its passes when it holds a
    # sixteenth of the row or more, and writes its ids as one block; the rows
    # here put that block at the start, inside and at the end of the order,
    # across several tiles of the sort, with and without the candidate outputs
    # (without them the block shares a buffer with the last pass's ids).
    rng = np.random.default_rng(2024 + candidates)
    V = 20011
    logits, names = hot_key_rows(rng, V)
    rows = logits.shape[0]
    choices = [(1.0, 0, 0.9, 0.0, 1.0), (0.7, 0, 0.99, 0.02, 1.0), (2.0, 0, 0.5, 0.0, 1.3),
               (1.0, 100, 0.95, 0.0, 1.0), (1.0, 7000, 0.999, 0.0, 0.8), (1.0, V - 1, 0.9, 0.05, 1.0)]
    settings = [R.sampling(*choices[r % len(choices)], 16, r) for r in range(rows)]
    windows = rng.integers(0, V, (rows, 16)).astype(np.uint32)
    wlen = np.full(rows, 16, np.uint32)
    uniforms = rng.random(rows).astype(np.float32)
    print("dominant-key rows: %d x %d, candidates %s" % (rows, V, candidates), flush=True)
    if candidates:
        got, want = run_both(device, logits, settings, windows, wlen, uniforms)
        assert_match("dominant key", got, want, settings)
        return
    import torch
    ctx = R.DeviceSampler(rows, V, max_window=16)
    ctx.configure(settings)
    tok = torch.empty(rows, dtype=torch.int32, device=device)
    kept = torch.empty_like(tok)
    used = torch.empty(rows, dtype=torch.uint8, device=device)
    ctx.sample_rows(torch.from_numpy(logits.reshape(-1)).to(device), rows, V, tok, kept, used,
                    windows=torch.from_numpy(windows.view(np.int32)).to(device), window_stride=16,
                    window_len=torch.from_numpy(wlen.view(np.int32)).to(device),
                    uniforms=torch.from_numpy(uniforms).to(device))
    torch.cuda.synchronize()
    want = O.pick_rows(logits, [as_oracle_settings(s) for s in settings], windows, wlen, uniforms)
    t, k = tok.cpu().numpy().view(np.uint32), kept.cpu().numpy().view(np.uint32)
    for r in range(rows):
        assert (t[r], k[r]) == (want["token"][r], want["kept"][r]), "%s %r" % (names[r], settings[r])


@pytest.mark.parametrize("V", [151936, 100003])
def test_split_rows_with_windows(device, V):
    """Rows split into one-tile chunks, where each chunk penalises the window
    ids that fall in it: window ids on chunk edges and on the row's last
    vocab % 4 elements, penalties above and below 1 on positive and negative
    logits, repeats and ids past the vocabulary, and rows whose k best are
    all NaN (the rescan, which needs the whole window)."""
    rng = np.random.default_rng(V + 5)
    rows, W = 6, 48
    n4 = V // 4
    chunks = min(1024 // rows, 32, -(-n4 // 2048))
    edges = [4 * (c * n4 // chunks) for c in range(1, chunks)]
    x = rng.normal(0.0, 1.0, (rows, V)).astype(np.float32)
    windows = np.full((rows, W), V + 2, np.uint32)
    settings = []
    spread = rng.choice(V, 40, replace=False)
    # 0, 1: the 40 NaNs beat every value (k = 20): the rescan decides, with
    # the largest value on a window id that the penalty lowers or lifts.
    x[0, spread] = np.nan
    x[0, 777] = 10.0; x[0, V - 5] = 7.0
    windows[0, :3] = [777, 777, 12]
    settings.append(R.sampling(0.7, 20, 0.9, 0.0, 2.0, W, 1))
    x[1, spread] = np.nan
    x[1, 777] = 10.0; x[1, edges[0]] = 6.0
    windows[1, :2] = [edges[0], V + 9]
    settings.append(R.sampling(0.7, 20, 0.9, 0.0, 0.5, W, 2))
    # 2: the row's best values sit on window ids at the chunk edges.
    ids = sorted({e + d for e in edges for d in (-1, 0, 1)})[:W]
    x[2, ids] = rng.uniform(5.0, 9.0, len(ids))
    windows[2, :len(ids)] = ids
    settings.append(R.sampling(1.0, 40, 0.95, 0.0, 1.5, W, 3))
    # 3: the last elements of the row (vocab % 4 of them when V is not a
    # multiple of 4) and repeats.
    x[3, V - 3:] = [8.0, 9.0, 10.0]
    windows[3, :6] = [V - 1, V - 2, V - 1, V - 3, V, V + 1]
    settings.append(R.sampling(0.8, 5, 1.0, 0.0, 3.0, W, 4))
    # 4: a penalty below 1 lifts a negative window logit toward 0, above the rest.
    x[4] = -np.abs(x[4]) - 1.0
    x[4, 5000] = -1.2; x[4, 9000] = -1.1
    windows[4, :2] = [5000, 5000]
    settings.append(R.sampling(0.5, 10, 0.9, 0.05, 0.25, W, 5))
    # 5: a full window of random ids with min-p.
    windows[5] = rng.integers(0, V, W)
    x[5, windows[5]] += 4.0
    settings.append(R.sampling(0.6, 64, 0.99, 0.02, 1.3, W, 6))
    wlen = np.full(rows, W, np.uint32)
    uniforms = rng.random(rows).astype(np.float32)
    print("split rows with windows: V=%d chunks=%d" % (V, chunks), flush=True)
    got, want = run_both(device, x, settings, windows, wlen, uniforms)
    assert_match("split V=%d" % V, got, want, settings)


@pytest.mark.parametrize("V", [9000, 16400, 40000, 100003, 248320])
def test_split_rows_across_chunk_counts(device, V):
    """Rows split into 2 to 31 one-tile chunks, with top-k on both sides of
    32 (lists of at most 32 entries are merged two to a wave), a penalty
    window and ties at the top."""
    rng = np.random.default_rng(V)
    ks = [1, 5, 20, 32, 33, 64]
    rows, W = len(ks), 16
    x = rng.normal(0.0, 2.0, (rows, V)).astype(np.float32)
    x[:, rng.choice(V, 48, replace=False)] = 9.0  # ties among the best
    windows = rng.integers(0, V, (rows, W)).astype(np.uint32)
    settings = [R.sampling(0.8, k, 0.97, 0.0, 1.4 if k % 2 else 1.0, W, 10 + k) for k in ks]
    wlen = np.full(rows, W, np.uint32)
    uniforms = rng.random(rows).astype(np.float32)
    chunks = min(1024 // rows, 32, -(-(V // 4) // 2048))
    print("split rows: V=%d chunks=%d" % (V, chunks), flush=True)
    got, want = run_both(device, x, settings, windows, wlen, uniforms)
    assert_match("chunks V=%d" % V, got, want, settings)


@pytest.mark.parametrize("k", [1, 20, 32, 64])
def test_split_rows_of_ties(device, k):
    """Rows split into 19 one-tile chunks where a third of every chunk ties
    at the top value: the chunk's bound admits every tied element, each
    wave's buffer overflows and compacts, the candidates exceed one wave's
    sort, and the lists' order among equal keys is by id."""
    rng = np.random.default_rng(k)
    V, rows, W = 151936, 3, 8
    x = random_rows(rng, rows, V, "ties")
    windows = rng.integers(0, V, (rows, W)).astype(np.uint32)
    settings = [R.sampling(1.0, k, 0.9, 0.0, pen, W, 100 + k) for pen in (1.0, 1.3, 0.7)]
    wlen = np.full(rows, W, np.uint32)
    uniforms = rng.random(rows).astype(np.float32)
    print("split ties: k=%d" % k, flush=True)
    got, want = run_both(device, x, settings, windows, wlen, uniforms)
    assert_match("ties k=%d" % k, got, want, settings)
