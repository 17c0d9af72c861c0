"""The min-p path of the full-vocabulary rows, against the oracle.

Rows with top_k 0 and min_p > 0 first try a path that sorts only the
candidates with p >= min_p (sample.rs:326-340) and accepts the top-p cut
(sample.rs:313-324) only when a proven error interval around the reference's
sequential mass cannot move it; every other row goes through the full sort.
These cases aim at both outcomes and at the boundaries between them: cuts
inside and past the survivors, exact ties at the cut (the interval straddles
it, so the row must fall back), survivor counts at and just over the cap,
top-p off (the reference keeps id order), top_p <= 0, min_p > 1 (nothing
survives), penalised ids crossing the threshold both ways, NaNs, and rows of
every path in one call. Results must match bit for bit."""
import numpy as np
import pytest

from test_gpu_edges import assert_match, run_both
import rl_sampler as R

pytestmark = pytest.mark.gpu

CAP = 4096  # survivors the min-p path holds per row (full_kernels.h)


def case(device, rows, settings, windows=None, wlen=None, seed=0, label="min-p"):
    rng = np.random.default_rng(seed)
    n, V = rows.shape
    if windows is None:
        windows = rng.integers(0, V, (n, 16)).astype(np.uint32)
        wlen = np.zeros(n, np.uint32)
    uniforms = rng.random(n).astype(np.float32)
    got, want = run_both(device, rows.astype(np.float32), settings, windows, wlen, uniforms)
    assert_match(label, got, want, settings)
    return got


def test_cut_inside_and_past_the_survivors(device):
    rng = np.random.default_rng(11)
    V = 151936
    x = rng.normal(0.0, 1.0, (6, V)).astype(np.float32)
    for r in range(6):
        x[r, rng.choice(V, 12, replace=False)] = rng.uniform(8.0, 12.0, 12)
    settings = [R.sampling(1.0, 0, tp, mp, 1.0, 0, r)
                for r, (tp, mp) in enumerate([(0.5, 1e-4), (0.9, 1e-4), (0.95, 0.05), (0.3, 1e-3),
                                              (0.99, 1e-6), (0.7, 0.2)])]
    case(device, x, settings, label="peaked rows")


def test_an_exact_tie_at_the_cut_falls_back_to_the_sort(device):
    # Top candidates with p = 1 exactly and the rest of the row at -inf: the
    # mass is an integer, and top_p puts the target exactly on a partial sum,
    # inside any error interval, so the row must take the sorting path.
    V = 5000
    rows = []
    settings = []
    for r, (n_top, tp) in enumerate([(4, 0.5), (8, 0.25), (3, 1.0 / 3.0), (6, 0.5)]):
        x = np.full(V, -np.inf, np.float32)
        x[np.arange(n_top) * 97 + 11] = 5.0
        rows.append(x)
        settings.append(R.sampling(1.0, 0, tp, 1e-3, 1.0, 0, r))
    case(device, np.stack(rows), settings, label="exact ties at the cut")


@pytest.mark.parametrize("n_top", [CAP - 1, CAP, CAP + 1])
def test_survivors_at_the_cap(device, n_top):
    V = 10007
    x = np.full((3, V), -100.0, np.float32)  # p = exp(-100), a subnormal > 0: not survivors
    rng = np.random.default_rng(n_top)
    for r in range(3):
        x[r, rng.choice(V, n_top, replace=False)] = 0.0
    settings = [R.sampling(1.0, 0, 0.9, 0.5, 1.0, 0, 1), R.sampling(1.0, 0, 1.0, 0.5, 1.0, 0, 2),
                R.sampling(2.0, 0, 0.999, 0.25, 1.0, 0, 3)]
    case(device, x, settings, label="%d survivors" % n_top)


@pytest.mark.parametrize("n_top", [1, 2, 63, 64, 65, 200])
def test_survivor_counts_around_one_wave(device, n_top):
    # Up to 64 survivors finish on one wave (register sort, readlane
    # replays); more take the block path. Spikes in [9, 10] over N(0, 1)
    # noise: every spike survives min_p >= 0.05 at these temperatures and no
    # noise element does, so the survivor count is n_top exactly. Row 3 holds
    # half its spikes at one value (ties, ascending ids).
    V = 151936
    rng = np.random.default_rng(1000 + n_top)
    x = rng.normal(0.0, 1.0, (4, V)).astype(np.float32)
    for r in range(4):
        ids = rng.choice(V, n_top, replace=False)
        x[r, ids] = rng.uniform(9.0, 10.0, n_top)
        if r == 3:
            x[r, ids[: max(1, n_top // 2)]] = 9.5
    settings = [R.sampling(1.0, 0, 0.9, 0.05, 1.0, 0, 1), R.sampling(1.0, 0, 1.0, 0.05, 1.0, 0, 2),
                R.sampling(0.7, 0, 0.5, 0.1, 1.0, 0, 3), R.sampling(1.0, 0, 0.999, 0.05, 1.0, 0, 4)]
    got = case(device, x, settings, seed=n_top, label="%d survivors" % n_top)
    assert got["kept"][1] == n_top  # top-p off: every survivor is kept


def test_top_p_off_keeps_id_order(device):
    rng = np.random.default_rng(5)
    V = 30001
    x = rng.normal(0.0, 2.0, (5, V)).astype(np.float32)
    settings = [R.sampling(t, k, tp, mp, 1.0, 0, r)
                for r, (t, k, tp, mp) in enumerate([(1.0, 0, 1.0, 0.01), (0.6, 0, 1.0, 0.3), (1.0, 3 * V, 1.0, 0.05),
                                                    (4.0, V, float("nan"), 0.01), (0.3, 0, 1.5, 0.001)])]
    case(device, x, settings, label="top-p off")


def test_degenerate_top_p_and_min_p(device):
    rng = np.random.default_rng(6)
    V = 20000
    x = rng.normal(0.0, 2.0, (6, V)).astype(np.float32)
    x[3, 17] = 9.0
    x[3, 18] = 9.0
    settings = [R.sampling(1.0, 0, 0.0, 0.05, 1.0, 0, 0), R.sampling(1.0, 0, -0.5, 0.05, 1.0, 0, 1),
                R.sampling(1.0, 0, 0.9, 1.5, 1.0, 0, 2), R.sampling(1.0, 0, 0.0, 1.0, 1.0, 0, 3),
                R.sampling(1.0, 0, 0.9, float("nan"), 1.0, 0, 4), R.sampling(1.0, 0, 0.9, 1e-30, 1.0, 0, 5)]
    case(device, x, settings, label="degenerate settings")


def test_penalised_ids_cross_the_threshold(device):
    rng = np.random.default_rng(8)
    V = 50000
    x = rng.normal(0.0, 1.0, (6, V)).astype(np.float32)
    windows = np.zeros((6, 64), np.uint32)
    wlen = np.full(6, 64, np.uint32)
    for r in range(6):
        top = rng.choice(V, 10, replace=False)
        x[r, top] = rng.uniform(6.0, 9.0, 10)
        near = rng.choice(V, 20, replace=False)
        x[r, near] = rng.uniform(-3.0, 3.0, 20)
        win = np.concatenate([top[:5], near[:20], rng.integers(0, V + 100, 39)]).astype(np.uint32)
        windows[r] = win
    settings = [R.sampling(1.0, 0, tp, mp, pen, 64, r)
                for r, (tp, mp, pen) in enumerate([(0.9, 0.01, 2.0), (0.9, 0.01, 0.5), (1.0, 0.05, 1.5),
                                                   (0.5, 1e-4, 0.25), (0.99, 0.001, 4.0), (0.8, 0.3, -1.0)])]
    case(device, x, settings, windows, wlen, label="penalised survivors")


def test_nan_rows_and_mixed_paths_in_one_call(device):
    rng = np.random.default_rng(9)
    V = 40000
    x = rng.normal(0.0, 2.5, (10, V)).astype(np.float32)
    x[0, 123] = np.nan
    x[1, :100] = np.nan
    x[2, 5] = np.inf
    x[3, :] = -np.inf
    x[3, 7] = 1.0
    settings = [R.sampling(1.0, 0, 0.9, 0.05, 1.0, 0, 0), R.sampling(0.7, 0, 0.9, 0.05, 1.3, 8, 1),
                R.sampling(1.0, 0, 0.9, 0.05, 1.0, 0, 2), R.sampling(1.0, 0, 0.95, 0.02, 1.0, 0, 3),
                R.sampling(1.0, 0, 0.95, 0.0, 1.0, 0, 4), R.sampling(0.6, 20, 0.95, 0.0, 1.2, 64, 5),
                R.greedy_sampling(), R.sampling(1.0, 100, 0.9, 0.05, 1.0, 0, 7),
                R.sampling(1.0, 0, 0.95, 0.05, 1.1, 64, 8), R.sampling(0.01, 0, 0.99, 0.01, 1.0, 0, 9)]
    windows = rng.integers(0, V, (10, 64)).astype(np.uint32)
    wlen = np.full(10, 64, np.uint32)
    case(device, x, settings, windows, wlen, label="mixed paths")


def test_small_and_ragged_vocabularies(device):
    rng = np.random.default_rng(10)
    for V in (1, 2, 5, 63, 4097):
        x = rng.normal(0.0, 1.0, (4, V)).astype(np.float32)
        settings = [R.sampling(1.0, 0, 0.9, 0.05, 1.0, 0, 0), R.sampling(1.0, 0, 1.0, 0.5, 1.0, 0, 1),
                    R.sampling(0.5, 0, 0.5, 0.001, 1.0, 0, 2), R.sampling(1.0, 0, 0.0, 0.9, 1.0, 0, 3)]
        case(device, x, settings, seed=V, label="V=%d" % V)


def test_infinities_and_empty_chunks_across_the_single_read(device):
    # The single read keeps, per chunk and per wave, the lowest id holding
    # +inf, and a row's maximum from every chunk: +inf at several ids in
    # several chunks (the lowest wins), a chunk of -inf only next to finite
    # chunks, NaN inside a chunk of -inf only (the row must leave the min-p
    # path), and a maximum that rises steadily along the row (many stale
    # candidates).
    V = 151936
    rng = np.random.default_rng(21)
    x = rng.normal(0.0, 2.0, (8, V)).astype(np.float32)
    x[0, [140000, 70001, 70000, 99999]] = np.inf
    x[1, :20000] = -np.inf
    x[2, :20000] = -np.inf
    x[2, 777] = np.nan
    x[3] = np.linspace(-20.0, 10.0, V, dtype=np.float32)
    x[4, :] = -np.inf
    x[4, 151935] = -3.0
    x[5, :] = -np.inf
    x[5, 3] = np.nan
    x[6, 151935] = np.inf
    x[7] = np.linspace(10.0, -20.0, V, dtype=np.float32)
    settings = [R.sampling(1.0, 0, 0.9, 0.05, 1.0, 0, r) for r in range(8)]
    case(device, x, settings, label="infinities and empty chunks")


@pytest.mark.parametrize("n_top", [1000, 1024, 1025])
def test_survivors_at_the_in_kernel_cap(device, n_top):
    # Up to 1024 survivors finish inside the single read; more go to the sort.
    V = 151936
    rng = np.random.default_rng(2000 + n_top)
    x = rng.normal(0.0, 1.0, (3, V)).astype(np.float32)
    for r in range(3):
        x[r, rng.choice(V, n_top, replace=False)] = rng.uniform(9.0, 10.0, n_top)
    settings = [R.sampling(1.0, 0, 0.999, 0.05, 1.0, 0, 1), R.sampling(1.0, 0, 1.0, 0.05, 1.0, 0, 2),
                R.sampling(1.0, 0, 0.5, 0.05, 1.0, 0, 3)]
    got = case(device, x, settings, seed=n_top, label="%d survivors" % n_top)
    assert got["kept"][1] == n_top


def test_extreme_temperatures(device):
    # A temperature too small for the mass's exponent scale (the row leaves
    # the min-p path), huge ones (every element a candidate: the list
    # overflows), and ordinary ones beside them.
    V = 30000
    rng = np.random.default_rng(22)
    x = rng.normal(0.0, 2.0, (6, V)).astype(np.float32)
    settings = [R.sampling(t, 0, 0.9, 0.05, 1.0, 0, r)
                for r, t in enumerate([1e-30, 1e-6, 1e30, 3.0e38, 0.05, 20.0])]
    case(device, x, settings, label="extreme temperatures")
