"""The device replay of sequential sums (rust-llm_amd/csrc/rl_seqsum.h) on the
GPU, against plain sequential loops on the host, bit for bit.

The reference's sums are sequential: f64 for the probability mass, the top-p
cumulative sum and the normalising total (sample.rs:307-324, :342) and for
top_probability (forward.rs:1678), f32 for the draw (sample.rs:349-356). The
harness tests/native/seqsum_gpu.hip runs the device replay on arbitrary term
arrays, one workgroup per case, with 1024 threads, top_probability's shape
(256), a third one (128 threads of 3 terms), and the chunked replay the
sampler uses (chunk summaries chained by one wave, which replays the chunks
holding a binade crossing or the event term by term). Each case asks for the whole sum or for
the first partial sum >= or > a threshold (every partial sum, its neighbours,
0 and -1); numpy's cumulative sums (sequential, in the terms' precision) give
the expected index and value.

A second harness entry runs the chunked replay as the sampler's draw does:
in place (each staged round's terms written over its words) with a range of
words read as one value (memory there holds NaN); the written prefix, the
words past it and the results are checked against numpy.

Cases: uniform, wide and very wide ranges, narrow values whose sums stay
exact across binades, subnormals, mostly zeros, two values, short
significands, values near 1, runs of exact rounding ties in f32 and in f64,
constant runs, the exp terms of a 248 320-wide top_probability row, sorted
and unsorted, lengths 0 to 248 320.
"""
import ctypes
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "tests", "native", "libseqsum_gpu.so")


def harness():
    if not os.path.exists(LIB):
        raise RuntimeError("%s is not built (make -C tests/native)" % LIB)
    lib = ctypes.CDLL(LIB)
    lib.seqsum_gpu_run.argtypes = [ctypes.c_int, ctypes.c_int] + [ctypes.c_void_p] * 5 + [ctypes.c_uint32] + \
        [ctypes.c_void_p] * 3
    lib.seqsum_gpu_run.restype = ctypes.c_int
    return lib


def term_arrays(seed):
    g = np.random.default_rng(seed)
    out = []
    for rep in range(160):
        n = int(g.integers(1, 300 if rep < 80 else 5000))
        kind = rep % 13
        u = g.random(n)
        if kind == 0:
            x = u.astype(np.float32)
        elif kind == 1:
            x = np.exp(-40.0 * u).astype(np.float32)
        elif kind == 2:
            x = (1.0 + u * 1e-3).astype(np.float32)
        elif kind == 3:
            x = g.integers(0, 0x00800000, n, dtype=np.uint32).view(np.float32)
        elif kind == 4:
            x = np.where(g.integers(0, 4, n) == 0, u, 0.0).astype(np.float32)
        elif kind == 5:
            x = np.where(g.integers(0, 2, n) == 1, np.float32(0.75), np.float32(1.0 / 3.0)).astype(np.float32)
        elif kind == 6:
            x = np.ldexp(1.0 + g.integers(0, 8, n) / 8.0, -g.integers(0, 60, n)).astype(np.float32)
        elif kind == 7:
            x = (np.uint32(0x3F800000) + g.integers(0, 4, n, dtype=np.uint32)).view(np.float32)
        elif kind == 8:
            x = np.exp(-100.0 * u).astype(np.float32)
        elif kind == 9:
            x = (u * u * u).astype(np.float32)
        elif kind == 10:
            # f32 sums in [1, 2): every odd multiple of 2^-24 is an exact tie.
            x = np.ldexp(2.0 * g.integers(0, 64, n) + 1.0, -24).astype(np.float32)
            x[0] = 1.0
        elif kind == 11:
            # f64 sums in [1, 2): odd multiples of 2^-53 are exact ties.
            x = np.ldexp(2.0 * g.integers(0, 1 << 20, n) + 1.0, -53).astype(np.float32)
            x[0] = 1.0
        else:
            x = np.full(n, np.ldexp(float(g.integers(1, 256)), -int(g.integers(8, 28))), np.float32)
        if rep % 3 == 0:
            x = np.sort(x)[::-1].copy()
        out.append(x)
    out.append(np.zeros(0, np.float32))
    out.append(np.zeros(700, np.float32))
    # A top_probability row's terms: exp(l - max) of 248 320 logits N(0, 2^2)
    # with spikes in [8, 14) (numpy's f32 exp: any f32 terms will do here).
    lg = (g.standard_normal(248320) * 2.0).astype(np.float32)
    lg[g.choice(248320, 16, replace=False)] = g.uniform(8.0, 14.0, 16).astype(np.float32)
    out.append(np.exp(lg - lg.max()).astype(np.float32))
    # Short significands whose f64 sum crosses from 2^-8 to 2^0 in one step
    # (the 21st term, 1.75) and lands on a tie there, so that a step count one
    # off before the crossing changes the result; the crossing lane's own step
    # count is far above 2^53.
    out.append(np.array([
        0x24600000, 0x2FD00000, 0x2E800000, 0x2C700000, 0x2B400000, 0x29800000, 0x30100000, 0x3AA00000,
        0x37400000, 0x35100000, 0x2B300000, 0x25300000, 0x3B900000, 0x23700000, 0x24A00000, 0x36A00000,
        0x36E00000, 0x37E00000, 0x35700000, 0x24600000, 0x3FE00000, 0x39C00000, 0x3DC00000, 0x2C100000,
        0x32800000, 0x25D00000, 0x3D600000, 0x3B000000, 0x37D00000, 0x37F00000, 0x37000000, 0x2E200000,
        0x2D800000, 0x2E500000, 0x34200000, 0x3C500000, 0x2A400000, 0x2FA00000, 0x3BD00000, 0x36300000],
        np.uint32).view(np.float32))
    # A sampler draw's terms: 150 000 near-equal probabilities normalised
    # to sum to about 1, descending (the running f32 sum crosses 17 binades).
    q = np.sort((0.9 + 0.1 * g.random(150000)) / 142500.0)[::-1].astype(np.float32)
    out.append(q)
    # Ties-heavy rows long enough for many tiles, and a long constant run.
    out.append(np.ldexp(2.0 * g.integers(0, 64, 60000) + 1.0, -24).astype(np.float32))
    out.append(np.full(100000, np.float32(3.0 / 1024.0)))
    return out


def expected(x, precision, thr, mode):
    n = x.size
    p = np.cumsum(x) if precision == 24 else np.cumsum(x.astype(np.float64))
    p = p.astype(np.float64)
    if mode == 0:
        return n, (float(p[-1]) if n else 0.0)
    hit = p >= thr if mode == 1 else p > thr
    i = int(np.argmax(hit)) if n and hit.any() else n
    return i, (float(p[i]) if i < n else (float(p[-1]) if n else 0.0))


def run_cases(device, precision, shape, seed):
    import torch
    arrays = term_arrays(seed)
    g = np.random.default_rng(seed + 1)
    offs, ns, thrs, modes, want = [], [], [], [], []
    flat, at = [], 0
    for x in arrays:
        flat.append(x)
        p = np.cumsum(x) if precision == 24 else np.cumsum(x.astype(np.float64))
        p = p.astype(np.float64)
        picks = [(0.0, 0)]
        for t in range(4):
            if x.size == 0:
                break
            v = float(p[int(g.integers(0, x.size))])
            w = int(g.integers(-1, 2))
            if w:
                v = float(np.nextafter(v, np.inf if w > 0 else -np.inf))
            picks.append((v, 1 + (t % 2)))
        picks += [(0.0, 1), (-1.0, 2), (float(p[-1]) if x.size else 0.0, 2)]
        for thr, mode in picks:
            offs.append(at)
            ns.append(x.size)
            thrs.append(thr)
            modes.append(mode)
            want.append(expected(x, precision, thr, mode))
        at += x.size
    terms = torch.from_numpy(np.concatenate(flat)).to(device)
    d = lambda a, dt: torch.from_numpy(np.asarray(a, dt)).to(device)
    d_off, d_n = d(offs, np.int64), d(np.asarray(ns, np.uint32).view(np.int32), np.int32)
    d_thr, d_mode = d(thrs, np.float64), d(np.asarray(modes, np.uint32).view(np.int32), np.int32)
    cases = len(offs)
    out_idx = torch.empty(cases, dtype=torch.int32, device=device)
    out_sum = torch.empty(cases, dtype=torch.float64, device=device)
    print("seqsum P=%d shape=%d: %d cases, %d terms" % (precision, shape, cases, at), flush=True)
    rc = harness().seqsum_gpu_run(precision, shape, terms.data_ptr(), d_off.data_ptr(), d_n.data_ptr(),
                                  d_thr.data_ptr(), d_mode.data_ptr(), cases, out_idx.data_ptr(),
                                  out_sum.data_ptr(), torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    torch.cuda.synchronize()
    gi = out_idx.cpu().numpy().view(np.uint32)
    gs = out_sum.cpu().numpy()
    bad = [c for c in range(cases) if gi[c] != want[c][0] or gs[c].tobytes() != np.float64(want[c][1]).tobytes()]
    assert not bad, "P=%d shape=%d: %d of %d cases differ, first %s: got (%d, %r) want %r (n=%d thr=%r mode=%d)" % (
        precision, shape, len(bad), cases, bad[0], gi[bad[0]], gs[bad[0]], want[bad[0]], ns[bad[0]], thrs[bad[0]],
        modes[bad[0]])


@pytest.mark.parametrize("precision", [24, 53])
@pytest.mark.parametrize("shape", [0, 1, 2, 3])
def test_replay_matches_sequential_loops(device, precision, shape):
    run_cases(device, precision, shape, seed=1000 + precision + shape)


def run_wb_cases(device, precision, seed):
    """The chunked replay as the draw runs it (rust-llm_amd/csrc/full_rest.h):
    in place, each staged round's terms written over its words, with a range
    of words read as one value whatever memory holds there (the row's
    commonest key, whose block the sort does not store). The harness's term
    doubles the word (exact). Memory under the range holds NaN, so a read of
    it shows in the sum; the expected results are numpy's sequential cumulative
    sums of the doubled effective terms, and every written word must be its
    doubled effective term while the words past the written prefix keep
    theirs."""
    import torch
    g = np.random.default_rng(seed)
    base = term_arrays(seed)
    picks_from = [x for x in base if x.size > 0]
    cases = []
    for c in range(48):
        x = picks_from[int(g.integers(0, len(picks_from)))] if c % 4 else picks_from[-1 - (c // 4) % 4]
        x = x.copy()
        n = x.size
        kind = c % 6
        if kind == 0:
            lo = hi = 0                        # no range
        elif kind == 1:
            lo, hi = 0, n                      # every word
        elif kind == 2:
            lo = int(g.integers(0, n)); hi = n + int(g.integers(0, 5000))  # to the end and past it
        else:
            lo = int(g.integers(0, n)); hi = min(n, lo + int(g.integers(1, max(2, n // 2))))
        word = x[lo] if lo < n else np.float32(0.5)
        eff = x.copy()
        eff[lo:min(hi, n)] = word
        mem = x.view(np.uint32).copy()
        mem[lo:min(hi, n)] = 0x7FC00000         # NaN: must never be read
        t = (eff.astype(np.float32) * np.float32(2.0)).astype(np.float32)
        p = np.cumsum(t) if precision == 24 else np.cumsum(t.astype(np.float64))
        p = p.astype(np.float64)
        r = int(g.integers(0, 4))
        if r == 0 or n == 0:
            thr, mode = 0.0, 0
        elif r == 1:
            thr, mode = float(p[int(g.integers(0, n))]), 1 + int(g.integers(0, 2))
        elif r == 2:
            thr, mode = float(np.nextafter(p[int(g.integers(0, n))], np.inf)), 2
        else:
            thr, mode = -1.0, 1                # met at +0: the first term's sum
        cases.append((mem, n, thr, mode, lo, hi, np.float32(word).view(np.uint32), t))
    offs, at = [], 0
    for mem, *_ in cases:
        offs.append(at)
        at += mem.size
    words = torch.from_numpy(np.concatenate([c[0] for c in cases]).view(np.int32)).to(device)
    d = lambda a, dt: torch.from_numpy(np.asarray(a, dt)).to(device)
    u32 = lambda a: d(np.asarray(a, np.uint32).view(np.int32), np.int32)
    k = len(cases)
    out_idx = torch.empty(k, dtype=torch.int32, device=device)
    out_sum = torch.empty(k, dtype=torch.float64, device=device)
    out_staged = torch.empty(k, dtype=torch.int32, device=device)
    lib = harness()
    lib.seqsum_gpu_run_wb.argtypes = [ctypes.c_int] + [ctypes.c_void_p] * 8 + [ctypes.c_uint32] + [ctypes.c_void_p] * 4
    lib.seqsum_gpu_run_wb.restype = ctypes.c_int
    args = [d(offs, np.int64), u32([c[1] for c in cases]), d([c[2] for c in cases], np.float64),
            u32([c[3] for c in cases]), u32([c[4] for c in cases]), u32([c[5] for c in cases]),
            u32([c[6] for c in cases])]
    print("seqsum in place P=%d: %d cases, %d words" % (precision, k, at), flush=True)
    rc = lib.seqsum_gpu_run_wb(precision, words.data_ptr(), *[a.data_ptr() for a in args], k, out_idx.data_ptr(),
                               out_sum.data_ptr(), out_staged.data_ptr(), torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    torch.cuda.synchronize()
    gi = out_idx.cpu().numpy().view(np.uint32)
    gs = out_sum.cpu().numpy()
    gst = out_staged.cpu().numpy().view(np.uint32)
    back = words.cpu().numpy().view(np.uint32)
    for c, (mem, n, thr, mode, lo, hi, wbits, t) in enumerate(cases):
        want_i, want_s = expected(t, precision, thr, mode)
        assert gi[c] == want_i and gs[c].tobytes() == np.float64(want_s).tobytes(), (
            "case %d (n=%d, range [%d, %d), thr %r mode %d): got (%d, %r) want (%d, %r)" % (
                c, n, lo, hi, thr, mode, gi[c], gs[c], want_i, want_s))
        st = int(gst[c])
        assert st <= n, (c, st, n)
        if want_i < n and not (mode == 1 and thr < 0.0):
            assert st >= want_i + 1, (c, st, want_i)
        if want_i == n:
            assert st == n, (c, st, n)
        seg = back[offs[c]:offs[c] + n]
        assert np.array_equal(seg[:st], t[:st].view(np.uint32)), "case %d: written prefix" % c
        assert np.array_equal(seg[st:], mem[st:]), "case %d: words past the prefix" % c


@pytest.mark.parametrize("precision", [24, 53])
def test_chunked_replay_in_place_with_a_hot_range(device, precision):
    run_wb_cases(device, precision, seed=3000 + precision)
