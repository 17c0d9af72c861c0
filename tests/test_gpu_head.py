"""The device output head (rl_head_logits, rl_quantize_rows) against the oracle,
bit for bit.

The reference's tiers agree bit for bit (crates/llm-core/src/kernels/
avx2.rs:480-523), so the device must too: every logit equal to the oracle's
q6k_matvec (the scalar tier, kernels/mod.rs:273-300, after quant.rs:337-375),
NaN where it is NaN. Cases follow the reference's kernel tests
(crates/llm-core/tests/kernels.rs): its awkward shapes (k = 1 ... 16384), the
head's full shape (2560 x 248320), batches that straddle the device's pass size
and tile sizes, the saturation extremes with their closed-form answers, zero
weights and activations, rows with NaN, infinities and subnormals, a vocabulary
that is not a whole number of 64-row groups, a padded row stride, and the head
feeding the sampler with the logits left in HBM.
"""
import numpy as np
import pytest
import torch

import oracle as O
import rl_sampler as R
from conftest import as_oracle_settings
from head_fixtures import (AWKWARD_SHAPES, HEAD_K, HEAD_ROWS, QK, SAT_PATTERNS, XorShiftRng, bulk_weights,
                           random_weights, saturated_activations, saturated_known_answer, saturated_weights,
                           signed_row)

pytestmark = pytest.mark.gpu


def bits_equal(got, want):
    got = np.asarray(got, np.float32)
    want = np.asarray(want, np.float32)
    nan = np.isnan(want)
    if not np.array_equal(np.isnan(got), nan):
        return False
    return np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def device_head(device, w, k, rows, max_batch=40):
    torch.cuda.synchronize()
    return R.DeviceHead(w, k, rows, max_batch=max_batch, device=device.index or 0)


def run_head(head, x, device):
    xd = torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(device)
    out = head.logits(xd)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def test_quantize_rows_matches_the_oracle(device):
    g = np.random.default_rng(3)
    for k in (1, 37, 255, 256, 257, 300, 2560, 9216):
        x = (g.standard_normal((6, k)) * g.uniform(0.001, 80, (6, 1))).astype(np.float32)
        x[1, :: max(1, k // 5)] = np.nan
        x[2] = 0.0
        x[3, 0] = np.inf
        x[4, : min(k, 40)] = np.float32(1e-40)  # subnormal inputs
        if k >= 2:
            x[5, 1] = -np.float32(3e38)
        print("quantize k=%d" % k, flush=True)
        d, qs, bs = R.quantize_rows(torch.from_numpy(x).to(device))
        torch.cuda.synchronize()
        wd, wq, wb = O.quantize_rows(x)
        assert bits_equal(d.cpu().numpy(), wd), k
        assert np.array_equal(qs.cpu().numpy(), wq), k
        assert np.array_equal(bs.cpu().numpy(), wb), k


@pytest.mark.parametrize("i", range(len(AWKWARD_SHAPES)))
def test_awkward_shapes(device, i):
    k, rows = AWKWARD_SHAPES[i]
    nb = -(-k // QK)
    rng = XorShiftRng(0x51ED + i)
    w = random_weights(rng, nb * rows)
    head = device_head(device, w, k, rows)
    for t in (1, 2, 3, 5, 9, 17, 33):
        print("awkward k=%d rows=%d t=%d" % (k, rows, t), flush=True)
        x = np.stack([signed_row(rng, k) for _ in range(t)])
        got = run_head(head, x, device)
        want = O.q6k_matvec(w, k, x)
        assert bits_equal(got, want), (k, rows, t)
    head.close()


def test_batches_straddle_passes_and_tiles(device):
    # 1000 rows: 15 full 64-row groups and one of 40. k = 2560 holds 19
    # activation rows per pass; 20 and 35 take two passes.
    k, rows = 2560, 1000
    rng = XorShiftRng(0xBA7C4)
    w = random_weights(rng, 10 * rows)
    head = device_head(device, w, k, rows)
    x_all = np.stack([signed_row(rng, k) for _ in range(35)])
    singles = [run_head(head, x_all[j:j + 1], device)[0] for j in range(35)]
    want_all = O.q6k_matvec(w, k, x_all)
    for j in range(35):
        assert bits_equal(singles[j], want_all[j]), j
    for t in (1, 2, 3, 4, 5, 6, 7, 8, 9, 12, 15, 16, 17, 18, 19, 20, 33, 35):
        print("batch t=%d" % t, flush=True)
        got = run_head(head, x_all[:t], device)
        for j in range(t):
            # A batch gives each row what it gives alone (kernels/mod.rs:208-217).
            assert bits_equal(got[j], singles[j]), (t, j)
    head.close()


@pytest.mark.parametrize("k", [2560, 300, 256])
def test_saturation_extremes(device, k):
    nb = -(-k // QK)
    rows = 70
    for wi, s in enumerate((127, -128)):
        w = saturated_weights(nb * rows)[wi]
        head = device_head(device, w, k, rows)
        for t in (1, 19):
            print("saturated k=%d s=%d t=%d" % (k, s, t), flush=True)
            x = saturated_activations(k, t)
            got = run_head(head, x, device)
            for j in range(t):
                want = saturated_known_answer(k, SAT_PATTERNS[j % 4], s)
                assert np.all(got[j] == want), (k, s, t, j)
        head.close()


def test_zero_weights_and_special_activation_rows(device):
    k, rows = 512, 130
    rng = XorShiftRng(7)
    w = random_weights(rng, 2 * rows)
    x = np.stack([signed_row(rng, k) for _ in range(8)])
    x[0] = 0.0
    x[1, 17] = np.nan
    x[2, 300] = np.inf
    x[3, :] = np.float32(1e-42)
    x[4, :] = np.float32(3e38) * np.sign(x[4])
    x[5, 5] = -np.inf
    x[6, :256] = 0.0
    head = device_head(device, w, k, rows)
    got = run_head(head, x, device)
    want = O.q6k_matvec(w, k, x)
    assert bits_equal(got, want)
    assert np.all(got[0] == 0.0)
    head.close()
    zero = np.zeros(2 * rows * 210, np.uint8)
    head = device_head(device, zero, k, rows)
    got = run_head(head, x, device)
    assert bits_equal(got, O.q6k_matvec(zero, k, x))
    # Zero weights give 0, except where an infinity made a block's scale
    # infinite: (inf * 0) * 0 is NaN in the reference's f32 line too.
    finite_rows = [0, 1, 3, 4, 6, 7]
    assert np.all(got[finite_rows] == 0.0)
    assert np.all(np.isnan(got[[2, 5]]))
    head.close()


def test_padded_row_stride_and_ragged_vocabulary(device):
    for k, rows in ((2560, 63), (2560, 65), (768, 1)):
        nb = -(-k // QK)
        rng = XorShiftRng(rows)
        w = random_weights(rng, nb * rows)
        head = device_head(device, w, k, rows)
        t, stride = 3, rows + 37
        x = np.stack([signed_row(rng, k) for _ in range(t)])
        out = torch.full((t, stride), -7.0, dtype=torch.float32, device=device)
        head.logits_into(torch.from_numpy(x).to(device), out, row_stride=stride)
        torch.cuda.synchronize()
        o = out.cpu().numpy()
        assert bits_equal(o[:, :rows], O.q6k_matvec(w, k, x)), (k, rows)
        assert np.all(o[:, rows:] == -7.0), (k, rows)
        head.close()


@pytest.fixture(scope="module")
def full_head(device):
    w = bulk_weights(0x7E4D, HEAD_ROWS, HEAD_K)
    head = device_head(device, w, HEAD_K, HEAD_ROWS, max_batch=32)
    yield w, head
    head.close()


def test_full_vocabulary_head(device, full_head):
    w, head = full_head
    g = np.random.default_rng(11)
    x = (g.standard_normal((17, HEAD_K)) * 1.5).astype(np.float32)
    print("full head t=1", flush=True)
    got1 = run_head(head, x[:1], device)
    assert bits_equal(got1, O.q6k_matvec(w, HEAD_K, x[:1]))
    print("full head t=17", flush=True)
    got = run_head(head, x, device)
    assert bits_equal(got[:1], got1)
    for lo in (0, 123456, HEAD_ROWS - 6000):
        hi = min(HEAD_ROWS, lo + 6000)
        assert bits_equal(got[:, lo:hi], O.q6k_matvec(w, HEAD_K, x, lo, hi)), lo


def test_head_feeds_the_sampler(device, full_head):
    # Nine verify-shaped rows: the head writes logits into HBM and the sampler
    # reads them there; the oracle runs its head and its sampler on the host.
    w, head = full_head
    g = np.random.default_rng(12)
    t = 9
    x = (g.standard_normal((t, HEAD_K)) * 2.0).astype(np.float32)
    xd = torch.from_numpy(x).to(device)
    logits = head.logits(xd)
    settings = [R.sampling(0.6, 20, 0.95, 0.0, 1.3, 64, 0) if j % 3 else R.greedy_sampling(repeat_penalty=1.3,
                                                                                           repeat_last_n=64)
                for j in range(t)]
    windows = g.integers(0, HEAD_ROWS, (t, 64)).astype(np.uint32)
    wlen = np.full(t, 64, np.uint32)
    uniforms = g.random(t).astype(np.float32)
    ctx = R.DeviceSampler(t, HEAD_ROWS, max_window=64)
    got = R.sample_batch(ctx, logits, settings, windows=torch.from_numpy(windows.view(np.int32)).to(device),
                         window_len=torch.from_numpy(wlen.view(np.int32)).to(device),
                         uniforms=torch.from_numpy(uniforms).to(device))
    host_logits = O.q6k_matvec(w, HEAD_K, x)
    want = O.pick_rows(host_logits, [as_oracle_settings(s) for s in settings], windows, wlen, uniforms,
                       cand_cap=got.ids.shape[1])
    assert np.array_equal(got.token, want["token"])
    assert np.array_equal(got.kept, want["kept"])
    for r in range(t):
        k = int(want["kept"][r])
        assert np.array_equal(got.ids[r, :k], want["ids"][r, :k]), r
        assert np.array_equal(got.probs[r, :k].view(np.uint32), want["probs"][r, :k].view(np.uint32)), r
    ctx.close()
