"""rl_argmax_rows_noalloc, the argmax entry point that allocates nothing (its
partial results live in a fixed device array in the library), against
rl_argmax_rows, the context entry point whose kernels it shares, and against
the oracle's argmax (sample.rs:118-128): bit-exact token ids on two calls in a
row, the second smaller than the first, plus the row limit and device memory
left unchanged."""
import numpy as np
import pytest

import oracle as O
import rl_sampler as R

pytestmark = pytest.mark.gpu


def tricky_rows(rows, vocab, seed):
    """Random rows with the argmax's corners planted: ties for the maximum,
    NaN, +-inf, -0/+0 and rows with nothing above -inf."""
    g = np.random.default_rng(seed)
    x = g.standard_normal((rows, vocab)).astype(np.float32) * 3
    for r in range(rows):
        kind = r % 7
        if kind == 1:  # a tie: the lowest id wins
            a, b = sorted(g.choice(vocab, 2, replace=False))
            x[r, a] = x[r, b] = 40.0
        elif kind == 2:
            x[r, g.integers(0, vocab, 8)] = np.nan
        elif kind == 3:
            x[r, :] = -np.inf
        elif kind == 4:
            x[r, g.integers(0, vocab)] = np.inf
        elif kind == 5:
            x[r, :] = -1.0
            x[r, g.integers(0, vocab)] = -0.0
            x[r, g.integers(0, vocab)] = 0.0
        elif kind == 6:
            x[r, :] = np.nan
    return x


def run_both(device, x, stride_pad=0):
    import torch
    rows, vocab = x.shape
    buf = np.zeros((rows, vocab + stride_pad), np.float32)
    buf[:, :vocab] = x
    d = torch.from_numpy(buf).to(device)
    want = np.array([O.argmax(x[r]) for r in range(rows)], np.uint32)
    out_new = torch.full((rows,), -1, dtype=torch.int32, device=device)
    R.argmax_rows_noalloc(d, rows, d.stride(0), out_new, vocab)
    ctx = R.DeviceSampler(rows, vocab, max_window=1)
    out_old = torch.full((rows,), -1, dtype=torch.int32, device=device)
    ctx.argmax_rows(d, rows, d.stride(0), out_old)
    torch.cuda.synchronize()
    return out_new.cpu().numpy().view(np.uint32), out_old.cpu().numpy().view(np.uint32), want


def test_two_calls_in_a_row_match_the_context_entry_point_and_the_oracle(device):
    for what, rows, vocab, pad, seed in (("300 x 151936", 300, 151936, 0, 1),
                                         ("5 x 1003, padded stride", 5, 1003, 5, 2)):
        print("noalloc argmax:", what, flush=True)
        x = tricky_rows(rows, vocab, seed)
        new, old, want = run_both(device, x, pad)
        assert np.array_equal(old, want), what
        assert np.array_equal(new, want), "%s: rows %s differ" % (what, np.nonzero(new != want)[0][:10])


def test_the_row_limit_and_one_row(device):
    import torch
    print("noalloc argmax: 8192 x 4096 and 1 x 248320", flush=True)
    x = tricky_rows(8192, 4096, 3)
    new, old, want = run_both(device, x)
    assert np.array_equal(new, want) and np.array_equal(old, want)
    x = tricky_rows(1, 248320, 4)
    new, old, want = run_both(device, x)
    assert np.array_equal(new, want) and np.array_equal(old, want)
    d = torch.zeros((8193, 4), dtype=torch.float32, device=device)
    out = torch.empty(8193, dtype=torch.int32, device=device)
    with pytest.raises(R.SamplerError) as e:
        R.argmax_rows_noalloc(d, 8193, 4, out, 4)
    assert e.value.code == R.RL_ERR_CAPACITY


def test_it_allocates_no_device_memory(device):
    import torch
    x = torch.from_numpy(tricky_rows(64, 151936, 5)).to(device)
    out = torch.empty(64, dtype=torch.int32, device=device)
    R.argmax_rows_noalloc(x, 64, x.stride(0), out, 151936)
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info()[0]
    for _ in range(16):
        R.argmax_rows_noalloc(x, 64, x.stride(0), out, 151936)
    torch.cuda.synchronize()
    assert torch.cuda.mem_get_info()[0] == free0
    want = np.array([O.argmax(r) for r in x.cpu().numpy()], np.uint32)
    assert np.array_equal(out.cpu().numpy().view(np.uint32), want)
