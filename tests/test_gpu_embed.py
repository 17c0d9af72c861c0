"""The device embedding lookup (rl_head_embed_rows) against the oracle, bit for
bit.

The reference's lookup (crates/rust-llm/src/forward.rs:1127-1138) expands
rows of the tied Q6_K `token_embd` with dequantize_row
(crates/llm-core/src/quant.rs:177-203); the device reads the same tensor from
the head's repacked layout. Cases: the reference's awkward widths (k = 1 ...
16384) with every row looked up, the head's full tensor (2560 x 248320) at the
first, last and random rows, f16 block scales that are infinite, NaN,
subnormal or negative zero, a padded row stride, tokens past the vocabulary,
and a token drawn by the sampler in HBM fed back into the lookup.
"""
import numpy as np
import pytest
import torch

import oracle as O
import rl_sampler as R
from conftest import as_oracle_settings
from head_fixtures import AWKWARD_SHAPES, HEAD_K, HEAD_ROWS, QK, XorShiftRng, bulk_weights, random_weights

pytestmark = pytest.mark.gpu


def bits_equal(got, want):
    got = np.asarray(got, np.float32)
    want = np.asarray(want, np.float32)
    nan = np.isnan(want)
    if not np.array_equal(np.isnan(got), nan):
        return False
    return np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def device_tokens(tokens, device):
    return torch.from_numpy(np.asarray(tokens, np.uint32).view(np.int32).copy()).to(device)


def embed(head, tokens, device):
    out = head.embed(device_tokens(tokens, device))
    torch.cuda.synchronize()
    return out.cpu().numpy()


@pytest.mark.parametrize("i", range(len(AWKWARD_SHAPES)))
def test_awkward_widths_every_row(device, i):
    k, rows = AWKWARD_SHAPES[i]
    nb = -(-k // QK)
    w = random_weights(XorShiftRng(0xE3B + i), nb * rows)
    torch.cuda.synchronize()
    head = R.DeviceHead(w, k, rows, max_batch=1, device=device.index or 0)
    tokens = list(range(rows)) + list(range(rows - 1, -1, -1)) + [0]
    print("embed k=%d rows=%d" % (k, rows), flush=True)
    assert bits_equal(embed(head, tokens, device), O.embed_rows(w, k, tokens)), (k, rows)
    head.close()


def test_special_block_scales(device):
    # f16 d = +inf, -inf, NaN, the smallest subnormal, -0 and the largest
    # finite, over random quants and scales: inf * 0 is NaN, -0 * x keeps its
    # sign, as in the reference's f32 multiply.
    k, rows = 512, 70
    nb = 2
    w = random_weights(XorShiftRng(0x5CA1E), nb * rows).reshape(rows * nb, 210)
    specials = [0x7C00, 0xFC00, 0x7E00, 0x0001, 0x8000, 0x7BFF]
    for j, bits in enumerate(specials):
        w[j * 3, 208:210] = np.array([bits & 0xFF, bits >> 8], np.uint8)
    w = w.reshape(-1)
    torch.cuda.synchronize()
    head = R.DeviceHead(w, k, rows, max_batch=1, device=device.index or 0)
    tokens = list(range(rows))
    got = embed(head, tokens, device)
    want = O.embed_rows(w, k, tokens)
    assert bits_equal(got, want)
    assert np.isnan(got).any() and np.isinf(got).any()
    head.close()


def test_padded_stride_and_tokens_past_the_vocabulary(device):
    k, rows = 300, 130
    nb = 2
    w = random_weights(XorShiftRng(0xD0D), nb * rows)
    torch.cuda.synchronize()
    head = R.DeviceHead(w, k, rows, max_batch=1, device=device.index or 0)
    tokens = [5, rows, 129, 0xFFFFFFFF, 64, 63]
    stride = k + 13
    out = torch.full((len(tokens), stride), -7.0, dtype=torch.float32, device=device)
    head.embed_into(device_tokens(tokens, device), out, row_stride=stride)
    torch.cuda.synchronize()
    o = out.cpu().numpy()
    assert np.all(o[:, k:] == -7.0)
    for i, t in enumerate(tokens):
        if t < rows:
            assert bits_equal(o[i, :k], O.embed_rows(w, k, [t])[0]), t
        else:
            # The reference asserts here (forward.rs:1130-1134); the device
            # writes the row as NaN.
            assert np.all(np.isnan(o[i, :k])), t
    head.close()


@pytest.fixture(scope="module")
def full_head(device):
    w = bulk_weights(0xE3BD, HEAD_ROWS, HEAD_K)
    torch.cuda.synchronize()
    head = R.DeviceHead(w, HEAD_K, HEAD_ROWS, max_batch=9, device=device.index or 0)
    yield w, head
    head.close()


def test_full_tensor(device, full_head):
    w, head = full_head
    g = np.random.default_rng(21)
    tokens = [0, HEAD_ROWS - 1, 1, 63, 64, 248319 - 64] + g.integers(0, HEAD_ROWS, 2000).tolist()
    print("embed full tensor, %d tokens" % len(tokens), flush=True)
    assert bits_equal(embed(head, tokens, device), O.embed_rows(w, HEAD_K, tokens))


def test_drawn_tokens_feed_the_lookup(device, full_head):
    # head -> sampler -> lookup, all in HBM: the next step's input rows come
    # from the tokens the sampler drew, with no host round trip.
    w, head = full_head
    g = np.random.default_rng(22)
    t = 9
    x = (g.standard_normal((t, HEAD_K)) * 2.0).astype(np.float32)
    logits = head.logits(torch.from_numpy(x).to(device))
    settings = [R.sampling(0.7, 40, 0.9, 0.0, 1.0, 64, 0) for _ in range(t)]
    uniforms = g.random(t).astype(np.float32)
    ctx = R.DeviceSampler(t, HEAD_ROWS, max_window=64)
    ctx.configure(settings)
    tok = torch.empty(t, dtype=torch.int32, device=device)
    kept = torch.empty(t, dtype=torch.int32, device=device)
    used = torch.empty(t, dtype=torch.uint8, device=device)
    ctx.sample_rows(logits, t, logits.stride(0), tok, kept, used, uniforms=torch.from_numpy(uniforms).to(device),
                    vocab=HEAD_ROWS)
    emb = head.embed(tok)  # stream-ordered after the draw
    torch.cuda.synchronize()
    want = O.pick_rows(O.q6k_matvec(w, HEAD_K, x), [as_oracle_settings(s) for s in settings], uniforms=uniforms)
    assert np.array_equal(tok.cpu().numpy().view(np.uint32), want["token"])
    assert bits_equal(emb.cpu().numpy(), O.embed_rows(w, HEAD_K, want["token"]))
    ctx.close()
