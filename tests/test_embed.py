"""The embedding lookup's oracle (orc_dequantize_row, oracle/head_ref.c), pinned
on the CPU.

The reference's lookup (crates/rust-llm/src/forward.rs:1127-1138) expands one
row of the tied Q6_K `token_embd` with dequantize_row
(crates/llm-core/src/quant.rs:177-203): value = d * (float)(s * (q - 32)).
What pins the restatement:
  - the reference test's own check (crates/llm-core/tests/kernels.rs:631-668):
    against the ggml dequantization written out separately (head_fixtures.
    dequantize, which scales in f32 twice), within 1e-6 relative, on the
    reference's awkward and model widths; a wrong nibble, lane, shift, scale
    index or sign lands far outside it;
  - exact known answers: blocks packed from chosen quants and scales by the
    ggml layout's definition (a packer written here, the inverse of the
    decode) give exactly s * (q - 32) at d = 1 and that times 2^-3 at d =
    0.125; the saturated block gives 0.0625 * 127 * 31 everywhere;
  - where the two f32 forms must agree bit for bit (d a power of two, so both
    products are exact), they do;
  - nothing past k is written.
"""
import numpy as np
import pytest

import oracle as O
from head_fixtures import AWKWARD_SHAPES, MODEL_SHAPES, QK, XorShiftRng, dequantize, f16_bytes, random_weights, \
    saturated_weights


def pack_q6k(quants, scales, d):
    """One ggml Q6_K block from 256 unsigned 6-bit quants, 16 i8 scales and an
    f32 d (stored as f16). Index h*128 + g*32 + l keeps its low nibble in
    ql[h*64 + (g % 2)*32 + l] (low half for g < 2, high half otherwise) and its
    top two bits in bits 2g..2g+1 of qh[h*32 + l]."""
    quants = np.asarray(quants, np.int64)
    ql = np.zeros(128, np.int64)
    qh = np.zeros(64, np.int64)
    for i in range(QK):
        h, g, l = i // 128, (i // 32) % 4, i % 32
        ql[h * 64 + (g % 2) * 32 + l] |= (quants[i] & 15) << (4 * (g // 2))
        qh[h * 32 + l] |= (quants[i] >> 4) << (2 * g)
    sc = np.asarray(scales, np.int64) & 0xFF
    return np.concatenate([ql, qh, sc, f16_bytes(d)]).astype(np.uint8)


def test_matches_the_reference_tests_dequantization():
    rng = XorShiftRng(0x5EED5EED)
    for k in sorted({k for k, _ in AWKWARD_SHAPES + MODEL_SHAPES}):
        nb = -(-k // QK)
        row = random_weights(rng, nb)
        got = O.embed_rows(row, k, [0])[0]
        want = dequantize(row, nb)[:k]
        tol = np.abs(want) * np.float32(1e-6) + np.float32(1e-12)
        assert np.all(np.abs(got - want) <= tol), k


def test_packed_blocks_give_the_integers_exactly():
    g = np.random.default_rng(5)
    for d, scale in ((1.0, 1.0), (0.125, 0.125), (-2.0, -2.0)):
        quants = g.integers(0, 64, QK)
        scales = g.integers(-128, 128, 16)
        blk = pack_q6k(quants, scales, d)
        got = O.embed_rows(blk, QK, [0])[0]
        want = np.float32(scale) * (np.repeat(scales, 16) * (quants - 32)).astype(np.float32)
        assert np.array_equal(got, want), d
    # Every quant value and both scale extremes, at each position.
    quants = np.arange(QK) % 64
    for s in (127, -128, 1, -1, 0):
        got = O.embed_rows(pack_q6k(quants, [s] * 16, 1.0), QK, [0])[0]
        assert np.array_equal(got, (s * (quants - 32)).astype(np.float32)), s


def test_saturated_block_known_answer():
    w127, w128 = saturated_weights(2)
    assert np.all(O.embed_rows(w127, 300, [0, 1]) == np.float32(0.0625 * 127 * 31))
    assert np.all(O.embed_rows(w128, 300, [1]) == np.float32(0.0625 * -128 * 31))


def test_power_of_two_scales_agree_bit_for_bit():
    # With d a power of two, (d * s) * q in f32 and d * (s * q) are both exact;
    # they differ only in the sign of a zero (a negative scale times q = 32
    # is -0 in the two-multiply form, while s * 0 is the integer 0 here).
    g = np.random.default_rng(9)
    for e in (-14, -6, 0, 5):
        blocks = np.concatenate([pack_q6k(g.integers(0, 64, QK), g.integers(-128, 128, 16), 2.0 ** e)
                                 for _ in range(3)])
        got = O.embed_rows(blocks, 3 * QK, [0])[0]
        want = dequantize(blocks, 3)
        nz = want != 0
        assert np.array_equal(got[nz].view(np.uint32), want[nz].view(np.uint32)), e
        assert np.all(got[~nz].view(np.uint32) == 0), e  # +0: d > 0 times the integer 0


@pytest.mark.parametrize("k", [1, 37, 255, 257, 300])
def test_nothing_past_k_is_written(k):
    import ctypes
    nb = -(-k // QK)
    row = random_weights(XorShiftRng(k), nb)
    out = np.full(nb * QK + 8, np.nan, np.float32)
    O.lib().orc_dequantize_row(row.ctypes.data_as(ctypes.POINTER(ctypes.c_uint8)), k,
                               out.ctypes.data_as(ctypes.POINTER(ctypes.c_float)))
    assert not np.any(np.isnan(out[:k]))
    assert np.all(np.isnan(out[k:]))


def test_rows_are_looked_up_by_token():
    k, rows = 300, 7
    nb = -(-k // QK)
    w = random_weights(XorShiftRng(77), nb * rows)
    tokens = [6, 0, 3, 3]
    got = O.embed_rows(w, k, tokens)
    stride = nb * 210
    for i, t in enumerate(tokens):
        assert np.array_equal(got[i], O.embed_rows(w[t * stride:(t + 1) * stride], k, [0])[0])
