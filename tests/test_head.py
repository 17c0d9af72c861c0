"""The output head's oracle (oracle/head_ref.c), pinned on the CPU.

The reference's head (crates/rust-llm/src/forward.rs:932-937) quantizes the
activations (crates/llm-core/src/quant.rs:337-375) and takes Q6_K dot products
(crates/llm-core/src/kernels/mod.rs:273-300). What pins the restatement:
  - the reference tests' own check: an f64 dot of the dequantized ggml layout,
    within 1e-5 of the sum of absolute terms (crates/llm-core/tests/
    kernels.rs:172-226), on the reference's awkward and model shapes — a wrong
    nibble, lane, shift, scale index or sign lands far outside it;
  - exact known answers: saturated weights against +/-1 patterns
    (kernels.rs:400-590) have closed-form integer sums; zero weights or zero
    activations give 0 (kernels.rs:228-254); a block past k adds nothing
    (kernels.rs:256-293);
  - the AVX2 tier's arithmetic restated in numpy (unsigned quants minus 32
    times the group sums; kernels/avx2.rs:304-348), bit for bit — this pins the
    f32 line per block and its order, which the tolerance above cannot;
  - the quantizer: rows of +/-amax give +/-127 (kernels.rs:575-590), zero rows
    give d = 0, NaN is left out of the maximum and quantizes to 0, halves round
    away from zero, and a numpy restatement matches on random rows.
"""
import numpy as np
import pytest

import oracle as O
from head_fixtures import (AWKWARD_SHAPES, QK, SAT_PATTERNS, XorShiftRng, avx2_head, numpy_quantize,
                           random_weights, reference_dot, saturated_activations, saturated_known_answer,
                           saturated_weights, signed_row)


def _check_against_reference(k, rows, seed, t=1):
    nb = -(-k // QK)
    rng = XorShiftRng(seed)
    w = random_weights(rng, nb * rows)
    x = np.stack([signed_row(rng, k) for _ in range(t)])
    got = O.q6k_matvec(w, k, x)
    d, qs, bs = O.quantize_rows(x)
    stride = nb * 210
    for tt in range(t):
        for r in range(rows):
            want, mag = reference_dot(w[r * stride:(r + 1) * stride], k, d[tt], qs[tt])
            tol = max(mag * 1e-5, 1e-12)
            assert abs(float(got[tt, r]) - want) <= tol, (k, rows, seed, tt, r, got[tt, r], want, tol)
    return w, x, got, (d, qs, bs)


@pytest.mark.parametrize("i", range(len(AWKWARD_SHAPES)))
def test_awkward_shapes_match_the_f64_reference(i):
    k, rows = AWKWARD_SHAPES[i]
    _check_against_reference(k, rows, 0x51ED + i)


def test_model_width_rows_match_the_f64_reference():
    # k of the head (2560) and of ffn_down (9216), a few hundred rows each.
    _check_against_reference(2560, 300, 0x51A9E, t=2)
    _check_against_reference(9216, 40, 0x51A9F)


@pytest.mark.parametrize("k,rows,t", [(2560, 200, 3), (300, 50, 2), (16384, 8, 1), (37, 20, 5)])
def test_avx2_decomposition_gives_the_oracle_bits(k, rows, t):
    nb = -(-k // QK)
    rng = XorShiftRng(0xBA7C4 + k)
    w = random_weights(rng, nb * rows)
    x = np.stack([signed_row(rng, k) for _ in range(t)])
    got = O.q6k_matvec(w, k, x)
    d, qs, bs = O.quantize_rows(x)
    want = avx2_head(w, k, d, qs, bs)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("k", [2560, 300, 256])
def test_saturation_extremes_have_closed_form_answers(k):
    nb = -(-k // QK)
    x = saturated_activations(k, 4)
    d, qs, _ = O.quantize_rows(x)
    assert np.all(np.abs(qs[:, :k].astype(np.int32)) == 127)
    assert np.all(qs[:, k:] == 0)
    for wi, s in enumerate((127, -128)):
        w = saturated_weights(nb * 3)[wi]
        got = O.q6k_matvec(w, k, x)
        for tt in range(4):
            want = saturated_known_answer(k, SAT_PATTERNS[tt], s)
            assert np.all(got[tt] == want), (k, s, tt, got[tt], want)
    # Alternating signs zero every group sum: the output is exactly 0.
    assert saturated_known_answer(k, SAT_PATTERNS[1], 127) == 0.0


def test_zero_activations_and_zero_weights_give_zero():
    k = 512
    rng = XorShiftRng(7)
    w = random_weights(rng, 2)
    assert O.q6k_matvec(w, k, np.zeros((1, k), np.float32))[0, 0] == 0.0
    x = signed_row(rng, k)[None, :]
    assert O.q6k_matvec(np.zeros(2 * 210, np.uint8), k, x)[0, 0] == 0.0


def test_a_block_past_k_adds_nothing():
    short, long_ = QK, QK + 5
    rng = XorShiftRng(0xBEEF)
    w = random_weights(rng, 2)
    x = signed_row(rng, short)
    a = O.q6k_matvec(w[:210], short, x[None, :])
    b = O.q6k_matvec(w, long_, np.concatenate([x, np.zeros(5, np.float32)])[None, :])
    assert a.view(np.uint32)[0, 0] == b.view(np.uint32)[0, 0]


def test_quantizer_known_answers():
    amax = np.float32(3.25)
    x = np.zeros((1, 256), np.float32)
    x[0, 0], x[0, 1], x[0, 2] = amax, -amax, 0.0
    d, qs, bs = O.quantize_rows(x)
    assert d[0, 0] == amax / np.float32(127.0)
    assert qs[0, 0] == 127 and qs[0, 1] == -127 and qs[0, 2] == 0
    # amax 127 makes id exactly 1: halves round away from zero.
    x = np.zeros((1, 300), np.float32)
    x[0, :6] = [127.0, 0.5, -0.5, 1.5, -2.5, 2.4999998]
    d, qs, bs = O.quantize_rows(x)
    assert list(qs[0, :6]) == [127, 1, -1, 2, -3, 2]
    assert bs[0, 0, 0] == 127 + 1 - 1 + 2 - 3 + 2
    # The second block holds 44 values of 300 and zeros after them.
    assert np.all(qs[0, 256 + 44:] == 0)
    # Zero rows: d = 0 and every quant 0.
    d, qs, bs = O.quantize_rows(np.zeros((2, 256), np.float32))
    assert np.all(d == 0) and np.all(qs == 0) and np.all(bs == 0)
    # NaN is left out of the maximum and quantizes to 0.
    x = np.full((1, 256), 0.5, np.float32)
    x[0, 3] = np.nan
    x[0, 9] = -2.0
    d, qs, bs = O.quantize_rows(x)
    assert d[0, 0] == np.float32(2.0) / np.float32(127.0)
    assert qs[0, 3] == 0 and qs[0, 9] == -127
    # An infinity makes d infinite and id 0: every quant is 0 (inf * 0 is NaN).
    x = np.ones((1, 256), np.float32)
    x[0, 5] = np.inf
    d, qs, bs = O.quantize_rows(x)
    assert np.isinf(d[0, 0]) and np.all(qs == 0)


@pytest.mark.parametrize("k", [1, 37, 255, 256, 257, 2560, 9216])
def test_quantizer_matches_numpy_restatement(k):
    g = np.random.default_rng(k)
    x = (g.standard_normal((5, k)) * g.uniform(0.01, 50, (5, 1))).astype(np.float32)
    x[1, :: max(1, k // 7)] = np.nan
    x[2] = 0.0
    d, qs, bs = O.quantize_rows(x)
    d2, qs2, bs2 = numpy_quantize(x)
    assert np.array_equal(d.view(np.uint32), d2.view(np.uint32))
    assert np.array_equal(qs, qs2)
    assert np.array_equal(bs, bs2)


def test_f16_scale_decoding():
    bits = np.arange(0, 1 << 16, 37, dtype=np.uint16)
    want = bits.view(np.float16).astype(np.float32)
    got = np.array([O.f16_to_f32(b) for b in bits], np.float32)
    finite = np.isfinite(want)
    assert np.array_equal(got[finite].view(np.uint32), want[finite].view(np.uint32))
    assert np.all(np.isnan(got[np.isnan(want)]))
    assert np.array_equal(got[np.isinf(want)], want[np.isinf(want)])
