"""The full path's bulk loops compute the reference's (l - max) / t
(sample.rs:309) as a product with 1 / t when t is a power of two whose
reciprocal is a normal f32 (TempScale in full_kernels.h). Both are the exact
quotient rounded once, so they agree bit for bit; this pins that claim and
the reciprocal's bit construction on the host, including subnormal results,
the largest finite values and the ends of the exponent range."""
import numpy as np


def recip_bits(t):
    """1 / t as TempScale builds it from t's biased exponent e: (254 - e) << 23."""
    e = (np.float32(t).view(np.uint32) >> np.uint32(23)) & np.uint32(0xFF)
    return np.uint32((254 - int(e)) << 23).view(np.float32)


def test_product_with_the_reciprocal_equals_the_division():
    rng = np.random.default_rng(7)
    bits = rng.integers(0, 2**32, 400_000, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    x = x[np.isfinite(x)]
    specials = np.array([0.0, -0.0, 1.0, -1.0, 3.4028235e38, -3.4028235e38, 1e-45, -1e-45, 1.1754944e-38,
                         -30.5, -104.0], np.float32)
    x = np.concatenate([x, specials])
    for k in list(range(-125, 126, 7)) + [-125, -1, 0, 1, 125]:
        t = np.float32(2.0) ** np.float32(k)
        inv = recip_bits(t)
        assert inv == np.float32(1.0) / t
        with np.errstate(over="ignore", under="ignore"):
            q = x / t
            m = x * inv
        assert np.array_equal(q.view(np.uint32), m.view(np.uint32)), k


def test_non_powers_of_two_are_not_taken():
    # The bit test of TempScale: sign clear, mantissa zero, biased exponent 2..252.
    def pow2(t):
        b = int(np.float32(t).view(np.uint32))
        e = (b >> 23) & 0xFF
        return (b & 0x807FFFFF) == 0 and 2 <= e <= 252
    assert pow2(1.0) and pow2(0.5) and pow2(2.0) and pow2(2.0 ** -125) and pow2(2.0 ** 125)
    for t in (0.6, 0.7, 1.5, -1.0, -2.0, 0.0, 2.0 ** -126, 2.0 ** 126, 2.0 ** 127, float("inf"), float("nan"),
              1e-40):
        assert not pow2(t), t
