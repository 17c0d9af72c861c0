"""Inputs and independent checks for the Q6_K output head, shared by the CPU
pins of the oracle (test_head.py) and the device parity tests
(test_gpu_head.py).

Restated from the reference's kernel tests (crates/llm-core/tests/kernels.rs):
the xorshift64* generator and random well-formed weights (:45-95), the
dequantize-then-f64 reference with its tolerance (:130-200), the saturation
fixtures (:507-590). Plus a numpy restatement of the AVX2 tier's integer
decomposition (crates/llm-core/src/kernels/avx2.rs:304-348: unsigned 6-bit
quants dotted with the activations, minus 32 times the sub-block scales dotted
with the activation group sums), which must give the oracle's bits.
"""
import numpy as np

QK = 256
Q6K_BYTES = 210
M64 = (1 << 64) - 1

# Shapes as (k, rows) (kernels.rs:22-40).
AWKWARD_SHAPES = [(256, 1), (1, 1), (32, 3), (37, 3), (255, 2), (257, 2), (300, 4), (512, 5), (8192, 2),
                  (16384, 1)]
MODEL_SHAPES = [(2560, 8192), (2560, 9216), (9216, 2560), (4096, 2560), (2560, 1024)]
HEAD_K, HEAD_ROWS = 2560, 248320  # token_embd [2560, 248320] Q6_K (docs/models.md:107)


class XorShiftRng:
    """xorshift64* (kernels.rs:45-71)."""

    def __init__(self, seed):
        self.s = seed | 1

    def next_u64(self):
        x = self.s
        x ^= x >> 12
        x ^= (x << 25) & M64
        x ^= x >> 27
        self.s = x
        return (x * 0x2545F4914F6CDD1D) & M64

    def byte(self):
        return (self.next_u64() >> 33) & 0xFF

    def signed(self):
        """Uniform in [-1, 1), f32."""
        return np.float32(np.float32(self.next_u64() >> 40) / np.float32(1 << 23) - np.float32(1.0))

    def bytes(self, n):
        return [self.byte() for _ in range(n)]


def f16_bytes(x):
    return np.array([x], np.float32).astype(np.float16).view(np.uint8).tolist()


def random_weights(rng, n):
    """n Q6_K blocks: 208 random bytes, then d = f16(signed * 0.01)
    (kernels.rs:78-82)."""
    out = []
    for _ in range(n):
        out += rng.bytes(208)
        out += f16_bytes(rng.signed() * np.float32(0.01))
    return np.array(out, np.uint8)


def bulk_weights(seed, rows, k):
    """A full-size random tensor (numpy generator; the byte-per-call generator
    above is too slow for 500 MB): random quant and scale bytes, d uniform in
    [-0.01, 0.01) as f16, as the reference's fixture draws it."""
    nb = -(-k // QK)
    g = np.random.default_rng(seed)
    w = g.integers(0, 256, size=(rows * nb, Q6K_BYTES), dtype=np.uint8)
    d = (g.random(rows * nb, dtype=np.float32) * 2 - 1) * np.float32(0.01)
    w[:, 208:210] = d.astype(np.float16).view(np.uint8).reshape(-1, 2)
    return w.reshape(-1)


def signed_row(rng, n, scale=3.0):
    return np.array([rng.signed() * np.float32(scale) for _ in range(n)], np.float32)


# ------------------------------------------------------------- reference

def dequantize(row, nb):
    """The ggml Q6_K layout to f32 (kernels.rs:130-150)."""
    blocks = np.asarray(row, np.uint8).reshape(nb, Q6K_BYTES)
    out = np.zeros((nb, QK), np.float32)
    d = blocks[:, 208:210].copy().view(np.float16).astype(np.float32)[:, 0]
    for n in range(2):
        ql = blocks[:, n * 64:n * 64 + 64].astype(np.int32)
        qh = blocks[:, 128 + n * 32:128 + n * 32 + 32].astype(np.int32)
        sc = blocks[:, 192 + n * 8:192 + n * 8 + 8].view(np.int8).astype(np.float32)
        l = np.arange(32)
        isx = l // 16
        q1 = ((ql[:, l] & 0xF) | ((qh[:, l] & 3) << 4)) - 32
        q2 = ((ql[:, 32 + l] & 0xF) | (((qh[:, l] >> 2) & 3) << 4)) - 32
        q3 = ((ql[:, l] >> 4) | (((qh[:, l] >> 4) & 3) << 4)) - 32
        q4 = ((ql[:, 32 + l] >> 4) | (((qh[:, l] >> 6) & 3) << 4)) - 32
        for o, q, s in ((0, q1, isx), (32, q2, isx + 2), (64, q3, isx + 4), (96, q4, isx + 6)):
            out[:, n * 128 + o:n * 128 + o + 32] = (d[:, None] * sc[:, s]) * q.astype(np.float32)
    return out.reshape(-1)


def reference_dot(row, k, d, qs):
    """(f64 dot, f64 sum of |terms|) of one weight row with one quantized
    activation row (kernels.rs:172-186)."""
    nb = -(-k // QK)
    w = dequantize(row, nb).astype(np.float64)
    x = (np.repeat(d, QK) * qs.astype(np.float32)).astype(np.float64)
    terms = w[:k] * x[:k]
    return terms.sum(), np.abs(terms).sum()


def avx2_head(w, k, d, qs, bsums):
    """The AVX2 tier's arithmetic (avx2.rs:304-348, :493-523) in numpy: per
    block, isum = sum(u6 * a * s) - 32 * sum(s * bsum) with u6 the unsigned
    6-bit quants (exact in int64), then (act.d * w.d) * f32(isum) accumulated in
    f32, block by block from 0. Returns out [t][rows]."""
    nb = -(-k // QK)
    blocks = np.asarray(w, np.uint8).reshape(-1, nb, Q6K_BYTES)
    rows = blocks.shape[0]
    ql = blocks[:, :, 0:128].astype(np.int64)
    qh = blocks[:, :, 128:192].astype(np.int64)
    sc = blocks[:, :, 192:208].view(np.int8).astype(np.int64)
    dw = blocks[:, :, 208:210].copy().view(np.float16).astype(np.float32)[:, :, 0]
    u6 = np.zeros((rows, nb, QK), np.int64)
    for h in range(2):
        for g in range(4):
            qlv = ql[:, :, 64 * h + 32 * (g % 2):64 * h + 32 * (g % 2) + 32]
            nib = qlv & 0xF if g < 2 else (qlv >> 4) & 0xF
            high = (qh[:, :, 32 * h:32 * h + 32] >> (2 * g)) & 3
            u6[:, :, 128 * h + 32 * g:128 * h + 32 * g + 32] = nib | (high << 4)
    t = d.shape[0]
    a = qs.reshape(t, nb, QK).astype(np.int64)
    out = np.zeros((t, rows), np.float32)
    scale_per_value = np.repeat(sc, 16, axis=2)  # [rows][nb][256]
    for tt in range(t):
        raw = np.einsum("rbi,bi->rb", u6 * scale_per_value, a[tt])
        bias = np.einsum("rbj,bj->rb", sc, bsums[tt].astype(np.int64))
        isum = raw - 32 * bias
        assert np.all(np.abs(isum) < 2 ** 31)
        acc = np.zeros(rows, np.float32)
        for ib in range(nb):
            scale = np.float32(d[tt, ib]) * dw[:, ib]
            acc = acc + scale * isum[:, ib].astype(np.float32)
        out[tt] = acc
    return out


def numpy_quantize(x):
    """quant.rs:337-375 in numpy (vectorised; independent of the C oracle)."""
    x = np.asarray(x, np.float32)
    t, k = x.shape
    nb = -(-k // QK)
    pad = np.zeros((t, nb * QK), np.float32)
    pad[:, :k] = x
    blocks = pad.reshape(t, nb, QK)
    a = np.abs(blocks)
    amax = np.where(np.isnan(a), np.float32(0), a).max(axis=2).astype(np.float32)
    d = (amax / np.float32(127.0)).astype(np.float32)
    with np.errstate(divide="ignore"):
        idv = np.where(amax > 0, np.float32(127.0) / amax, np.float32(0)).astype(np.float32)
    with np.errstate(invalid="ignore"):
        p = (blocks * idv[:, :, None]).astype(np.float32)
        # Half away from zero; p + 0.5 is exact in f64 for every f32 p.
        p64 = p.astype(np.float64)
        r = np.where(p64 >= 0, np.floor(p64 + 0.5), np.ceil(p64 - 0.5))
        r = np.clip(r, -127, 127)
        q = np.where(np.isnan(r), 0, r).astype(np.int8)
    bs = q.reshape(t, nb, 16, 16).astype(np.int16).sum(axis=3).astype(np.int16)
    return d, q.reshape(t, nb * QK), bs


# ------------------------------------------------------------ saturation

def saturated_weights(n):
    """n blocks with every quant at 63 and every sub-block scale at +127 or
    -128, d = 0.0625 (kernels.rs:514-558, the Q6_K arm)."""
    out = []
    for s in (0x7F, 0x80):
        blk = [0xFF] * 128 + [0xFF] * 64 + [s] * 16 + f16_bytes(0.0625)
        out.append(np.array(blk * n, np.uint8))
    return out


SAT_PATTERNS = [
    lambda i: 1.0,
    lambda i: 1.0 if i % 2 == 0 else -1.0,
    lambda i: 1.0 if (i // 16) % 2 == 0 else -1.0,
    lambda i: -1.0 if (i // 128) % 3 == 0 else 1.0,
]


def saturated_activations(k, t):
    """t rows of +/-1 (pattern t % 4), which quantize to +/-127 exactly
    (kernels.rs:560-590)."""
    return np.array([[SAT_PATTERNS[r % 4](i) for i in range(k)] for r in range(t)], np.float32)


def saturated_known_answer(k, pattern, s):
    """The head's output for saturated weights (q - 32 = 31 everywhere, scale
    s, d = 1/16) and a +/-1 pattern: isum per block is s * 31 * 127 * (sum of
    the pattern's signs over the block's first k values), exact integers; the
    f32 line then applies (1/127 as f32 * 1/16) * isum block by block."""
    nb = -(-k // QK)
    ad = np.float32(1.0) / np.float32(127.0)  # amax 1: d = 1/127
    scale = ad * np.float32(0.0625)
    acc = np.float32(0.0)
    for ib in range(nb):
        lo, hi = ib * QK, min(k, ib * QK + QK)
        signs = sum(int(pattern(i)) for i in range(lo, hi))
        isum = s * 31 * 127 * signs
        acc = acc + scale * np.float32(isum)
    return acc
