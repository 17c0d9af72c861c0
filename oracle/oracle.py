"""ORACLE loader — test infrastructure only.

ctypes bindings for liboracle.so, the C restatement of rust-llm's sampler
(crates/rust-llm/src/sample.rs) and of its tests' naive f64 reference
(crates/rust-llm/tests/sample.rs:16-83). Only tests/, the smoke check and
bench.py's CPU-baseline leg import this module, and only to check results
against (or, in bench.py, to time the CPU baseline).
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")


class Sampling(ctypes.Structure):
    """Same layout as rl_sampling; mirrors Sampling (sample.rs:50-67)."""

    _fields_ = [
        ("temperature", ctypes.c_float),
        ("top_p", ctypes.c_float),
        ("min_p", ctypes.c_float),
        ("repeat_penalty", ctypes.c_float),
        ("top_k", ctypes.c_uint64),
        ("repeat_last_n", ctypes.c_uint64),
        ("seed", ctypes.c_uint64),
    ]


class Rng(ctypes.Structure):
    _fields_ = [("s", ctypes.c_uint64 * 4)]


_P = ctypes.POINTER
_f32p = _P(ctypes.c_float)
_f64p = _P(ctypes.c_double)
_u32p = _P(ctypes.c_uint32)
_u8p = _P(ctypes.c_uint8)
_u64p = _P(ctypes.c_uint64)
_lib = None


def build():
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        L.orc_splitmix64_next.argtypes = [_u64p]
        L.orc_splitmix64_next.restype = ctypes.c_uint64
        L.orc_rng_seeded.argtypes = [_P(Rng), ctypes.c_uint64]
        L.orc_rng_from_state.argtypes = [_P(Rng), _u64p]
        L.orc_rng_next_u64.argtypes = [_P(Rng)]
        L.orc_rng_next_u64.restype = ctypes.c_uint64
        L.orc_rng_next_f32.argtypes = [_P(Rng)]
        L.orc_rng_next_f32.restype = ctypes.c_float
        L.orc_argmax.argtypes = [_f32p, ctypes.c_size_t]
        L.orc_argmax.restype = ctypes.c_uint32
        L.orc_pick_rows.argtypes = [
            _f32p, ctypes.c_uint64, ctypes.c_size_t, ctypes.c_size_t, _P(Sampling), ctypes.c_int,
            _u32p, ctypes.c_size_t, _u32p, _f32p, _u32p, _u32p, _u8p, _u32p, _f32p, ctypes.c_size_t,
        ]
        L.orc_pick_rows.restype = ctypes.c_int
        L.orc_sampler_new.argtypes = [ctypes.c_size_t, _P(Sampling)]
        L.orc_sampler_new.restype = ctypes.c_void_p
        L.orc_sampler_free.argtypes = [ctypes.c_void_p]
        L.orc_sampler_reset.argtypes = [ctypes.c_void_p]
        L.orc_sampler_remember.argtypes = [ctypes.c_void_p, ctypes.c_uint32]
        L.orc_sampler_sample.argtypes = [ctypes.c_void_p, _f32p, ctypes.c_size_t]
        L.orc_sampler_sample.restype = ctypes.c_uint32
        L.orc_sampler_candidates.argtypes = [ctypes.c_void_p, _P(_u32p), _P(_f32p)]
        L.orc_sampler_candidates.restype = ctypes.c_size_t
        L.orc_sampler_filled.argtypes = [ctypes.c_void_p]
        L.orc_sampler_filled.restype = ctypes.c_size_t
        L.orc_sampler_recent.argtypes = [ctypes.c_void_p]
        L.orc_sampler_recent.restype = _u32p
        L.orc_sampler_rng_state.argtypes = [ctypes.c_void_p, _u64p]
        L.orc_naive.argtypes = [_f32p, ctypes.c_size_t, _P(Sampling), _u32p, ctypes.c_size_t, _u32p, _f64p]
        L.orc_naive.restype = ctypes.c_size_t
        L.orc_test_logits.argtypes = [_f32p, ctypes.c_size_t, ctypes.c_uint64, ctypes.c_float]
        L.orc_alloc_test_logits.argtypes = [_f32p, ctypes.c_size_t, ctypes.c_uint64]
        L.orc_top_probability.argtypes = [_f32p, ctypes.c_size_t, _f32p]
        L.orc_top_probability.restype = ctypes.c_uint32
        L.orc_top_probability_rows.argtypes = [_f32p, ctypes.c_uint64, ctypes.c_size_t, ctypes.c_size_t, _u32p,
                                               _f32p]
        L.orc_libm_expf.argtypes = [ctypes.c_float]
        L.orc_libm_expf.restype = ctypes.c_float
        L.orc_expf_compare.argtypes = [_f32p, ctypes.c_uint32, ctypes.c_uint64, _u32p, ctypes.c_uint64]
        L.orc_expf_compare.restype = ctypes.c_uint64
        L.orc_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.orc_f16_to_f32.restype = ctypes.c_float
        L.orc_quantize_rows.argtypes = [_f32p, ctypes.c_size_t, ctypes.c_size_t, _f32p, _P(ctypes.c_int8),
                                        _P(ctypes.c_int16)]
        L.orc_q6k_matvec.argtypes = [_u8p, ctypes.c_size_t, ctypes.c_size_t, ctypes.c_size_t, _f32p,
                                     ctypes.c_size_t, _f32p]
        L.orc_q6k_matvec.restype = ctypes.c_int
        L.orc_dequantize_row.argtypes = [_u8p, ctypes.c_size_t, _f32p]
        L.orc_dequantize_row.restype = None
        _lib = L
    return _lib


def _ptr(a, t):
    return a.ctypes.data_as(t) if a is not None else None


def sampling(temperature=0.6, top_k=20, top_p=0.95, min_p=0.0, repeat_penalty=1.0, repeat_last_n=64, seed=0):
    """Sampling::default() (sample.rs:88-100) unless overridden."""
    return Sampling(temperature, top_p, min_p, repeat_penalty, top_k, repeat_last_n, seed)


GREEDY = dict(temperature=0.0, top_k=0, top_p=1.0, min_p=0.0, repeat_penalty=1.0, repeat_last_n=0, seed=0)


class OracleRng:
    """The reference's Rng (sample.rs:368-404)."""

    def __init__(self, seed=None, state=None):
        self.r = Rng()
        if state is not None:
            arr = (ctypes.c_uint64 * 4)(*state)
            lib().orc_rng_from_state(ctypes.byref(self.r), arr)
        else:
            lib().orc_rng_seeded(ctypes.byref(self.r), seed)

    def next_u64(self):
        return lib().orc_rng_next_u64(ctypes.byref(self.r))

    def next_f32(self):
        return lib().orc_rng_next_f32(ctypes.byref(self.r))

    def state(self):
        return tuple(self.r.s)


def splitmix64_stream(seed, n):
    z = ctypes.c_uint64(seed)
    return [lib().orc_splitmix64_next(ctypes.byref(z)) for _ in range(n)]


def argmax(logits):
    a = np.ascontiguousarray(logits, dtype=np.float32)
    return lib().orc_argmax(_ptr(a, _f32p), a.size)


def pick_rows(logits, settings, windows=None, wlen=None, uniforms=None, cand_cap=None):
    """Runs the restated pick over each row. `settings` is one Sampling or a
    list (one per row). Returns dict of numpy arrays."""
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    if logits.ndim == 1:
        logits = logits[None, :]
    rows, n = logits.shape
    per_row = isinstance(settings, (list, tuple))
    if per_row:
        sarr = (Sampling * rows)(*settings)
    else:
        sarr = (Sampling * 1)(settings)
    if cand_cap is None:
        cand_cap = n
    if windows is not None:
        windows = np.ascontiguousarray(windows, dtype=np.uint32)
        if windows.ndim == 1:
            windows = windows[None, :]
        wstride = windows.shape[1]
        wlen = np.ascontiguousarray(
            wlen if wlen is not None else np.full(rows, wstride), dtype=np.uint32)
    else:
        wstride = 0
        wlen = None
    uni = np.ascontiguousarray(uniforms if uniforms is not None else np.zeros(rows), dtype=np.float32)
    tok = np.zeros(rows, np.uint32)
    kept = np.zeros(rows, np.uint32)
    used = np.zeros(rows, np.uint8)
    ids = np.zeros((rows, cand_cap), np.uint32)
    probs = np.zeros((rows, cand_cap), np.float32)
    rc = lib().orc_pick_rows(
        _ptr(logits, _f32p), n, rows, n, sarr, 1 if per_row else 0,
        _ptr(windows, _u32p), wstride, _ptr(wlen, _u32p), _ptr(uni, _f32p),
        _ptr(tok, _u32p), _ptr(kept, _u32p), _ptr(used, _u8p), _ptr(ids, _u32p), _ptr(probs, _f32p), cand_cap)
    if rc != 0:
        raise RuntimeError("oracle pick failed (vocabulary mismatch or out of memory)")
    return dict(token=tok, kept=kept, used=used, ids=ids, probs=probs)


class OracleSampler:
    """The stateful Sampler (sample.rs:132-219)."""

    def __init__(self, vocab, set_):
        self.vocab = vocab
        self.h = lib().orc_sampler_new(vocab, ctypes.byref(set_))
        if not self.h:
            raise MemoryError

    def __del__(self):
        if getattr(self, "h", None) and _lib is not None:
            _lib.orc_sampler_free(self.h)
            self.h = None

    def remember(self, t):
        lib().orc_sampler_remember(self.h, t)

    def reset(self):
        lib().orc_sampler_reset(self.h)

    def sample(self, logits):
        a = np.ascontiguousarray(logits, dtype=np.float32)
        t = lib().orc_sampler_sample(self.h, _ptr(a, _f32p), a.size)
        if t == 0xFFFFFFFF:
            raise ValueError("this sampler was built for a different vocabulary")
        return t

    def candidates(self):
        ip = _u32p()
        pp = _f32p()
        n = lib().orc_sampler_candidates(self.h, ctypes.byref(ip), ctypes.byref(pp))
        ids = np.ctypeslib.as_array(ip, shape=(max(n, 1),))[:n].copy()
        probs = np.ctypeslib.as_array(pp, shape=(max(n, 1),))[:n].copy()
        return ids, probs

    def window(self):
        n = lib().orc_sampler_filled(self.h)
        if n == 0:
            return np.zeros(0, np.uint32)
        p = lib().orc_sampler_recent(self.h)
        return np.ctypeslib.as_array(p, shape=(n,)).copy()

    def rng_state(self):
        a = (ctypes.c_uint64 * 4)()
        lib().orc_sampler_rng_state(self.h, a)
        return tuple(a)


def naive(logits, set_, recent=()):
    a = np.ascontiguousarray(logits, dtype=np.float32)
    rec = np.ascontiguousarray(np.asarray(recent, dtype=np.uint32))
    ids = np.zeros(a.size, np.uint32)
    probs = np.zeros(a.size, np.float64)
    n = lib().orc_naive(_ptr(a, _f32p), a.size, ctypes.byref(set_), _ptr(rec, _u32p), rec.size,
                        _ptr(ids, _u32p), _ptr(probs, _f64p))
    return ids[:n], probs[:n]


def test_logits(n, seed, spread):
    """tests/sample.rs:87-98."""
    out = np.zeros(n, np.float32)
    lib().orc_test_logits(_ptr(out, _f32p), n, seed, spread)
    return out


def alloc_test_logits(n, seed):
    """tests/sample_allocations.rs:63-73."""
    out = np.zeros(n, np.float32)
    lib().orc_alloc_test_logits(_ptr(out, _f32p), n, seed)
    return out


def top_probability(logits):
    """forward.rs:1671-1680: (argmax, 1 / sum exp(v - max)) of one row."""
    a = np.ascontiguousarray(logits, dtype=np.float32)
    p = ctypes.c_float()
    t = lib().orc_top_probability(_ptr(a, _f32p), a.size, ctypes.byref(p))
    return int(t), np.float32(p.value)


def top_probability_rows(logits):
    a = np.ascontiguousarray(logits, dtype=np.float32)
    rows, n = a.shape
    tok = np.zeros(rows, np.uint32)
    prob = np.zeros(rows, np.float32)
    lib().orc_top_probability_rows(_ptr(a, _f32p), n, rows, n, _ptr(tok, _u32p), _ptr(prob, _f32p))
    return tok, prob


def libm_expf(x):
    return lib().orc_libm_expf(x)


def expf_compare(got, lo_bits, report_max=16):
    got = np.ascontiguousarray(got, dtype=np.float32)
    rep = np.zeros(report_max, np.uint32)
    bad = lib().orc_expf_compare(_ptr(got, _f32p), lo_bits, got.size, _ptr(rep, _u32p), report_max)
    return bad, rep[: min(bad, report_max)]


QK = 256
Q6K_BYTES = 210


def f16_to_f32(bits):
    return np.float32(lib().orc_f16_to_f32(int(bits)))


def quantize_rows(x):
    """Activations::quantize_batch (quant.rs:337-375) of x [t][k]:
    (d [t][nb] f32, qs [t][nb*256] i8, bsums [t][nb][16] i16)."""
    a = np.ascontiguousarray(x, dtype=np.float32)
    if a.ndim == 1:
        a = a[None, :]
    t, k = a.shape
    nb = -(-k // QK)
    d = np.zeros((t, nb), np.float32)
    qs = np.zeros((t, nb * QK), np.int8)
    bs = np.zeros((t, nb, 16), np.int16)
    lib().orc_quantize_rows(_ptr(a, _f32p), t, k, _ptr(d, _f32p), _ptr(qs, _P(ctypes.c_int8)),
                            _ptr(bs, _P(ctypes.c_int16)))
    return d, qs, bs


def q6k_matvec(w, k, x, row_lo=0, row_hi=None):
    """The head (forward.rs:932-937): logits [t][row_hi-row_lo] of the Q6_K
    tensor w (bytes, [rows][ceil(k/256)*210]) times the rows of x [t][k]."""
    w = np.ascontiguousarray(w, dtype=np.uint8)
    a = np.ascontiguousarray(x, dtype=np.float32)
    if a.ndim == 1:
        a = a[None, :]
    t = a.shape[0]
    assert a.shape[1] == k
    row_bytes = -(-k // QK) * Q6K_BYTES
    rows = w.size // row_bytes
    if row_hi is None:
        row_hi = rows
    assert 0 <= row_lo <= row_hi <= rows
    out = np.zeros((t, row_hi - row_lo), np.float32)
    rc = lib().orc_q6k_matvec(_ptr(w, _u8p), k, row_lo, row_hi, _ptr(a, _f32p), t, _ptr(out, _f32p))
    if rc != 0:
        raise MemoryError("orc_q6k_matvec")
    return out


def embed_rows(w, k, tokens):
    """The embedding lookup (forward.rs:1127-1138) of each token: [len][k] f32."""
    w = np.ascontiguousarray(w, dtype=np.uint8)
    row_bytes = -(-k // QK) * Q6K_BYTES
    out = np.zeros((len(tokens), k), np.float32)
    for i, t in enumerate(tokens):
        r = np.ascontiguousarray(w[int(t) * row_bytes:(int(t) + 1) * row_bytes])
        lib().orc_dequantize_row(_ptr(r, _u8p), k, _ptr(out[i], _f32p))
    return out
