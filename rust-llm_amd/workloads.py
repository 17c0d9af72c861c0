"""The sampler's five workload shapes: synthetic logits, windows, per-row
settings and uniforms.

Logits and windows come from librl_workloads.so (deterministic per row, see
csrc/workloads.c for the distributions); uniforms come from the reference's Rng
(sample.rs:368-404) as implemented by librl_sampler.so: each row of an
independent batch has its own Sampler seeded `seed_base + row`, the
speculative-verify batch walks one stream in row order.
"""
import ctypes
import os

import numpy as np

import rl_sampler

HERE = os.path.dirname(os.path.abspath(__file__))
WL_PATH = os.path.join(HERE, "librl_workloads.so")

V1 = 151936
V2 = 248320
WINDOW = 64

WL_SINGLE, WL_ZIPF, WL_SPIKES, WL_VERIFY, WL_TIES = 1, 2, 3, 4, 5

_wl = None


def wl_lib():
    global _wl
    if _wl is None:
        if not os.path.exists(WL_PATH):
            raise RuntimeError("%s is missing: build it with `make -C rust-llm_amd`" % WL_PATH)
        L = ctypes.CDLL(WL_PATH)
        L.wl_generate.argtypes = [ctypes.c_int, ctypes.c_uint64, ctypes.c_uint32, ctypes.c_uint32,
                                  ctypes.c_uint32, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                  ctypes.c_int]
        L.wl_verify_drafts.argtypes = [ctypes.c_uint64, ctypes.c_uint32, ctypes.c_void_p, ctypes.c_uint32]
        L.wl_verify_history.argtypes = [ctypes.c_uint64, ctypes.c_uint32, ctypes.c_void_p]
        _wl = L
    return _wl


class Workload:
    """One benchmark shape. `settings(row)` is the row's Sampling; the whole
    batch is rows x vocab f32 logits."""

    def __init__(self, name, kind, rows, vocab, seed, settings, uniform_seed, one_stream=False, description=""):
        self.name = name
        self.kind = kind
        self.rows = rows
        self.vocab = vocab
        self.seed = seed
        self._settings = settings
        self.uniform_seed = uniform_seed
        self.one_stream = one_stream
        self.description = description

    def settings(self, row=0):
        s = self._settings(row)
        return s

    def settings_list(self, row0=0, rows=None):
        rows = self.rows - row0 if rows is None else rows
        return [self.settings(row0 + r) for r in range(rows)]

    def generate(self, row0=0, rows=None, threads=None):
        """Returns (logits [rows][vocab] f32, windows [rows][64] u32, wlen [rows] u32)."""
        rows = self.rows - row0 if rows is None else rows
        threads = threads or min(16, os.cpu_count() or 1)
        logits = np.empty((rows, self.vocab), np.float32)
        windows = np.empty((rows, WINDOW), np.uint32)
        wlen = np.empty(rows, np.uint32)
        rc = wl_lib().wl_generate(self.kind, self.seed, self.vocab, row0, rows, logits.ctypes.data,
                                  windows.ctypes.data, wlen.ctypes.data, threads)
        if rc != 0:
            raise RuntimeError("workload generation failed")
        return logits, windows, wlen

    def uniforms(self, row0=0, rows=None):
        """The value each row's Rng::next_f32 would give for its draw."""
        rows = self.rows - row0 if rows is None else rows
        out = np.empty(rows, np.float32)
        if self.one_stream:
            r = rl_sampler.RngStream(self.uniform_seed)
            vals = [r.next_f32() for _ in range(row0 + rows)]
            out[:] = vals[row0:]
        else:
            for i in range(rows):
                out[i] = rl_sampler.RngStream(self.uniform_seed + row0 + i).next_f32()
        return out

    def drafts(self):
        d = np.zeros(self.rows - 1, np.uint32)
        wl_lib().wl_verify_drafts(self.seed, self.vocab, d.ctypes.data, d.size)
        return d

    def history(self):
        h = np.zeros(WINDOW, np.uint32)
        wl_lib().wl_verify_history(self.seed, self.vocab, h.ctypes.data)
        return h

    def algorithmic_bytes(self, kept_total):
        """HBM bytes one call must move: per row the logits once, the window,
        the uniform, the token and the kept count; plus one (id, prob) pair per
        candidate the call keeps. `kept_total` is the sum over rows of the
        kept counts the call returned (Sampler::kept, sample.rs:342-347), or 0
        when the candidates are not written."""
        per_row = self.vocab * 4 + WINDOW * 4 + 4 + 4 + 4
        return self.rows * per_row + int(kept_total) * 8


S = rl_sampler.sampling

WORKLOADS = {
    "single": Workload(
        "single", WL_SINGLE, 1, V1, 0x5EED0001,
        lambda r: S(0.6, 20, 0.95, 0.0, 1.0, 64, 1001), 1001,
        description="1 x 151936, N(0, 2.5^2) + 8 spikes at +12; defaults (T 0.6, top-k 20, top-p 0.95)"),
    "single_greedy": Workload(
        "single_greedy", WL_SINGLE, 1, V1, 0x5EED0001,
        lambda r: rl_sampler.greedy_sampling(), 1001,
        description="1 x 151936, same logits, greedy"),
    "zipf": Workload(
        "zipf", WL_ZIPF, 64, V1, 0x5EED0002,
        lambda r: S(1.0, 0, 0.95, 0.05, 1.1, 64, 2000 + r), 2000,
        description="64 x 151936, N(0, 3^2) - 1.1 ln(rank); T 1, top-k 0, top-p 0.95, min-p 0.05, penalty 1.1/64"),
    "spikes": Workload(
        "spikes", WL_SPIKES, 1024, V2, 0x5EED0003,
        lambda r: S(0.6, 20, 0.95, 0.0, 1.2, 64, 3000 + r), 3000,
        description="1024 x 248320, N(0, 2^2) + 16 spikes in [8, 14); T 0.6, top-k 20, top-p 0.95, penalty 1.2/64"),
    "verify": Workload(
        "verify", WL_VERIFY, 9, V1, 0x5EED0004,
        lambda r: S(0.6, 20, 0.95, 0.0, 1.3, 64, 4000), 4000, one_stream=True,
        description="9 x 151936 speculative-verify rows; penalty 1.3 over history + drafts; T 0.6/top-k 20/top-p 0.95"),
    "verify_greedy": Workload(
        "verify_greedy", WL_VERIFY, 9, V1, 0x5EED0004,
        lambda r: rl_sampler.greedy_sampling(repeat_penalty=1.3, repeat_last_n=64), 4000, one_stream=True,
        description="9 x 151936 speculative-verify rows, greedy with penalty 1.3"),
    "ties": Workload(
        "ties", WL_TIES, 256, V1, 0x5EED0005,
        lambda r: S(1.0, 0, 0.99, 0.02, 1.0, 64, 5000 + r), 5000,
        description="256 x 151936 bf16-grid logits, 40% tied at -0.0234375; T 1, top-k 0, top-p 0.99, min-p 0.02"),
}

BENCH_WORKLOAD = "spikes"


# The output head's workload: the tied embedding token_embd [2560, 248320]
# Q6_K of the reference's model (docs/models.md:107) with synthetic weights.
HEAD_K = 2560
HEAD_ROWS = V2
Q6K_BLOCK_BYTES = 210


def head_weights(seed=0x7E4D, rows=HEAD_ROWS, k=HEAD_K):
    """A Q6_K tensor of `rows` rows of `k` values as the GGUF stores it: random
    quant and scale bytes (every bit pattern is a valid block) and block scales
    d uniform in [-0.01, 0.01) as f16, drawn from numpy's PCG64 with `seed`."""
    nb = -(-k // 256)
    g = np.random.default_rng(seed)
    w = g.integers(0, 256, size=(rows * nb, Q6K_BLOCK_BYTES), dtype=np.uint8)
    d = (g.random(rows * nb, dtype=np.float32) * 2 - 1) * np.float32(0.01)
    w[:, 208:210] = d.astype(np.float16).view(np.uint8).reshape(-1, 2)
    return w.reshape(-1)


def head_inputs(t, seed=0x4EAD, k=HEAD_K):
    """t normed hidden rows, N(0, 1.5^2) f32."""
    return (np.random.default_rng(seed).standard_normal((t, k)) * 1.5).astype(np.float32)
