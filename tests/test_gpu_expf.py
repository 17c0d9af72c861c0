"""The device expf against this host's libm expf, on every f32 input.

sample.rs:309 takes `.exp()` of an f32, which Rust lowers to libm expf; the
kept probabilities and the draw depend on its exact bits. The device evaluates
the same published method in double precision (rust-llm_amd/csrc/rl_expf.h).
This compares all 2^32 bit patterns (NaN results compare equal to NaN), and
the branch-free variant that top_probability uses for its arguments l - best
(never positive, never NaN) with the general one on every such argument.
"""
import concurrent.futures as cf
import ctypes
import os
import time

import numpy as np
import pytest

import oracle as O
import rl_sampler as R

pytestmark = pytest.mark.gpu

CHUNK = 1 << 26


def test_device_expf_equals_host_libm_everywhere(device):
    import torch
    out = torch.empty(CHUNK, dtype=torch.float32, device=device)
    pool = cf.ThreadPoolExecutor(max_workers=8)
    futures = []
    t0 = time.time()
    for c in range((1 << 32) // CHUNK):
        lo = c * CHUNK
        R.expf_range(lo, out)
        host = out.cpu().numpy()

        def check(h=host, lo=lo):
            # split each chunk over workers for the libm side
            n = h.size // 8
            res = [O.expf_compare(h[i * n:(i + 1) * n], lo + i * n) for i in range(8)]
            return sum(r[0] for r in res), np.concatenate([r[1] for r in res])

        futures.append(pool.submit(check))
        while sum(not f.done() for f in futures) > 12:  # bound host memory
            time.sleep(0.01)
        if c % 16 == 15:
            print("expf: %d/64 chunks queued, %.1fs" % (c + 1, time.time() - t0), flush=True)
    bad = 0
    examples = []
    for f in futures:
        b, ex = f.result()
        bad += b
        examples.extend(int(x) for x in ex[:4])
    pool.shutdown()
    print("expf: all 2^32 inputs compared in %.1fs, %d differ" % (time.time() - t0, bad), flush=True)
    assert bad == 0, "device expf differs from libm on %d inputs, e.g. bit patterns %s" % (
        bad, [hex(x) for x in examples[:8]])


def test_branch_free_expf_equals_general_on_non_positive_inputs(device):
    """+0, and every bit pattern from -0 (0x80000000) to -inf (0xFF800000)."""
    import torch
    lib = os.path.join(os.path.dirname(os.path.abspath(__file__)), "native", "libexp2_gpu.so")
    assert os.path.exists(lib), "%s is missing: build it with `make -C tests/native`" % lib
    L = ctypes.CDLL(lib)
    L.expf_nonpos_diff.argtypes = [ctypes.c_uint32, ctypes.c_uint64, ctypes.c_void_p, ctypes.c_void_p]
    count = torch.zeros(1, dtype=torch.int32, device=device)
    stream = torch.cuda.current_stream().cuda_stream
    ranges = [(0, 1), (0x80000000, 0x7F800001)]
    for lo, n in ranges:
        for at in range(lo, lo + n, 1 << 30):
            assert L.expf_nonpos_diff(at, min(1 << 30, lo + n - at), count.data_ptr(), stream) == 0
    torch.cuda.synchronize()
    assert int(count.item()) == 0, "branch-free expf differs on %d non-positive inputs" % int(count.item())
