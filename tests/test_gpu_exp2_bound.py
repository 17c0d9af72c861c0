"""The hardware base-2 exponential against exp2 in f64, on every f32 input
the min-p path can give it.

k_full_pass (rust-llm_amd/csrc/full_kernels.h) bounds the reference's mass
from a sum of v_exp_f32 terms and assumes each is within 2^-21 relative of the
exact 2^z for results at or above 2^-126 (HW_EXP2_REL, minp_bound.h), and
within 2^-126 absolute below that (flushed or subnormal). It gives v_exp_f32
two kinds of argument: the terms' z <= 0, and, in the rescaling of a partial
sum as the running maximum rises, the fraction z - floor(z) in [0, 1). This
checks every f32 in [-160, 0] (bit patterns 0x80000000 .. 0xC3200000), which
covers every term that is not 0 in f32 and the flush region beyond, and every
f32 in [0, 1) (bit patterns 0x00000000 .. 0x3F7FFFFF).
"""
import ctypes
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "native", "libexp2_gpu.so")
CHUNK = 1 << 25
RANGES = [(0x80000000, 0xC3200000),  # -0.0 .. -160.0: the terms
          (0x00000000, 0x3F800000)]  # +0.0 .. 1 - 2^-24: the rescalings' fractions


def test_hardware_exp2_is_within_the_assumed_bound(device):
    import torch
    assert os.path.exists(LIB), "%s is missing: build it with `make -C tests/native`" % LIB
    L = ctypes.CDLL(LIB)
    L.exp2_hw_range.argtypes = [ctypes.c_uint32, ctypes.c_uint64, ctypes.c_void_p, ctypes.c_void_p]
    out = torch.empty(CHUNK, dtype=torch.float32, device=device)
    worst_rel = 0.0
    worst_abs = 0.0
    for lo, n in ((lo, min(CHUNK, HI - lo)) for LO, HI in RANGES for lo in range(LO, HI, CHUNK)):
        assert L.exp2_hw_range(lo, n, out.data_ptr(), torch.cuda.current_stream().cuda_stream) == 0
        bits = torch.arange(lo, lo + n, dtype=torch.int64, device=device).to(torch.int32)
        z = bits.view(torch.float32).double()
        ref = torch.exp2(z)
        got = out[:n].double()
        normal = ref >= 2.0 ** -126
        if bool(normal.any()):
            rel = ((got - ref).abs() / ref)[normal].max().item()
            worst_rel = max(worst_rel, rel)
        if bool((~normal).any()):
            ab = (got - ref).abs()[~normal].max().item()
            worst_abs = max(worst_abs, ab)
    print("v_exp_f32 on [-160, 0] and [0, 1): worst relative error %.3g (%.2f x 2^-24), worst absolute below 2^-126 %.3g"
          % (worst_rel, worst_rel / 2.0 ** -24, worst_abs))
    assert worst_rel <= 2.0 ** -21, worst_rel
    assert worst_abs <= 2.0 ** -126, worst_abs
