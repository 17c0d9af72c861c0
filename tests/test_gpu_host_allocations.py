"""The host Sampler allocates nothing per call: the reference's
tests/sample_allocations.rs:75-136 (four settings that reach different stages,
a full penalty window, two warm-up calls, 8 counted calls over 248 320
logits), plus the verify/commit walk and a batched call.

The count is taken by tests/native/alloc_count, a host program that defines
malloc itself, so every heap allocation in the process passes through it, and
charges each allocation to the innermost caller outside the C and C++ runtime
libraries. The library's own allocations must be zero; what the HIP runtime
allocates for the copies and launches a call issues is printed, not asserted
(it is the runtime's, and the reference has no device runtime to count).
"""
import json
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
PROG = os.path.join(HERE, "native", "alloc_count")


def test_the_host_sampler_allocates_nothing_per_call(device):
    assert os.path.exists(PROG), "%s is missing: build it with `make -C tests/native`" % PROG
    print("alloc_count: 4 settings x (device, host logits), verify+commit, batch of 4; 8 counted calls each",
          flush=True)
    res = subprocess.run([PROG], capture_output=True, text=True, timeout=300)
    assert res.returncode == 0, "alloc_count failed (%d): %s" % (res.returncode, res.stderr[-2000:])
    counts = json.loads(res.stdout)
    assert len(counts) == 10, counts
    for what, c in counts.items():
        print("%s: library %d, HIP runtime %d, other %d allocations over %d calls"
              % (what, c["library"], c["hip_runtime"], c["other"], c["calls"]))
    mine = {what: c["library"] for what, c in counts.items() if c["library"]}
    assert not mine, "the sampler library allocated on the heap during sampling: %s" % mine
