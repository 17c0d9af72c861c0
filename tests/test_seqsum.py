"""The exact parallel replay of sequential sums (rust-llm_amd/csrc/rl_seqsum.h),
checked on the host.

The device replays the reference's sequential f64 and f32 sums
(sample.rs:307-324, :342, :349-356) with a workgroup: per binade of the running
sum, each term is a map parity -> (grid steps, parity), composed by a scan.
tests/native/seqsum_check.cpp runs the same algorithm serially with the same
header and compares every final sum and every first-crossing index (for
thresholds at, just below and just above each partial sum, and 0) with plain
sequential loops, bit for bit: uniform, very wide, narrow, subnormal, zero-
heavy, tie-heavy and constant inputs, sorted and unsorted, tiles of 1 to 2048
terms. It also checks that the term maps compose associatively.
"""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SRC = os.path.join(ROOT, "tests", "native", "seqsum_check.cpp")
INC = os.path.join(ROOT, "rust-llm_amd", "csrc")


def test_replay_equals_sequential_sums(tmp_path):
    exe = str(tmp_path / "seqsum_check")
    # -ffp-contract=off: the plain loops must round every addition on its own.
    subprocess.run(["g++", "-O2", "-std=c++17", "-ffp-contract=off", "-I" + INC, "-o", exe, SRC], check=True)
    out = subprocess.run([exe], capture_output=True, text=True)
    assert out.returncode == 0, out.stdout + out.stderr
    assert out.stdout.startswith("ok "), out.stdout
