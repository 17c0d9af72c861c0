"""The C ABI library without a GPU: it loads, exports every entry point the
headers declare, refuses bad arguments with status codes, and its host-side
pieces (the Rng, the settings constants) match the reference and the oracle."""
import ctypes
import os
import re

import pytest

import oracle as O
import rl_sampler as R

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    names = set()
    for h in sorted(f for f in os.listdir(os.path.join(ROOT, "include")) if f.endswith(".h")):
        text = open(os.path.join(ROOT, "include", h)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names.update(re.findall(r"\b(rl_\w+)\s*\(", text))
    return sorted(names)


def test_the_library_exports_every_declared_entry_point():
    lib = R.lib()
    names = declared_functions()
    assert len(names) >= 20, names
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, "declared but not exported: %s" % missing


def test_status_codes_without_a_device():
    lib = R.lib()
    h = ctypes.c_void_p()
    assert lib.rl_sampler_create(0, 0, 100, 64, ctypes.byref(h)) == R.RL_ERR_ARGUMENT
    # Windows of any length are accepted (sample.rs:166): with no GPU here the
    # call gets as far as selecting the device.
    assert lib.rl_sampler_create(0, 4, 100, 5000, ctypes.byref(h)) == R.RL_ERR_DEVICE
    assert lib.rl_sampler_create(0, 4, (1 << 21) + 1, 64, ctypes.byref(h)) == R.RL_ERR_CAPACITY
    assert b"vocab" in lib.rl_sampler_last_error()
    assert lib.rl_sampler_create(0, 4, 100, 64, None) == R.RL_ERR_ARGUMENT
    assert lib.rl_sampler_configure(None, None, 1) == R.RL_ERR_ARGUMENT
    assert lib.rl_sampler_sample_rows(None, None, 0, 1, 1, None, 0, None, None, None, None, None, None,
                                      None, 0, None) == R.RL_ERR_ARGUMENT
    lib.rl_sampler_destroy(None)  # accepted


def test_head_status_codes_without_a_device():
    lib = R.lib()
    h = ctypes.c_void_p()
    buf = (ctypes.c_uint8 * (2 * 210))()
    assert lib.rl_head_create(0, 256, 2, 4, buf, 2 * 210, None) == R.RL_ERR_ARGUMENT
    assert lib.rl_head_create(0, 256, 2, 4, None, 2 * 210, ctypes.byref(h)) == R.RL_ERR_ARGUMENT
    assert lib.rl_head_create(0, 0, 2, 4, buf, 0, ctypes.byref(h)) == R.RL_ERR_ARGUMENT
    assert lib.rl_head_create(0, 256, 2, 0, buf, 2 * 210, ctypes.byref(h)) == R.RL_ERR_ARGUMENT
    # Two rows of one block are 420 bytes, not 419.
    assert lib.rl_head_create(0, 256, 2, 4, buf, 419, ctypes.byref(h)) == R.RL_ERR_ARGUMENT
    assert b"210" in lib.rl_sampler_last_error()
    assert lib.rl_head_logits(None, None, 1, None, 0, None) == R.RL_ERR_ARGUMENT
    assert lib.rl_head_embed_rows(None, None, 1, None, 0, None) == R.RL_ERR_ARGUMENT
    assert lib.rl_quantize_rows(None, 1, 256, None, None, None, None) == R.RL_ERR_ARGUMENT
    assert lib.rl_quantize_rows(None, 0, 256, None, None, None, None) == R.RL_OK  # nothing to do
    lib.rl_head_destroy(None)  # accepted


@pytest.mark.skipif(os.path.exists("/dev/kfd") and os.access("/dev/kfd", os.R_OK),
                    reason="a GPU is present")
def test_create_fails_cleanly_where_there_is_no_device():
    lib = R.lib()
    h = ctypes.c_void_p()
    rc = lib.rl_sampler_create(0, 4, 100, 64, ctypes.byref(h))
    assert rc == R.RL_ERR_DEVICE, rc
    assert lib.rl_sampler_last_error()


def test_the_host_rng_matches_the_oracle():
    for seed in (0, 1, 7, 42, 0xFEED, 2**64 - 1):
        a, b = R.RngStream(seed), O.OracleRng(seed)
        assert a.state() == b.state()
        assert [a.next_u64() for _ in range(16)] == [b.next_u64() for _ in range(16)]
        assert [a.next_f32() for _ in range(16)] == [b.next_f32() for _ in range(16)]


def test_settings_constants():  # sample.rs:71-79, :88-100
    d = R.lib().rl_sampling_default()
    assert (d.temperature, d.top_k, d.top_p, d.min_p, d.repeat_penalty, d.repeat_last_n, d.seed) == (
        pytest.approx(0.6), 20, pytest.approx(0.95), 0.0, 1.0, 64, 0)
    g = R.lib().rl_sampling_greedy()
    assert (g.temperature, g.top_k, g.top_p, g.min_p, g.repeat_penalty, g.repeat_last_n, g.seed) == (
        0.0, 0, 1.0, 0.0, 1.0, 0, 0)
    assert ctypes.sizeof(R.Sampling) == ctypes.sizeof(O.Sampling) == 40


def test_the_product_path_fails_loudly_without_its_library(monkeypatch, tmp_path):
    monkeypatch.setattr(R, "_lib", None)
    monkeypatch.setattr(R, "LIB_PATH", str(tmp_path / "missing.so"))
    with pytest.raises(RuntimeError, match="missing"):
        R.lib()


def test_entropy_seed_comes_from_the_os_and_needs_no_device():
    """entropy_seed (sample.rs:107-112) is a host-only seed from OS entropy:
    it runs here without a GPU, and successive calls differ (64 bits each: a
    repeat among 64 calls has probability about 1e-16)."""
    seeds = [R.entropy_seed() for _ in range(64)]
    assert len(set(seeds)) == len(seeds)
    assert all(0 <= s < 1 << 64 for s in seeds)
    assert any(s >= 1 << 32 for s in seeds), "the high half is never filled"
    # Each bit position takes both values over the calls.
    ones = [sum((s >> b) & 1 for s in seeds) for b in range(64)]
    assert all(0 < c < len(seeds) for c in ones), ones
