"""The GPU sampler against the committed golden fixtures (tests/golden/):
workload rows through the batched device entry point, and the reference's 72
pipeline cases through the host Sampler API."""
import numpy as np
import pytest

import oracle as O
import rl_sampler as R
import workloads as W
from test_golden import golden_rows, load

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("name", ["single", "single_greedy", "zipf", "spikes", "verify", "verify_greedy", "ties"])
def test_device_reproduces_the_workload_fixture(device, name):
    import torch
    g = load("workloads.npz")
    logits, windows, wlen, uniforms, settings = golden_rows(g, name)
    ctx = R.DeviceSampler(logits.shape[0], logits.shape[1], max_window=W.WINDOW)
    got = R.sample_batch(ctx, torch.from_numpy(logits).to(device), settings,
                         windows=torch.from_numpy(windows.view(np.int32)).to(device),
                         window_len=torch.from_numpy(wlen.view(np.int32)).to(device),
                         uniforms=torch.from_numpy(uniforms).to(device))
    assert np.array_equal(got.token, g[name + "/token"]), name
    assert np.array_equal(got.kept, g[name + "/kept"]), name
    assert np.array_equal(got.used, g[name + "/used"]), name
    for r in range(got.token.size):
        k = int(got.kept[r])
        assert np.array_equal(got.ids[r, :k], g[name + "/ids"][r, :k]), (name, r)
        assert np.array_equal(got.probs[r, :k].view(np.uint32), g[name + "/probs"][r, :k].view(np.uint32)), (name, r)


def test_host_sampler_reproduces_the_reference_case_fixture(device):
    g = load("reference_cases.npz")
    for i in range(g["token"].size):
        t = g["settings"][i]
        set_ = R.sampling(float(t[0]), int(t[1]), float(t[2]), float(t[3]), float(t[4]), int(t[5]), int(t[6]))
        l = O.test_logits(2048, int(g["seed"][i]), float(g["spread"][i]))
        s = R.HostSampler(l.size, set_)
        for tok in (3, 11, 400, 11, 7, 1999, 0, 3):
            s.remember(tok)
        assert s.sample(l) == g["token"][i], g["names"][i]
        ids, probs = s.candidates()
        k = int(g["kept"][i])
        assert np.array_equal(ids, g["ids"][i, :k]), g["names"][i]
        assert np.array_equal(probs.view(np.uint32), g["probs"][i, :k].view(np.uint32)), g["names"][i]
