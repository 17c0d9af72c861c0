"""The oracle against its committed golden fixtures (tests/golden/), so a
change to the restatement or to the workload generator shows up as a diff."""
import hashlib
import os

import numpy as np
import pytest

import oracle as O
import workloads as W
from conftest import as_oracle_settings

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    return np.load(os.path.join(GOLD, name), allow_pickle=False)


def golden_rows(g, name):
    wl = W.WORKLOADS[name]
    rows = g[name + "/rows"].tolist()
    parts = [wl.generate(r, 1) for r in rows]
    logits = np.concatenate([p[0] for p in parts])
    windows = np.concatenate([p[1] for p in parts])
    wlen = np.concatenate([p[2] for p in parts])
    uniforms = np.concatenate([wl.uniforms(r, 1) for r in rows])
    assert hashlib.sha256(logits.tobytes()).hexdigest() == str(g[name + "/logits_sha256"]), \
        "%s: the workload generator no longer produces the fixture's inputs" % name
    assert np.array_equal(uniforms, g[name + "/uniforms"])
    return logits, windows, wlen, uniforms, [wl.settings(r) for r in rows]


@pytest.mark.parametrize("name", ["single", "single_greedy", "zipf", "spikes", "verify", "verify_greedy", "ties"])
def test_oracle_reproduces_the_workload_fixture(name):
    g = load("workloads.npz")
    logits, windows, wlen, uniforms, settings = golden_rows(g, name)
    res = O.pick_rows(logits, [as_oracle_settings(s) for s in settings], windows, wlen, uniforms)
    for key in ("token", "kept", "used"):
        assert np.array_equal(res[key], g[name + "/" + key]), (name, key)
    k = g[name + "/ids"].shape[1]
    assert np.array_equal(res["ids"][:, :k], g[name + "/ids"])
    assert np.array_equal(res["probs"][:, :k].view(np.uint32), g[name + "/probs"].view(np.uint32))


def test_oracle_reproduces_the_reference_case_fixture():
    g = load("reference_cases.npz")
    for i in range(g["token"].size):
        t = g["settings"][i]
        set_ = O.sampling(float(t[0]), int(t[1]), float(t[2]), float(t[3]), float(t[4]), int(t[5]), int(t[6]))
        l = O.test_logits(2048, int(g["seed"][i]), float(g["spread"][i]))
        s = O.OracleSampler(l.size, set_)
        for tok in (3, 11, 400, 11, 7, 1999, 0, 3):
            s.remember(tok)
        assert s.sample(l) == g["token"][i], g["names"][i]
        ids, probs = s.candidates()
        k = int(g["kept"][i])
        assert ids.size == k
        assert np.array_equal(ids, g["ids"][i, :k])
        assert np.array_equal(probs.view(np.uint32), g["probs"][i, :k].view(np.uint32))
