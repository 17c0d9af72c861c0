"""Writes the golden fixtures under tests/golden/ from the oracle.

    python tests/golden/make_golden.py

workloads.npz: selected rows of every workload shape (inputs are regenerated
from the workload seeds; a SHA-256 of the regenerated logits is stored with
them) and the oracle's token, kept count, used flag and kept candidates.

reference_cases.npz: the 72 cases of crates/rust-llm/tests/sample.rs:128-232
(8 settings x 3 logit seeds x 3 spreads at V = 2048, window
[3, 11, 400, 11, 7, 1999, 0, 3]) sampled by a fresh Sampler each, as that
test does: token, kept candidates and their probabilities.
"""
import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "rust-llm_amd"))
sys.path.insert(0, os.path.join(ROOT, "oracle"))

import oracle as O  # noqa: E402
import rl_sampler as R  # noqa: E402
import workloads as W  # noqa: E402

ROWS = {
    "single": [0], "single_greedy": [0], "zipf": [0, 1, 63], "spikes": [0, 511, 1023],
    "verify": list(range(9)), "verify_greedy": list(range(9)), "ties": [0],
}

REF_CASES = [  # tests/sample.rs:129-209
    ("temperature only", (0.7, 0, 1.0, 0.0, 1.0, 0, 1)),
    ("a cold temperature", (0.05, 0, 1.0, 0.0, 1.0, 64, 0)),
    ("a hot temperature", (4.0, 0, 1.0, 0.0, 1.0, 64, 0)),
    ("top-k only", (1.0, 17, 1.0, 0.0, 1.0, 0, 2)),
    ("top-p only", (1.0, 0, 0.6, 0.0, 1.0, 0, 3)),
    ("min-p only", (1.0, 0, 1.0, 0.3, 1.0, 0, 4)),
    ("the defaults", (0.6, 20, 0.95, 0.0, 1.0, 64, 0)),
    ("everything at once", (0.8, 40, 0.9, 0.02, 1.3, 16, 5)),
]
REF_WINDOW = [3, 11, 400, 11, 7, 1999, 0, 3]


def rows_of(wl, rows):
    parts = [wl.generate(r, 1) for r in rows]
    logits = np.concatenate([p[0] for p in parts])
    windows = np.concatenate([p[1] for p in parts])
    wlen = np.concatenate([p[2] for p in parts])
    uniforms = np.concatenate([wl.uniforms(r, 1) for r in rows])
    settings = [wl.settings(r) for r in rows]
    return logits, windows, wlen, uniforms, settings


def digest(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def oracle_settings(s):
    return O.Sampling(s.temperature, s.top_p, s.min_p, s.repeat_penalty, s.top_k, s.repeat_last_n, s.seed)


def make_workloads():
    out = {}
    for name, rows in ROWS.items():
        wl = W.WORKLOADS[name]
        logits, windows, wlen, uniforms, settings = rows_of(wl, rows)
        res = O.pick_rows(logits, [oracle_settings(s) for s in settings], windows, wlen, uniforms)
        kmax = int(res["kept"].max())
        out[name + "/rows"] = np.array(rows, np.uint32)
        out[name + "/logits_sha256"] = np.array(digest(logits))
        out[name + "/uniforms"] = uniforms
        for key in ("token", "kept", "used"):
            out[name + "/" + key] = res[key]
        out[name + "/ids"] = res["ids"][:, :kmax]
        out[name + "/probs"] = res["probs"][:, :kmax]
    np.savez_compressed(os.path.join(HERE, "workloads.npz"), **out)


def make_reference_cases():
    out = {"names": [], "settings": [], "seed": [], "spread": [], "token": [], "kept": []}
    ids, probs = [], []
    for what, t in REF_CASES:
        for seed in (1, 2, 3):
            for spread in (0.5, 4.0, 30.0):
                l = O.test_logits(2048, seed, spread)
                s = O.OracleSampler(l.size, O.sampling(*t))
                for tok in REF_WINDOW:
                    s.remember(tok)
                token = s.sample(l)
                ci, cp = s.candidates()
                out["names"].append(what)
                out["settings"].append(t)
                out["seed"].append(seed)
                out["spread"].append(spread)
                out["token"].append(token)
                out["kept"].append(ci.size)
                ids.append(np.pad(ci, (0, 2048 - ci.size)))
                probs.append(np.pad(cp, (0, 2048 - cp.size)))
    np.savez_compressed(
        os.path.join(HERE, "reference_cases.npz"), names=np.array(out["names"]),
        settings=np.array(out["settings"], np.float64), seed=np.array(out["seed"], np.uint64),
        spread=np.array(out["spread"], np.float32), token=np.array(out["token"], np.uint32),
        kept=np.array(out["kept"], np.uint32), ids=np.array(ids, np.uint32), probs=np.array(probs, np.float32))


if __name__ == "__main__":
    make_workloads()
    make_reference_cases()
    for f in ("workloads.npz", "reference_cases.npz"):
        print(f, os.path.getsize(os.path.join(HERE, f)), "bytes")
