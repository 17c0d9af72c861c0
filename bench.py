"""Benchmark: rows/s and achieved HBM GB/s of the full sampling chain.

One step is one rl_sampler_sample_rows call over the whole batch of logit rows
already resident in HBM: repetition penalty over each row's 64-id window,
temperature, top-k, top-p, min-p and the draw against a host-drawn uniform,
writing token, kept count, used flag and the kept (id, prob) candidates.

Default workload: 1024 rows x 248320 f32 logits, N(0, 2^2) plus 16 spikes per
row in [8, 14); T 0.6, top-k 20, top-p 0.95, min-p 0, repeat penalty 1.2 over
64-id windows. Other workload shapes are parity cases (tests/) and can be timed
with --workload.

--op embed times the embedding lookup from the same resident tensor
(rl_head_embed_rows: --tokens rows of 2560 f32 each).

--op host_verify times the host Sampler's speculative-verify walk on the host
wall clock (rl_host_sampler_verify over the 9-row verify workload, then
rl_host_sampler_commit_verified row by row, every draft accepted), --op
host_batch one rl_host_sample_batch call over 16 host Samplers, --op
host_sample one rl_host_sampler_sample_device call on one row; each timed from
C++ (rust-llm_amd/librl_hostbench.so) and printed beside the device time of
the same rows' rl_sampler_sample_rows call.

--op head times the output head instead (rl_head_logits: t normed hidden rows
times the tied Q6_K embedding [2560, 248320], logits into HBM); --op head_sample
times the head followed by sampling its logits, the device path from hidden
state to token.

Prints one JSON line. `roofline.achieved` is the workload's algorithmic bytes
per call divided by the average duration of a call: the timed calls run back
to back between one pair of HIP events on the stream the kernels run on, and
the region's time is divided by the number of calls. `cpu_baseline` times the
oracle (the C restatement of the reference sampler) on one host core over a
bounded sample of the same rows, `cpu_baseline_threads` on the host's threads.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "rust-llm_amd"))

HBM_PEAK_GBS = 8000.0


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default=None)
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="budget for the CPU-baseline sample (0 skips it)")
    ap.add_argument("--no-candidates", action="store_true",
                    help="skip the candidate outputs (tokens only)")
    ap.add_argument("--op", default="sample",
                    choices=["sample", "top_probability", "argmax", "head", "head_sample", "embed", "host_verify",
                             "host_batch", "host_sample"],
                    help="sample: rl_sampler_sample_rows (the benchmark); top_probability and argmax time "
                         "rl_top_probability_rows and rl_argmax_rows on the same logits; head times "
                         "rl_head_logits, head_sample the head followed by sampling its logits; embed times "
                         "rl_head_embed_rows, the embedding lookup from the same tensor; host_verify and "
                         "host_batch time the host Sampler's verify+commit walk and a 16-sampler batch on the "
                         "host wall clock")
    ap.add_argument("--tokens", type=int, default=1,
                    help="tokens per embedding lookup (1 = a decode step, more = a prompt)")
    ap.add_argument("--head-rows", type=int, default=1,
                    help="activation rows per head call (1 = a decode step, 9 or 17 = a verify batch)")
    ap.add_argument("--max-window", type=int, default=None,
                    help="the sampling context's max_window (default: the workload's 64-id windows); the "
                         "call's windows stay 64 ids")
    ap.add_argument("--calibration-copy", type=int, default=0,
                    help="after the timed steps, run this many plain device copies of the logits "
                         "(known bytes) so profiler byte counters can be scaled")
    return ap.parse_args()


def traffic_bytes(workload):
    """HBM bytes per launch of the dominant kernel, from the PMC runs recorded
    in profiles/traffic.json (FETCH_SIZE + WRITE_SIZE scaled by a copy of known
    size): a figure of the profile named in `source`, not of this run. None
    where no such run has been recorded for the workload."""
    try:
        with open(os.path.join(ROOT, "profiles", "traffic.json")) as f:
            return json.load(f)[workload]["traffic_bytes_per_launch"]
    except (OSError, KeyError, ValueError):
        return None


def traffic_source(workload):
    try:
        with open(os.path.join(ROOT, "profiles", "traffic.json")) as f:
            e = json.load(f)[workload]
        return "profile: %s (%s)" % (e["source"], e["kernel"])
    except (OSError, KeyError, ValueError):
        return None


def cpu_baseline(wl, logits, windows, wlen, uniforms, settings, budget_s):
    """The oracle on one host core over rows of the same workload, cycling
    until the time budget is spent. Returns rows/s and the sample size."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import numpy as np

    import oracle
    osets = [oracle.Sampling(s.temperature, s.top_p, s.min_p, s.repeat_penalty, s.top_k, s.repeat_last_n, s.seed)
             for s in settings]
    rows = logits.shape[0]
    batch = min(rows, 16)
    done = 0
    t0 = time.perf_counter()
    r0 = 0
    while True:
        sl = slice(r0, r0 + batch)
        oracle.pick_rows(logits[sl], osets[sl], windows[sl], wlen[sl], uniforms[sl], cand_cap=1)
        done += batch
        r0 = (r0 + batch) % (rows - batch + 1)
        el = time.perf_counter() - t0
        if el >= budget_s:
            break
    return done / el, done, el


def host_info():
    """What a CPU baseline ran on, as the reference's bench reports it
    (crates/rust-llm/src/bench.rs:457-487): the CPU model, the CPUs the kernel
    reports (nproc), the affinity mask, the cgroup quota, the one-minute load
    average and the C library (whose expf the oracle calls). `available` is
    Rust's available_parallelism: the affinity mask, limited by the quota."""
    model = None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    affinity = len(os.sched_getaffinity(0))
    available = affinity
    quota = None
    try:
        with open("/sys/fs/cgroup/cpu.max") as f:
            quota = f.read().strip()
        q, period = quota.split()[:2]
        if q != "max":
            available = min(available, max(1, int(q) // int(period)))
    except (OSError, ValueError):
        pass
    load = None
    try:
        with open("/proc/loadavg") as f:
            load = float(f.read().split()[0])
    except (OSError, ValueError, IndexError):
        pass
    return {"cpu_model": model, "nproc": os.cpu_count(), "affinity": affinity, "cpu_max": quota,
            "available_parallelism": available, "load_average_1m": load,
            "libc": " ".join(os.confstr("CS_GNU_LIBC_VERSION").split()) if hasattr(os, "confstr") else None}


# One GPU's share of a host's cores: the threaded baseline uses no more
# threads than this even where the affinity mask shows more CPUs.
GPU_CPU_SHARE = 16


def host_threads(info):
    """Threads for the threaded CPU baseline: available_parallelism, capped at
    one GPU's share of the host (GPU_CPU_SHARE)."""
    return max(1, min(info["available_parallelism"], GPU_CPU_SHARE))


def cpu_baseline_threads(wl, logits, windows, wlen, uniforms, settings, budget_s, threads):
    """The oracle on `threads` host threads (rows split over them, each thread
    cycling over its own slice; the oracle's C calls run without the GIL),
    until the time budget is spent. Returns rows/s and the sample size."""
    import threading

    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle
    osets = [oracle.Sampling(s.temperature, s.top_p, s.min_p, s.repeat_penalty, s.top_k, s.repeat_last_n, s.seed)
             for s in settings]
    rows = logits.shape[0]
    per = max(1, rows // threads)
    batch = min(per, 16)
    counts = [0] * threads
    t0 = time.perf_counter()

    def work(i):
        lo = (i * per) % rows
        hi = min(rows, lo + per)
        r0 = lo
        while time.perf_counter() - t0 < budget_s:
            r1 = min(hi, r0 + batch)
            sl = slice(r0, r1)
            oracle.pick_rows(logits[sl], osets[sl], windows[sl], wlen[sl], uniforms[sl], cand_cap=1)
            counts[i] += r1 - r0
            r0 = r1 if r1 < hi else lo

    ts = [threading.Thread(target=work, args=(i,)) for i in range(threads)]
    for t in ts:
        t.start()
    for t in ts:
        t.join()
    el = time.perf_counter() - t0
    return sum(counts) / el, sum(counts), el


def head_cpu_baseline(w, x, budget_s):
    """The oracle head on one host core over slices of the vocabulary, until
    the time budget is spent. Returns full-vocabulary head calls/s."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle
    import workloads as W
    rows = W.HEAD_ROWS
    chunk = 2048
    done = 0
    lo = 0
    t0 = time.perf_counter()
    while True:
        hi = min(rows, lo + chunk)
        oracle.q6k_matvec(w, W.HEAD_K, x, lo, hi)
        done += hi - lo
        lo = 0 if hi == rows else hi
        el = time.perf_counter() - t0
        if el >= budget_s:
            break
    return done / rows / el, done, el


def time_calls(step, args, stream):
    """args.warmup untimed calls, then args.steps timed ones, back to back,
    bracketed by one HIP-event pair on `stream` (an event recorded between two
    calls delays the next launch by several microseconds, so none is). Returns
    (wall ms per step, HIP-event ms per call over the timed region, sorted
    per-call HIP-event ms from a separate, untimed pass of args.steps calls
    each between its own events: the spread, not the throughput)."""
    import torch
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t_start = torch.cuda.Event(enable_timing=True)
    t_end = torch.cuda.Event(enable_timing=True)
    t_wall = time.perf_counter()
    t_start.record(stream)
    for _ in range(args.steps):
        step()
    t_end.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t_wall
    region_ms = t_start.elapsed_time(t_end) / args.steps
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps)]
    for i in range(args.steps):
        starts[i].record(stream)
        step()
        ends[i].record(stream)
    torch.cuda.synchronize()
    return wall * 1e3 / args.steps, region_ms, sorted(a.elapsed_time(b) for a, b in zip(starts, ends))


def bench_embed(args):
    """--op embed: the embedding lookup of --tokens tokens from the resident
    Q6_K tensor."""
    import numpy as np
    import torch

    import rl_sampler as R
    import workloads as W

    n = args.tokens
    dev = torch.device("cuda:0")
    t0 = time.time()
    w = W.head_weights()
    head = R.DeviceHead(w, W.HEAD_K, W.HEAD_ROWS, max_batch=1)
    print("[bench] head weights generated and uploaded in %.1fs" % (time.time() - t0), file=sys.stderr, flush=True)
    tokens = np.random.default_rng(6).integers(0, W.HEAD_ROWS, n).astype(np.int32)
    d_tok = torch.from_numpy(tokens).to(dev)
    d_out = torch.empty((n, W.HEAD_K), dtype=torch.float32, device=dev)
    stream = torch.cuda.current_stream()

    def step():
        head.embed_into(d_tok, d_out, stream=stream.cuda_stream)

    ms_per_step, mean_ms, per_call_ms = time_calls(step, args, stream)
    median_ms = per_call_ms[len(per_call_ms) // 2]
    nb = -(-W.HEAD_K // 256)
    # Per token: the id, its row's blocks, the f32 row written.
    alg_bytes = n * (4 + nb * W.Q6K_BLOCK_BYTES + W.HEAD_K * 4)
    achieved = alg_bytes / (mean_ms / 1e3) / 1e9
    print("[bench] embed %d tokens: wall %.4f ms/step, events %.4f ms per call over the timed region; alone: median %.4f min %.4f max %.4f ms" % (
        n, ms_per_step, mean_ms, median_ms, per_call_ms[0], per_call_ms[-1]), file=sys.stderr, flush=True)
    if args.calibration_copy > 0:
        dst = torch.empty_like(d_out)
        for _ in range(args.calibration_copy):
            dst.copy_(d_out)
        torch.cuda.synchronize()
        print("[bench] calibration: %d copies of %d bytes" % (args.calibration_copy, d_out.numel() * 4),
              file=sys.stderr, flush=True)
        del dst
    cpu = None
    if args.cpu_seconds > 0:
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import oracle
        done, t_cpu = 0, time.perf_counter()
        while time.perf_counter() - t_cpu < min(args.cpu_seconds, 3.0):
            oracle.embed_rows(w, W.HEAD_K, tokens)
            done += n
        el = time.perf_counter() - t_cpu
        cpu = {"value": round(done / el, 1), "unit": "tokens/s", "cores": 1, "kind": "port",
               "sample": "%d lookups through the oracle's dequantize_row on one host core in %.1f s" % (done, el)}
    line = {
        "metric": "tokens/s + achieved HBM GB/s, embedding lookup from Q6_K [%d, %d], %d token%s" % (
            W.HEAD_K, W.HEAD_ROWS, n, "" if n == 1 else "s"),
        "value": round(n * 1e3 / ms_per_step, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q6_k -> f32",
        "data": "synthetic (seeded Q6_K weights and token ids, rust-llm_amd/workloads.py)",
        "config": {"workload": "embed: token_embd [%d, %d] Q6_K, %d tokens" % (W.HEAD_K, W.HEAD_ROWS, n),
                   "tokens": n, "k": W.HEAD_K},
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic_bytes("embed_n%d" % n),
            "traffic_source": traffic_source("embed_n%d" % n),
            "algorithmic_bytes_per_call": alg_bytes,
            "call_ms_mean": round(mean_ms, 5),
            "call_ms_median_alone": round(median_ms, 5),
        },
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


def bench_head(args):
    """--op head / head_sample: the output head, and the head then sampling."""
    import numpy as np
    import torch

    import rl_sampler as R
    import workloads as W

    t = args.head_rows
    dev = torch.device("cuda:0")
    t0 = time.time()
    w = W.head_weights()
    x = W.head_inputs(t)
    head = R.DeviceHead(w, W.HEAD_K, W.HEAD_ROWS, max_batch=max(t, 1))
    print("[bench] head weights generated and uploaded in %.1fs" % (time.time() - t0), file=sys.stderr, flush=True)
    d_x = torch.from_numpy(x).to(dev)
    d_logits = torch.empty((t, W.HEAD_ROWS), dtype=torch.float32, device=dev)
    stream = torch.cuda.current_stream()
    sample = args.op == "head_sample"
    if sample:
        # The verify batch's settings (penalty 1.3 over 64-id windows, T 0.6,
        # top-k 20, top-p 0.95), one stream of uniforms in row order.
        settings = [R.sampling(0.6, 20, 0.95, 0.0, 1.3, 64, 0) for _ in range(t)]
        g = np.random.default_rng(5)
        d_win = torch.from_numpy(g.integers(0, W.HEAD_ROWS, (t, W.WINDOW)).astype(np.int32)).to(dev)
        d_wlen = torch.full((t,), W.WINDOW, dtype=torch.int32, device=dev)
        d_uni = torch.from_numpy(g.random(t).astype(np.float32)).to(dev)
        ctx = R.DeviceSampler(t, W.HEAD_ROWS, max_window=W.WINDOW)
        ctx.configure(settings)
        cs = ctx.required_cand_stride()
        out_tok = torch.empty(t, dtype=torch.int32, device=dev)
        out_kept = torch.empty(t, dtype=torch.int32, device=dev)
        out_used = torch.empty(t, dtype=torch.uint8, device=dev)
        out_ids = torch.empty((t, cs), dtype=torch.int32, device=dev)
        out_probs = torch.empty((t, cs), dtype=torch.float32, device=dev)

    def step():
        head.logits_into(d_x, d_logits, stream=stream.cuda_stream)
        if sample:
            ctx.sample_rows(d_logits, t, d_logits.stride(0), out_tok, out_kept, out_used, windows=d_win,
                            window_stride=W.WINDOW, window_len=d_wlen, uniforms=d_uni, out_ids=out_ids,
                            out_probs=out_probs, cand_stride=cs, stream=stream.cuda_stream)

    ms_per_step, mean_ms, per_call_ms = time_calls(step, args, stream)
    median_ms = per_call_ms[len(per_call_ms) // 2]
    weight_bytes = W.HEAD_ROWS * (-(-W.HEAD_K // 256)) * W.Q6K_BLOCK_BYTES
    # Weights once, the hidden rows, the logits written; sampling re-reads the
    # logits and writes (token, kept, used, 20 candidates) per row.
    alg_bytes = weight_bytes + t * W.HEAD_K * 4 + t * W.HEAD_ROWS * 4
    if sample:
        alg_bytes += t * (W.HEAD_ROWS * 4 + W.WINDOW * 4 + 4 + 4 + 4 + 1 + 20 * 8)
    achieved = alg_bytes / (mean_ms / 1e3) / 1e9
    print("[bench] head t=%d%s: wall %.3f ms/step, events %.3f ms per call over the timed region; alone: median %.3f min %.3f max %.3f ms" % (
        t, " + sample" if sample else "", ms_per_step, mean_ms, median_ms, per_call_ms[0], per_call_ms[-1]),
        file=sys.stderr, flush=True)
    if args.calibration_copy > 0:
        src = torch.zeros(weight_bytes // 4, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(args.calibration_copy):
            dst.copy_(src)
        torch.cuda.synchronize()
        print("[bench] calibration: %d copies of %d bytes" % (args.calibration_copy, weight_bytes),
              file=sys.stderr, flush=True)
        del src, dst
    cpu = None
    if args.cpu_seconds > 0:
        rate, n, el = head_cpu_baseline(w, x, args.cpu_seconds)
        cpu = {"value": round(rate, 4), "unit": "head calls/s", "cores": 1, "kind": "port",
               "sample": "%d vocabulary rows x %d activation rows through the oracle's scalar Q6_K head on "
                         "one host core in %.1f s, scaled to full-vocabulary calls" % (n, t, el)}
        print("[bench] cpu baseline %.4f head calls/s" % rate, file=sys.stderr, flush=True)
    line = {
        "metric": "head calls/s + achieved HBM GB/s, Q6_K [%d, %d] output head, %d activation row%s%s" % (
            W.HEAD_K, W.HEAD_ROWS, t, "" if t == 1 else "s", ", then sampling" if sample else ""),
        "value": round(1e3 / ms_per_step, 2),
        "unit": "head calls/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q6_k x int8 (exact integer sums, f32 scaling)",
        "data": "synthetic (seeded Q6_K weights and hidden rows, rust-llm_amd/workloads.py)",
        "config": {"workload": "head: token_embd [%d, %d] Q6_K, %d rows" % (W.HEAD_K, W.HEAD_ROWS, t),
                   "rows": t, "vocab": W.HEAD_ROWS, "k": W.HEAD_K, "sampling": sample},
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": None if sample else traffic_bytes("head_t%d" % t),
            "traffic_source": None if sample else traffic_source("head_t%d" % t),
            "algorithmic_bytes_per_call": alg_bytes,
            "call_ms_mean": round(mean_ms, 5),
            "call_ms_median_alone": round(median_ms, 5),
        },
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)

def device_call_ms(ctx, d_logits, rows, settings, windows, wlen, uniforms, calls, stream):
    """Median HIP-event time of rl_sampler_sample_rows alone over `rows` rows
    (each call between its own events), candidates out."""
    import numpy as np
    import torch

    import rl_sampler as R
    dev = d_logits.device
    ctx.configure(settings)
    cs = ctx.required_cand_stride()
    tok = torch.empty(rows, dtype=torch.int32, device=dev)
    kept = torch.empty_like(tok)
    used = torch.empty(rows, dtype=torch.uint8, device=dev)
    ids = torch.empty((rows, cs), dtype=torch.int32, device=dev)
    probs = torch.empty((rows, cs), dtype=torch.float32, device=dev)
    d_win = torch.from_numpy(np.ascontiguousarray(windows).view(np.int32)).to(dev)
    d_wlen = torch.from_numpy(wlen.view(np.int32)).to(dev)
    d_uni = torch.from_numpy(uniforms).to(dev)
    out = []
    for i in range(calls + 3):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        ctx.sample_rows(d_logits, rows, d_logits.stride(0), tok, kept, used, windows=d_win,
                        window_stride=windows.shape[1], window_len=d_wlen, uniforms=d_uni, out_ids=ids,
                        out_probs=probs, cand_stride=cs, stream=stream.cuda_stream)
        b.record(stream)
        torch.cuda.synchronize()
        if i >= 3:
            out.append(a.elapsed_time(b))
    return sorted(out)[len(out) // 2]


def hostbench_lib():
    """librl_hostbench.so: the host Sampler's calls timed from C++ (no
    interpreter between the calls)."""
    import ctypes
    path = os.path.join(ROOT, "rust-llm_amd", "librl_hostbench.so")
    if not os.path.exists(path):
        raise RuntimeError("%s is missing: build it with `make -C rust-llm_amd`" % path)
    L = ctypes.CDLL(path)
    vp, u64, sz, u32 = ctypes.c_void_p, ctypes.c_uint64, ctypes.c_size_t, ctypes.c_uint32
    L.rlb_verify_walks.argtypes = [ctypes.c_int, vp, u64, sz, vp, vp, sz, u32, u32, vp, vp]
    L.rlb_batch_calls.argtypes = [ctypes.c_int, vp, u64, sz, vp, u32, vp, u32, vp, u32, vp]
    L.rlb_sample_calls.argtypes = [ctypes.c_int, vp, sz, vp, vp, sz, u32, vp]
    return L


def bench_host(args):
    """--op host_verify / host_batch / host_sample: the host Sampler's calls on
    the host wall clock, timed natively, beside the device time of the same
    rows' rl_sampler_sample_rows call."""
    import ctypes

    import numpy as np
    import torch

    import rl_sampler as R
    import workloads as W

    L = hostbench_lib()
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream()
    calls = args.warmup + args.steps
    us = np.zeros(calls, np.float64)
    if args.op == "host_verify":
        name = args.workload or "verify"
        wl = W.WORKLOADS[name]
        rows, windows, wlen = wl.generate()
        n = wl.rows
        d_rows = torch.from_numpy(rows).to(dev)
        set_ = wl.settings(0)
        history = np.ascontiguousarray(wl.history(), np.uint32)
        committed = np.zeros(calls, np.uint32)
        torch.cuda.synchronize()
        rc = L.rlb_verify_walks(0, d_rows.data_ptr(), d_rows.stride(0), wl.vocab, ctypes.addressof(set_),
                                history.ctypes.data, history.size, n, calls, us.ctypes.data, committed.ctypes.data)
        if rc != 0:
            raise RuntimeError("rlb_verify_walks: %d (%s)" % (rc, R.lib().rl_sampler_last_error().decode()))
        ctx = R.DeviceSampler(n, wl.vocab, max_window=W.WINDOW)
        dev_ms = device_call_ms(ctx, d_rows, n, wl.settings_list(), windows, wlen, wl.uniforms(), 20, stream)
        what = "%s: one rl_host_sampler_verify of %d rows, then rl_host_sampler_commit_verified row by row " \
               "(%.1f rows committed a walk)" % (name, n, committed[args.warmup:].mean())
        metric = "host walks/s, speculative verify+commit over %d x %d fp32 logits" % (n, wl.vocab)
        unit = "walks/s"
    elif args.op == "host_batch":
        name = args.workload or "spikes"
        wl = W.WORKLOADS[name]
        n = 16
        rows, windows, wlen = wl.generate(0, n)
        settings = wl.settings_list(0, n)
        sets = (R.Sampling * n)(*settings)
        d_rows = torch.from_numpy(rows).to(dev)
        torch.cuda.synchronize()
        rc = L.rlb_batch_calls(0, d_rows.data_ptr(), d_rows.stride(0), wl.vocab, ctypes.addressof(sets), n,
                               windows.ctypes.data, windows.shape[1], wlen.ctypes.data, calls, us.ctypes.data)
        if rc != 0:
            raise RuntimeError("rlb_batch_calls: %d (%s)" % (rc, R.lib().rl_sampler_last_error().decode()))
        ctx = R.DeviceSampler(n, wl.vocab, max_window=W.WINDOW)
        dev_ms = device_call_ms(ctx, d_rows, n, settings, windows, wlen, wl.uniforms(0, n), 20, stream)
        what = "%s rows 0..15: one rl_host_sample_batch call over 16 host Samplers" % name
        metric = "host batch calls/s, 16 host Samplers over 16 x %d fp32 logits" % wl.vocab
        unit = "calls/s"
    else:
        name = args.workload or "single"
        wl = W.WORKLOADS[name]
        n = 1
        rows, windows, wlen = wl.generate(0, 1)
        set_ = wl.settings(0)
        d_rows = torch.from_numpy(rows).to(dev)
        hist = np.ascontiguousarray(windows[0, :wlen[0]], np.uint32)
        torch.cuda.synchronize()
        rc = L.rlb_sample_calls(0, d_rows.data_ptr(), wl.vocab, ctypes.addressof(set_), hist.ctypes.data, hist.size,
                                calls, us.ctypes.data)
        if rc != 0:
            raise RuntimeError("rlb_sample_calls: %d (%s)" % (rc, R.lib().rl_sampler_last_error().decode()))
        ctx = R.DeviceSampler(1, wl.vocab, max_window=W.WINDOW)
        dev_ms = device_call_ms(ctx, d_rows, 1, [set_], windows, wlen, wl.uniforms(0, 1), 20, stream)
        what = "%s: rl_host_sampler_sample_device on one device row" % name
        metric = "host samples/s, one host Sampler over 1 x %d fp32 logits" % wl.vocab
        unit = "samples/s"
    walls = np.sort(us[args.warmup:] / 1e3)
    med = float(walls[len(walls) // 2])
    mean = float(walls.mean())
    print("[bench] %s: host wall median %.4f ms (min %.4f, max %.4f); device call alone median %.4f ms" % (
        what, med, walls[0], walls[-1], dev_ms), file=sys.stderr, flush=True)
    line = {
        "metric": metric,
        "value": round(1e3 / mean, 1),
        "unit": unit,
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(mean, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded generator, rust-llm_amd/csrc/workloads.c)",
        "config": {"workload": what, "rows": n, "vocab": wl.vocab},
        "host_wall_ms_median": round(med, 5),
        "host_wall_ms_min": round(float(walls[0]), 5),
        "device_call_ms_median": round(dev_ms, 5),
        "host_over_device_ms": round(med - dev_ms, 5),
        "roofline": None,
        "cpu_baseline": None,
    }
    print(json.dumps(line), flush=True)


def main():
    args = parse()
    if args.gpus != 1:
        print("bench.py measures one GPU: every box here has one GPU and the sampler's rows are "
              "independent, so a multi-GPU run is not part of this build (asked for --gpus %d)" % args.gpus,
              file=sys.stderr)
        sys.exit(2)
    if args.op == "embed":
        bench_embed(args)
        return
    if args.op in ("head", "head_sample"):
        bench_head(args)
        return
    if args.op in ("host_verify", "host_batch", "host_sample"):
        bench_host(args)
        return
    import numpy as np
    import torch

    import rl_sampler as R
    import workloads as W

    name = args.workload or W.BENCH_WORKLOAD
    wl = W.WORKLOADS[name]
    dev = torch.device("cuda:0")
    t0 = time.time()
    logits, windows, wlen = wl.generate()
    settings = wl.settings_list()
    uniforms = wl.uniforms()
    print("[bench] generated %s (%d x %d) in %.1fs" % (name, wl.rows, wl.vocab, time.time() - t0),
          file=sys.stderr, flush=True)
    d_logits = torch.from_numpy(logits).to(dev)
    d_win = torch.from_numpy(windows.view(np.int32)).to(dev)
    d_wlen = torch.from_numpy(wlen.view(np.int32)).to(dev)
    d_uni = torch.from_numpy(uniforms).to(dev)
    ctx = R.DeviceSampler(wl.rows, wl.vocab, max_window=args.max_window or W.WINDOW)
    ctx.configure(settings)
    cs = 0 if args.no_candidates else ctx.required_cand_stride()
    out_tok = torch.empty(wl.rows, dtype=torch.int32, device=dev)
    out_kept = torch.empty(wl.rows, dtype=torch.int32, device=dev)
    out_used = torch.empty(wl.rows, dtype=torch.uint8, device=dev)
    out_ids = torch.empty((wl.rows, cs), dtype=torch.int32, device=dev) if cs else None
    out_probs = torch.empty((wl.rows, cs), dtype=torch.float32, device=dev) if cs else None
    stream = torch.cuda.current_stream()

    out_prob = torch.empty(wl.rows, dtype=torch.float32, device=dev)

    def step():
        if args.op == "sample":
            ctx.sample_rows(d_logits, wl.rows, d_logits.stride(0), out_tok, out_kept, out_used, windows=d_win,
                            window_stride=W.WINDOW, window_len=d_wlen, uniforms=d_uni, out_ids=out_ids,
                            out_probs=out_probs, cand_stride=cs, stream=stream.cuda_stream)
        elif args.op == "top_probability":
            ctx.top_probability_rows(d_logits, wl.rows, d_logits.stride(0), out_tok, out_prob,
                                     stream=stream.cuda_stream)
        else:
            ctx.argmax_rows(d_logits, wl.rows, d_logits.stride(0), out_tok, stream=stream.cuda_stream)

    ms_per_step, mean_ms, per_call_ms = time_calls(step, args, stream)
    median_ms = per_call_ms[len(per_call_ms) // 2]
    rows_per_s = wl.rows / (ms_per_step / 1e3)
    kept_total = None
    if args.op == "sample":
        # Every call returns the same kept counts (the calls are idempotent):
        # the candidates written are the kept set the last call returned.
        kept_total = int(out_kept.to(torch.int64).sum().item()) if cs else 0
        alg_bytes = wl.algorithmic_bytes(kept_total)
    else:  # the logits once, and a token (and a probability) per row
        alg_bytes = wl.rows * (wl.vocab * 4 + 4 + (4 if args.op == "top_probability" else 0))
    achieved = alg_bytes / (mean_ms / 1e3) / 1e9
    print("[bench] %s: wall %.4f ms/step, events %.4f ms per call over the timed region; alone: median %.4f min %.4f max %.4f ms" % (
        name, ms_per_step, mean_ms, median_ms, per_call_ms[0], per_call_ms[-1]), file=sys.stderr, flush=True)

    if args.calibration_copy > 0:
        dst = torch.empty_like(d_logits)
        for _ in range(args.calibration_copy):
            dst.copy_(d_logits)
        torch.cuda.synchronize()
        print("[bench] calibration: %d copies of %d bytes" % (args.calibration_copy, d_logits.numel() * 4),
              file=sys.stderr, flush=True)
        del dst

    cpu = None
    cpu_n = None
    if args.cpu_seconds > 0 and args.op == "sample":
        info = host_info()
        rate, n, el = cpu_baseline(wl, logits, windows, wlen, uniforms, settings, args.cpu_seconds)
        cpu = {"value": round(rate, 2), "unit": "rows/s", "cores": 1, "kind": "port",
               "sample": "%d rows of the same workload (%s) through the oracle (the C restatement of the "
                         "reference sampler) on one host core in %.1f s; the reference's own Rust sampler is "
                         "published at 0.62-0.65 ms a row (1 540-1 610 rows/s, one thread) for these settings "
                         "at V = 248 320 (docs/decisions.md:969-970), on another host" % (n, name, el),
               "host": info}
        print("[bench] cpu baseline %.1f rows/s over %d rows" % (rate, n), file=sys.stderr, flush=True)
        nt = host_threads(info)
        if nt > 1:
            rate_n, n_n, el_n = cpu_baseline_threads(wl, logits, windows, wlen, uniforms, settings,
                                                     args.cpu_seconds / 2, nt)
            cpu_n = {"value": round(rate_n, 2), "unit": "rows/s", "cores": nt, "kind": "port",
                     "sample": "%d rows of the same workload (%s) through the oracle on %d host threads, rows "
                               "split over them, in %.1f s (available_parallelism %d, at most %d: one GPU's "
                               "share of the host)" % (n_n, name, nt, el_n, info["available_parallelism"],
                                                      GPU_CPU_SHARE),
                     "host": info}
            print("[bench] cpu baseline, %d threads: %.1f rows/s over %d rows" % (nt, rate_n, n_n),
                  file=sys.stderr, flush=True)

    s0 = settings[0]
    line = {
        "metric": ("rows/s + achieved HBM GB/s, %dx%d fp32 logits, full sampling chain" % (wl.rows, wl.vocab)
                   if args.op == "sample" else
                   "rows/s + achieved HBM GB/s, %dx%d fp32 logits, %s" % (wl.rows, wl.vocab, args.op)),
        "value": round(rows_per_s, 1),
        "unit": "rows/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded generator, rust-llm_amd/csrc/workloads.c)",
        "config": {
            "workload": "%s: %s" % (name, wl.description),
            "rows": wl.rows,
            "vocab": wl.vocab,
            "temperature": s0.temperature, "top_k": s0.top_k, "top_p": s0.top_p, "min_p": s0.min_p,
            "repeat_penalty": s0.repeat_penalty, "repeat_last_n": s0.repeat_last_n,
            "candidates_out": bool(cs),
            "max_window": args.max_window or W.WINDOW,
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            # The same bytes over the wall-clock time per step, and over the
            # median time of a call launched on its own.
            "frac_ms_per_step": round(alg_bytes / (ms_per_step / 1e3) / 1e9 / HBM_PEAK_GBS, 4),
            "frac_alone": round(alg_bytes / (median_ms / 1e3) / 1e9 / HBM_PEAK_GBS, 4),
            "traffic": traffic_bytes(name) if args.op == "sample" else None,
            "traffic_source": traffic_source(name) if args.op == "sample" else None,
            "algorithmic_bytes_per_call": alg_bytes,
            "kept_per_call": kept_total,
            "call_ms_mean": round(mean_ms, 5),
            "call_ms_median_alone": round(median_ms, 5),
        },
        "cpu_baseline": cpu,
        "cpu_baseline_threads": cpu_n,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
