#!/usr/bin/env python3
"""Benchmark of the GemmaEdge token-sampling path on one MI355X.

Headline metric: rows/s of the sampler at V=262144, batch 64
(config C2: fp32 N(0,3) + peaks, softcap 30, T 0.7, top-k 40, top-p 0.9,
penalty 1.15 over 2048-id histories), with the dominant kernel's achieved HBM
bandwidth against the 8 TB/s peak; batch-1 latency (C1), C3, C4, C4's rows in
f32 (the f32 full-order path) and the C5 decode sweep are reported as extra
fields.

A "step" is one ge_sample call over the whole batch with every input already
resident in HBM. The K timed steps are one HIP-graph replay of K captured
launches, bracketed by torch.cuda.synchronize(), so the host's launch rate does
not limit the figure. Kernel durations for the roofline are measured with HIP
events on the launch stream, queued behind a spin kernel so that no host gap
falls inside an event pair.

The CPU baseline leg times the oracle (oracle/ge_oracle.cpp, a C++ restatement
of the reference sampler) on the same C2 rows on the host's cores; its outputs
also give the same-run parity counts.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--extras C1,C3,C4,C5]

Prints progress to stderr and ONE JSON line to stdout.
"""
from __future__ import annotations

import argparse
import ctypes
import dataclasses
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E peak, GB/s
PROFILE_TRAFFIC = os.path.join(ROOT, "profiles", "stream_kernel_C2_traffic.txt")
DROP_IN_BIN = os.path.join(ROOT, "tests", "cpp", "bin", "drop_in_test")


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


def parse_args():
    ap = argparse.ArgumentParser(description="GemmaEdge sampler benchmark (one MI355X)")
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--extras", default="C1,C2cold,C3,C4,C4f32,C5,dropin",
                    help="comma list of extra configs to report (C1,C2cold,C3,C4,C4f32,C5,dropin) or ''")
    ap.add_argument("--c5-steps", type=int, default=1024)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=12.0,
                    help="target wall time of the oracle baseline sample")
    ap.add_argument("--profile-pass", action="store_true",
                    help="short run for rocprofv3: --steps launches of one config plus a copy-kernel calibration")
    ap.add_argument("--profile-config", default="C2", choices=["C1", "C1g", "C1f", "C2", "C3", "C4", "C4f32", "C5"],
                    help="config of the profile pass (C5: --steps consecutive decode steps on the device ring)")
    return ap.parse_args()


class Bound:
    """A workload resident on the device with a prebuilt ge_sample_args."""

    def __init__(self, sampler, w, torch):
        from gemmaedge_amd import sampler as S
        from gemmaedge_amd.workloads import to_device

        self.w = w
        self.torch = torch
        self.logits, self.hist, self.offs, self.uni = to_device(w)
        rows = w.rows
        self.tokens = torch.empty(rows, dtype=torch.int32, device="cuda")
        self.probs = torch.empty(rows, dtype=torch.float32, device="cuda")
        self.flags = torch.empty(rows, dtype=torch.int32, device="cuda")
        a = S.SampleArgs()
        a.logits = self.logits.data_ptr()
        a.dtype = S.GE_DTYPE_BF16 if w.dtype == "bf16" else S.GE_DTYPE_F32
        a.rows = rows
        a.vocab = w.vocab
        a.row_stride = w.vocab
        a.params = S.SamplingConfig(**w.params).params()
        a.history = None if self.hist is None else self.hist.data_ptr()
        a.history_offsets = None if self.offs is None else self.offs.data_ptr()
        a.uniforms = self.uni.data_ptr()
        a.tokens_out = self.tokens.data_ptr()
        a.probs_out = self.probs.data_ptr()
        a.flags_out = self.flags.data_ptr()
        self.args = a
        self.sampler = sampler
        self.lib = S.load_library()
        self.S = S

    def launch(self, stream_ptr):
        rc = self.lib.ge_sample(self.sampler._h, ctypes.c_void_p(stream_ptr), ctypes.byref(self.args))
        if rc != 0:
            raise RuntimeError(f"ge_sample failed ({rc}): {self.S.last_error()}")

    def run_once(self):
        self.launch(self.torch.cuda.current_stream().cuda_stream)
        return self.outputs()

    def outputs(self):
        self.torch.cuda.synchronize()
        return (self.tokens.cpu().numpy(), self.probs.cpu().numpy(), self.flags.cpu().numpy())


def kernel_durations_us(torch, b: Bound, n: int):
    """Per-launch durations from HIP events on the launch stream; a spin kernel
    first keeps the GPU busy while the host queues every event pair."""
    stream = torch.cuda.current_stream()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(n)]
    torch.cuda.synchronize()
    torch.cuda._sleep(int(2.5e7))
    for e0, e1 in ev:
        e0.record(stream)
        b.launch(stream.cuda_stream)
        e1.record(stream)
    torch.cuda.synchronize()
    return np.array([e0.elapsed_time(e1) * 1000.0 for e0, e1 in ev])


def capture(torch, b: Bound, steps: int):
    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        with torch.cuda.graph(g, stream=side):
            cap = torch.cuda.current_stream()
            for _ in range(steps):
                b.launch(cap.cuda_stream)
    torch.cuda.synchronize()
    return g


def timed_graph(torch, b: Bound, steps: int, warmup: int):
    """W eager warmup launches, then EXACTLY `steps` launches as one graph
    replay bracketed by synchronize(). Returns (wall seconds, seconds between
    HIP events recorded on the launch stream around the replay)."""
    stream = torch.cuda.current_stream()
    for _ in range(warmup):
        b.launch(stream.cuda_stream)
    torch.cuda.synchronize()
    g = capture(torch, b, steps)
    g.replay()  # untimed: first replay uploads the graph
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record(stream)
    g.replay()
    e1.record(stream)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    return t1 - t0, e0.elapsed_time(e1) * 1e-3


def read_traffic():
    """HBM bytes per launch from the committed rocprofv3 PMC summary, if any."""
    if not os.path.exists(PROFILE_TRAFFIC):
        return None
    vals = {}
    for line in open(PROFILE_TRAFFIC):
        if "=" in line and not line.lstrip().startswith("#"):
            k, v = line.split("=", 1)
            vals[k.strip()] = v.strip()
    try:
        return float(vals["traffic_bytes_per_launch"])
    except (KeyError, ValueError):
        return None


def _oracle():
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import ge_oracle as O

    return O


def host_threads() -> int:
    n = os.cpu_count() or 1
    return max(1, min(n, int(os.environ.get("OMP_NUM_THREADS", n))))


def oracle_pass(w, nthreads, history=None, offsets=None):
    """One oracle pass over the workload's rows; returns (outputs, seconds)."""
    O = _oracle()
    if history is None and w.history.size:
        history, offsets = w.history, w.offsets
    t0 = time.perf_counter()
    ora = O.run(w.logits, O.make_params(**w.params), history=history, offsets=offsets,
                uniforms=w.uniforms, nthreads=nthreads)
    return ora, time.perf_counter() - t0


def parity_of(gpu_out, ora):
    """Same-run parity against the oracle: token mismatches (lowest-index tie
    rule), draws within 1e-6 of a CDF boundary (counted separately), and the
    largest relative error of the selected probability."""
    tokens, probs, flags = gpu_out
    rel = np.abs(probs.astype(np.float64) - ora.probs) / np.maximum(np.abs(ora.probs), 1e-30)
    bad = tokens != ora.tokens
    near = ora.flags != 0
    return {"rows": int(tokens.size), "token_mismatches": int(np.sum(bad)),
            "token_mismatches_outside_boundary": int(np.sum(bad & ~near)),
            "near_boundary_draws": int(np.sum(near)),
            "max_prob_rel_err": float(np.nanmax(rel)) if rel.size else 0.0}


def cpu_rate(w, seconds, nthreads, first=None):
    """Oracle rows/s on `nthreads` host threads: passes over the workload's
    rows repeated for about `seconds` (one pass at least)."""
    if first is None:
        _, first = oracle_pass(w, nthreads)
    reps = max(1, int(seconds / max(first, 1e-3)))
    t0 = time.perf_counter()
    for _ in range(reps):
        oracle_pass(w, nthreads)
    dt = time.perf_counter() - t0
    rows = reps * w.rows
    return {"rows_per_s": rows / dt, "us_per_row": dt / rows * 1e6, "threads": nthreads,
            "sample": f"{reps} pass(es) over the {w.rows}-row {w.name} batch ({rows} rows, {dt:.2f} s)"}


def cpu_baseline_leg(w, seconds: float, gpu_out):
    """CPU baseline: the oracle over the same C2 rows, one row per thread on
    the host's cores (capped by OMP_NUM_THREADS), repeated for about `seconds`.
    Its outputs are also the same-run parity reference."""
    nthreads = host_threads()
    ora, first = oracle_pass(w, nthreads)
    r = cpu_rate(w, seconds, nthreads, first)
    base = {"value": r["rows_per_s"], "unit": "rows/s", "cores": nthreads, "kind": "port",
            "sample": r["sample"] + ", oracle/ge_oracle.cpp, one row per thread"}
    return base, parity_of(gpu_out, ora)


def reference_c1(w, seconds=2.0):
    """The reference's own gemmaedge::sample_token (oracle/_ref, compiled from
    its src/generation.cpp when that checkout was present at build time) on
    C1's row after the oracle's softcap, with C1's T, k, p and no penalty (the
    reference has none): one thread, as its decode loop calls it. None when
    the library was not built."""
    O = _oracle()
    if not O.ref_available():
        return None
    p = O.make_params(**dict(w.params, repetition_penalty=1.0))
    capped = O.transform_row(w.logits[0], p)[None, :].astype(np.float32)
    kw = dict(temperature=w.params["temperature"], top_k=w.params["top_k"], top_p=w.params["top_p"],
              min_p=w.params["min_p"], seed=1)
    O.ref_sample_sequence(capped, **kw)
    reps, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        O.ref_sample_sequence(capped, **kw)
        reps += 1
    dt = time.perf_counter() - t0
    return {"us_per_token": dt / reps * 1e6, "threads": 1, "kind": "reference",
            "sample": f"{reps} calls of the reference's sample_token on C1's capped row ({dt:.2f} s), "
                      "oracle/_ref/libge_ref.so; softcap not included, the shim's copy of the row into a std::vector is"}


def bench_c1(torch, sampler, W):
    """Batch-1 latency (C1 and its greedy run). Returns (extras, {name: (workload, outputs)})."""
    out, runs = {}, {}
    for greedy in (False, True):
        w = W.c1(greedy=greedy)
        b = Bound(sampler, w, torch)
        gpu_out = b.run_once()
        d = kernel_durations_us(torch, b, 200)
        g, _ = timed_graph(torch, b, 200, 10)
        name = "C1_greedy" if greedy else "C1"
        out[name] = {
            "us_per_token_kernel_p50": float(np.median(d)),
            "us_per_token_kernel_p99": float(np.percentile(d, 99)),
            "us_per_token_graph_back_to_back": g / 200 * 1e6,
            "bytes_per_launch": w.bytes_per_row()}
        runs[name] = (w, gpu_out)
    # The reference's own dtype with top-k disabled (k = V): the f32 full-order
    # path for one row (not one of the headline configs; its latency is reported).
    w = dataclasses.replace(W.c1(), name="C1-f32-full-order", params=dict(W.c1().params, top_k=0))
    b = Bound(sampler, w, torch)
    gpu_out = b.run_once()
    d = kernel_durations_us(torch, b, 10)
    out["C1_f32_full_order"] = {"us_per_token_kernel_p50": float(np.median(d)),
                                "us_per_token_kernel_max": float(np.max(d)),
                                "bytes_per_launch": w.bytes_per_row()}
    runs["C1_f32_full_order"] = (w, gpu_out)
    return out, runs


def bench_throughput(torch, sampler, w, name):
    """Rows/s of one config. Returns (extras, {name: (workload, outputs)})."""
    b = Bound(sampler, w, torch)
    gpu_out = b.run_once()
    if np.any(gpu_out[2] & 2):
        return {name: {"status": "unsupported in this build (rows flagged GE_FLAG_UNSUPPORTED)"}}, {}
    d = kernel_durations_us(torch, b, 30)
    bytes_launch = w.bytes_per_row() * w.rows
    gbs = bytes_launch / (np.mean(d) * 1e-6) / 1e9
    return ({name: {"rows": w.rows, "rows_per_s": w.rows / (np.mean(d) * 1e-6),
                    "kernel_us": float(np.mean(d)), "GBps": gbs, "frac_peak": gbs / HBM_PEAK_GBS}},
            {name: (w, gpu_out)})


def bench_c2_cold(torch, sampler, w, copies=5, steps=100):
    """C2 with inputs that do not fit the 256 MB Infinity Cache: `copies`
    distinct copies of the batch (5 x 67.6 MB), launch i reading copy i %
    copies, all captured in one graph; average launch time from HIP events."""
    b = Bound(sampler, w, torch)
    bufs = [b.logits] + [b.logits.clone() for _ in range(copies - 1)]
    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        with torch.cuda.graph(g, stream=side):
            cs = torch.cuda.current_stream().cuda_stream
            for i in range(steps):
                b.args.logits = bufs[i % copies].data_ptr()
                b.launch(cs)
    b.args.logits = bufs[0].data_ptr()
    torch.cuda.synchronize()
    g.replay()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    g.replay()
    e1.record(stream)
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1000.0 / steps
    gbs = w.bytes_per_row() * w.rows / (us * 1e-6) / 1e9
    return {"C2_cold": {"copies": copies, "resident_bytes": int(copies * b.logits.numel() * 4),
                        "kernel_us": us, "GBps": gbs, "frac_peak": gbs / HBM_PEAK_GBS}}


def copy_peak(torch, nbytes=64 * 2**20, buffers=6, copies=60):
    """Cold device-copy rate: `buffers` source/destination pairs of `nbytes`
    each (6 x 2 x 64 MiB = 805 MB, beyond the 256 MB Infinity Cache), copy i
    moving pair i % buffers, all captured in one graph. GB/s counts bytes read
    plus bytes written."""
    n = nbytes // 4
    src = [torch.empty(n, dtype=torch.float32, device="cuda").fill_(float(i)) for i in range(buffers)]
    dst = [torch.empty_like(x) for x in src]
    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        with torch.cuda.graph(g, stream=side):
            for i in range(copies):
                dst[i % buffers].copy_(src[i % buffers])
    torch.cuda.synchronize()
    g.replay()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    g.replay()
    e1.record(stream)
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1000.0 / copies
    ok = all(bool(torch.equal(d, s_)) for d, s_ in zip(dst, src))
    del g, src, dst
    torch.cuda.empty_cache()
    return {"GBps": 2 * nbytes / (us * 1e-6) / 1e9, "us_per_copy": us, "bytes_per_copy": 2 * nbytes,
            "buffers": buffers, "resident_bytes": 2 * buffers * nbytes, "copies_checked": ok,
            "note": "torch copy_ (read + write), pair i % 6 per copy, one graph replay"}


def drop_in_latency(W, calls=400):
    """Wall-clock latency of gemmaedge::sample_token as the reference's decode
    loop calls it (a host std::vector<float> of V logits in, a token out:
    host-to-device copy, launch, device-to-host read), timed by
    tests/cpp/bin/drop_in_test in a child process over 4 C1-shaped rows."""
    import subprocess
    import tempfile

    if not os.path.exists(DROP_IN_BIN):
        return {"status": f"{os.path.relpath(DROP_IN_BIN, ROOT)} not built"}
    rows = [W.c1(seed=s) for s in (1, 2, 3, 4)]
    x = np.concatenate([w.logits for w in rows]).astype(np.float32)
    h = np.concatenate([w.history for w in rows]).astype(np.int32)
    with tempfile.TemporaryDirectory() as d:
        xf, hf = os.path.join(d, "rows.bin"), os.path.join(d, "hist.bin")
        x.tofile(xf)
        h.tofile(hf)
        r = subprocess.run([DROP_IN_BIN, "bench", xf, str(len(rows)), str(x.shape[1]), str(calls), hf,
                            str(h.size // len(rows))], capture_output=True, text=True, timeout=300)
    if r.returncode != 0:
        return {"error": f"exit {r.returncode}: {r.stderr[-300:]}"}
    out = {}
    for line in r.stdout.splitlines():
        parts = line.split()
        if len(parts) > 1 and all("=" in q for q in parts[1:]):
            out[parts[0]] = {k: float(v) for k, v in (q.split("=") for q in parts[1:])}
    out["note"] = ("wall clock per call, host vector in, token out: reference_signature = "
                   "sample_token(logits, config, rng) with T 1.0, k 64, p 0.95; penalty_overload adds "
                   "softcap 30 and penalty 1.1 over 128 ids")
    return out


def c5_sweep(torch, sampler, W, steps):
    """Batch-1 decode sweep: one captured graph (the sampling launch) replayed
    per step; the history ring and its length live on the device and grow by
    each sampled token. New logits/uniform are copied in outside the timed pair."""
    from gemmaedge_amd import sampler as S

    w = W.c5_steps(steps=steps)
    cap = int(w.notes["ring_capacity"])
    all_logits = torch.from_numpy(w.logits).cuda()
    uni_all = torch.from_numpy(w.uniforms).cuda()
    logits = torch.empty(w.vocab, dtype=torch.float32, device="cuda")
    uni = torch.empty(1, dtype=torch.float32, device="cuda")
    ring = torch.zeros((1, cap), dtype=torch.int32, device="cuda")
    ring_len = torch.zeros(1, dtype=torch.int32, device="cuda")
    tokens = torch.empty(1, dtype=torch.int32, device="cuda")
    probs = torch.empty(1, dtype=torch.float32, device="cuda")
    flags = torch.empty(1, dtype=torch.int32, device="cuda")
    a = S.SampleArgs()
    a.logits = logits.data_ptr()
    a.dtype = S.GE_DTYPE_F32
    a.rows = 1
    a.vocab = w.vocab
    a.row_stride = w.vocab
    a.params = S.SamplingConfig(**w.params).params()
    a.ring = ring.data_ptr()
    a.ring_len = ring_len.data_ptr()
    a.ring_capacity = cap
    a.uniforms = uni.data_ptr()
    a.tokens_out = tokens.data_ptr()
    a.probs_out = probs.data_ptr()
    a.flags_out = flags.data_ptr()
    lib = S.load_library()
    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        with torch.cuda.graph(g, stream=side):
            rc = lib.ge_sample(sampler._h, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream),
                               ctypes.byref(a))
    if rc != 0:
        raise RuntimeError(S.last_error())
    torch.cuda.synchronize()
    ring.zero_()
    ring_len.zero_()
    stream = torch.cuda.current_stream()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    step_tokens = torch.empty(steps, dtype=torch.int32, device="cuda")
    step_probs = torch.empty(steps, dtype=torch.float32, device="cuda")
    step_flags = torch.empty(steps, dtype=torch.int32, device="cuda")
    torch.cuda.synchronize()
    for i in range(steps):
        logits.copy_(all_logits[i])
        uni.copy_(uni_all[i:i + 1])
        ev[i][0].record(stream)
        g.replay()
        ev[i][1].record(stream)
        step_tokens[i:i + 1].copy_(tokens)
        step_probs[i:i + 1].copy_(probs)
        step_flags[i:i + 1].copy_(flags)
    torch.cuda.synchronize()
    gpu_out = (step_tokens.cpu().numpy(), step_probs.cpu().numpy(), step_flags.cpu().numpy())
    us = np.array([e0.elapsed_time(e1) * 1000.0 for e0, e1 in ev])
    out = {"steps": steps,
           "graph_replay_per_step": {
               "p50_us": float(np.median(us)), "p99_us": float(np.percentile(us, 99)),
               "mean_us": float(np.mean(us)),
               "note": "one-node graph replay per step between HIP events: includes the runtime's graph launch"},
           "history_len_final": int(ring_len.item())}

    # Device-timed steps: the same decode loop as direct ge_sample launches
    # (step i reads its logits and uniform in place), queued in blocks behind
    # a spin kernel so that no host gap falls inside an event pair; the events
    # bracket the sampler's own launch on the device.
    dev_tokens = torch.empty(steps, dtype=torch.int32, device="cuda")
    dev_ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    ring.zero_()
    ring_len.zero_()
    torch.cuda.synchronize()
    block = 128
    for lo in range(0, steps, block):
        torch.cuda._sleep(int(4e7))
        for i in range(lo, min(steps, lo + block)):
            a.logits = all_logits[i].data_ptr()
            a.uniforms = uni_all[i:i + 1].data_ptr()
            a.tokens_out = dev_tokens[i:i + 1].data_ptr()
            dev_ev[i][0].record(stream)
            rc = lib.ge_sample(sampler._h, ctypes.c_void_p(stream.cuda_stream), ctypes.byref(a))
            dev_ev[i][1].record(stream)
            if rc != 0:
                raise RuntimeError(S.last_error())
    torch.cuda.synchronize()
    dus = np.array([e0.elapsed_time(e1) * 1000.0 for e0, e1 in dev_ev])
    top = np.argsort(dus)[-8:]
    log("C5 device-timed slowest steps: " + ", ".join(f"{int(i)}:{dus[i]:.1f}us" for i in top))
    out["device_per_step"] = {
        "p50_us": float(np.median(dus)), "p99_us": float(np.percentile(dus, 99)),
        "mean_us": float(np.mean(dus)), "max_us": float(np.max(dus)),
        "tokens_match": bool(torch.equal(dev_tokens, step_tokens)),
        "note": "direct launches queued behind a spin kernel, HIP events around each launch"}

    # The same decode loop with every step captured in one graph: launch i
    # reads step i's logits and uniform in place and appends to the device
    # history ring, so the per-step cost is the sampler's own, without a graph
    # launch per step. Its tokens must equal the step-by-step run's.
    graph_tokens = torch.empty(steps, dtype=torch.int32, device="cuda")
    g_all = torch.cuda.CUDAGraph()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        with torch.cuda.graph(g_all, stream=side):
            cs = torch.cuda.current_stream().cuda_stream
            for i in range(steps):
                a.logits = all_logits[i].data_ptr()
                a.uniforms = uni_all[i:i + 1].data_ptr()
                a.tokens_out = graph_tokens[i:i + 1].data_ptr()
                rc = lib.ge_sample(sampler._h, ctypes.c_void_p(cs), ctypes.byref(a))
                if rc != 0:
                    raise RuntimeError(S.last_error())
    torch.cuda.synchronize()
    # The first replay uploads the graph. The second is timed as replayed; the
    # third behind a spin kernel, so that the runtime's submission of the
    # graph's nodes is done before the first event (the device's own time).
    timed = []
    for spin in (False, False, True):
        ring.zero_()
        ring_len.zero_()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        if spin:
            torch.cuda._sleep(int(1e8))
        e0.record(stream)
        g_all.replay()
        e1.record(stream)
        torch.cuda.synchronize()
        timed.append(e0.elapsed_time(e1) * 1000.0 / steps)
    out["one_graph_us_per_step"] = timed[2]
    out["one_graph_us_per_step_with_submission"] = timed[1]
    out["one_graph_tokens_match"] = bool(torch.equal(graph_tokens, step_tokens))
    # For the oracle: step i's history is the tokens sampled before it (the
    # window never wraps: steps <= ring capacity).
    toks = gpu_out[0]
    lens = np.array([min(i, cap) for i in range(steps)], np.int64)
    offs = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    hist = np.concatenate([toks[max(0, i - cap):i] for i in range(steps)]).astype(np.int32)
    return out, (w, gpu_out, hist, offs)


def main():
    args = parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on exactly one GPU; --gpus must be 1 "
                                   "(rows shard across GPUs without communication)"}))
        sys.exit(2)
    import torch

    from gemmaedge_amd import Sampler, available
    from gemmaedge_amd import workloads as W

    if not torch.cuda.is_available() or not available():
        print(json.dumps({"error": "no gfx950 GPU visible"}))
        sys.exit(1)
    sampler = Sampler(max_rows=512, max_vocab=W.VOCAB, max_history=8192)

    log("generating C2 (64 x 262144 fp32)")
    w = W.c2()
    b = Bound(sampler, w, torch)
    bytes_launch = w.bytes_per_row() * w.rows

    if args.profile_pass:
        stream = torch.cuda.current_stream()
        pc = args.profile_config
        if pc == "C5":
            c5_sweep(torch, sampler, W, args.steps)
        else:
            pw = {"C1": lambda: W.c1(), "C1g": lambda: W.c1(greedy=True),
                  "C1f": lambda: dataclasses.replace(W.c1(), name="C1-f32-full-order",
                                                     params=dict(W.c1().params, top_k=0)),
                  "C2": lambda: w, "C3": W.c3, "C4": W.c4, "C4f32": lambda: W.c4(f32=True)}[pc]()
            pb = b if pc == "C2" else Bound(sampler, pw, torch)
            for _ in range(args.steps):
                pb.launch(stream.cuda_stream)
        torch.cuda.synchronize()
        src = torch.empty(256 * 2**20 // 4, dtype=torch.float32, device="cuda").fill_(1.0)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        log(f"profile pass: {args.steps} {pc} launches, 5 copies of {src.numel() * 4} bytes")
        print(json.dumps({"profile_pass": True, "config": pc, "launches": args.steps, "copy_bytes": src.numel() * 4}))
        return

    log(f"timing {args.steps} steps (warmup {args.warmup})")
    seconds, ev_seconds = timed_graph(torch, b, args.steps, args.warmup)
    ms = seconds / args.steps * 1e3
    rows_per_s = w.rows * args.steps / seconds
    launch_us = ev_seconds / args.steps * 1e6  # average launch duration, HIP events
    achieved = bytes_launch / (launch_us * 1e-6) / 1e9
    d = kernel_durations_us(torch, b, 100)   # one launch per event pair
    log(f"C2: {ms * 1e3:.2f} us/step, {launch_us:.2f} us/launch (events), isolated {np.mean(d):.2f} us, "
        f"{achieved:.0f} GB/s")
    gpu_out = b.run_once()
    log("cold copy peak")
    cp = copy_peak(torch)
    log(f"copy peak {cp['GBps']:.0f} GB/s")

    extras = {}
    runs = {}  # name -> (workload, gpu outputs[, history, offsets]) for the same-run parity
    for name in [x for x in args.extras.split(",") if x]:
        log(f"extra {name}")
        try:
            if name == "C1":
                e, r = bench_c1(torch, sampler, W)
            elif name == "C2cold":
                e, r = bench_c2_cold(torch, sampler, w), {}
            elif name == "C3":
                e, r = bench_throughput(torch, sampler, W.c3(), "C3")
            elif name == "C4":
                e, r = bench_throughput(torch, sampler, W.c4(), "C4")
            elif name == "C4f32":
                # not one of the headline configs: C4's rows kept in f32 (the f32 full-order path)
                e, r = bench_throughput(torch, sampler, W.c4(f32=True), "C4_f32")
            elif name == "C5":
                c5, run = c5_sweep(torch, sampler, W, args.c5_steps)
                e, r = {"C5": c5}, {"C5": run}
            elif name == "dropin":
                e, r = {"C1_drop_in": drop_in_latency(W)}, {}
            else:
                raise ValueError(f"unknown extra {name}")
            extras.update(e)
            runs.update(r)
        except Exception as ex:  # report, do not hide
            extras[name] = {"error": repr(ex)}
        torch.cuda.empty_cache()

    cpu, parity = None, {}
    if not args.no_cpu_baseline:
        log("CPU baseline leg (oracle) ...")
        cpu, parity["C2"] = cpu_baseline_leg(w, args.cpu_seconds, gpu_out)
        log(f"C2 parity: {parity['C2']}")
        nthreads = host_threads()
        per_config = {}
        for name, run in runs.items():
            rw, rout = run[0], run[1]
            hist, offs = (run[2], run[3]) if len(run) > 2 else (None, None)
            ora, first = oracle_pass(rw, nthreads, hist, offs)
            parity[name] = parity_of(rout, ora)
            log(f"{name} parity: {parity[name]}")
            if hist is None:
                per_config[name] = cpu_rate(rw, min(args.cpu_seconds / 4, 4.0), nthreads, first)
            else:  # the decode sweep: its rows have growing histories
                per_config[name] = {"rows_per_s": rw.rows / first, "us_per_row": first / rw.rows * 1e6,
                                    "threads": nthreads,
                                    "sample": f"one pass over the {rw.rows} decode steps ({first:.2f} s)"}
        if "C1" in runs:
            # Batch 1 as the reference runs it: the softcap loop OpenMP-parallel
            # over the host's threads (generation.cpp:433), the rest of the
            # sampler on one thread; and the whole token on one thread.
            # The "C1" entry above is the first (its softcap over `nthreads`).
            w1 = runs["C1"][0]
            r1 = cpu_rate(w1, 2.0, 1)
            per_config["C1_single_thread"] = {"us_per_token": r1["us_per_row"], "threads": 1,
                                              "sample": r1["sample"]}
            ref = reference_c1(w1)
            if ref is not None:
                per_config["C1_reference_sample_token"] = ref
        cpu["per_config"] = per_config

    result = {
        "metric": "sampler rows/s at V=262144, batch 64 (C2)",
        "value": rows_per_s,
        "unit": "rows/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded Philox logits, mt19937_64 uniforms)",
        "config": {"workload": "C2: 64 rows x V=262144 fp32, softcap 30, T 0.7, top-k 40, "
                               "top-p 0.9, penalty 1.15, H=2048", "rows": w.rows, "vocab": w.vocab},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": read_traffic(),
                     "copy_peak_GBps": cp["GBps"], "frac_of_copy_peak": achieved / cp["GBps"],
                     "copy_peak": cp,
                     "kernel": "stream_kernel<float,64>", "kernel_us_mean": launch_us,
                     "kernel_us_isolated_p50": float(np.median(d)), "bytes_per_launch": bytes_launch},
        "cpu_baseline": cpu,
        "parity": parity,
        "extras": extras,
    }
    print(json.dumps(result))


if __name__ == "__main__":
    main()
