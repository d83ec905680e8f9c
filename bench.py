#!/usr/bin/env python3
"""Sampling-chain benchmark: sampled rows/s and achieved HBM GB/s, one MI355X.

With no flags it measures the headline workload -- 256 rows x 128256 vocab
fp32 with configuration 2's logits and filter chain (T 1.0, top-k 40, top-p
0.95, min-p 0.05) -- and prints ONE JSON line.  ``--workload c1 .. c5`` measures
the reference's other configurations, ``headline-exact``, ``headline-post``,
``headline-penalty`` and ``headline-default`` the headline's logits with the
exact outputs, the decode loop's post-processing, the repetition penalty or
the reference's default chain, ``c1-decode`` configuration 1's one-row calls
with the post-processing and the penalty (the reference's decode step), and
``all`` every line, one JSON line each.

A step is one llz_sample_rows call over one resident batch.  Inputs rotate
over enough distinct device buffers that each step reads its logits from HBM,
not from the 256 MB Infinity Cache.  Each line carries the roofline of the
step's one kernel (k_stats; k_split for token-only calls of at most 32 rows,
which read each row with several workgroups), the fraction of rows on each
path, and the CPU baseline (the reference sampler restated in C) timed on
this host with one thread and with the host's share of threads.
"""
from __future__ import annotations

import argparse
import dataclasses
import json
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (os.path.join(ROOT, "llama.zig_amd"), os.path.join(ROOT, "tests")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

PEAK_HBM_GBPS = 8000.0  # MI355X HBM3E, AMD public specification
MALL_BYTES = 256 << 20  # MI355X Infinity Cache
HOST_THREADS = 16       # the CPU share of one GPU on the GPU box
METRIC = "sampled rows/sec + achieved HBM GB/s, batch 256 x vocab 128256 fp32"


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def cpu_baseline(w, x_host, u_host, threads: int, budget_s: float, params=None, post=None, prev=None) -> dict:
    """The oracle (sampler.zig restated in C, -O2, no fast-math) on host cores:
    whole batches of the workload's first rows, repeated until budget_s.  With
    post (soft-cap, logit scale) the rows are post-processed inside the timed
    loop, as the decode loop does before sampling (main.zig:653-666)."""
    import oracle_lib as O

    params = params if params is not None else w.params
    rows = x_host.shape[0]
    n_rows = 0
    t0 = time.perf_counter()
    while True:
        x = x_host if post is None else O.logit_post(x_host, post.final_logit_softcapping, post.logit_scale)
        O.sample_rows(x, params, u_host, prev_tokens=prev, threads=threads)
        n_rows += rows
        dt = time.perf_counter() - t0
        if dt >= budget_s:
            break
    return {
        "value": round(n_rows / dt, 2),
        "unit": "rows/s",
        "cores": threads,
        "kind": "port",
        "cpu_model": cpu_model(),
        "nproc": os.cpu_count(),
        "sample": f"{n_rows} rows ({rows} distinct) of the {w.name} workload ({w.vocab} vocab), "
                  f"sampler.zig restated in C (oracle/llz_oracle.c, std stable sort in place of Zig's "
                  f"block sort), rows split over {threads} thread(s), {dt:.2f} s wall",
    }


def calibrate_copy(mib: int) -> int:
    """A plain device-to-device copy of known size (torch's copy kernel), so the
    HBM counters' bytes per dispatch can be scaled against bytes actually moved."""
    import torch

    n = mib << 20
    src = [torch.empty(n, dtype=torch.uint8, device="cuda:0").fill_(i + 1) for i in range(3)]
    dst = torch.empty(n, dtype=torch.uint8, device="cuda:0")
    torch.cuda.synchronize()
    for i in range(6):
        dst.copy_(src[i % 3])
    torch.cuda.synchronize()
    print(json.dumps({"calibration": "copy", "bytes_read": n, "bytes_written": n, "dispatches": 6}), flush=True)
    return 0


def c1_latency(w, x_host, u_host, reps: int) -> dict:
    """Configuration 1 is one row per decode step (main.zig:667): its latency
    per call, rotating over the given rows, for the device-resident batched
    entry point and for the host Sampler that takes host logits (H2D copy,
    sampling, D2H, synchronisation)."""
    import numpy as np
    import torch

    import llz

    dev = torch.device("cuda:0")
    cfg = llz.SamplerConfig.of(w.params)
    nr = x_host.shape[0]
    xs = [torch.from_numpy(x_host[b:b + 1].copy()).to(dev) for b in range(nr)]
    us = [torch.from_numpy(u_host[b:b + 1].copy()).to(dev) for b in range(nr)]
    call = llz.PreparedCall(1, w.vocab, cfg, dev)
    for i in range(20):
        call(xs[i % nr], us[i % nr])
    torch.cuda.synchronize()
    per_row = np.zeros(nr)
    for i in range(reps * nr):
        t0 = time.perf_counter()
        call(xs[i % nr], us[i % nr])
        torch.cuda.synchronize()
        per_row[i % nr] += time.perf_counter() - t0
    per_row *= 1e6 / reps

    s = llz.Sampler(llz.SamplerConfig.of(w.params, seed=0))
    rows = [np.ascontiguousarray(x_host[b]) for b in range(nr)]
    for i in range(20):
        s.sample(rows[i % nr])
    t0 = time.perf_counter()
    for i in range(reps * nr):
        s.sample(rows[i % nr])
    host_us = (time.perf_counter() - t0) * 1e6 / (reps * nr)
    s.close()
    return {"device_rows_us_per_call": round(float(per_row.mean()), 2),
            "device_rows_us_per_row": [round(float(v), 1) for v in per_row],
            "host_sampler_us_per_call": round(host_us, 2), "reps_per_row": reps, "rows": nr,
            "note": "one row per call, each call synchronised, rotating over the configuration's first rows: "
                    "llz_sample_rows on device logits, and llz_sampler_sample on host logits (513 KB H2D copy + "
                    "sampling + token D2H)"}


# bench lines: (workload, mode).  "token": the call asks for the token alone
# (the reference's Sampler.sample returns only the token, sampler.zig:26-28);
# "exact": it also asks for the kept probabilities and the row statistics
# (the exact normaliser on every row); "post": the token call after the
# decode loop's post-processing, soft-cap 30 and logit scale 0.5
# (main.zig:653-666); "penalty": the token call with the reference's default
# repetition penalty (window 32, 1.1, sampler.zig:54-75) over 32 history
# tokens per row; "decode": both, on configuration 1's one-row calls (the
# reference's decode step, main.zig:653-667).
LINES = {
    "headline": ("headline", "token"),
    "headline-exact": ("headline", "exact"),
    "headline-post": ("headline", "post"),
    "headline-penalty": ("headline", "penalty"),
    "headline-default": ("headline-default", "token"),
    "c1": ("c1", "token"),
    "c1-decode": ("c1", "decode"),
    "c2": ("c2", "token"),
    "c3": ("c3", "token"),
    "c4": ("c4", "token"),
    "c5": ("c5", "token"),
}
C1_ROWS = 8  # configuration 1 is one row per call: the steps rotate over this many rows of its generator


def run_workload(line: str, steps: int, warmup: int, args) -> dict:
    import numpy as np
    import torch

    import llz
    import oracle_lib as O
    from llz.workloads import WORKLOADS, algorithmic_bytes

    name, mode = LINES[line]
    w = WORKLOADS[name]
    dev = torch.device("cuda:0")
    rows, vocab = w.rows, w.vocab
    batch_bytes = rows * vocab * 4
    params = w.params
    post = prev = None
    if mode in ("post", "decode"):
        post = llz.LogitPost(final_logit_softcapping=30.0, logit_scale=0.5)
    if mode in ("penalty", "decode"):
        params = dataclasses.replace(params, repetition_window=32, repetition_penalty=1.1)
        prev_host = np.random.default_rng(41).integers(0, vocab, size=(rows, 32)).astype(np.int32)
        prev = torch.from_numpy(prev_host).to(dev)
    cfg = llz.SamplerConfig.of(params)
    exact = mode == "exact"
    stream = torch.cuda.current_stream()

    if name == "c1":
        # one row per call, rotating over C1_ROWS rows of the generator (each
        # step reads a row the previous steps did not)
        nbuf = C1_ROWS
        x_host = w.logits(nbuf)
        u_host = llz.rng_uniforms(w.uniform_seed, nbuf)
        xs = [torch.from_numpy(x_host[b:b + 1].copy()).to(dev) for b in range(nbuf)]
        us = [torch.from_numpy(u_host[b:b + 1].copy()).to(dev) for b in range(nbuf)]
    else:
        # one batch generated on the host; the other buffers hold its rows
        # rotated (same data, other addresses: each step reads memory the
        # previous steps did not leave in the Infinity Cache)
        nbuf = max(2, -(-2 * MALL_BYTES // batch_bytes) + 1)
        x_host = w.logits(rows)
        u_host = llz.rng_uniforms(w.uniform_seed, rows)
        x0 = torch.from_numpy(x_host).to(dev)
        u0 = torch.from_numpy(u_host).to(dev)
        xs = [torch.roll(x0, shifts=b * max(1, rows // nbuf), dims=0).contiguous() for b in range(nbuf)]
        us = [torch.roll(u0, shifts=b * max(1, rows // nbuf), dims=0).contiguous() for b in range(nbuf)]
        del x0
    call = llz.PreparedCall(rows, vocab, cfg, dev, kept_cap=64 if exact else 0, probs=exact, stats=exact,
                            stream=stream, post=post, prev_tokens=prev)

    def step(i):
        b = i % nbuf
        call(xs[b], us[b])

    # parity spot check of the timed call against the oracle, and the path
    # each row takes (the same call with the path bits asked for)
    probe = llz.PreparedCall(rows, vocab, cfg, dev, kept_cap=64 if exact else 0, probs=exact, stats=exact,
                             path=True, stream=stream, post=post, prev_tokens=prev)
    tok0, con0, paths = [], [], []
    for b in range(nbuf if name == "c1" else 1):
        r = probe(xs[b], us[b])
        torch.cuda.synchronize()
        tok0.append(r.tokens.cpu().numpy().view(np.uint32).copy())
        con0.append(r.consumed.cpu().numpy().copy())
        paths.append(r.row_path.cpu().numpy().view(np.uint32).copy())
    tok0, con0, paths = np.concatenate(tok0), np.concatenate(con0), np.concatenate(paths)
    nchk = min(8, tok0.shape[0])
    x_chk = x_host[:nchk]
    if post is not None:
        x_chk = O.logit_post(x_chk, post.final_logit_softcapping, post.logit_scale)
    p_chk = None
    if prev is not None:  # configuration 1's calls share the one history row
        p_chk = prev_host[:nchk] if prev_host.shape[0] >= nchk else np.tile(prev_host[:1], (nchk, 1))
    o_tok, o_con, _ = O.sample_rows(x_chk, params, u_host[:nchk], prev_tokens=p_chk, threads=HOST_THREADS)
    parity_ok = bool(np.array_equal(tok0[:nchk], o_tok) and np.array_equal(con0[:nchk], o_con))
    frac = lambda bit: round(float(np.mean((paths & bit) != 0)), 4)  # noqa: E731
    path_fracs = {"stream_norm": frac(llz.PATH_STREAM_NORM), "full_sort": frac(llz.PATH_FULL_SORT),
                  "entropy": frac(llz.PATH_ENTROPY), "sum_le0": frac(llz.PATH_SUM_LE0),
                  "walk_rounds": frac(llz.PATH_WALK_ROUNDS), "resolve_generic": frac(llz.PATH_RESOLVE_GENERIC),
                  "buckets": frac(llz.PATH_BUCKETS), "token_only": frac(llz.PATH_TOKEN_ONLY),
                  "recollect": frac(llz.PATH_RECOLLECT), "split": frac(llz.PATH_SPLIT),
                  "single_pass": round(float(np.mean((paths & (llz.PATH_STREAM_NORM | llz.PATH_FULL_SORT)) == 0)), 4)}
    del probe

    # W untimed warmup steps right before the timed region (after the spot
    # check, whose host work leaves the GPU idle), a synchronisation, then the
    # timed region: K steps back to back on one stream, bracketed by HIP
    # events on that stream.  The sampling kernel is the only kernel of a step, so the
    # events' interval over K is its average launch duration (the host
    # enqueues faster than the GPU runs, so launches follow each other with
    # no idle gap).  The first dispatch after the synchronisation's idle gap
    # runs about 12 us longer than the others (kernel trace of this command),
    # so one untimed lead-in step goes ahead of the start event: the events
    # time exactly the K steps, and the wall clock (from the synchronisation
    # on) includes the lead-in, so ms_per_step and value err on the slow side.
    cb = torch.cuda.Event(enable_timing=True)
    ce = torch.cuda.Event(enable_timing=True)
    for ev in (cb, ce):  # materialise the underlying HIP events
        ev.record(stream)
    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    step(warmup)  # the lead-in (untimed by the events)
    cb.record(stream)
    for i in range(steps):
        step(warmup + 1 + i)
    ce.record(stream)
    torch.cuda.synchronize()
    t1 = time.perf_counter()

    ms_per_step = (t1 - t0) * 1e3 / steps
    ms_events = cb.elapsed_time(ce) / steps
    alg = algorithmic_bytes(rows, vocab)
    achieved = alg / (ms_events * 1e-3) / 1e9
    # HBM bytes per launch from the committed counter runs of this line
    # (rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE, scaled by a device copy),
    # not measured by this run
    traffic = None
    kernel = "k_split" if path_fracs["split"] >= 0.5 else "k_stats"
    traffic_src = os.path.join("profiles", f"{kernel}_{line}_traffic.json")
    if os.path.exists(os.path.join(ROOT, traffic_src)):
        with open(os.path.join(ROOT, traffic_src)) as f:
            traffic = json.load(f).get("hbm_bytes_per_launch")

    out = {
        "metric": METRIC,
        "value": round(rows / (ms_per_step * 1e-3), 1),
        "unit": "rows/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": f"synthetic ({w.text}); numpy default_rng per row; inputs resident in HBM, "
                f"{nbuf} rotating buffers ({nbuf * batch_bytes / 2**20:.0f} MiB) to defeat the Infinity Cache",
        "config": {"workload": line, "rows": rows, "vocab": vocab, "temperature": params.temperature,
                   "top_k": params.top_k, "top_p": params.top_p, "min_p": params.min_p,
                   "typical_p": params.typical_p,
                   "call": ("token, kept probabilities (64) and row statistics" if exact else "token alone"),
                   "parallelism": "none (1 GPU)"},
        "gbps": round(alg / (ms_per_step * 1e-3) / 1e9, 1),
        "ms_per_step_events": round(ms_events, 5),
        "roofline": {"bound": "hbm", "kernel": kernel, "achieved": round(achieved, 1),
                     "peak": PEAK_HBM_GBPS, "unit": "GB/s", "frac": round(achieved / PEAK_HBM_GBPS, 4),
                     "traffic": traffic, "traffic_source": traffic_src if traffic is not None else None,
                     "kernel_ms": round(ms_events, 5),
                     "algorithmic_bytes": alg},
        "paths": path_fracs,
        "parity_spot_check": {"rows": nchk, "ok": parity_ok},
    }
    if post is not None:
        out["config"].update(final_logit_softcapping=post.final_logit_softcapping, logit_scale=post.logit_scale)
    if prev is not None:
        out["config"].update(repetition_window=params.repetition_window,
                             repetition_penalty=params.repetition_penalty, history_tokens=int(prev_host.shape[1]))
    if line == "c1":
        out["latency"] = c1_latency(w, x_host, u_host, reps=50)
    del xs, us, call
    torch.cuda.empty_cache()
    if not args.no_cpu_baseline:
        # 64 rows (a batch of fewer rows is repeated), so that every thread has rows
        reps = -(-64 // min(rows, 64))
        sample = np.ascontiguousarray(np.tile(x_host[: min(rows, 64)], (reps, 1))[:64])
        usample = np.ascontiguousarray(np.tile(u_host[: min(rows, 64)], reps)[:64])
        psample = None
        if prev is not None:
            psample = np.ascontiguousarray(np.tile(prev_host[: min(rows, 64)], (reps, 1))[:64])
        out["cpu_baseline"] = cpu_baseline(w, sample, usample, HOST_THREADS, args.cpu_seconds, params, post, psample)
        k1 = min(16, sample.shape[0])
        out["cpu_baseline_1core"] = cpu_baseline(w, sample[:k1], usample[:k1], 1, args.cpu_seconds, params, post,
                                                 None if psample is None else psample[:k1])
    return out


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=400)
    ap.add_argument("--warmup", type=int, default=40)
    ap.add_argument("--workload", default="headline",
                    help="headline (default), headline-exact, headline-post, headline-penalty, headline-default, "
                         "c1 .. c5, c1-decode, or all (one JSON line each)")
    ap.add_argument("--cpu-seconds", type=float, default=5.0,
                    help="wall-clock budget of each CPU baseline mode")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="instead of the benchmark: launch a plain device copy of MIB MiB a few times, "
                         "the known-size reference for rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE")
    args = ap.parse_args()
    if args.calibrate_copy:
        return calibrate_copy(args.calibrate_copy)

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(json.dumps({"error": "this build measures one GPU only: the sampling chain is per row and "
                                   "shards by rows with no exchange, so N>1 is not run",
                          "n_gpus": args.gpus}))
        return 2

    from llz.workloads import WORKLOADS

    names = list(LINES) if args.workload == "all" else [args.workload]
    head_rows = WORKLOADS["headline"].rows * WORKLOADS["headline"].vocab
    ok = True
    for name in names:
        w = WORKLOADS[LINES[name][0]]
        # the headline takes the given K; the others scale K by their batch size
        # (at least 10 steps), so each line times a comparable amount of work
        steps = args.steps if name == "headline" else max(10, args.steps * head_rows // (w.rows * w.vocab))
        steps = min(steps, args.steps) if name != "c1" else min(args.steps, 200)
        warmup = min(args.warmup, max(2, steps // 4))
        out = run_workload(name, steps, warmup, args)
        ok = ok and out["parity_spot_check"]["ok"]
        print(json.dumps(out), flush=True)
    return 0 if ok else 1


if __name__ == "__main__":
    sys.exit(main())
