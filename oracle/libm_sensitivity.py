#!/usr/bin/env python3
"""How much would an ulp-level difference in Zig's f32 exp / log change the
sampler's results?

The reference's std.math.exp (sampler.zig:85) and @log (sampler.zig:131,136)
cannot be run here (no Zig toolchain), so the oracle restates the msun
algorithms Zig's compiler_rt carries.  This study re-runs the oracle with the
C library's expf / logf (glibc's: a different algorithm, nearly correctly
rounded) and counts, per configuration family, the rows whose normaliser,
kept set, kept probabilities or token change.  Results are recorded in the
project's design notes; rerun with

    python oracle/libm_sensitivity.py [--rows N] [--threads T]

Test infrastructure only (it drives the oracle, never the shipped library).
"""
from __future__ import annotations

import argparse
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (os.path.join(ROOT, "llama.zig_amd"), os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)

import oracle_lib as O  # noqa: E402
from llz.workloads import WORKLOADS  # noqa: E402


def run(name: str, rows: int, threads: int) -> dict:
    w = WORKLOADS[name]
    x = w.logits(rows)
    u = O.uniforms(w.uniform_seed, rows)
    res = {}
    for mode in (0, 1):
        O.lib().llz_oracle_use_libm(mode)
        out = []
        for r in range(rows):
            o = O.sample_row(x[r], w.params, u[r])
            out.append((o.token, o.consumed, np.float32(o.sum).view(np.uint32), o.kept_ids().tobytes(),
                        o.probs[o.kept_ids()].view(np.uint32).tobytes()))
        res[mode] = out
    O.lib().llz_oracle_use_libm(0)
    a, b = res[0], res[1]
    return {
        "workload": name, "rows": rows,
        "sum_differs": sum(p[2] != q[2] for p, q in zip(a, b)),
        "kept_set_differs": sum(p[3] != q[3] for p, q in zip(a, b)),
        "kept_probs_differ": sum(p[4] != q[4] for p, q in zip(a, b)),
        "token_differs": sum(p[0] != q[0] or p[1] != q[1] for p, q in zip(a, b)),
    }


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--rows", type=int, default=64)
    ap.add_argument("--workloads", default="c1,c2,c3,c4,c5,headline")
    args = ap.parse_args()
    # how often the two libraries disagree on the arguments the chain evaluates
    import ctypes as C

    libm = C.CDLL("libm.so.6")
    libm.expf.restype = C.c_float
    libm.expf.argtypes = [C.c_float]
    xs = np.random.default_rng(0).uniform(-30.0, 0.0, 1 << 18).astype(np.float32)
    O.lib().llz_oracle_use_libm(0)
    msun = O.expf_array(xs)
    clib = np.array([libm.expf(float(v)) for v in xs], np.float32)
    print(f"expf on 2^18 arguments in [-30, 0]: the msun restatement and the C library's expf differ on "
          f"{np.mean(msun.view(np.uint32) != clib.view(np.uint32)):.3%}")
    print("| workload | rows | normaliser differs | kept set differs | kept probabilities differ | token differs |")
    print("|---|---|---|---|---|---|")
    for name in args.workloads.split(","):
        rows = 1 if name == "c1" else args.rows
        r = run(name, rows, 1)
        print(f"| {r['workload']} | {r['rows']} | {r['sum_differs']} | {r['kept_set_differs']} | "
              f"{r['kept_probs_differ']} | {r['token_differs']} |", flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
