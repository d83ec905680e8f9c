"""Phase timings of the fused sampling kernel, per row, from the measurement
build (libllzsample_stamp.so: ``make -C llama.zig_amd stamp``).

Thread 0 of each row's workgroup records s_memrealtime (100 MHz, 10 ns) at
the phase boundaries; this script runs a workload a few times through that
build and prints, per phase, the median and the largest duration over the
rows that reached both of its boundaries, in microseconds.

    python llama.zig_amd/llz/phases.py --workload headline [--rows R] [--reps K]
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.dirname(HERE)
STAMP_LIB = os.path.join(PKG, "libllzsample_stamp.so")

# slot -> boundary (slots as the kernel writes them)
SLOTS = {
    0: "start", 1: "L end", 2: "M end", 3: "S end", 4: "F+X end", 5: "B end", 6: "C end (walk)",
    7: "streaming normaliser end", 8: "full row: buffers claimed", 9: "full row: keys written",
    10: "full row: sorted", 11: "full row: prefix filters", 12: "entropy end", 13: "typical head end",
    14: "full row end", 15: "row end",
    16: "F+X: re-reads landed (wave 0)", 17: "F+X: slots done (wave 0)", 18: "F+X: first segment summed (wave 0)",
    19: "F+X: specials settled (wave 0)", 20: "C: walk start", 21: "C: walk done (wave 0)",
    22: "S: LDS-resident batches done",
    23: "buckets: keys and coarse histogram", 24: "buckets: fine histogram", 25: "buckets: top-p classes",
    26: "buckets: top-p walk", 27: "buckets: draw classes", 28: "buckets: draw walk",
    29: "buckets (draw): sums", 30: "buckets (draw): first batch gathered", 31: "buckets (draw): first batch walked",
    32: "token-only: candidate lanes queued", 33: "token-only: candidates evaluated", 34: "token-only: sorted",
    38: "token-only: row maximum read", 39: "token-only: candidate segments scanned",
    35: "token-only: prefix and min-p counted", 36: "token-only: top-p and order checked", 37: "token-only: drawn",
    40: "recollect: histogram", 41: "recollect: cut", 42: "recollect: collected",
    43: "penalty: shared list built (wave 0)", 44: "penalty: elements patched", 45: "transforms: maximum settled",
    46: "L: load loop done (wave 0)",
    48: "entropy: first 512 terms", 49: "entropy: tile 0", 50: "entropy: tile 1", 51: "entropy: tile 16",
    52: "entropy: last tile",
}
# phases as (name, from slot, to slot)
PHASES = [
    ("L (loads)", 0, 1), ("M", 1, 2), ("S", 2, 3), ("F+X", 3, 4), ("B", 4, 5), ("C (walk)", 5, 6),
    ("selection (single pass)", 6, 15), ("streaming normaliser", 6, 7),
    ("full row: claim", 7, 8), ("full row: keys", 8, 9), ("full row: sort", 9, 10),
    ("full row: prefix filters", 10, 11), ("entropy pass", 11, 12), ("entropy pass (after short list)", 6, 12),
    ("typical head", 12, 13), ("full row: rest", 13, 14), ("whole row", 0, 15),
    ("S: LDS-resident batches", 2, 22), ("S: register batches", 22, 3),
    ("F+X: wait for re-reads (w0)", 3, 16), ("F+X: slots (w0)", 16, 17), ("F+X: first segment (w0)", 17, 18),
    ("F+X: settle (w0)", 18, 19), ("F+X: barrier wait (w0)", 19, 4), ("C: candidate reads", 5, 20),
    ("C: walk (w0)", 20, 21), ("C: after walk", 21, 6),
    ("buckets: keys + coarse histogram", 8, 23), ("buckets: fine histogram", 23, 24),
    ("buckets: top-p classes", 24, 25), ("buckets: top-p chain", 25, 26), ("buckets: draw classes", 26, 27),
    ("buckets: draw chain", 27, 28), ("buckets draw: sums", 27, 29), ("buckets draw: 1st gather+sort", 29, 30),
    ("buckets draw: 1st walk", 30, 31), ("buckets draw: rest", 31, 28),
    ("token-only: scan", 2, 32), ("M start (max, barrier)", 1, 38), ("token: estimate + scan", 38, 39),
    ("token: queue + loads issued + barrier", 39, 32), ("token-only: re-read and exact terms", 32, 33), ("token-only: sort", 33, 34),
    ("token-only: decisions", 34, 15), ("decisions: entry + counts", 34, 35), ("decisions: top-p + order", 35, 36),
    ("decisions: draw", 36, 37), ("decisions: outputs + barrier", 37, 15),
    ("recollect: histogram pass", 6, 40), ("recollect: cut", 40, 41), ("recollect: collect pass", 41, 42),
    ("after recollect: sort, filters, draw", 42, 15),
    ("penalty: list -> L end", 43, 1), ("penalty: patch (after loads)", 0, 44), ("penalty: loop end -> patched", 46, 44),
    ("penalty: patched -> list built", 44, 43),
    ("transforms: maximum (from start)", 0, 45), ("transforms: patch -> maximum", 44, 45),
    ("L: load loop (w0)", 0, 46), ("L: loop end -> L end", 46, 1), ("transforms: maximum -> L end", 45, 1),
    ("entropy: before it", 6, 48), ("entropy: first 512 terms -> tile 0", 48, 49), ("entropy: tile 1", 49, 50),
    ("entropy: tiles 2..16", 50, 51), ("entropy: tiles 17..", 51, 52), ("entropy: after it", 52, 12),
    ("entropy tile 20: loads + arguments", 53, 54), ("entropy tile 20: accumulate", 54, 55), ("entropy tile 16 end -> 20 start", 51, 53),
]


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--workload", default="headline")
    ap.add_argument("--rows", type=int, default=0, help="rows (default: the workload's batch)")
    ap.add_argument("--reps", type=int, default=3)
    ap.add_argument("--exact", action="store_true", help="ask for row statistics (the exact phases on every row)")
    ap.add_argument("--chain-params", default="", help="override the workload's chain, e.g. T=0.8,top_p=0.9,min_p=0,top_k=0")
    ap.add_argument("--dump", default="", help="also save every row's raw timestamps (.npy)")
    ap.add_argument("--post", default="", help="soft-cap and logit scale, e.g. 30,0.5 (main.zig:653-666)")
    ap.add_argument("--penalty", default="", help="repetition window and penalty over as many random history "
                                                  "tokens per row, e.g. 32,1.1 (sampler.zig:54-75)")
    ap.add_argument("--no-split", action="store_true",
                    help="one workgroup per row also for token-only calls of few rows (the split rows off)")
    ap.add_argument("--chain", type=int, default=1,
                    help="launches back to back before reading (the last one's stamps, as in a benchmark loop)")
    a = ap.parse_args()
    os.environ["LLZ_LIBRARY"] = STAMP_LIB
    sys.path.insert(0, PKG)
    import numpy as np
    import torch

    import llz
    from llz.workloads import WORKLOADS

    w = WORKLOADS[a.workload]
    rows = a.rows or w.rows
    L = llz.library()
    L.llz_debug_phase_stamps.argtypes = [C.c_void_p, C.c_int, C.c_int]
    L.llz_debug_phase_stamps.restype = C.c_int
    rows_st = min(rows, 4096)
    buf = np.zeros((rows_st, 60), np.uint64)
    x = torch.from_numpy(w.logits(rows)).cuda()
    u = torch.from_numpy(llz.rng_uniforms(w.uniform_seed, rows)).cuda()
    params = w.params
    if a.chain_params:
        import dataclasses

        names = {"T": "temperature", "top_p": "top_p", "min_p": "min_p", "top_k": "top_k", "typical_p": "typical_p"}
        kv = dict(item.split("=") for item in a.chain_params.split(","))
        params = dataclasses.replace(params, **{names[k]: (int(v) if k == "top_k" else float(v)) for k, v in kv.items()})
    post = prev = None
    if a.post:
        cap, scale = (float(v) for v in a.post.split(","))
        post = llz.LogitPost(final_logit_softcapping=cap, logit_scale=scale)
    if a.penalty:
        import dataclasses

        win, rp = a.penalty.split(",")
        params = dataclasses.replace(params, repetition_window=int(win), repetition_penalty=float(rp))
        prev = torch.from_numpy(np.random.default_rng(41).integers(0, w.vocab, size=(rows, int(win)))
                                .astype(np.int32)).cuda()
    cfg = llz.SamplerConfig.of(params)
    if a.no_split:
        llz.debug_set_split(1)
    res = None
    for _ in range(a.reps):
        assert L.llz_debug_phase_stamps(buf.ctypes.data, rows_st, 1) == 0
        torch.cuda.synchronize()
        for _ in range(a.chain):
            res = llz.sample_rows(x, cfg, u, prev, post=post, path=True, stats=a.exact)
        torch.cuda.synchronize()
    assert L.llz_debug_phase_stamps(buf.ctypes.data, rows_st, 0) == 0
    if a.dump:
        np.save(a.dump, buf)
    paths = res.row_path.cpu().numpy()
    st = buf.astype(np.int64)
    t0 = st[:, 0][st[:, 0] > 0].min()
    out = {"workload": w.name, "rows": rows, "paths": {int(k): int(v) for k, v in zip(*np.unique(paths, return_counts=True))},
           "phases_us": {}}
    for name, f, to in PHASES:
        ok = (st[:, f] > 0) & (st[:, to] > 0)
        if not ok.any():
            continue
        d = (st[ok, to] - st[ok, f]) / 100.0  # 100 MHz ticks -> us
        out["phases_us"][name] = {"rows": int(ok.sum()), "median": round(float(np.median(d)), 2),
                                  "max": round(float(d.max()), 2)}
    end = st[:, 15][st[:, 15] > 0]
    out["kernel_span_us"] = round(float((end.max() - t0) / 100.0), 2)
    print(json.dumps(out, indent=1))
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
