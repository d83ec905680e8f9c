#!/usr/bin/env python3
"""Writes tests/golden/sampler_golden.npz: input/output vectors of the CPU
oracle (oracle/llz_oracle.c, the restatement of src/sampler.zig:43-169).

Test infrastructure.  The reference is Zig and cannot run here (no Zig
toolchain), so these vectors come from the oracle after it has been pinned
by tests/test_oracle_cpu.py (published RNG vectors, exp/log error bounds,
the reference's own unit tests in closed form, invariants).  They freeze the
oracle's behaviour so a regression in it, or in the GPU path, shows up as a
diff against committed data.

Cases:
  * hand-built rows (ties, -inf entries, a dominant token, crossing
    equalities) under every filter combination the reference has;
  * two rows of each configuration's logit family at vocab 4096;
  * configuration 1 at its full vocab (logits regenerated from the seed,
    guarded by a SHA-256 of the bytes).

Run: python tests/golden/make_golden.py   (rewrites the .npz)
"""
from __future__ import annotations

import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
for p in (os.path.join(ROOT, "llama.zig_amd"), os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)

import oracle_lib as O  # noqa: E402
from llz.workloads import WORKLOADS, Params  # noqa: E402

OUT = os.path.join(HERE, "sampler_golden.npz")
KEPT_CAP = 64
NO_REP = dict(repetition_window=0, repetition_penalty=1.0)


def hand_cases():
    """(name, logits, params, uniform, prev_tokens) built by hand."""
    c = []
    eq4 = np.zeros(4, np.float32)
    for u in (0.1, 0.25, 0.5, 0.75, 0.9999999):
        c.append((f"ref-equal4-u{u}", eq4, Params(temperature=1.0, top_k=0, top_p=1.0, **NO_REP), u, None))
    c.append(("ref-topk1", np.array([2.0, 1.9, 1.8], np.float32),
              Params(temperature=1.0, top_k=1, top_p=1.0, **NO_REP), 0.7, None))
    # four finite logits and -inf: p = 0.25 exactly, top-p 0.5 keeps exactly two (cum == top_p keeps)
    q = np.array([0.0, -np.inf, 0.0, 0.0, -np.inf, 0.0], np.float32)
    c.append(("quarters-topp-equal", q, Params(temperature=1.0, top_p=0.5, **NO_REP), 0.6, None))
    c.append(("quarters-topp-below", q, Params(temperature=1.0, top_p=0.4999, **NO_REP), 0.6, None))
    c.append(("quarters-minp", q, Params(temperature=1.0, top_p=1.0, min_p=1.0, **NO_REP), 0.3, None))
    c.append(("quarters-typical", q, Params(temperature=1.0, top_p=1.0, typical_p=0.6, **NO_REP), 0.3, None))
    dom = np.full(50, -1.0, np.float32)
    dom[17] = 30.0
    c.append(("dominant-empty-set", dom, Params(temperature=0.8, top_p=0.9, **NO_REP), 0.5, None))
    c.append(("greedy", dom, Params(temperature=0.0, **NO_REP), 0.5, None))
    g = np.random.default_rng(99)
    r = g.normal(0, 2, 300).astype(np.float32)
    r[::7] = r[3]  # many exact ties
    for name, p in [
        ("ties-all-filters", Params(temperature=1.3, top_k=20, top_p=0.8, min_p=0.01, typical_p=0.9, **NO_REP)),
        ("ties-typical", Params(temperature=0.7, top_p=1.0, typical_p=0.5, **NO_REP)),
        ("ties-topk", Params(temperature=0.9, top_k=7, top_p=1.0, **NO_REP)),
        ("ties-no-filters", Params(temperature=1.0, top_p=1.0, **NO_REP)),
    ]:
        c.append((name, r, p, 0.37, None))
    prev = np.array([10, 11, 11, 299, 7, 10, 123, 6000], np.uint32)
    rp = g.normal(0, 2, 300).astype(np.float32)
    rp[10], rp[11] = 4.0, -4.0
    for w in (0, 3, 8, 32):
        c.append((f"repetition-w{w}", rp,
                  Params(temperature=0.9, top_p=0.95, repetition_window=w, repetition_penalty=1.3), 0.42, prev))
    return c


def family_cases():
    c = []
    for name in ("c1", "c2", "c3", "c4", "c5", "headline"):
        w = WORKLOADS[name]
        u = O.uniforms(w.uniform_seed, 2)
        for r in range(2):
            gen = np.random.default_rng([w.data_seed, 1000 + r])
            x = w.gen_row(gen, 4096, r)
            c.append((f"{name}-v4096-row{r}", x, w.params, float(u[r]), None))
    return c


def main() -> None:
    cases = hand_cases() + family_cases()
    rec = {k: [] for k in ("name", "n", "offset", "prev_offset", "n_prev", "u", "params", "token", "consumed",
                           "kept_count", "exit_path", "stats_bits", "kept_ids", "kept_probs_bits")}
    xs, prevs = [], []
    off = poff = 0
    for name, x, p, u, prev in cases:
        o = O.sample_row(x, p, np.float32(u), prev_tokens=prev)
        rec["name"].append(name)
        rec["n"].append(x.size)
        rec["offset"].append(off)
        rec["prev_offset"].append(poff)
        rec["n_prev"].append(0 if prev is None else prev.size)
        rec["u"].append(np.float32(u))
        rec["params"].append([p.temperature, p.top_k, p.top_p, p.min_p, p.typical_p,
                              p.repetition_window, p.repetition_penalty])
        rec["token"].append(o.token)
        rec["consumed"].append(o.consumed)
        rec["kept_count"].append(o.kept_count)
        rec["exit_path"].append(o.exit_path)
        rec["stats_bits"].append(np.array([o.max_logit, o.sum, o.entropy, o.total], np.float32).view(np.uint32))
        ids = np.full(KEPT_CAP, 0xFFFFFFFF, np.uint32)
        pb = np.zeros(KEPT_CAP, np.uint32)
        if o.exit_path != O.EXIT_GREEDY:
            kept = o.kept_ids()[:KEPT_CAP]
            ids[: kept.size] = kept
            pb[: kept.size] = o.probs[kept].view(np.uint32)
        rec["kept_ids"].append(ids)
        rec["kept_probs_bits"].append(pb)
        xs.append(np.asarray(x, np.float32))
        off += x.size
        if prev is not None:
            prevs.append(prev)
            poff += prev.size

    # configuration 1 at full vocab: regenerated from its seed
    w = WORKLOADS["c1"]
    x1 = w.logits(1)[0]
    u1 = O.uniforms(w.uniform_seed, 1)[0]
    o1 = O.sample_row(x1, w.params, u1)
    kept1 = o1.kept_ids()[:KEPT_CAP]
    np.savez_compressed(
        OUT,
        name=np.array(rec["name"]), n=np.array(rec["n"], np.int64), offset=np.array(rec["offset"], np.int64),
        prev_offset=np.array(rec["prev_offset"], np.int64), n_prev=np.array(rec["n_prev"], np.int64),
        u=np.array(rec["u"], np.float32), params=np.array(rec["params"], np.float64),
        token=np.array(rec["token"], np.uint32), consumed=np.array(rec["consumed"], np.uint8),
        kept_count=np.array(rec["kept_count"], np.uint32), exit_path=np.array(rec["exit_path"], np.uint8),
        stats_bits=np.stack(rec["stats_bits"]), kept_ids=np.stack(rec["kept_ids"]),
        kept_probs_bits=np.stack(rec["kept_probs_bits"]),
        logits=np.concatenate(xs), prev_tokens=np.concatenate(prevs) if prevs else np.zeros(0, np.uint32),
        c1_sha256=np.array(hashlib.sha256(x1.tobytes()).hexdigest()),
        c1_u=np.float32(u1), c1_token=np.uint32(o1.token), c1_consumed=np.uint8(o1.consumed),
        c1_kept=np.uint32(o1.kept_count), c1_kept_ids=kept1.astype(np.uint32),
        c1_stats_bits=np.array([o1.max_logit, o1.sum, o1.entropy, o1.total], np.float32).view(np.uint32),
    )
    print(f"wrote {OUT}: {len(rec['name'])} cases + configuration 1 at full vocab")


if __name__ == "__main__":
    main()
