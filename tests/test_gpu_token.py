"""GPU parity of token-only rows: a call that asks for no probabilities and
no row statistics gets each row's token from the candidates' exact terms and
an interval for the normaliser, wherever every decision of the chain holds
over that interval (llz_token.h); other rows take the exact phases.

Bar: token, draw flag, kept count and kept ids bit for bit against the
oracle (sampler.zig restated), on every row, whichever path a row takes;
and the same outputs as a call asking for row statistics (the exact path).
"""
from __future__ import annotations

import dataclasses

import numpy as np
import pytest

import llz
import oracle_lib as O
from llz.workloads import WORKLOADS

pytestmark = pytest.mark.gpu

PATH_TOKEN_ONLY = 128
PATH_SPLIT = 1 << 17


def _run(cuda, x, params, u, stats=False, cap=64):
    import torch

    cfg = llz.SamplerConfig.of(params)
    res = llz.sample_rows(torch.from_numpy(np.ascontiguousarray(x)).to(cuda), cfg,
                          torch.from_numpy(np.ascontiguousarray(u, dtype=np.float32)).to(cuda),
                          kept_cap=cap, probs=stats, stats=stats, path=True)
    torch.cuda.synchronize()
    return dict(tokens=res.tokens.cpu().numpy().view(np.uint32), consumed=res.consumed.cpu().numpy(),
                kept_count=res.kept_count.cpu().numpy().view(np.uint32),
                kept_ids=res.kept_ids.cpu().numpy().view(np.uint32), path=res.row_path.cpu().numpy().view(np.uint32),
                cap=cap)


def _check_oracle(x, params, u, g, rows=None):
    rows = range(x.shape[0]) if rows is None else rows
    for r in rows:
        o = O.sample_row(x[r], params, u[r])
        ctx = f"row {r} (path {g['path'][r]:#x})"
        assert g["tokens"][r] == o.token, f"{ctx}: token {g['tokens'][r]} != {o.token}"
        assert g["consumed"][r] == o.consumed, f"{ctx}: consumed"
        assert g["kept_count"][r] == o.kept_count, f"{ctx}: kept {g['kept_count'][r]} != {o.kept_count}"
        k = min(o.kept_count, g["cap"])
        assert np.array_equal(g["kept_ids"][r, :k], o.kept_ids()[:k]), f"{ctx}: kept ids"


def test_headline_token_only_every_row(cuda):
    """Every headline row against the oracle; the rows certify without the exact normaliser."""
    w = WORKLOADS["headline"]
    x = w.logits()
    u = llz.rng_uniforms(w.uniform_seed, w.rows)
    g = _run(cuda, x, w.params, u)
    tok = (g["path"] & PATH_TOKEN_ONLY) != 0
    assert tok.mean() >= 0.99, f"{int((~tok).sum())} rows took the exact phases"
    _check_oracle(x, w.params, u, g)


def test_token_only_matches_exact_mode(cuda):
    """Configuration 2's rows: the token-only call and a call asking for row
    statistics (the exact phases) give the same outputs."""
    w = WORKLOADS["c2"]
    rows = 32
    x = w.logits(rows)
    u = llz.rng_uniforms(w.uniform_seed, rows)
    gt = _run(cuda, x, w.params, u)
    ge = _run(cuda, x, w.params, u, stats=True)
    assert np.all(gt["path"] & PATH_TOKEN_ONLY)
    assert not np.any(ge["path"] & PATH_TOKEN_ONLY)
    for k in ("tokens", "consumed", "kept_count", "kept_ids"):
        assert np.array_equal(gt[k], ge[k]), k
    _check_oracle(x, w.params, u, gt, rows=range(0, rows, 4))


@pytest.mark.parametrize("name", ["c1", "c3", "c5"])
def test_token_only_other_configs(cuda, name):
    """Top-p-only, typical-p and peaked rows: whichever path, the oracle's results."""
    w = WORKLOADS[name]
    rows = {"c1": 1, "c3": 4, "c5": 12}[name]
    x = w.logits(rows)
    u = llz.rng_uniforms(w.uniform_seed, rows)
    g = _run(cuda, x, w.params, u, cap=256)
    _check_oracle(x, w.params, u, g)


def test_token_only_undecidable_rows_fall_back(cuda):
    """Rows built so that a decision sits on its boundary: a term exactly at
    min-p, a draw on a CDF boundary, top-p binding.  They leave the
    token-only path and still match the oracle."""
    w = WORKLOADS["headline"]
    rows = 6
    x = w.logits(rows).copy()
    u = llz.rng_uniforms(w.uniform_seed, rows).copy()
    p = w.params
    # row 0: a term at min-p (v = m + T ln(min_p), rounded)
    m0 = x[0].max()
    x[0, 17] = np.float32(m0 + np.float32(np.log(np.float32(p.min_p))))
    # row 1: the draw on the boundary after the first kept term
    o1 = O.sample_row(x[1], p, np.float32(0.5))
    k1 = max(o1.kept_count, 1)
    probs = o1.probs[o1.kept_ids()[:k1]].astype(np.float64)
    u[1] = np.float32(probs[0] / probs.sum())
    g = _run(cuda, x, p, u)
    # row 0's min-p term may round clear of the band: only the oracle decides it.
    # Row 1's draw lands on a CDF boundary, inside the draw's margin: the row
    # must leave the token path
    assert not (g["path"][1] & PATH_TOKEN_ONLY), f"row 1 certified a boundary draw (path {g['path'][1]:#x})"
    _check_oracle(x, p, u, g)
    # top-p binding: configuration 2's logits with top-p 0.3
    p2 = dataclasses.replace(p, top_p=0.3)
    g2 = _run(cuda, x, p2, u)
    _check_oracle(x, p2, u, g2)


def test_token_only_top_p_cut_inside_interval_falls_back(cuda):
    """Ten equal terms over a low floor with top-p 0.3: the running sum after
    three terms is 3/S with S close to 10, and the reference's S is known
    only to (n - 1) 2^-24 (the recursive-summation bound), about 0.8%, so
    the cut cannot be decided without the exact normaliser.  The row leaves
    the token path and matches the oracle; the same logits with top-p 0.5
    (a cut clear of the interval) stay on it."""
    w = WORKLOADS["headline"]
    rows = 2
    rng = np.random.default_rng(5)
    x = rng.normal(-30.0, 1.0, size=(rows, w.vocab)).astype(np.float32)
    for r in range(rows):
        x[r, rng.choice(w.vocab, 10, replace=False)] = 0.0
    u = llz.rng_uniforms(w.uniform_seed, rows)
    p = dataclasses.replace(w.params, top_k=0, top_p=0.3)
    g = _run(cuda, x, p, u)
    assert not np.any(g["path"] & PATH_TOKEN_ONLY), f"paths {g['path']}"
    _check_oracle(x, p, u, g)
    p5 = dataclasses.replace(p, top_p=0.45)
    g5 = _run(cuda, x, p5, u)
    assert np.all(g5["path"] & PATH_TOKEN_ONLY), f"paths {g5['path']}"
    _check_oracle(x, p5, u, g5)


def test_token_only_top_p_without_min_p(cuda):
    """The reference's default chain (no min-p; top-p 0.9, T 0.8): the token
    path's list holds the terms e >= 2^-10, and a row certifies when its
    top-p cut falls inside the list and clear of the normaliser's interval
    (about 0.8% at 128k terms).  Configuration 1's rows 1-3 do (their cuts
    lie 2% or more from 0.9); row 0's running sum stops 0.04% short of 0.9,
    so it takes the exact phases.  On the headline's logits the nuclei are
    long and fine-grained, so most rows take the exact phases too.  Every row
    matches the oracle."""
    c1 = WORKLOADS["c1"]
    x1 = c1.logits(4)
    u1 = llz.rng_uniforms(c1.uniform_seed, 4)
    g1 = _run(cuda, x1, c1.params, u1)
    assert np.all(g1["path"][1:] & PATH_TOKEN_ONLY), f"paths {g1['path']}"
    assert not (g1["path"][0] & PATH_TOKEN_ONLY), f"path {g1['path'][0]:#x}"
    _check_oracle(x1, c1.params, u1, g1)
    w = WORKLOADS["headline"]
    rows = 48
    x = w.logits(rows)
    u = llz.rng_uniforms(w.uniform_seed, rows)
    p = dataclasses.replace(w.params, temperature=0.8, top_k=0, top_p=0.9, min_p=0.0)
    g = _run(cuda, x, p, u)
    _check_oracle(x, p, u, g)
    # with top-k inside the list as well
    pk = dataclasses.replace(p, top_k=20)
    gk = _run(cuda, x, pk, u)
    _check_oracle(x, pk, u, gk)


@pytest.mark.parametrize("kind", ["flat", "wide-nucleus"])
def test_token_only_top_p_without_min_p_falls_back(cuda, kind):
    """Top-p without min-p where the cut is not inside the list: a near-flat
    row (every term past the list's reach) and top-p 0.999 on peaked rows
    (the list holds less than 0.999 of the mass).  The rows take the exact
    phases and match the oracle."""
    w = WORKLOADS["headline"]
    rows = 4
    if kind == "flat":
        x = np.random.default_rng(3).normal(0.0, 0.3, size=(rows, 100000)).astype(np.float32)
        p = dataclasses.replace(w.params, temperature=1.2, top_k=0, top_p=0.9, min_p=0.0)
    else:
        x = WORKLOADS["c1"].logits(rows)
        p = dataclasses.replace(WORKLOADS["c1"].params, top_p=0.999)
    u = llz.rng_uniforms(w.uniform_seed, rows)
    g = _run(cuda, x, p, u, cap=256)
    assert not np.any(g["path"] & PATH_TOKEN_ONLY), f"paths {g['path']}"
    _check_oracle(x, p, u, g)


def test_token_only_kept_ids_without_cap(cuda):
    """No kept ids asked for (the benchmark's call): tokens and flags only."""
    import torch

    w = WORKLOADS["headline"]
    rows = 64
    x = w.logits(rows)
    u = llz.rng_uniforms(w.uniform_seed, rows)
    cfg = llz.SamplerConfig.of(w.params)
    res = llz.sample_rows(torch.from_numpy(x).to(cuda), cfg, torch.from_numpy(u).to(cuda))
    torch.cuda.synchronize()
    tok = res.tokens.cpu().numpy().view(np.uint32)
    con = res.consumed.cpu().numpy()
    ot, oc, _ = O.sample_rows(x, w.params, u, threads=8)
    assert np.array_equal(tok, ot)
    assert np.array_equal(con, oc)


@pytest.mark.parametrize("kind", ["flat", "many"])
def test_token_only_overflow_falls_back(cuda, kind):
    """Min-p rows whose candidates overflow the token path: a flat row (its
    candidate lanes overflow every wave's queue) and 600 terms near the
    maximum over a low floor without top-k (the lanes fit, the 512-entry list
    does not, and no top-k lets it be collected again).  The exact phases
    follow, with the oracle's results."""
    w = WORKLOADS["headline"]
    rows = 4
    rng = np.random.default_rng(7)
    params = w.params
    if kind == "flat":
        x = rng.normal(0.0, 0.3, size=(rows, w.vocab)).astype(np.float32)
    else:
        x = _many_near_max(rng, rows, w.vocab, 600)
        params = dataclasses.replace(params, top_k=0)
    u = llz.rng_uniforms(w.uniform_seed, rows)
    g = _run(cuda, x, params, u, cap=256)
    assert not np.any(g["path"] & PATH_TOKEN_ONLY)
    _check_oracle(x, params, u, g)


@pytest.mark.parametrize("terms", [600, 700])
def test_token_only_list_collected_again(cuda, terms):
    """More terms above min-p's threshold than the 512-entry list holds (40
    of them 1% apart at the top, the rest in [-1.5, -0.5] below the maximum,
    over a low floor), under top-k 40 and typical-p 0.98 (the token call's
    second collection round is built into the typical-p instantiation): the
    list is collected again above just below the 41st largest term
    collected, and every row decides on the token path (min-p's count beyond
    the list unknown: top-k cuts inside it; the kept surprises lie below the
    entropy).  Every row against the oracle; without typical-p the same rows
    take the exact phases, also against the oracle."""
    w = WORKLOADS["headline"]
    rows = 4
    rng = np.random.default_rng(11)
    x = rng.normal(-30.0, 1.0, size=(rows, w.vocab)).astype(np.float32)
    for r in range(rows):
        idx = rng.choice(w.vocab, terms, replace=False)
        x[r, idx[:40]] = (-0.01 * np.arange(40)).astype(np.float32)
        x[r, idx[40:]] = rng.uniform(-1.5, -0.5, terms - 40).astype(np.float32)
    u = llz.rng_uniforms(w.uniform_seed, rows)
    params = dataclasses.replace(w.params, typical_p=0.98)
    g = _run(cuda, x, params, u, cap=256)
    _check_oracle(x, params, u, g)
    assert np.all(g["path"] & PATH_TOKEN_ONLY), f"paths {g['path']}"
    g0 = _run(cuda, x, w.params, u, cap=256)
    _check_oracle(x, w.params, u, g0)
    assert not np.any(g0["path"] & PATH_TOKEN_ONLY), f"paths {g0['path']}"


def _many_near_max(rng, rows, n, k):
    x = rng.normal(-30.0, 1.0, size=(rows, n)).astype(np.float32)
    for r in range(rows):
        idx = rng.choice(n, k, replace=False)
        x[r, idx] = rng.uniform(-1.0, 0.0, k).astype(np.float32)
    return x


@pytest.mark.parametrize("split", [False, True])
def test_token_only_long_list(cuda, split):
    """300 terms near the maximum over a low floor: a list between 256 and
    512 terms (rank sort with two keys a lane and up to 38 a wave's eighth),
    decided on the token path, with one workgroup per row or split rows."""
    w = WORKLOADS["headline"]
    rows = 4
    x = _many_near_max(np.random.default_rng(7), rows, w.vocab, 300)
    u = llz.rng_uniforms(w.uniform_seed, rows)
    if not split:
        llz.debug_set_split(1)
    try:
        g = _run(cuda, x, w.params, u, cap=256)
    finally:
        llz.debug_set_split(0)
    assert np.all(g["path"] & PATH_TOKEN_ONLY)
    assert np.all(((g["path"] & PATH_SPLIT) != 0) == split)
    _check_oracle(x, w.params, u, g)


def test_token_only_wave_with_many_candidates(cuda):
    """About 100 terms near the maximum, all in one wave's segments (segment
    g belongs to wave g mod 8), over a low floor: that wave has more than 64
    candidate elements, so it evaluates its queued lanes' four terms each
    instead of staging one element per lane.  The list (100 terms) fits and
    the rows still certify on the token path."""
    w = WORKLOADS["headline"]
    rows = 6
    rng = np.random.default_rng(11)
    x = rng.normal(-30.0, 1.0, size=(rows, w.vocab)).astype(np.float32)
    pos = np.arange(w.vocab)
    for r in range(rows):
        wave = r % 8
        own = pos[((pos // 256) % 8) == wave]
        idx = rng.choice(own, 90 + 5 * r, replace=False)
        x[r, idx] = rng.uniform(-1.0, 0.0, idx.size).astype(np.float32)
    u = llz.rng_uniforms(w.uniform_seed, rows)
    g = _run(cuda, x, w.params, u)
    assert np.all(g["path"] & PATH_TOKEN_ONLY), f"rows off the token path: {g['path']}"
    _check_oracle(x, w.params, u, g)


def test_token_only_typical_rows(cuda):
    """Typical-p on the token path (configuration 5: top-k 50, top-p 0.9,
    min-p 0.02, typical-p 0.98): the kept terms in the order of their
    distance to an interval of the row's entropy, every decision checked over
    the intervals.  Every row against the oracle; the rows decide on the
    token path (the N(0, 2) rows' kept surprises lie far below their entropy,
    the peaked rows keep nothing before typical-p)."""
    w = WORKLOADS["c5"]
    rows = 64
    x = w.logits(rows)
    u = llz.rng_uniforms(w.uniform_seed, rows)
    g = _run(cuda, x, w.params, u)
    _check_oracle(x, w.params, u, g)
    tok = (g["path"] & PATH_TOKEN_ONLY) != 0
    assert tok.mean() >= 0.9, f"{int((~tok).sum())} rows took the exact phases"


def test_token_only_typical_entropy_among_kept_falls_back(cuda):
    """Rows whose entropy lies among the kept terms' surprises (30 tokens near
    +10 over N(0, 1) logits) and whose typical-p cut falls inside the kept
    terms (typical-p 0.5): their typical order depends on the exact entropy,
    so they take the exact phases.  With typical-p 0.98 nothing is cut (the
    kept terms' sum stays below it whatever the normaliser), the order does
    not matter, and the same rows decide on the token path (most of them).
    Every row against the oracle."""
    rng = np.random.default_rng(7)
    rows, n = 8, 32768
    x = rng.normal(0.0, 1.0, (rows, n)).astype(np.float32)
    for r in range(rows):
        ids = rng.choice(n, 30, replace=False)
        x[r, ids] = (10.0 + rng.normal(0.0, 0.5, 30)).astype(np.float32)
    params = dataclasses.replace(WORKLOADS["c5"].params, typical_p=0.5)
    u = llz.rng_uniforms(5, rows)
    g = _run(cuda, x, params, u)
    _check_oracle(x, params, u, g)
    # the premise, from the oracle: the entropy lies inside the kept surprises
    for r in range(rows):
        o = O.sample_row(x[r], params, u[r])
        s = -np.log(o.probs[o.order[:20]].astype(np.float64))
        assert s.min() < o.entropy < s.max()
    assert np.all((g["path"] & PATH_TOKEN_ONLY) == 0)
    p98 = WORKLOADS["c5"].params
    g98 = _run(cuda, x, p98, u)
    _check_oracle(x, p98, u, g98)
    # (a row may still leave the token path for another decision, e.g. top-p's cut near S's interval)
    assert np.mean((g98["path"] & PATH_TOKEN_ONLY) != 0) >= 0.75, f"paths {g98['path']}"
