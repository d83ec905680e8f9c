"""GPU parity of split rows: token-only calls of at most 64 plain rows read
each row with several workgroups, one chunk each; the workgroup that
finishes a row merges the chunks' maxima, sums and short lists, then makes
the chain's decisions as the token path does (llz_split.h), or finishes the
row with the single-row path when a check fails.

Bar: token, draw flag, kept count and kept ids bit for bit against the
oracle (sampler.zig restated) on every row, and against the same call with
split rows off, whichever path a row takes.
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


def _run(cuda, x, params, u, cap=64, split=True, post=None, prev=None):
    """split: True (the library's choice), False (off), or the chunk width
    nv in float4 per thread (2, 4, 8: at least that)."""
    import torch

    cfg = llz.SamplerConfig.of(params)
    pt = None if prev is None else torch.from_numpy(np.ascontiguousarray(prev, dtype=np.int32)).to(cuda)
    llz.debug_set_split(0 if split is True else (1 if split is False else int(split)))
    try:
        res = llz.sample_rows(torch.from_numpy(np.ascontiguousarray(x)).to(cuda), cfg,
                              torch.from_numpy(np.ascontiguousarray(u, dtype=np.float32)).to(cuda), pt,
                              post=post, kept_cap=cap, probs=False, stats=False, path=True)
        torch.cuda.synchronize()
    finally:
        llz.debug_set_split(False)
    return dict(tokens=res.tokens.cpu().numpy().view(np.uint32), consumed=res.consumed.cpu().numpy(),
                kept_count=res.kept_count.cpu().numpy().view(np.uint32),
                kept_ids=res.kept_ids.cpu().numpy().view(np.uint32), path=res.row_path.cpu().numpy().view(np.uint32),
                cap=cap)


def _check_oracle(x, params, u, g, rows=None, post=None, prev=None):
    rows = range(x.shape[0]) if rows is None else rows
    if post is not None:
        x = O.logit_post(x, post.final_logit_softcapping, post.logit_scale)
    for r in rows:
        o = O.sample_row(x[r], params, u[r], prev_tokens=None if prev is None else prev[r])
        ctx = f"row {r} (path {g['path'][r]:#x})"
        assert g["tokens"][r] == o.token, f"{ctx}: token {g['tokens'][r]} != {o.token}"
        assert g["consumed"][r] == o.consumed, f"{ctx}: consumed"
        assert g["kept_count"][r] == o.kept_count, f"{ctx}: kept {g['kept_count'][r]} != {o.kept_count}"
        k = min(o.kept_count, g["cap"])
        assert np.array_equal(g["kept_ids"][r, :k], o.kept_ids()[:k]), f"{ctx}: kept ids"


def _same(a, b):
    for k in ("tokens", "consumed", "kept_count", "kept_ids"):
        assert np.array_equal(a[k], b[k]), k


def _split_frac(g):
    return float(np.mean((g["path"] & PATH_SPLIT) != 0))


def _split_covers(g, g_off):
    """Rows the unsplit call finishes on its token path are split rows (both
    certify from the same kind of interval for the normaliser); returns how
    many such rows there were."""
    tok = (g_off["path"] & PATH_TOKEN_ONLY) != 0
    miss = np.flatnonzero(tok & ((g["path"] & PATH_SPLIT) == 0))
    assert miss.size <= tok.sum() // 10, f"token-path rows not split: {miss.tolist()}"
    return int(tok.sum())


@pytest.mark.parametrize("rows", [1, 2, 8, 16, 32, 64])
def test_split_rows_c2(cuda, rows):
    """Configuration 2 (min-p): chunk widths 1, 2, 4 and 8 float4 per thread as
    the row count grows (64 rows: not split, one workgroup per row), against
    the oracle and the unsplit call."""
    w = WORKLOADS["c2"]
    x = w.logits(rows)
    u = llz.rng_uniforms(w.uniform_seed, rows)
    g = _run(cuda, x, w.params, u)
    assert _split_frac(g) >= (0.9 if rows <= 32 else 0.0), f"paths {[hex(p) for p in g['path']]}"
    assert np.all(g["path"][(g["path"] & PATH_SPLIT) != 0] & PATH_TOKEN_ONLY)
    _same(g, _run(cuda, x, w.params, u, split=False))
    _check_oracle(x, w.params, u, g, rows=range(0, rows, max(1, rows // 8)))


@pytest.mark.parametrize("nv", [2, 4, 8])
def test_split_rows_chunk_widths(cuda, nv):
    """Every chunk width on few rows (the library picks 1 for them), against
    the unsplit call and the oracle."""
    w = WORKLOADS["c2"]
    rows = 3
    x = w.logits(rows)
    u = llz.rng_uniforms(w.uniform_seed, rows)
    g = _run(cuda, x, w.params, u, split=nv)
    assert _split_frac(g) >= 2 / 3, f"paths {[hex(p) for p in g['path']]}"
    _same(g, _run(cuda, x, w.params, u, split=False))
    _check_oracle(x, w.params, u, g)


def test_split_hook_rejects_other_modes(cuda):
    for bad in (3, 5, 16, -1):
        with pytest.raises(llz.LlzError):
            llz.debug_set_split(bad)
    llz.debug_set_split(0)


@pytest.mark.parametrize("rows", [1, 4, 24])
def test_split_rows_c1(cuda, rows):
    """Configuration 1 (top-p alone, eight boosted tokens) against the oracle."""
    w = WORKLOADS["c1"]
    x = w.logits(rows)
    u = llz.rng_uniforms(w.uniform_seed, rows)
    g = _run(cuda, x, w.params, u, cap=256)
    g_off = _run(cuda, x, w.params, u, cap=256, split=False)
    # top-p alone: a row whose cut lies within the normaliser's interval
    # (the sequential sum's bound, (n - 1) 2^-24 ~ 2^-7 here) needs the exact
    # normaliser on either path
    _split_covers(g, g_off)
    _same(g, g_off)
    _check_oracle(x, w.params, u, g)


def test_split_rows_headline_params(cuda):
    """The headline's rows and chain (top-k, top-p, min-p), 24 rows."""
    w = WORKLOADS["headline"]
    rows = 24
    x = w.logits(rows)
    u = llz.rng_uniforms(w.uniform_seed, rows)
    g = _run(cuda, x, w.params, u)
    assert _split_frac(g) >= 0.9
    _same(g, _run(cuda, x, w.params, u, split=False))
    _check_oracle(x, w.params, u, g, rows=range(0, rows, 6))


@pytest.mark.parametrize("vocab", [4096, 50000, 151936, 256000])
def test_split_rows_vocab_sizes(cuda, vocab):
    """Chunk counts from 2 upwards, a last chunk shorter than the others, and
    vocabularies that need wider chunks to stay within 64 of them."""
    rng = np.random.default_rng(vocab)
    rows = 3
    x = rng.normal(0.0, 2.0, size=(rows, vocab)).astype(np.float32)
    for r in range(rows):
        x[r, rng.choice(vocab, 5, replace=False)] += np.float32(9.0)
    u = rng.random(rows, dtype=np.float32)
    p = dataclasses.replace(WORKLOADS["c2"].params)
    g = _run(cuda, x, p, u)
    assert _split_frac(g) >= 2 / 3, f"paths {[hex(q) for q in g['path']]}"
    _same(g, _run(cuda, x, p, u, split=False))
    _check_oracle(x, p, u, g)


def test_split_rows_special_values(cuda):
    """Rows the merge must not certify, or whose chunks hold nothing: a NaN,
    +inf, a flat row (every chunk's list overflows at its first bin), chunks
    of -inf only, a row of -inf with one finite logit, huge negative padding.
    Every row gets the oracle's results."""
    w = WORKLOADS["c2"]
    rows = 8
    x = w.logits(rows).copy()
    u = llz.rng_uniforms(w.uniform_seed, rows)
    x[0, 1234] = np.nan
    x[1, 99999] = np.inf
    x[2, :] = np.float32(0.5)
    x[3, : 70000] = -np.inf
    x[4, :] = -np.inf
    x[4, 77777] = np.float32(3.0)
    x[5, 100000:] = np.float32(-1.0e30)
    x[6, 4096: 8192] = np.float32(x[6].max() + 30.0)  # one chunk far above the rest, flat inside
    g = _run(cuda, x, w.params, u, cap=256)
    for r in (0, 1, 2, 6):
        assert not (g["path"][r] & PATH_SPLIT), f"row {r} certified by the merge (path {g['path'][r]:#x})"
    _same(g, _run(cuda, x, w.params, u, cap=256, split=False))
    _check_oracle(x, w.params, u, g)


def test_split_rows_boundary_decisions(cuda):
    """A term exactly at min-p and a draw on a CDF boundary: the merge leaves
    the row to the single-row path, which matches the oracle."""
    w = WORKLOADS["headline"]
    rows = 4
    x = w.logits(rows).copy()
    u = llz.rng_uniforms(w.uniform_seed, rows).copy()
    p = w.params
    m0 = x[0].max()
    x[0, 17] = np.float32(m0 + np.float32(np.log(np.float32(p.min_p))))
    o1 = O.sample_row(x[1], p, np.float32(0.5))
    k1 = max(o1.kept_count, 1)
    probs = o1.probs[o1.kept_ids()[:k1]].astype(np.float64)
    u[1] = np.float32(probs[0] / probs.sum())
    g = _run(cuda, x, p, u)
    assert not (g["path"][1] & PATH_TOKEN_ONLY), f"row 1 certified a boundary draw (path {g['path'][1]:#x})"
    _same(g, _run(cuda, x, p, u, split=False))
    _check_oracle(x, p, u, g)


def test_split_rows_workspace_reuse(cuda):
    """Calls in a row on one workspace with different row counts and chunk
    counts: a chunk record counts only under its own call's tag."""
    import torch

    w = WORKLOADS["c2"]
    cfg = llz.SamplerConfig.of(w.params)
    xs = {r: w.logits(r) for r in (32, 1, 17)}
    dev = torch.device(cuda)
    ws = torch.empty(llz.workspace_bytes(32, w.vocab, cfg), dtype=torch.uint8, device=dev)
    ws.fill_(0xA5)  # not cleared: arbitrary bytes
    for it in range(2):
        for r, x in xs.items():
            u = llz.rng_uniforms(w.uniform_seed + it, r)
            res = llz.sample_rows(torch.from_numpy(x).to(dev), cfg, torch.from_numpy(u).to(dev), kept_cap=64,
                                  probs=False, path=True, workspace=ws)
            torch.cuda.synchronize()
            g = dict(tokens=res.tokens.cpu().numpy().view(np.uint32), consumed=res.consumed.cpu().numpy(),
                     kept_count=res.kept_count.cpu().numpy().view(np.uint32),
                     kept_ids=res.kept_ids.cpu().numpy().view(np.uint32),
                     path=res.row_path.cpu().numpy().view(np.uint32), cap=64)
            assert _split_frac(g) >= 0.9
            _check_oracle(x, w.params, u, g, rows=range(0, r, max(1, r // 4)))


# ---- rows read through the decode loop's post-processing and the penalty

POSTS = {"cap+scale": (30.0, 0.5), "scale": (0.0, 0.5), "cap": (30.0, 1.0), "none": None}


def _histories(x, n_prev, seed, top=4):
    """History rows of n_prev random ids whose last `top` are the row's
    largest logits (the penalty then moves the maximum and the kept set)."""
    rows, n = x.shape
    prev = np.random.default_rng(seed).integers(0, n, (rows, n_prev)).astype(np.uint32)
    for r in range(rows):
        prev[r, -top:] = np.argsort(-x[r], kind="stable")[:top]
    return prev


@pytest.mark.parametrize("rows", [1, 8])
@pytest.mark.parametrize("pen", [False, True])
@pytest.mark.parametrize("post_name", list(POSTS))
def test_split_rows_transformed(cuda, post_name, pen, rows):
    """Soft-cap and/or logit scale (main.zig:653-666) and the repetition
    penalty over a 32-token window (sampler.zig:54-75), applied exactly to
    every logit of a chunk: the same outputs as the unsplit call, and the
    oracle's on the post-processed rows with the same histories."""
    if post_name == "none" and not pen:
        pytest.skip("plain rows: covered above")
    w = WORKLOADS["c2"]
    x = w.logits(rows)
    u = llz.rng_uniforms(w.uniform_seed, rows)
    post = None if POSTS[post_name] is None else llz.LogitPost(final_logit_softcapping=POSTS[post_name][0],
                                                               logit_scale=POSTS[post_name][1])
    params = w.params
    prev = None
    if pen:
        params = dataclasses.replace(params, repetition_window=32, repetition_penalty=1.1)
        prev = _histories(x, 32, seed=rows)
    g = _run(cuda, x, params, u, post=post, prev=prev)
    assert _split_frac(g) >= 0.5, f"paths {[hex(p) for p in g['path']]}"
    _same(g, _run(cuda, x, params, u, split=False, post=post, prev=prev))
    _check_oracle(x, params, u, g, post=post, prev=prev)


def test_split_rows_decode_loop_shape(cuda):
    """The reference's decode step: one row, the default chain (T 0.8, top-p
    0.9), soft-cap 30 and logit scale 0.5, the default penalty over the last
    32 tokens; eight rows of configuration 1's generator, one call each."""
    w = WORKLOADS["c1"]
    x = w.logits(8)
    u = llz.rng_uniforms(w.uniform_seed, 8)
    post = llz.LogitPost(final_logit_softcapping=30.0, logit_scale=0.5)
    params = dataclasses.replace(w.params, repetition_window=32, repetition_penalty=1.1)
    prev = _histories(x, 32, seed=5)
    for r in range(8):
        g = _run(cuda, x[r:r + 1], params, u[r:r + 1], cap=256, post=post, prev=prev[r:r + 1])
        _check_oracle(x[r:r + 1], params, u[r:r + 1], g, post=post, prev=prev[r:r + 1])


# ---- the interval of S weighted by where the row's mass lies

def _late_mass_rows(rows, n, seed):
    """Rows whose largest terms lie in their last 1,000 positions, with a
    top-p whose cut sits 0.3% past a cumulative sum: inside the
    recursive-summation interval of S (about 0.77% at 128k terms), outside
    the same bound weighted by position (about 0.01% here)."""
    rng = np.random.default_rng(seed)
    x = rng.normal(0.0, 2.0, size=(rows, n)).astype(np.float32)
    for r in range(rows):
        x[r, n - 1000 + rng.choice(1000, 8, replace=False)] += np.float32(12.0)
    base = dataclasses.replace(WORKLOADS["c1"].params, top_p=0.9)
    u = rng.random(rows, dtype=np.float32)
    tps = []
    for r in range(rows):
        o = O.sample_row(x[r], base, u[r])
        c = np.cumsum(np.sort(o.probs.astype(np.float64))[::-1])
        q = next(q for q in range(1, 8) if c[q + 1] > c[q] * 1.02)
        tps.append(float(np.float32(c[q] * 1.003)))
    return x, u, base, tps


@pytest.mark.parametrize("split", [True, False], ids=["split", "one-workgroup"])
def test_top_p_cut_certified_by_position_weighted_interval(cuda, split):
    """Top-p cuts 0.3% from a cumulative sum, in rows whose mass lies at
    their end: certified on the token path (both launches) and the oracle's
    results."""
    n = 128256
    x, u, base, tps = _late_mass_rows(4, n, seed=77)
    for r in range(4):
        params = dataclasses.replace(base, top_p=tps[r])
        g = _run(cuda, x[r:r + 1], params, u[r:r + 1], cap=256, split=split)
        assert g["path"][0] & PATH_TOKEN_ONLY, f"row {r}: path {g['path'][0]:#x}"
        _check_oracle(x[r:r + 1], params, u[r:r + 1], g)
