"""GPU parity of the bucket path: rows without typical-p whose kept prefix
overflows the candidate list get top-k / top-p / min-p, the total and the
draw from buckets of the p keys instead of a sort of the row
(sampler.zig:106-126, 156-168).

The path runs when the caller asks for no kept ids (their p order needs the
sort), so these tests compare what it returns -- token, draw flag, kept
count, row maximum, normaliser and kept total -- bit for bit with the oracle,
and with the sorting path on the same rows.  The kept count fixes the kept
set: it is the first K elements of (p desc, id asc).
"""
from __future__ import annotations

import dataclasses

import numpy as np
import pytest

import llz
import oracle_lib as O
from llz.workloads import WORKLOADS, Params

pytestmark = pytest.mark.gpu


def _bits(a) -> np.ndarray:
    return np.asarray(a, dtype=np.float32).view(np.uint32)


def _run(cuda, x, params, u, kept_cap=0):
    import torch

    cfg = llz.SamplerConfig.of(params)
    res = llz.sample_rows(torch.from_numpy(np.ascontiguousarray(x)).to(cuda), cfg,
                          torch.from_numpy(np.ascontiguousarray(u, dtype=np.float32)).to(cuda),
                          kept_cap=kept_cap, stats=True, path=True)
    torch.cuda.synchronize()
    return dict(tokens=res.tokens.cpu().numpy().view(np.uint32), consumed=res.consumed.cpu().numpy(),
                kept_count=res.kept_count.cpu().numpy().view(np.uint32), stats=res.row_stats.cpu().numpy(),
                path=res.row_path.cpu().numpy().view(np.uint32))


def _check_oracle(x, params, u, g):
    for r in range(x.shape[0]):
        o = O.sample_row(x[r], params, u[r])
        ctx = f"row {r} (path {g['path'][r]:#x})"
        assert g["tokens"][r] == o.token, f"{ctx}: token {g['tokens'][r]} != {o.token}"
        assert g["consumed"][r] == o.consumed, f"{ctx}: consumed"
        assert g["kept_count"][r] == o.kept_count, f"{ctx}: kept {g['kept_count'][r]} != {o.kept_count}"
        st = g["stats"][r]
        assert _bits(st[0]) == _bits(o.max_logit), f"{ctx}: max"
        assert _bits(st[1]) == _bits(o.sum), f"{ctx}: sum"
        assert _bits(st[3]) == _bits(o.total), f"{ctx}: total {st[3]!r} != {o.total!r}"


def test_bucket_path_c4_rows(cuda):
    """Configuration 4 (256000 near-flat logits, top-p 0.9): every row on the bucket path."""
    w = WORKLOADS["c4"]
    rows = 8
    x = w.logits(rows)
    u = llz.rng_uniforms(w.uniform_seed, rows)
    g = _run(cuda, x, w.params, u)
    assert np.all(g["path"] & llz.PATH_BUCKETS), f"rows off the bucket path: {g['path']}"
    _check_oracle(x, w.params, u, g)


def test_bucket_path_agrees_with_sort_path(cuda):
    """The same rows through the sorting path (kept ids requested) give the same results."""
    w = WORKLOADS["c4"]
    rows = 4
    x = w.logits(rows, first_row=100)
    u = llz.rng_uniforms(w.uniform_seed + 1, rows)
    gb = _run(cuda, x, w.params, u)
    gs = _run(cuda, x, w.params, u, kept_cap=8)
    assert np.all(gb["path"] & llz.PATH_BUCKETS)
    assert not np.any(gs["path"] & llz.PATH_BUCKETS)
    for k in ("tokens", "consumed", "kept_count"):
        assert np.array_equal(gb[k], gs[k]), k
    assert np.array_equal(_bits(gb["stats"]), _bits(gs["stats"]))


_NEAR_FLAT = [
    ("top-p 0.5", Params(temperature=1.0, top_k=0, top_p=0.5, min_p=0.0, typical_p=1.0,
                         repetition_window=0, repetition_penalty=1.0)),
    ("top-p 0.99", Params(temperature=1.2, top_k=0, top_p=0.99, min_p=0.0, typical_p=1.0,
                          repetition_window=0, repetition_penalty=1.0)),
    ("top-k 150000, top-p 0.9", Params(temperature=0.9, top_k=150000, top_p=0.9, min_p=0.0, typical_p=1.0,
                                       repetition_window=0, repetition_penalty=1.0)),
    ("top-k 30000 alone", Params(temperature=1.0, top_k=30000, top_p=1.0, min_p=0.0, typical_p=1.0,
                                 repetition_window=0, repetition_penalty=1.0)),
    ("min-p 0.6 alone", Params(temperature=1.0, top_k=0, top_p=1.0, min_p=0.6, typical_p=1.0,
                               repetition_window=0, repetition_penalty=1.0)),
    ("all three", Params(temperature=0.8, top_k=100000, top_p=0.8, min_p=0.2, typical_p=1.0,
                         repetition_window=0, repetition_penalty=1.0)),
]


@pytest.mark.parametrize("name,params", _NEAR_FLAT, ids=[c[0] for c in _NEAR_FLAT])
def test_bucket_path_filters(cuda, name, params):
    rng = np.random.default_rng(1234)
    rows, n = 4, 200000
    x = rng.normal(0.0, 0.3, (rows, n)).astype(np.float32)
    u = llz.rng_uniforms(99, rows)
    g = _run(cuda, x, params, u)
    assert np.any(g["path"] & llz.PATH_BUCKETS), f"no row on the bucket path: {g['path']}"
    _check_oracle(x, params, u, g)


def test_bucket_path_duplicate_keys(cuda):
    """Logits on a coarse grid: long runs of equal p (order by id) and rounding ties.
    Rows whose buckets overflow the sort list take the sorting path; every row
    matches the oracle either way."""
    rng = np.random.default_rng(77)
    rows, n = 4, 160000
    x = (np.round(rng.normal(0.0, 0.4, (rows, n)) * 64.0) / 64.0).astype(np.float32)
    x[1] = (np.round(rng.normal(0.0, 0.4, n) * 4096.0) / 4096.0).astype(np.float32)
    params = dataclasses.replace(WORKLOADS["c4"].params, top_p=0.7)
    u = llz.rng_uniforms(5, rows)
    g = _run(cuda, x, params, u)
    _check_oracle(x, params, u, g)
