"""GPU parity of rows whose candidate list floods: more than 2048 terms above
the candidate threshold (2^-16 without min-p), while the kept prefix is short.
The selection collects the row's largest terms again (recollect_top in
llz_select.h) and runs on that list, certified by the bound of the terms it
left out; rows whose kept prefix is not inside it take the full-row
fallback.  Bar: every output against the oracle, bit for bit (exact mode:
kept ids and probabilities, row maximum, normaliser, total; token-only
calls: token, draw flag, kept count and ids).
"""
from __future__ import annotations

import numpy as np
import pytest

import llz
import oracle_lib as O
from llz.workloads import WORKLOADS, Params
from test_gpu_parity import compare_rows

pytestmark = pytest.mark.gpu

PATH_FULL_SORT = 4
PATH_TOKEN_ONLY = 128
PATH_RECOLLECT = 1 << 16

DEFAULT_CHAIN = Params(temperature=0.8, top_k=0, top_p=0.9, min_p=0.0, typical_p=1.0, repetition_window=0,
                       repetition_penalty=1.0)


def _run(cuda, x, params, u, exact, cap=512):
    import torch

    cfg = llz.SamplerConfig.of(params)
    res = llz.sample_rows(torch.from_numpy(np.ascontiguousarray(x)).to(cuda), cfg,
                          torch.from_numpy(np.ascontiguousarray(u, dtype=np.float32)).to(cuda), kept_cap=cap,
                          probs=exact, stats=exact, path=True)
    torch.cuda.synchronize()
    g = dict(tokens=res.tokens.cpu().numpy().view(np.uint32), consumed=res.consumed.cpu().numpy(),
             kept_count=res.kept_count.cpu().numpy().view(np.uint32),
             kept_ids=res.kept_ids.cpu().numpy().view(np.uint32), path=res.row_path.cpu().numpy().view(np.uint32),
             cap=cap)
    if exact:
        g["kept_probs"] = res.kept_probs.cpu().numpy()
        g["stats"] = res.row_stats.cpu().numpy()
    return g


def _check_token_call(x, params, u, g):
    for r in range(x.shape[0]):
        o = O.sample_row(x[r], params, u[r])
        ctx = f"row {r} (path {g['path'][r]:#x})"
        assert (g["tokens"][r], g["consumed"][r], g["kept_count"][r]) == (o.token, o.consumed, o.kept_count), ctx
        k = min(o.kept_count, g["cap"])
        assert np.array_equal(g["kept_ids"][r, :k], o.kept_ids()[:k]), f"{ctx}: kept ids"


@pytest.mark.parametrize("exact", [True, False], ids=["exact", "token-call"])
def test_default_chain_flooded_rows(cuda, exact):
    """The reference's default chain (T 0.8, top-p 0.9, no min-p) on the
    headline's logits: 1000 to 4000 terms above 2^-16 per row, nuclei of 10
    to 300.  Flooded rows finish on a list collected again, none on the
    full-row fallback."""
    w = WORKLOADS["headline"]
    rows = 48
    x = w.logits(rows)
    u = llz.rng_uniforms(w.uniform_seed, rows)
    g = _run(cuda, x, DEFAULT_CHAIN, u, exact)
    rec = (g["path"] & PATH_RECOLLECT) != 0
    assert rec.sum() >= rows // 4, f"{int(rec.sum())} rows collected again"
    assert not np.any(g["path"] & PATH_FULL_SORT), f"full-row rows: {np.flatnonzero(g['path'] & PATH_FULL_SORT)}"
    if exact:
        compare_rows(x, DEFAULT_CHAIN, u, g)
    else:
        _check_token_call(x, DEFAULT_CHAIN, u, g)


def test_top_k_only_flooded_rows(cuda):
    """Top-k 50 alone on rows flattened by T 2.5 (every term above 2^-16):
    the list collected again holds the top 1536 terms, top-k cuts inside it."""
    w = WORKLOADS["headline"]
    rows = 8
    x = w.logits(rows)
    u = llz.rng_uniforms(w.uniform_seed, rows)
    p = Params(temperature=2.5, top_k=50, top_p=1.0, min_p=0.0, typical_p=1.0, repetition_window=0,
               repetition_penalty=1.0)
    g = _run(cuda, x, p, u, exact=True, cap=64)
    assert np.all(g["path"] & PATH_RECOLLECT), f"paths {g['path']}"
    compare_rows(x, p, u, g)


def test_flooded_rows_nucleus_past_the_list(cuda):
    """Near-flat rows with top-p 0.9: the nucleus holds most of the row, so
    the list collected again cannot hold it and the full-row fallback
    decides; and all-equal rows, where no cut separates the top terms."""
    rows, n = 4, 30000
    rng = np.random.default_rng(13)
    x = rng.normal(0.0, 0.3, size=(rows, n)).astype(np.float32)
    x[3] = np.float32(0.25)
    u = llz.rng_uniforms(17, rows)
    g = _run(cuda, x, DEFAULT_CHAIN, u, exact=True, cap=64)
    assert np.all(g["path"] & PATH_FULL_SORT), f"paths {g['path']}"
    compare_rows(x, DEFAULT_CHAIN, u, g)
