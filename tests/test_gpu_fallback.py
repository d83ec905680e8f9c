"""GPU tests of the full-row fallback's bounded buffer pool and of the
largest configurations at their full batch.

Rows whose kept set outgrows the candidate list take the full-row fallback
(a stable radix sort of the row in the workspace).  A call holds at most
min(rows, 256) such buffer sets; rows beyond wait for one.  The first test
makes every row of a 320-row batch take the fallback and compares all of
them with the oracle.  The others run configurations 4 and 5 at their full
batch (1024 x 256000 and 4096 x 128256): determinism, the per-row outputs'
invariants, and oracle parity on rows spread over the batch.
"""
from __future__ import annotations

import numpy as np
import pytest

import llz
import oracle_lib as O
from llz.workloads import WORKLOADS, Params
from test_gpu_parity import compare_rows, run_gpu

pytestmark = pytest.mark.gpu


def test_fallback_pool_contention(cuda):
    rows, n = 320, 20000
    x = np.random.default_rng(21).normal(0, 0.3, (rows, n)).astype(np.float32)
    p = Params(temperature=1.2, top_k=0, top_p=0.9, min_p=0.0, repetition_penalty=1.0)
    u = llz.rng_uniforms(31, rows)
    g = run_gpu(x, p, u, cuda, kept_cap=64)
    compare_rows(x, p, u, g)


def test_lean_fallback_pool_contention(cuda):
    """With min-p >= 2^-10 a call holds 8 full-row buffer sets: here 96
    near-flat rows all need one (every term passes min-p 0.05, far more than
    the candidate list holds), so rows wait for sets in turn.  Every row
    against the oracle."""
    rows, n = 96, 20000
    x = np.random.default_rng(23).normal(0, 0.3, (rows, n)).astype(np.float32)
    p = Params(temperature=1.0, top_k=0, top_p=0.95, min_p=0.05, repetition_penalty=1.0)
    u = llz.rng_uniforms(37, rows)
    g = run_gpu(x, p, u, cuda, kept_cap=64)
    compare_rows(x, p, u, g)


@pytest.mark.parametrize("name,check_rows", [("c4", (0, 137, 511, 1023)), ("c5", (0, 1, 1001, 2048, 4095))])
def test_full_batch(cuda, name, check_rows):
    import torch

    w = WORKLOADS[name]
    x = w.logits(w.rows)
    u = llz.rng_uniforms(w.uniform_seed, w.rows)
    cfg = llz.SamplerConfig.of(w.params)
    xt = torch.from_numpy(x).to(cuda)
    ut = torch.from_numpy(u).to(cuda)
    ws = torch.empty(llz.workspace_bytes(w.rows, w.vocab, cfg), dtype=torch.uint8, device=cuda)
    a = llz.sample_rows(xt, cfg, ut, stats=True, path=True, workspace=ws)
    b = llz.sample_rows(xt, cfg, ut, stats=True, path=True, workspace=ws)
    torch.cuda.synchronize()
    ta, tb = a.tokens.cpu().numpy().view(np.uint32), b.tokens.cpu().numpy().view(np.uint32)
    assert np.array_equal(ta, tb), "not deterministic"
    assert np.array_equal(a.consumed.cpu().numpy(), b.consumed.cpu().numpy())
    paths = a.row_path.cpu().numpy().view(np.uint32)
    assert not np.any(paths & 0x80000000), "a row reported an error"
    assert np.all(ta < w.vocab)
    kc = a.kept_count.cpu().numpy()
    con = a.consumed.cpu().numpy()
    assert np.all((kc > 0) == (con == 1))  # a row draws exactly when its kept set is non-empty
    for r in check_rows:
        o = O.sample_row(x[r], w.params, u[r])
        assert ta[r] == o.token and con[r] == o.consumed and kc[r] == o.kept_count, r
        st = a.row_stats.cpu().numpy()[r]
        assert np.float32(st[1]).view(np.uint32) == np.float32(o.sum).view(np.uint32), r
