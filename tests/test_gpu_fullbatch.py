"""GPU parity over whole configuration batches, every row against the oracle
(sampler.zig restated in C, on the host's threads).

* Configurations 3 (256 x 151936, typical-p), 4 (1024 x 256000, near-flat
  top-p) and 5 (4096 x 128256, the full chain) with row statistics asked
  for (the exact phases on every row): token, draw flag and kept count, and
  the row maximum, the sequential normaliser, the entropy (typical-p rows
  that keep something) and the kept total, bit for bit.
* Configuration 2's 64 rows in a token-only call (the benchmark's call):
  token, draw flag, kept count and kept ids, every row on the token path.
* Configuration 5's 4,096 rows in a token-only call (the benchmark's call,
  typical-p decided on the token path): token, draw flag and kept count of
  every row, kept ids of every eighth.

Parity over the batch is the bar, whatever path each row takes.
"""
from __future__ import annotations

import numpy as np
import pytest

import llz
import oracle_lib as O
from llz.workloads import WORKLOADS

pytestmark = pytest.mark.gpu

HOST_THREADS = 16
PATH_TOKEN_ONLY = 128


def _bits(a) -> np.ndarray:
    return np.asarray(a, dtype=np.float32).view(np.uint32)


@pytest.mark.parametrize("name", ["c3", "c4", "c5"])
def test_full_batch_every_row_matches_oracle(cuda, name):
    import torch

    w = WORKLOADS[name]
    x = w.logits(w.rows)
    u = llz.rng_uniforms(w.uniform_seed, w.rows)
    cfg = llz.SamplerConfig.of(w.params)
    print(f"{name}: {w.rows} x {w.vocab}", flush=True)
    res = llz.sample_rows(torch.from_numpy(x).to(cuda), cfg, torch.from_numpy(u).to(cuda), stats=True, path=True)
    torch.cuda.synchronize()
    tok = res.tokens.cpu().numpy().view(np.uint32)
    con = res.consumed.cpu().numpy()
    kept = res.kept_count.cpu().numpy().view(np.uint32)
    st = res.row_stats.cpu().numpy()
    path = res.row_path.cpu().numpy().view(np.uint32)
    del res
    torch.cuda.empty_cache()
    ot, oc, ok, ost = O.sample_rows_stats(x, w.params, u, threads=HOST_THREADS)

    def first_bad(mask, what):
        bad = np.flatnonzero(mask)
        assert bad.size == 0, (f"{name}: {bad.size} rows differ in {what}; first row {bad[0]} "
                               f"(path {path[bad[0]]:#x})")

    first_bad(tok != ot, "token")
    first_bad(con != oc, "draw flag")
    first_bad(kept != ok, "kept count")
    first_bad(_bits(st[:, 0]) != _bits(ost[:, 0]), "row maximum")
    first_bad(_bits(st[:, 1]) != _bits(ost[:, 1]), "normaliser")
    first_bad(_bits(st[:, 3]) != _bits(ost[:, 3]), "kept total")
    if 0.0 < w.params.typical_p < 1.0:
        # the entropy wherever a row computed it (typical-p rows that keep something)
        has = (ok >= 1) & (st[:, 2] != 0.0)
        assert has.any()
        first_bad(has & (_bits(st[:, 2]) != _bits(ost[:, 2])), "entropy")


def test_c2_full_batch_token_only(cuda):
    import torch

    w = WORKLOADS["c2"]
    x = w.logits(w.rows)
    u = llz.rng_uniforms(w.uniform_seed, w.rows)
    cfg = llz.SamplerConfig.of(w.params)
    cap = 64
    res = llz.sample_rows(torch.from_numpy(x).to(cuda), cfg, torch.from_numpy(u).to(cuda), kept_cap=cap,
                          probs=False, path=True)
    torch.cuda.synchronize()
    tok = res.tokens.cpu().numpy().view(np.uint32)
    con = res.consumed.cpu().numpy()
    kept = res.kept_count.cpu().numpy().view(np.uint32)
    ids = res.kept_ids.cpu().numpy().view(np.uint32)
    path = res.row_path.cpu().numpy().view(np.uint32)
    assert np.all(path & PATH_TOKEN_ONLY), f"rows off the token path: {np.flatnonzero((path & PATH_TOKEN_ONLY) == 0)}"
    for r in range(w.rows):
        o = O.sample_row(x[r], w.params, u[r])
        assert (tok[r], con[r], kept[r]) == (o.token, o.consumed, o.kept_count), f"row {r}"
        k = min(o.kept_count, cap)
        assert np.array_equal(ids[r, :k], o.kept_ids()[:k]), f"row {r}: kept ids"


def test_c5_full_batch_token_only(cuda):
    import torch

    w = WORKLOADS["c5"]
    x = w.logits(w.rows)
    u = llz.rng_uniforms(w.uniform_seed, w.rows)
    cfg = llz.SamplerConfig.of(w.params)
    cap = 64
    print(f"c5 token-only: {w.rows} x {w.vocab}", flush=True)
    res = llz.sample_rows(torch.from_numpy(x).to(cuda), cfg, torch.from_numpy(u).to(cuda), kept_cap=cap,
                          probs=False, path=True)
    torch.cuda.synchronize()
    tok = res.tokens.cpu().numpy().view(np.uint32)
    con = res.consumed.cpu().numpy()
    kept = res.kept_count.cpu().numpy().view(np.uint32)
    ids = res.kept_ids.cpu().numpy().view(np.uint32)
    path = res.row_path.cpu().numpy().view(np.uint32)
    del res
    torch.cuda.empty_cache()
    ot, oc, ok = O.sample_rows(x, w.params, u, threads=HOST_THREADS)
    for what, a, b in (("token", tok, ot), ("draw flag", con, oc), ("kept count", kept, ok)):
        bad = np.flatnonzero(a != b)
        assert bad.size == 0, f"c5: {bad.size} rows differ in {what}; first row {bad[0]} (path {path[bad[0]]:#x})"
    for r in range(0, w.rows, 8):
        o = O.sample_row(x[r], w.params, u[r])
        k = min(o.kept_count, cap)
        assert np.array_equal(ids[r, :k], o.kept_ids()[:k]), f"row {r} (path {path[r]:#x}): kept ids"
    # the rows off the token path: N(0, 2) rows with more than 512 terms above
    # min-p's threshold (about one in nine rows)
    on_tok = (path & PATH_TOKEN_ONLY) != 0
    assert on_tok.mean() >= 0.85, f"{int((~on_tok).sum())} rows off the token path"
