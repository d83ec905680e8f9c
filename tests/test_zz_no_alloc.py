"""llz_sample_rows_noalloc (the entry point that allocates nothing: its
kernels' scratch is the library's static device array) against
llz_sample_rows with a caller workspace, through the C ABI, on two calls in a
row, the second with a smaller input.  Bar: bit-exact outputs."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

import llz
from llz.workloads import WORKLOADS, Params

pytestmark = pytest.mark.gpu


def _outputs(torch, rows, cap, dev):
    return dict(tokens=torch.full((rows,), -1, dtype=torch.int32, device=dev),
                consumed=torch.full((rows,), 7, dtype=torch.uint8, device=dev),
                kept_count=torch.full((rows,), -1, dtype=torch.int32, device=dev),
                kept_ids=torch.full((rows, cap), -1, dtype=torch.int32, device=dev),
                kept_probs=torch.full((rows, cap), float("nan"), dtype=torch.float32, device=dev),
                stats=torch.zeros((rows, 4), dtype=torch.float32, device=dev),
                path=torch.full((rows,), -1, dtype=torch.int32, device=dev))


def _extras(o, cap):
    ex = llz.CExtras()
    ex.d_kept_count = o["kept_count"].data_ptr()
    ex.d_kept_ids = o["kept_ids"].data_ptr()
    ex.d_kept_probs = o["kept_probs"].data_ptr()
    ex.kept_cap = cap
    ex.d_row_stats = o["stats"].data_ptr()
    ex.d_row_path = o["path"].data_ptr()
    return ex


def _run_both(torch, cuda, x, params, u, cap):
    L = llz.library()
    rows, vocab = x.shape
    xt = torch.from_numpy(np.ascontiguousarray(x)).to(cuda)
    ut = torch.from_numpy(np.ascontiguousarray(u, dtype=np.float32)).to(cuda)
    cfg = llz.SamplerConfig.of(params).to_c()
    stream = torch.cuda.current_stream().cuda_stream
    a, b = _outputs(torch, rows, cap, cuda), _outputs(torch, rows, cap, cuda)
    ea, eb = _extras(a, cap), _extras(b, cap)
    ws = torch.empty(L.llz_sample_workspace_bytes(rows, vocab, C.byref(cfg), 0), dtype=torch.uint8, device=cuda)
    rc = L.llz_sample_rows(xt.data_ptr(), vocab, rows, vocab, C.byref(cfg), None, None, 0, 0, ut.data_ptr(),
                           a["tokens"].data_ptr(), a["consumed"].data_ptr(), C.byref(ea), ws.data_ptr(),
                           ws.numel(), stream)
    assert rc == llz.LLZ_OK
    rc = L.llz_sample_rows_noalloc(xt.data_ptr(), vocab, rows, vocab, C.byref(cfg), None, None, 0, 0,
                                   ut.data_ptr(), b["tokens"].data_ptr(), b["consumed"].data_ptr(), C.byref(eb),
                                   stream)
    assert rc == llz.LLZ_OK, L.llz_strerror(rc)
    torch.cuda.synchronize()
    for k in a:
        va, vb = a[k].cpu().numpy(), b[k].cpu().numpy()
        assert np.array_equal(va.view(np.uint8), vb.view(np.uint8)), f"{k} differs"
    return a


def test_noalloc_matches_workspace_entry_point(cuda):
    import torch

    # call 1: headline rows at full vocab (the single-pass path)
    w = WORKLOADS["headline"]
    x1 = w.logits(64)
    a = _run_both(torch, cuda, x1, w.params, llz.rng_uniforms(w.uniform_seed, 64), cap=64)
    assert (a["path"].cpu().numpy() & 0xC) .sum() == 0
    # call 2, smaller: near-flat rows whose kept sets outgrow the candidate
    # list, so every row takes the full-row fallback from the scratch's slots
    x2 = np.random.default_rng(8).normal(0, 0.3, (16, 20000)).astype(np.float32)
    p2 = Params(temperature=1.2, top_k=0, top_p=0.9, min_p=0.0, repetition_penalty=1.0)
    b = _run_both(torch, cuda, x2, p2, llz.rng_uniforms(3, 16), cap=64)
    assert np.all(b["path"].cpu().numpy() & 4)


def test_noalloc_rejects_what_does_not_fit(cuda):
    import torch

    L = llz.library()
    rows, vocab = 4096, 256000  # 4096 rows x 32 KB of per-row scratch alone exceed 96 MiB
    cfg = llz.SamplerConfig(temperature=1.0).to_c()
    # full-size buffers (4 GB of logits), so that the call stays in bounds even
    # if it were accepted; it is rejected before any launch
    x = torch.empty((rows, vocab), dtype=torch.float32, device=cuda)
    u = torch.full((rows,), 0.5, dtype=torch.float32, device=cuda)
    tok = torch.zeros(rows, dtype=torch.int32, device=cuda)
    rc = L.llz_sample_rows_noalloc(x.data_ptr(), vocab, rows, vocab, C.byref(cfg), None, None, 0, 0,
                                   u.data_ptr(), tok.data_ptr(), None, None, None)
    assert rc == llz.LLZ_E_SCRATCH
    assert b"static scratch" in L.llz_strerror(rc)
