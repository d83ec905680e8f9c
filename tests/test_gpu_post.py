"""GPU parity of the decode loop's logit post-processing and the fused
repetition penalty, against the oracle, through the C ABI.

main.zig:653-666 soft-caps the final logits (v = tanh(v / s) * s) and
scales them (v *= 1 / logit_scale) before Sampler.sample; sampler.zig:54-75
then penalises the window's ids.  The kernels apply all three as they read
each logit.  The oracle applies main.zig's loops to a copy and samples it
(llz_oracle_logit_post, llz_oracle_sample_row).  Bar: bit-exact, as in
test_gpu_parity.py.
"""
from __future__ import annotations

import numpy as np
import pytest

import llz
import oracle_lib as O
from llz.workloads import WORKLOADS, Params
from test_gpu_parity import _bits_range, _f32bits, compare_rows, run_gpu

pytestmark = pytest.mark.gpu


# ---------------------------------------------------------------------------
# device expm1 / tanh against the oracle's restatement (musl expm1f / tanhf)
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("name,lo,hi,step", [
    ("tanh-positive", 0x00000000, 0x7f800001, 61),    # +0 .. +inf
    ("tanh-negative", 0x80000000, 0xff800001, 67),    # -0 .. -inf
    ("tanh-branches", 0x3e700000, 0x3f200000, 1),     # 0.23 .. 0.625: both branch edges, dense
    ("tanh-saturation", 0x41000000, 0x41300000, 1),   # 8 .. 11: the |x| > 10 edge, dense
])
def test_device_tanh_matches_oracle(cuda, name, lo, hi, step):
    import torch

    x = _bits_range(lo, hi, step)
    for a in range(0, x.size, 1 << 25):
        xs = x[a:a + (1 << 25)]
        _, _, em1, th = llz.debug_math(torch.from_numpy(xs).to(cuda), extra=True)
        torch.cuda.synchronize()
        gt, ge = th.cpu().numpy(), em1.cpu().numpy()
        bad = np.flatnonzero(_f32bits(gt) != _f32bits(O.tanhf_array(xs)))
        assert bad.size == 0, f"{name}: tanh {bad.size} mismatches, first x={xs[bad[0]]!r}"
        bad = np.flatnonzero(_f32bits(ge) != _f32bits(O.expm1f_array(xs)))
        assert bad.size == 0, f"{name}: expm1 {bad.size} mismatches, first x={xs[bad[0]]!r}"


# ---------------------------------------------------------------------------
# post-processing through the sampling chain
# ---------------------------------------------------------------------------
POSTS = [
    ("softcap30", llz.LogitPost(final_logit_softcapping=30.0, logit_scale=1.0)),
    ("softcap5", llz.LogitPost(final_logit_softcapping=5.0, logit_scale=1.0)),
    ("scale-half", llz.LogitPost(final_logit_softcapping=0.0, logit_scale=0.5)),
    ("scale-odd", llz.LogitPost(final_logit_softcapping=0.0, logit_scale=1.7)),
    ("softcap-and-scale", llz.LogitPost(final_logit_softcapping=20.0, logit_scale=0.3)),
    ("scale-zero-ignored", llz.LogitPost(final_logit_softcapping=-1.0, logit_scale=0.0)),
]


def _oracle_post(x, post):
    return O.logit_post(x, post.final_logit_softcapping, post.logit_scale)


@pytest.mark.parametrize("name,post", POSTS)
@pytest.mark.parametrize("wl,rows", [("headline", 6), ("c1", 1), ("c5", 4)])
def test_post_processing_matches_oracle(cuda, name, post, wl, rows):
    w = WORKLOADS[wl]
    x = w.logits(rows)
    u = llz.rng_uniforms(w.uniform_seed + 101, rows)
    g = run_gpu(x, w.params, u, cuda, kept_cap=256, post=post)
    compare_rows(_oracle_post(x, post), w.params, u, g)


def test_post_processing_unaligned_rows(cuda):
    """The element-load kernel (rows not 16-byte aligned, odd vocab)."""
    import torch

    n, rows, stride = 3001, 3, 3007
    base = np.random.default_rng(15).normal(0, 9, rows * stride + 1).astype(np.float32)
    p = Params(temperature=0.8, top_k=30, top_p=0.9, min_p=0.02, repetition_penalty=1.0)
    post = llz.LogitPost(final_logit_softcapping=10.0, logit_scale=1.3)
    u = llz.rng_uniforms(19, rows)
    full = torch.from_numpy(base).to(cuda)
    view = full[1:1 + rows * stride].view(rows, stride)[:, :n]
    res = llz.sample_rows(view, llz.SamplerConfig.of(p), torch.from_numpy(u).to(cuda), post=post,
                          kept_cap=64, stats=True)
    torch.cuda.synchronize()
    x = base[1:1 + rows * stride].reshape(rows, stride)[:, :n].copy()
    g = dict(tokens=res.tokens.cpu().numpy().view(np.uint32), consumed=res.consumed.cpu().numpy(),
             kept_count=res.kept_count.cpu().numpy().view(np.uint32),
             kept_ids=res.kept_ids.cpu().numpy().view(np.uint32),
             kept_probs=res.kept_probs.cpu().numpy(), stats=res.row_stats.cpu().numpy(), cap=64)
    compare_rows(_oracle_post(x, post), p, u, g)


def test_greedy_with_post_processing(cuda):
    """sampleArgmax of the post-processed logits, through llz_argmax_rows and
    through the T <= 0 exit of llz_sample_rows (main.zig:663-667 then
    sampler.zig:50): values that tie after the scale keep the first index."""
    import torch

    post = llz.LogitPost(final_logit_softcapping=0.0, logit_scale=0.3)
    inv = np.float32(1.0) / np.float32(0.3)
    x = np.random.default_rng(4).normal(0, 2, (4, 1000)).astype(np.float32)
    # two different logits whose scaled values are equal: a tie only after the scale
    a = np.float32(50.0)
    b = np.nextafter(a, np.float32(0))
    assert a != b and a * inv == b * inv
    x[0, 700], x[0, 300] = a, b          # the smaller logit comes first: it wins after scaling
    x[1, 5] = x[1, 600] = 80.0
    x[2, :] = np.float32(-3.0)
    cap = llz.LogitPost(final_logit_softcapping=2.0, logit_scale=1.0)
    x[3, 10], x[3, 20] = 40.0, 41.0      # both saturate to 2.0 under the soft-cap: index 10 wins
    for pp in (post, cap):
        want = [int(O.lib().llz_oracle_argmax(O._fptr(np.ascontiguousarray(r)), r.size))
                for r in _oracle_post(x, pp)]
        t = llz.argmax_rows(torch.from_numpy(x).to(cuda), post=pp).cpu().numpy().tolist()
        assert t == want, (pp, t, want)
        g = run_gpu(x, Params(temperature=0.0, repetition_penalty=1.0), np.zeros(4, np.float32), cuda,
                    post=pp)
        assert g["tokens"].tolist() == want
        assert not g["consumed"].any()
        if pp is post:
            assert want[0] == 300   # without the scale, 700 (the larger logit) would win
        else:
            assert want[3] == 10


# ---------------------------------------------------------------------------
# the repetition penalty applied as the rows are read
# ---------------------------------------------------------------------------
def _histories(rows, n, n_prev, seed):
    g = np.random.default_rng(seed)
    prev = g.integers(0, n, (rows, n_prev)).astype(np.uint32)
    prev[:, 1] = prev[:, 0]              # a repeated id is penalised once
    prev[:, 2] = n + 5                   # ids >= n never match (sampler.zig:64)
    return prev


@pytest.mark.parametrize("window,n_prev,rp", [
    (32, 40, 1.3),            # fused: last 32 of 40
    (0xFFFFFFFF, 40, 1.3),    # u32 window beyond the history: the whole history (sampler.zig:60)
    (64, 64, 0.7),            # fused at its limit; a penalty below 1 boosts
    (0xFFFFFFFF, 200, 1.25),  # 200 > 64 ids: the penalised copy
])
def test_penalty_at_full_vocab(cuda, window, n_prev, rp):
    w = WORKLOADS["headline"]
    rows = 6
    x = w.logits(rows)
    prev = _histories(rows, w.vocab, n_prev, seed=n_prev)
    # put the row maximum and some candidates in the window, so the penalty
    # moves the maximum and the kept set
    for r in range(rows):
        top = np.argsort(-x[r])[:4]
        prev[r, -4:] = top
    p = Params(temperature=1.0, top_k=40, top_p=0.95, min_p=0.05, repetition_window=window,
               repetition_penalty=rp)
    u = llz.rng_uniforms(77, rows)
    g = run_gpu(x, p, u, cuda, prev=prev, kept_cap=256)
    compare_rows(x, p, u, g, prev=prev)


def test_penalty_with_post_processing(cuda):
    w = WORKLOADS["c5"]
    rows = 4
    x = w.logits(rows)
    prev = _histories(rows, w.vocab, 48, seed=3)
    for r in range(rows):
        prev[r, -3:] = np.argsort(-x[r])[:3]
    post = llz.LogitPost(final_logit_softcapping=15.0, logit_scale=0.8)
    for window in (16, 48):
        p = dataclasses_replace(w.params, repetition_window=window, repetition_penalty=1.4)
        u = llz.rng_uniforms(window, rows)
        g = run_gpu(x, p, u, cuda, prev=prev, kept_cap=256, post=post)
        compare_rows(_oracle_post(x, post), p, u, g, prev=prev)


def dataclasses_replace(params, **kw):
    import dataclasses

    return dataclasses.replace(params, **kw)


def test_sampler_object_ignores_post(cuda):
    """llz_sampler_sample takes logits already post-processed on the host
    (main.zig applies 653-666 itself): the caller-uniform entry point returns
    the oracle's token and consumed flag for the same uniform."""
    w = WORKLOADS["c1"]
    x = w.logits(1)[0]
    s = llz.Sampler(llz.SamplerConfig.of(w.params))
    for i, u in enumerate(llz.rng_uniforms(5, 6)):
        tok, con = s.sample_uniform(x, float(u))
        o = O.sample_row(x, w.params, u)
        assert (tok, con) == (o.token, bool(o.consumed)), i
    s.close()


def test_shared_handle_takes_each_calls_config(cuda):
    """llz_sampler_sample_config: one handle serves samplers of different
    configurations (the Zig drop-in shares one per process), each call with
    its own configuration and uniform, against the oracle."""
    w = WORKLOADS["c1"]
    x = w.logits(2)
    s = llz.Sampler(llz.SamplerConfig.of(w.params))
    chains = [w.params, dataclasses_replace(w.params, temperature=1.3, top_k=5, top_p=1.0),
              dataclasses_replace(w.params, min_p=0.2), dataclasses_replace(w.params, temperature=0.0)]
    for i, u in enumerate(llz.rng_uniforms(11, 8)):
        p = chains[i % len(chains)]
        row = x[i % 2]
        tok, con = s.sample_config(llz.SamplerConfig.of(p), row, float(u))
        o = O.sample_row(row, p, u)
        assert (tok, con) == (o.token, bool(o.consumed)), (i, p)
    s.close()
