"""GPU parity of the single pass's transform modes: the logit scale and the
repetition penalty applied exactly as the row is read (kXmLight), and
soft-capping, whose single pass estimates the capped logits from a closed
form and takes the exact values where they decide something (kXmCap).

* tanh_f32 on every non-negative float: bit-equal to the oracle's tanhf
  (musl tanhf, the function behind Zig's std.math.tanh) and within
  3 * 2^-24 of tanh (the soft-cap estimates' error bound takes that figure).
  It is not monotone (it steps down by an ulp at places), so nothing in the
  kernels takes f(max) for max(f): the soft-cap mode finds the maximum from
  its estimates and evaluates the largest elements exactly.
* Token-only calls (the benchmark's call: no probabilities, no statistics)
  under every mode, with the row maximum inside the penalty window (the
  penalised maximum makes the kernel take the maximum again from the
  estimates), against the oracle: token, draw flag, kept count and ids.
* Exact calls (kept probabilities and row statistics) under the same modes.
* Rows the single pass leaves to the exact streaming path (a soft-cap whose
  estimates would be too coarse at a low temperature, a negative logit
  scale), NaN and infinite logits, saturated soft-caps (many equal maxima).
* The benchmark's transformed batches (256 x 128256: soft-cap 30 with logit
  scale 0.5; the repetition penalty 1.1 over a 32-token window), every row.

The oracle post-processes a copy (llz_oracle_logit_post, main.zig:653-666)
and penalises inside its sampler (sampler.zig:54-75).  Bar: bit-exact.
"""
from __future__ import annotations

import dataclasses
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest

import llz
import oracle_lib as O
from llz.workloads import WORKLOADS, Params
from test_gpu_parity import _f32bits, compare_rows, run_gpu

pytestmark = pytest.mark.gpu

HOST_THREADS = 16
PATH_TOKEN_ONLY = 128


@pytest.fixture(autouse=True)
def _one_workgroup_per_row():
    """These tests exercise k_stats's transform modes, so calls of few rows
    run one workgroup per row here (split rows, which apply the same
    transforms in their chunk pass, are tested in test_gpu_split.py)."""
    llz.debug_set_split(1)
    yield
    llz.debug_set_split(0)


def _oracle_post(x, post):
    if post is None:
        return x
    return O.logit_post(x, post.final_logit_softcapping, post.logit_scale)


def _token_call(cuda, x, params, u, post=None, prev=None, cap=64):
    import torch

    cfg = llz.SamplerConfig.of(params)
    pt = None
    if prev is not None:
        pt = torch.from_numpy(np.ascontiguousarray(prev, dtype=np.int32)).to(cuda)
    res = llz.sample_rows(torch.from_numpy(np.ascontiguousarray(x)).to(cuda), cfg,
                          torch.from_numpy(np.ascontiguousarray(u, dtype=np.float32)).to(cuda), pt, post=post,
                          kept_cap=cap, probs=False, stats=False, path=True)
    torch.cuda.synchronize()
    return dict(tokens=res.tokens.cpu().numpy().view(np.uint32), consumed=res.consumed.cpu().numpy(),
                kept_count=res.kept_count.cpu().numpy().view(np.uint32),
                kept_ids=res.kept_ids.cpu().numpy().view(np.uint32), path=res.row_path.cpu().numpy().view(np.uint32),
                cap=cap)


def _check_token_rows(x, params, u, g, post=None, prev=None):
    xo = _oracle_post(x, post)
    for r in range(x.shape[0]):
        o = O.sample_row(xo[r], params, u[r], prev_tokens=None if prev is None else prev[r])
        ctx = f"row {r} (path {g['path'][r]:#x})"
        assert (g["tokens"][r], g["consumed"][r], g["kept_count"][r]) == (o.token, o.consumed, o.kept_count), ctx
        k = min(o.kept_count, g["cap"])
        assert np.array_equal(g["kept_ids"][r, :k], o.kept_ids()[:k]), f"{ctx}: kept ids"


def _histories(x, n_prev, seed, top=4):
    """History rows of n_prev random ids whose last `top` are the row's
    largest logits (the penalty then moves the maximum and the kept set)."""
    rows, n = x.shape
    prev = np.random.default_rng(seed).integers(0, n, (rows, n_prev)).astype(np.uint32)
    for r in range(rows):
        if top:
            prev[r, -top:] = np.argsort(-x[r], kind="stable")[:top]
    return prev


# ---------------------------------------------------------------------------
# tanh_f32 on every non-negative float
# ---------------------------------------------------------------------------
def test_tanh_every_float_exact_and_accurate(cuda):
    import torch

    chunk = 1 << 26
    top = 0x7f800000  # +inf (NaNs above it propagate)
    worst = 0.0
    steps_down = 0
    pool = ThreadPoolExecutor(HOST_THREADS)
    try:
        for lo in range(0, top + 1, chunk):
            hi = min(lo + chunk, top + 1)
            xb = torch.arange(lo, hi, dtype=torch.int32, device=cuda)
            x = xb.view(torch.float32)
            _, _, _, th = llz.debug_math(x, extra=True)
            steps_down += int((th[1:] < th[:-1]).sum())  # recorded, not required
            # within 3 * 2^-24 of tanh (float64 on the device as the reference)
            err = (th.double() - torch.tanh(x.double())).abs().max().item()
            worst = max(worst, err)
            assert err <= 3.0 * 2.0 ** -24, f"tanh error {err / 2.0 ** -24:.3f} * 2^-24 in [{lo:#x}, {hi:#x})"
            # bit for bit the oracle's tanhf (the reference's restated)
            xs = xb.cpu().numpy().view(np.float32)
            gs = th.cpu().numpy()
            del xb, x, th
            step = chunk // HOST_THREADS

            def bad_in(a):
                want = O.tanhf_array(xs[a:a + step])
                return int(np.count_nonzero(_f32bits(want) != _f32bits(gs[a:a + step])))

            nbad = sum(pool.map(bad_in, range(0, xs.size, step)))
            assert nbad == 0, f"{nbad} tanh mismatches with the oracle in [{lo:#x}, {hi:#x})"
    finally:
        pool.shutdown()
    print(f"tanh_f32: max error {worst / 2.0 ** -24:.3f} * 2^-24; {steps_down} steps down between "
          f"adjacent non-negative floats", flush=True)


# ---------------------------------------------------------------------------
# token-only calls under every mode
# ---------------------------------------------------------------------------
POST_CAP = llz.LogitPost(final_logit_softcapping=30.0, logit_scale=0.5)
MODES = [
    # name, post, penalty window (0: none), penalty
    ("scale", llz.LogitPost(final_logit_softcapping=0.0, logit_scale=0.5), 0, 1.0),
    ("penalty", None, 32, 1.1),
    ("penalty-boost", None, 32, 0.7),
    ("scale-penalty", llz.LogitPost(final_logit_softcapping=0.0, logit_scale=1.7), 32, 1.3),
    ("softcap-scale", POST_CAP, 0, 1.0),
    ("softcap5", llz.LogitPost(final_logit_softcapping=5.0, logit_scale=1.0), 0, 1.0),
    ("softcap-penalty", POST_CAP, 32, 1.1),
    ("softcap-penalty-boost", llz.LogitPost(final_logit_softcapping=20.0, logit_scale=1.0), 48, 0.8),
]


@pytest.mark.parametrize("name,post,window,rp", MODES, ids=[m[0] for m in MODES])
@pytest.mark.parametrize("chain", ["headline", "headline-default"])
def test_token_calls_under_each_mode(cuda, name, post, window, rp, chain):
    w = WORKLOADS[chain]
    rows = 16
    x = w.logits(rows)
    u = llz.rng_uniforms(w.uniform_seed + 3, rows)
    p = w.params
    prev = None
    if window:
        p = dataclasses.replace(p, repetition_window=window, repetition_penalty=rp)
        # half the rows with their maximum in the window, half without
        prev = _histories(x, window + 8, seed=window, top=4)
        prev[rows // 2:] = _histories(x[rows // 2:], window + 8, seed=window + 1, top=0)
    g = _token_call(cuda, x, p, u, post=post, prev=prev)
    _check_token_rows(x, p, u, g, post=post, prev=prev)
    if chain == "headline":
        # the token path decides the rows (the mode's single pass did not fall back)
        assert np.mean((g["path"] & PATH_TOKEN_ONLY) != 0) >= 0.5, f"paths {g['path']}"


@pytest.mark.parametrize("name,post,window,rp", MODES, ids=[m[0] for m in MODES])
def test_exact_calls_under_each_mode(cuda, name, post, window, rp):
    w = WORKLOADS["headline"]
    rows = 8
    x = w.logits(rows)
    u = llz.rng_uniforms(w.uniform_seed + 5, rows)
    p = w.params
    prev = None
    if window:
        p = dataclasses.replace(p, repetition_window=window, repetition_penalty=rp)
        prev = _histories(x, window, seed=window + 7, top=3)
    g = run_gpu(x, p, u, cuda, prev=prev, kept_cap=256, post=post)
    compare_rows(_oracle_post(x, post), p, u, g, prev=prev)


# ---------------------------------------------------------------------------
# the exact streaming path, special values, saturation
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("post,temperature,single_pass", [
    (POST_CAP, 0.1, False),                                                    # estimates too coarse at T 0.1
    (llz.LogitPost(final_logit_softcapping=30.0, logit_scale=-0.5), 1.0, True),  # a decreasing transform
])
@pytest.mark.parametrize("exact", [False, True], ids=["token-call", "exact"])
def test_soft_cap_coarse_and_decreasing(cuda, post, temperature, single_pass, exact):
    """A soft-cap whose estimates are too coarse at a low temperature (the
    exact streaming path), and a negative logit scale (a decreasing
    transform: the estimates still locate the maximum)."""
    w = WORKLOADS["headline"]
    rows = 4
    x = w.logits(rows)
    u = llz.rng_uniforms(23, rows)
    p = dataclasses.replace(w.params, temperature=temperature)
    if exact:
        g = run_gpu(x, p, u, cuda, kept_cap=256, post=post)
        compare_rows(_oracle_post(x, post), p, u, g)
    else:
        g = _token_call(cuda, x, p, u, post=post)
        _check_token_rows(x, p, u, g, post=post)
        streamed = (g["path"] & llz.PATH_STREAM_NORM) != 0
        assert (not streamed.any()) if single_pass else streamed.all(), f"paths {g['path']}"


@pytest.mark.parametrize("exact", [False, True], ids=["token-call", "exact"])
def test_soft_cap_special_values(cuda, exact):
    """Rows with +inf, -inf and NaN logits, and rows whose largest logits all
    saturate the soft-cap (tanh = 1 beyond 10 caps: many equal maxima)."""
    w = WORKLOADS["headline"]
    rows = 6
    x = w.logits(rows)
    x[0, 17] = np.inf
    x[1, 5] = -np.inf
    x[1, 99] = np.inf
    x[2, 1234] = np.nan
    x[3, ::997] = 400.0            # 129 positions beyond 10 caps: one value after the cap
    x[4, 3:60] = 25.0 + np.arange(57, dtype=np.float32) * 1e-3   # near-equal after the cap
    x[5, :] = np.float32(-7.0)     # a flat row
    post = llz.LogitPost(final_logit_softcapping=30.0, logit_scale=1.0)
    u = llz.rng_uniforms(29, rows)
    p = w.params
    prev = _histories(x, 32, seed=31, top=2)
    p2 = dataclasses.replace(p, repetition_window=32, repetition_penalty=1.2)
    for params, pv in ((p, None), (p2, prev)):
        if exact:
            g = run_gpu(x, params, u, cuda, prev=pv, kept_cap=256, post=post)
            compare_rows(_oracle_post(x, post), params, u, g, prev=pv)
        else:
            g = _token_call(cuda, x, params, u, post=post, prev=pv)
            _check_token_rows(x, params, u, g, post=post, prev=pv)


# ---------------------------------------------------------------------------
# the benchmark's transformed batches, every row
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("line", ["post", "penalty"])
def test_benchmark_transformed_batches_every_row(cuda, line):
    w = WORKLOADS["headline"]
    x = w.logits(w.rows)
    u = llz.rng_uniforms(w.uniform_seed, w.rows)
    p, post, prev = w.params, None, None
    if line == "post":
        post = POST_CAP
    else:
        p = dataclasses.replace(p, repetition_window=32, repetition_penalty=1.1)
        prev = np.random.default_rng(41).integers(0, w.vocab, size=(w.rows, 32)).astype(np.uint32)
    g = _token_call(cuda, x, p, u, post=post, prev=prev)
    ot, oc, ok = O.sample_rows(_oracle_post(x, post), p, u, prev_tokens=prev, threads=HOST_THREADS)
    for what, a, b in (("token", g["tokens"], ot), ("draw flag", g["consumed"], oc), ("kept count", g["kept_count"], ok)):
        bad = np.flatnonzero(np.asarray(a) != np.asarray(b))
        assert bad.size == 0, f"{line}: {bad.size} rows differ in {what}; first {bad[0]} (path {g['path'][bad[0]]:#x})"
    assert np.mean((g["path"] & PATH_TOKEN_ONLY) != 0) >= 0.8, f"token path on {np.mean((g['path'] & PATH_TOKEN_ONLY) != 0):.2f}"
