"""GPU parity: the HIP sampling chain against the CPU oracle, through the C ABI.

Bar (bit-exact): sampled token ids, draw-consumed flags, the kept set and its
order, the kept probabilities, the row maximum, the sequential normaliser,
the entropy and the kept total.  Rows run at the configurations' full vocab
sizes; row counts are cut to what the oracle finishes in seconds.
"""
from __future__ import annotations

import numpy as np
import pytest

import llz
import oracle_lib as O
from llz.workloads import WORKLOADS, Params

pytestmark = pytest.mark.gpu


def _f32bits(a) -> np.ndarray:
    return np.asarray(a, dtype=np.float32).view(np.uint32)


def run_gpu(x: np.ndarray, params, u: np.ndarray, cuda, prev=None, kept_cap: int = 0, post=None):
    import torch

    cfg = llz.SamplerConfig.of(params)
    xt = torch.from_numpy(np.ascontiguousarray(x)).to(cuda)
    ut = torch.from_numpy(np.ascontiguousarray(u, dtype=np.float32)).to(cuda)
    pt = None
    if prev is not None:
        pt = torch.from_numpy(np.ascontiguousarray(prev, dtype=np.int32)).to(cuda)
    cap = kept_cap or 64
    res = llz.sample_rows(xt, cfg, ut, pt, post=post, kept_cap=cap, stats=True)
    torch.cuda.synchronize()
    return dict(
        tokens=res.tokens.cpu().numpy().view(np.uint32),
        consumed=res.consumed.cpu().numpy(),
        kept_count=res.kept_count.cpu().numpy().view(np.uint32),
        kept_ids=res.kept_ids.cpu().numpy().view(np.uint32),
        kept_probs=res.kept_probs.cpu().numpy(),
        stats=res.row_stats.cpu().numpy(),
        cap=cap,
    )


def compare_rows(x, params, u, g, prev=None, rows=None, typical=None):
    rows = range(x.shape[0]) if rows is None else rows
    typical = (0.0 < params.typical_p < 1.0) if typical is None else typical
    for r in rows:
        o = O.sample_row(x[r], params, u[r], prev_tokens=None if prev is None else prev[r])
        ctx = f"row {r}"
        assert g["tokens"][r] == o.token, f"{ctx}: token {g['tokens'][r]} != {o.token}"
        assert g["consumed"][r] == o.consumed, f"{ctx}: consumed"
        assert g["kept_count"][r] == o.kept_count, f"{ctx}: kept {g['kept_count'][r]} != {o.kept_count}"
        if o.exit_path == O.EXIT_GREEDY:
            assert g["kept_count"][r] == 0
            continue
        st = g["stats"][r]
        assert _f32bits(st[0]) == _f32bits(o.max_logit), f"{ctx}: max"
        assert _f32bits(st[1]) == _f32bits(o.sum), f"{ctx}: sum {st[1]!r} != {o.sum!r}"
        if o.exit_path in (O.EXIT_EMPTY, O.EXIT_DRAW, O.EXIT_FALLBACK):
            assert _f32bits(st[3]) == _f32bits(o.total), f"{ctx}: total"
            if typical and o.kept_count >= 1 and st[2] != 0.0:
                assert _f32bits(st[2]) == _f32bits(o.entropy), f"{ctx}: entropy"
        k = min(o.kept_count, g["cap"])
        kept = o.kept_ids()[:k]
        assert np.array_equal(g["kept_ids"][r, :k], kept), f"{ctx}: kept ids differ"
        assert np.array_equal(_f32bits(g["kept_probs"][r, :k]), _f32bits(o.probs[kept])), f"{ctx}: probs"


# ---------------------------------------------------------------------------
# device exp / log against the oracle's restatement
# ---------------------------------------------------------------------------
def _bits_range(lo_bits: int, hi_bits: int, step: int) -> np.ndarray:
    return np.arange(lo_bits, hi_bits, step, dtype=np.uint32).view(np.float32)


@pytest.mark.parametrize("name,lo,hi,step", [
    ("exp-negative", 0x80000000, 0xc2d00000, 1),      # -0 .. -104, every input (the kernels' domain)
    ("exp-positive", 0x00000000, 0x42b20000, 7),      # 0 .. 89
    ("exp-near-zero", 0xb8000000, 0xb9800000, 1),     # -2^-15 .. -2^-12 (branch edges), dense
])
def test_device_exp_matches_oracle(cuda, name, lo, hi, step):
    import torch

    x = _bits_range(lo, hi, step)
    for a in range(0, x.size, 1 << 25):
        xs = x[a:a + (1 << 25)]
        e, _ = llz.debug_math(torch.from_numpy(xs).to(cuda))
        torch.cuda.synchronize()
        ge = e.cpu().numpy()
        oe = O.expf_array(xs)
        bad = np.flatnonzero(_f32bits(ge) != _f32bits(oe))
        assert bad.size == 0, f"{name}: {bad.size} mismatches, first x={xs[bad[0]]!r}"


@pytest.mark.parametrize("name,lo,hi,step", [
    ("log-unit", 0x00000001, 0x3f800001, 5),          # subnormals .. 1.0
    ("log-near-one", 0x3f700000, 0x3f800001, 1),      # dense just below 1
])
def test_device_log_matches_oracle(cuda, name, lo, hi, step):
    import torch

    x = _bits_range(lo, hi, step)
    for a in range(0, x.size, 1 << 25):
        xs = x[a:a + (1 << 25)]
        _, lg = llz.debug_math(torch.from_numpy(xs).to(cuda))
        torch.cuda.synchronize()
        gl = lg.cpu().numpy()
        ol = O.logf_array(xs)
        bad = np.flatnonzero(_f32bits(gl) != _f32bits(ol))
        assert bad.size == 0, f"{name}: {bad.size} mismatches, first x={xs[bad[0]]!r}"


@pytest.mark.parametrize("name,op,lo,hi", [
    ("exp2-negative", 0, 0x80000000, 0xc2fc0000),   # -0 .. -126 (every input with a normal result)
    ("exp2-positive", 0, 0x00000000, 0x42800000),   # 0 .. 64
    ("log2-entropy", 1, 0x08800000, 0x3e800000),    # 2^-110 .. 2^-2
    ("rcp-softcap", 2, 0x3f800000, 0x71800000),     # 1 .. 2^100 (exp2 + 1 in the soft-cap estimate)
])
def test_hardware_exp2_log2_within_one_ulp(cuda, name, op, lo, hi):
    """The certified estimates (the single-pass statistics, the streaming
    normaliser, the entropy pass, the soft-cap estimate) take the hardware
    exp2, log2 and reciprocal to be within 1 ulp of the exact result (relative
    error <= 2^-23); checked on every float of the ranges they evaluate,
    against double precision."""
    err = llz.debug_hw_error(op, lo, hi - lo + 1)
    assert err <= 1.0, f"{name}: {err} units of 2^-23"


def test_hardware_log2_entropy_estimate(cuda):
    """The token path's entropy estimate takes the hardware log2 of every
    estimate q in [2^-100, 2^64] (q < 2^-100 is left out) to be within
    2^-18 max(1, |log2 q|) of log2 q (32 units of 2^-23 relative to
    max(1, |log2 q|)); checked on every float of that range."""
    err = llz.debug_hw_error(3, 0x0D800000, 0x5F800000 - 0x0D800000 + 1)
    assert err <= 32.0, f"log2: {err} units of 2^-23 relative to max(1, |log2 x|)"



# ---------------------------------------------------------------------------
# the five configurations and the headline batch, full vocab
# ---------------------------------------------------------------------------
CASES = [("c1", 1), ("c2", 16), ("c3", 6), ("c4", 3), ("c5", 16), ("headline", 24)]


@pytest.mark.parametrize("name,rows", CASES)
def test_config_rows_match_oracle(cuda, name, rows):
    w = WORKLOADS[name]
    rows = min(rows, w.rows)
    x = w.logits(rows)
    u = llz.rng_uniforms(w.uniform_seed, rows)
    cap = 262144 if name == "c4" else 256
    g = run_gpu(x, w.params, u, cuda, kept_cap=cap)
    compare_rows(x, w.params, u, g)


def test_headline_full_batch_properties(cuda):
    """All 256 headline rows: determinism, kept-set membership, a row sample vs the oracle."""
    w = WORKLOADS["headline"]
    x = w.logits()
    u = llz.rng_uniforms(w.uniform_seed, w.rows)
    g1 = run_gpu(x, w.params, u, cuda, kept_cap=64)
    g2 = run_gpu(x, w.params, u, cuda, kept_cap=64)
    assert np.array_equal(g1["tokens"], g2["tokens"])
    assert np.array_equal(g1["kept_ids"], g2["kept_ids"])
    for r in range(w.rows):
        kc = int(g1["kept_count"][r])
        assert 0 <= kc <= w.params.top_k
        # an empty kept set (p_max > top_p) returns the top token without a draw
        assert g1["consumed"][r] == (1 if kc > 0 else 0)
        if kc:
            assert g1["tokens"][r] in g1["kept_ids"][r, :kc]
        # kept probabilities are non-increasing
        assert np.all(np.diff(g1["kept_probs"][r, :kc]) <= 0)
    compare_rows(x, w.params, u, g1)


def _run_paths(cuda, x, params, u, cap=64):
    import torch

    cfg = llz.SamplerConfig.of(params)
    res = llz.sample_rows(torch.from_numpy(np.ascontiguousarray(x)).to(cuda), cfg,
                          torch.from_numpy(np.ascontiguousarray(u, dtype=np.float32)).to(cuda),
                          kept_cap=cap, stats=True, path=True)
    torch.cuda.synchronize()
    out = dict(tokens=res.tokens.cpu().numpy().view(np.uint32), consumed=res.consumed.cpu().numpy(),
               kept_count=res.kept_count.cpu().numpy().view(np.uint32),
               kept_ids=res.kept_ids.cpu().numpy().view(np.uint32), kept_probs=res.kept_probs.cpu().numpy(),
               stats=res.row_stats.cpu().numpy(), cap=cap)
    return res.row_path.cpu().numpy().view(np.uint32), out


def test_walk_rare_paths_reached(cuda):
    """The single pass's rarer walk paths are exercised and exact:
    - later rounds of EXACT slots: rows whose running sum sits just above 1/2
      (one early term of e = 1/2, then terms far below the grid) for most of
      the row, so that every segment's prediction straddles the binade
      boundary and is EXACT (far more than one round's 48 slots);
    - a crossing beyond a segment's tabulated binades: configuration 5's
      peaked rows, whose dominant token lifts the sum across about 20
      binades inside one segment.
    Those rows are compared with the oracle."""
    n, rows = 128256, 4
    g = np.random.default_rng(41)
    x = g.normal(-20.0, 1.0, (rows, n)).astype(np.float32)
    for r in range(rows):
        x[r, 10 + 97 * r] = np.float32(-0.6931472)  # e = exp(v - max) = 1/2
        x[r, n - 1 - 311 * r] = 0.0                 # the row maximum, late in the row
    params = Params(temperature=1.0, top_k=40, top_p=0.95, min_p=0.0, repetition_penalty=1.0)
    u = llz.rng_uniforms(9, rows)
    paths, out = _run_paths(cuda, x, params, u)
    assert np.all(paths & llz.PATH_WALK_ROUNDS), f"rows without later rounds: {paths}"
    assert not np.any(paths & llz.PATH_STREAM_NORM), f"rows left the single pass: {paths}"
    compare_rows(x, params, u, out)

    w = WORKLOADS["c5"]
    x = w.logits(32)
    u = llz.rng_uniforms(w.uniform_seed, 32)
    paths, out = _run_paths(cuda, x, w.params, u)
    generic = np.flatnonzero(paths & llz.PATH_RESOLVE_GENERIC)
    assert generic.size > 0, f"no row reached resolve_generic: {paths}"
    assert not np.any(paths & llz.PATH_STREAM_NORM), f"rows left the single pass: {paths}"
    compare_rows(x, w.params, u, out, rows=generic[:8])


# ---------------------------------------------------------------------------
# edge cases of the reference's chain
# ---------------------------------------------------------------------------
def _rand_rows(rows, n, seed, scale=2.0):
    return np.random.default_rng(seed).normal(0, scale, (rows, n)).astype(np.float32)


EDGE = [
    ("greedy", Params(temperature=0.0, top_k=0, top_p=0.9, repetition_penalty=1.0)),
    ("greedy-neg", Params(temperature=-1.0, repetition_penalty=1.0)),
    ("defaults-no-rep", Params(repetition_penalty=1.0)),
    ("topk1", Params(temperature=1.0, top_k=1, top_p=1.0, repetition_penalty=1.0)),
    ("topk-only", Params(temperature=0.9, top_k=7, top_p=1.0, repetition_penalty=1.0)),
    ("tiny-top-p", Params(temperature=1.0, top_p=1e-6, repetition_penalty=1.0)),
    ("minp-only", Params(temperature=1.0, top_p=1.0, min_p=0.3, repetition_penalty=1.0)),
    ("minp-above-one", Params(temperature=1.0, top_p=1.0, min_p=1.5, repetition_penalty=1.0)),
    ("typical-only", Params(temperature=0.7, top_p=1.0, typical_p=0.5, repetition_penalty=1.0)),
    ("all-filters", Params(temperature=1.3, top_k=20, top_p=0.8, min_p=0.01, typical_p=0.9,
                           repetition_penalty=1.0)),
    ("no-filters", Params(temperature=1.0, top_p=1.0, repetition_penalty=1.0)),
    # wide kept sets (beyond the candidate list on flat rows): typical-p after
    # a prefix filter in the full-row fallback
    ("typical-wide-top-p", Params(temperature=2.0, top_p=0.99, typical_p=0.9, repetition_penalty=1.0)),
    ("typical-wide-min-p", Params(temperature=2.0, top_p=1.0, min_p=1e-3, typical_p=0.7,
                                  repetition_penalty=1.0)),
]


@pytest.mark.parametrize("n", [1, 2, 3, 257, 2048, 2049, 40000])
@pytest.mark.parametrize("name,params", EDGE, ids=[e[0] for e in EDGE])
def test_edge_configs(cuda, n, name, params):
    rows = 4
    x = _rand_rows(rows, n, seed=n)
    if n >= 3:
        x[1, :] = 0.5          # all-equal row: ties everywhere
        x[2, n // 2] = 9.0     # one dominant token
        x[3, : n // 3] = -np.inf if n > 3 else x[3, : n // 3]
    u = llz.rng_uniforms(11 + n, rows)
    g = run_gpu(x, params, u, cuda, kept_cap=max(n, 1))
    compare_rows(x, params, u, g)


@pytest.mark.parametrize("n", [100004, 129020, 129024, 129028])
def test_long_rows_lds_segments(cuda, n):
    """Rows long enough for LDS-resident segments (more than 45 segments a
    wave), with a partial last segment among them (100004, 129020: it is
    read straight to LDS through the buffer resource, which returns zeros
    past the row), the longest row the single pass holds (129024), and one
    element more (129028: the streaming normaliser)."""
    import torch

    rows = 3
    x = _rand_rows(rows, n, seed=n % 1000)
    x[1, n - 1] = 12.0  # the row maximum in the last (partial) segment
    p = Params(temperature=1.0, top_k=40, top_p=0.95, min_p=0.05, repetition_penalty=1.0)
    u = llz.rng_uniforms(n % 97, rows)
    cfg = llz.SamplerConfig.of(p)
    ws = torch.zeros(llz.workspace_bytes(rows, n, cfg), dtype=torch.uint8, device=cuda)
    res = llz.sample_rows(torch.from_numpy(x).to(cuda), cfg, torch.from_numpy(u).to(cuda), kept_cap=256,
                          stats=True, workspace=ws)
    torch.cuda.synchronize()
    status = ws[: rows * 4].view(torch.int32).cpu().numpy()  # per-row path bits (workspace offset 0)
    fast = (status & 8) == 0
    assert fast.all() if n <= 129024 else not fast.any(), status
    g = dict(tokens=res.tokens.cpu().numpy().view(np.uint32), consumed=res.consumed.cpu().numpy(),
             kept_count=res.kept_count.cpu().numpy().view(np.uint32),
             kept_ids=res.kept_ids.cpu().numpy().view(np.uint32),
             kept_probs=res.kept_probs.cpu().numpy(), stats=res.row_stats.cpu().numpy(), cap=256)
    compare_rows(x, p, u, g)


def test_repetition_penalty(cuda):
    n, rows = 5000, 4
    x = _rand_rows(rows, n, seed=3)
    x[:, 10] = 4.0
    x[:, 11] = -4.0
    prev = np.array([[10, 11, 11, 4999, 7, 10, 123, 6000],   # duplicates, id >= n ignored
                     [1, 2, 3, 4, 5, 6, 7, 8],
                     [10, 10, 10, 10, 10, 10, 10, 10],
                     [0, 4999, 11, 10, 2, 3, 4, 5]], dtype=np.uint32)
    for window in (0, 3, 8, 32):
        p = Params(temperature=0.9, top_k=0, top_p=0.95, min_p=0.0, repetition_window=window,
                   repetition_penalty=1.3)
        u = llz.rng_uniforms(window + 5, rows)
        g = run_gpu(x, p, u, cuda, prev=prev, kept_cap=n)
        compare_rows(x, p, u, g, prev=prev)


def test_strided_and_unaligned_rows(cuda):
    import torch

    n, rows, stride = 3001, 3, 3007
    base = np.random.default_rng(5).normal(0, 2, rows * stride + 1).astype(np.float32)
    p = Params(temperature=0.8, top_k=30, top_p=0.9, min_p=0.02, repetition_penalty=1.0)
    u = llz.rng_uniforms(9, rows)
    cfg = llz.SamplerConfig.of(p)
    full = torch.from_numpy(base).to(cuda)
    view = full[1:1 + rows * stride].view(rows, stride)[:, :n]   # 4-byte aligned only
    res = llz.sample_rows(view, cfg, torch.from_numpy(u).to(cuda), kept_cap=64, stats=True)
    torch.cuda.synchronize()
    x = base[1:1 + rows * stride].reshape(rows, stride)[:, :n].copy()
    g = dict(tokens=res.tokens.cpu().numpy().view(np.uint32), consumed=res.consumed.cpu().numpy(),
             kept_count=res.kept_count.cpu().numpy().view(np.uint32),
             kept_ids=res.kept_ids.cpu().numpy().view(np.uint32),
             kept_probs=res.kept_probs.cpu().numpy(), stats=res.row_stats.cpu().numpy(), cap=64)
    compare_rows(x, p, u, g)


@pytest.mark.parametrize("post", [None, "softcap"])
def test_unaligned_rows_beyond_the_grid(cuda, post):
    """More rows than the grid's workgroups (300 > 256) on rows that are only
    4-byte aligned: the workgroups claim rows (k_stats_rows's element-load
    instantiations), each with its own special-queue overflow block; with
    and without the logit post-processing.  Every row against the oracle."""
    import torch

    n, rows, stride = 3001, 300, 3007
    base = np.random.default_rng(8).normal(0, 2, rows * stride + 1).astype(np.float32)
    p = Params(temperature=0.8, top_k=30, top_p=0.9, min_p=0.02, repetition_penalty=1.0)
    u = llz.rng_uniforms(19, rows)
    cfg = llz.SamplerConfig.of(p)
    lp = llz.LogitPost(final_logit_softcapping=20.0, logit_scale=0.5) if post else None
    full = torch.from_numpy(base).to(cuda)
    view = full[1:1 + rows * stride].view(rows, stride)[:, :n]   # 4-byte aligned only
    res = llz.sample_rows(view, cfg, torch.from_numpy(u).to(cuda), post=lp, kept_cap=64, stats=True)
    torch.cuda.synchronize()
    x = base[1:1 + rows * stride].reshape(rows, stride)[:, :n].copy()
    if post:
        x = O.logit_post(x, softcap=20.0, logit_scale=0.5)
    g = dict(tokens=res.tokens.cpu().numpy().view(np.uint32), consumed=res.consumed.cpu().numpy(),
             kept_count=res.kept_count.cpu().numpy().view(np.uint32),
             kept_ids=res.kept_ids.cpu().numpy().view(np.uint32),
             kept_probs=res.kept_probs.cpu().numpy(), stats=res.row_stats.cpu().numpy(), cap=64)
    compare_rows(x, p, u, g, rows=range(0, rows, 7))


def test_argmax_rows(cuda):
    import torch

    x = _rand_rows(5, 1000, seed=1)
    x[1, 5] = x[1, 700] = 100.0          # tie: first index wins
    x[2, 0] = np.nan                      # NaN at index 0 is never replaced
    x[3, 17] = np.nan                     # NaN elsewhere is ignored
    x[4, :] = -np.inf
    t = llz.argmax_rows(torch.from_numpy(x).to(cuda)).cpu().numpy()
    want = [O.lib().llz_oracle_argmax(O._fptr(np.ascontiguousarray(r)), r.size) for r in x]
    assert t.tolist() == want


# ---------------------------------------------------------------------------
# the Sampler object: the reference's RNG lifecycle across calls
# ---------------------------------------------------------------------------
def test_sampler_lifecycle_matches_oracle(cuda):
    n = 20000
    p = Params(temperature=0.8, top_k=0, top_p=0.9, min_p=0.0, repetition_penalty=1.0)
    gen = np.random.default_rng(12)
    steps = []
    for i in range(24):
        row = gen.normal(0, 2, n).astype(np.float32)
        if i % 3 == 1:
            row[gen.integers(0, n)] += 30.0  # p_max > top_p: empty kept set, no draw
        steps.append(row)
    for seed in (0, 1, 1234):
        s = llz.Sampler(llz.SamplerConfig.of(p, seed=seed))
        o = O.Sampler(p, seed=seed)
        for i, row in enumerate(steps):
            a = s.sample(row)
            b = o.sample(row)
            assert a == b, (seed, i, a, b)
            assert s.state == o.state, (seed, i)
        s.close()


def test_reference_unit_tests_restated(cuda):
    """sampler.zig:171-213 through the GPU Sampler."""
    cfg = llz.SamplerConfig(temperature=1.0, top_k=0, top_p=1.0, min_p=0.0, typical_p=1.0,
                            seed=1234, repetition_window=0, repetition_penalty=1.0)
    logits = np.zeros(4, np.float32)
    s1, s2 = llz.Sampler(cfg), llz.Sampler(cfg)
    seq1 = [s1.sample(logits) for _ in range(8)]
    seq2 = [s2.sample(logits) for _ in range(8)]
    assert seq1 == seq2
    # closed form: four equal probabilities sum to exactly 1, token = ceil(4u) - 1
    prng = llz.Prng(1234)
    for tok in seq1:
        uu = float(prng.float32())
        assert tok == int(np.ceil(np.float32(4.0) * np.float32(uu))) - 1
    cfg2 = llz.SamplerConfig(temperature=1.0, top_k=1, top_p=1.0, min_p=0.0, typical_p=1.0, seed=1,
                             repetition_window=0, repetition_penalty=1.0)
    s = llz.Sampler(cfg2)
    assert [s.sample(np.array([2.0, 1.9, 1.8], np.float32)) for _ in range(16)] == [0] * 16


# ---------------------------------------------------------------------------
# the committed golden vectors (tests/golden/sampler_golden.npz)
# ---------------------------------------------------------------------------
def test_golden_vectors_on_gpu(cuda):
    import os

    g = np.load(os.path.join(os.path.dirname(__file__), "golden", "sampler_golden.npz"), allow_pickle=False)
    for i, name in enumerate(g["name"]):
        n, off = int(g["n"][i]), int(g["offset"][i])
        x = g["logits"][off:off + n].reshape(1, n)
        t, k, tp, mp, typ, win, rp = g["params"][i]
        p = Params(temperature=float(t), top_k=int(k), top_p=float(tp), min_p=float(mp), typical_p=float(typ),
                   repetition_window=int(win), repetition_penalty=float(rp))
        prev = None
        if g["n_prev"][i]:
            po = int(g["prev_offset"][i])
            prev = g["prev_tokens"][po:po + int(g["n_prev"][i])].reshape(1, -1)
        cap = g["kept_ids"].shape[1]
        r = run_gpu(x, p, g["u"][i:i + 1], cuda, prev=prev, kept_cap=cap)
        assert r["tokens"][0] == g["token"][i], name
        assert r["consumed"][0] == g["consumed"][i], name
        if g["exit_path"][i] == O.EXIT_GREEDY:
            continue
        assert r["kept_count"][0] == g["kept_count"][i], name
        kc = min(int(g["kept_count"][i]), cap)
        assert np.array_equal(r["kept_ids"][0, :kc], g["kept_ids"][i, :kc]), name
        assert np.array_equal(_f32bits(r["kept_probs"][0, :kc]), g["kept_probs_bits"][i, :kc]), name
        sb = g["stats_bits"][i]
        assert _f32bits(r["stats"][0, 0]) == sb[0] and _f32bits(r["stats"][0, 1]) == sb[1], name


def test_golden_config1_full_vocab_on_gpu(cuda):
    import os

    g = np.load(os.path.join(os.path.dirname(__file__), "golden", "sampler_golden.npz"), allow_pickle=False)
    w = WORKLOADS["c1"]
    x = w.logits(1)
    r = run_gpu(x, w.params, np.array([g["c1_u"]], np.float32), cuda, kept_cap=64)
    assert (r["tokens"][0], r["consumed"][0], r["kept_count"][0]) == (g["c1_token"], g["c1_consumed"], g["c1_kept"])
    k = g["c1_kept_ids"].size
    assert np.array_equal(r["kept_ids"][0, :k], g["c1_kept_ids"])
    assert _f32bits(r["stats"][0, 1]) == g["c1_stats_bits"][1]


def test_non_finite_rows(cuda):
    """A NaN logit or an infinite maximum makes the reference's normaliser NaN:
    every comparison is then false and sampler.zig returns index 0 after a draw."""
    n, rows = 3000, 6
    x = _rand_rows(rows, n, seed=21)
    x[0, 17] = np.nan
    x[1, :] = -np.inf
    x[2, 5] = np.inf
    x[3, :] = np.nan
    x[4, 2999] = np.nan
    x[5, ::2] = -np.inf  # finite maximum: an ordinary row
    for params in (Params(temperature=0.8, top_k=0, top_p=0.9, repetition_penalty=1.0),
                   Params(temperature=1.0, top_k=7, top_p=0.5, min_p=0.1, typical_p=0.9, repetition_penalty=1.0)):
        u = llz.rng_uniforms(5, rows)
        g = run_gpu(x, params, u, cuda, kept_cap=n)
        for r in range(rows):
            o = O.sample_row(x[r], params, u[r])
            assert g["tokens"][r] == o.token, r
            assert g["consumed"][r] == o.consumed, r
            assert g["kept_count"][r] == o.kept_count, r
            k = min(o.kept_count, g["cap"])
            assert np.array_equal(g["kept_ids"][r, :k], o.kept_ids()[:k]), r


# ---------------------------------------------------------------------------
# the fast path is the one taken (a row it cannot certify is still exact,
# through the streaming normaliser, but several times slower)
# ---------------------------------------------------------------------------
def test_headline_rows_take_fast_path(cuda):
    """Every row of the headline batch is certified by the single-pass
    statistics (path bit 8 clear); a few rows are also checked against the
    oracle."""
    import torch

    w = WORKLOADS["headline"]
    rows = w.rows
    x = w.logits(rows)
    u = llz.rng_uniforms(w.uniform_seed, rows)
    cfg = llz.SamplerConfig.of(w.params)
    ws = torch.zeros(llz.workspace_bytes(rows, w.vocab, cfg), dtype=torch.uint8, device=cuda)
    xt = torch.from_numpy(np.ascontiguousarray(x)).to(cuda)
    ut = torch.from_numpy(np.ascontiguousarray(u, dtype=np.float32)).to(cuda)
    res = llz.sample_rows(xt, cfg, ut, kept_cap=256, stats=True, workspace=ws)
    torch.cuda.synchronize()
    status = ws[: rows * 4].view(torch.int32).cpu().numpy()  # per-row path bits (workspace offset 0)
    slow = np.flatnonzero(status & 8)
    assert slow.size == 0, f"rows not certified by the fast path: {slow.tolist()}"
    tok = res.tokens.cpu().numpy().view(np.uint32)
    for r in range(0, rows, 37):
        assert tok[r] == O.sample_row(x[r], w.params, u[r]).token, r


# ---------------------------------------------------------------------------
# the special queue's chunks past the LDS queue
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("qcap", [8, 32, 64])
def test_special_queue_chunks(cuda, qcap):
    """llz_debug_set_queue_cap shrinks the special-queue chunk, so ordinary rows fill
    several chunks (kept in the workgroup's overflow block of the workspace);
    a batch with more specials than a chunk holds (the row's first segments
    have many large terms) sends its row to the streaming normaliser.
    Results stay bit-exact; at 32 and 64 some rows (each with over 64
    specials per wave, so several chunks) still take the fast path."""
    llz.debug_set_queue_cap(qcap)
    try:
        _queue_chunk_rows(cuda, qcap)
    finally:
        llz.debug_set_queue_cap(0)


def _queue_chunk_rows(cuda, qcap):
    import torch

    for name, rows in [("headline", 8), ("c2", 6)]:
        w = WORKLOADS[name]
        x = w.logits(rows)
        u = llz.rng_uniforms(w.uniform_seed, rows)
        cfg = llz.SamplerConfig.of(w.params)
        ws = torch.zeros(llz.workspace_bytes(rows, w.vocab, cfg), dtype=torch.uint8, device=cuda)
        xt = torch.from_numpy(np.ascontiguousarray(x)).to(cuda)
        ut = torch.from_numpy(np.ascontiguousarray(u, dtype=np.float32)).to(cuda)
        res = llz.sample_rows(xt, cfg, ut, kept_cap=256, stats=True, workspace=ws)
        torch.cuda.synchronize()
        status = ws[: rows * 4].view(torch.int32).cpu().numpy()  # per-row path bits (workspace offset 0)
        if qcap >= 32 and name == "headline":
            assert ((status & 8) == 0).any(), f"{name}: no row kept the fast path: {status}"
        g = dict(
            tokens=res.tokens.cpu().numpy().view(np.uint32),
            consumed=res.consumed.cpu().numpy(),
            kept_count=res.kept_count.cpu().numpy().view(np.uint32),
            kept_ids=res.kept_ids.cpu().numpy().view(np.uint32),
            kept_probs=res.kept_probs.cpu().numpy(),
            stats=res.row_stats.cpu().numpy(),
            cap=256,
        )
        compare_rows(x, w.params, u, g)
