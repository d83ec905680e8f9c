"""CPU checks that pin the oracle (oracle/llz_oracle.c) before it is trusted
as the parity checker of the HIP path.

What pins what:
  * RNG: published vectors -- SplitMix64 seeded with 0, and the sequence
    of Zig's own std.Random.Xoshiro256 test (init(0)); the xoshiro256++
    output of the state {1, 2, 3, 4} worked by hand; Random.float(f32)'s
    bit construction on states whose first draw is known.
  * exp / log: error at most one ulp against float64 over dense sweeps,
    plus the special values the msun algorithms fix.
  * the sampler: the reference's two unit tests (sampler.zig:171-213) in
    closed form, hand cases with exactly representable probabilities, and
    invariants on seeded rows computed independently with numpy (index-order
    float32 cumsum, lexsort order, top-k/min-p sets, the draw walk).
  * the committed golden vectors (tests/golden/), which freeze all of this.
"""
from __future__ import annotations

import ctypes as C
import hashlib
import math
import os

import numpy as np
import pytest

import oracle_lib as O
from llz.workloads import WORKLOADS, Params

HERE = os.path.dirname(os.path.abspath(__file__))
GOLDEN = os.path.join(HERE, "golden", "sampler_golden.npz")
NO_REP = dict(repetition_window=0, repetition_penalty=1.0)


def f32bits(a):
    return np.asarray(a, dtype=np.float32).view(np.uint32)


# ---------------------------------------------------------------------------
# RNG (sampler.zig:17,22,162 -> std.Random.DefaultPrng, Random.float(f32))
# ---------------------------------------------------------------------------
def test_splitmix64_published_vector():
    st = (C.c_uint64 * 1)(0)
    got = [O.lib().llz_oracle_splitmix64_next(st) for _ in range(3)]
    assert got == [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F]


def test_xoshiro256_zig_std_sequence():
    # Zig std lib/std/Random/Xoshiro256.zig, test "sequence": init(0)
    s = (C.c_uint64 * 4)()
    O.lib().llz_oracle_xoshiro_seed(s, 0)
    got = [O.lib().llz_oracle_xoshiro_next(s) for _ in range(6)]
    assert got == [0x53175D61490B23DF, 0x61DA6F3DC380D507, 0x5C0FDF91EC9A7BFC,
                   0x02EEBF8C3BBE5E1A, 0x7ECA04EBAF4A5EEA, 0x0543C37757F08D9A]


def test_xoshiro256pp_by_hand():
    # result = rotl(s0 + s3, 23) + s0 = (5 << 23) + 1 for the state {1, 2, 3, 4}
    s = (C.c_uint64 * 4)(1, 2, 3, 4)
    assert O.lib().llz_oracle_xoshiro_next(s) == (5 << 23) + 1


def test_random_float_construction():
    # first draw 0x2800001 from {1,2,3,4}: clz64 = 38 < 41, so exponent 126-38 and
    # mantissa = the low 23 bits (0x000001)
    s = (C.c_uint64 * 4)(1, 2, 3, 4)
    u = np.float32(O.lib().llz_oracle_random_f32(s))
    assert f32bits(u) == ((126 - 38) << 23) | 0x000001
    # a draw with its top bit set gives an exponent of 126: u in [0.5, 1)
    L = O.lib()
    for seed in (0, 1, 1234, 0xDEADBEEF):
        st = (C.c_uint64 * 4)()
        L.llz_oracle_xoshiro_seed(st, seed)
        st2 = (C.c_uint64 * 4)(*st)
        raw = L.llz_oracle_xoshiro_next(st2)
        u = np.float32(L.llz_oracle_random_f32(st))
        lz = 64 - int(raw).bit_length()
        assert lz < 41
        assert f32bits(u) == ((126 - lz) << 23) | (raw & 0x7FFFFF)
        assert 0.0 < u < 1.0
        assert tuple(st) == tuple(st2)  # exactly one next() consumed


def test_uniform_stream_properties():
    u = O.uniforms(0xDEADBEEF, 200000)
    assert np.all((u > 0) & (u < 1))
    assert abs(float(u.mean()) - 0.5) < 0.005
    assert np.array_equal(u, O.uniforms(0xDEADBEEF, 200000))


def _gof_checks(u: np.ndarray):
    """Goodness of fit of a Random.float(f32) stream (raises AssertionError).
    The construction: exponent 126 - clz(draw), mantissa = the draw's low 23
    bits, so (1) u is uniform on (0, 1); (2) the binade [2^-(k+1), 2^-k)
    holds a fraction 2^-(k+1) of the draws; (3) within a binade the mantissa
    is uniform and independent of the binade."""
    from scipy import stats

    n = u.size
    assert np.all((u > 0) & (u < 1)), "u outside (0, 1)"
    # (1) chi-square over 4096 equal bins
    counts = np.bincount(np.minimum((u.astype(np.float64) * 4096).astype(np.int64), 4095), minlength=4096)
    p1 = stats.chisquare(counts).pvalue
    assert p1 > 1e-6, f"bins: p = {p1:.3g}"
    # (2) binade frequencies 2^-(k+1), k = 0 .. 15 (and the rest pooled)
    e = (u.view(np.uint32) >> 23).astype(np.int64)
    k = np.minimum(126 - e, 16)
    obs = np.bincount(k, minlength=17)
    exp = np.array([2.0 ** -(i + 1) for i in range(16)] + [2.0 ** -16]) * n
    p2 = stats.chisquare(obs, exp).pvalue
    assert p2 > 1e-6, f"binades: p = {p2:.3g}"
    # (3) the top 6 mantissa bits are uniform within each of the first four binades
    m6 = (u.view(np.uint32) >> 17) & 63
    table = np.stack([np.bincount(m6[k == i], minlength=64) for i in range(4)])
    p3 = stats.chi2_contingency(table).pvalue
    assert p3 > 1e-6, f"mantissa vs binade: p = {p3:.3g}"
    for i in range(4):
        pi = stats.chisquare(table[i]).pvalue
        assert pi > 1e-6, f"mantissa in binade {i}: p = {pi:.3g}"
    # (4) the low mantissa bits stay random in smaller binades (a fixed-point
    # uniform has fewer random bits there: its lowest k bits are 0 in binade k)
    low2 = u.view(np.uint32) & 3
    for i in range(1, 7):
        c = np.bincount(low2[k == i], minlength=4)
        pi = stats.chisquare(c).pvalue
        assert pi > 1e-6, f"low mantissa bits in binade {i}: p = {pi:.3g}"


def test_random_float_goodness_of_fit():
    """Random.float(f32) (sampler.zig:162) over a long stream: the
    construction's three distributional properties hold."""
    _gof_checks(O.uniforms(0xDEADBEEF, 1 << 21))


def test_random_float_goodness_of_fit_catches_construction_mistakes():
    """Plausible restatement mistakes fail the same checks: an exponent off
    by one (127 - clz), the mantissa from the draw's top bits, and a plain
    24-bit uniform (no clz exponent)."""
    L = O.lib()
    st = (C.c_uint64 * 4)()
    L.llz_oracle_xoshiro_seed(st, 99)
    raw = np.array([L.llz_oracle_xoshiro_next(st) for _ in range(1 << 19)], dtype=np.uint64)
    lz = np.array([64 - int(r).bit_length() for r in raw.tolist()], dtype=np.int64)
    good = (((126 - lz) << 23) | (raw & 0x7FFFFF).astype(np.int64)).astype(np.uint32).view(np.float32)
    _gof_checks(good)  # the correct construction from the same draws passes
    off_by_one = (((127 - lz) << 23) | (raw & 0x7FFFFF).astype(np.int64)).astype(np.uint32).view(np.float32)
    top_bits = (((126 - lz) << 23) | ((raw >> 41) & 0x7FFFFF).astype(np.int64)).astype(np.uint32).view(np.float32)
    plain24 = ((raw >> 40).astype(np.float64) * 2.0 ** -24).astype(np.float32)
    plain24 = plain24[plain24 > 0]
    for name, bad in (("exponent off by one", off_by_one), ("mantissa from the top bits", top_bits),
                      ("plain 24-bit uniform", plain24)):
        with pytest.raises(AssertionError):
            _gof_checks(bad)
            raise RuntimeError(f"{name} passed the goodness-of-fit checks")


# ---------------------------------------------------------------------------
# exp / log (sampler.zig:85 std.math.exp, :131,136 @log) -- msun algorithms
# ---------------------------------------------------------------------------
def _ulp_err(got: np.ndarray, want64: np.ndarray) -> np.ndarray:
    w32 = want64.astype(np.float32)
    ulp = np.spacing(np.abs(w32)).astype(np.float64)
    return np.abs(got.astype(np.float64) - want64) / ulp


def test_expf_within_one_ulp():
    # every 101st bit pattern of (-103.9, 88.7): the whole finite, normal-output range
    neg = np.arange(0x80000000, 0xC2CFF1B5, 101, dtype=np.uint64).astype(np.uint32).view(np.float32)
    pos = np.arange(0x00000000, 0x42B17218, 101, dtype=np.uint32).view(np.float32)
    for x in (neg, pos):
        got = O.expf_array(x)
        want = np.exp(x.astype(np.float64))
        normal = want >= np.finfo(np.float32).tiny
        err = _ulp_err(got[normal], want[normal])
        assert err.max() <= 1.0, f"max error {err.max():.3f} ulp"


def test_expf_special_values():
    assert O.expf(0.0) == 1.0 and O.expf(-0.0) == 1.0
    assert O.expf(-np.inf) == 0.0
    assert O.expf(np.inf) == np.inf
    assert np.isnan(O.expf(np.nan))
    assert O.expf(-104.0) == 0.0  # below the underflow threshold
    assert O.expf(89.0) == np.inf
    t = np.float32(1e-5)  # |x| <= 2^-13 returns 1 + x
    assert O.expf(t) == np.float32(1.0) + t
    # subnormal results stay within one subnormal step of the true value
    for x in (-88.0, -95.0, -100.0, -103.0):
        assert abs(float(O.expf(x)) - math.exp(x)) <= 2.0 ** -149


def test_logf_within_one_ulp():
    x = np.arange(0x00000001, 0x7F800000, 97, dtype=np.uint32).view(np.float32)
    got = O.logf_array(x)
    want = np.log(x.astype(np.float64))
    nz = want != 0.0
    err = _ulp_err(got[nz], want[nz])
    assert err.max() <= 1.0, f"max error {err.max():.3f} ulp"


def test_logf_special_values():
    assert O.logf(1.0) == 0.0
    assert O.logf(0.0) == -np.inf and O.logf(-0.0) == -np.inf
    assert np.isnan(O.logf(-1.0))
    assert O.logf(np.inf) == np.inf
    assert np.isnan(O.logf(np.nan))
    for k in (-149, -126, -20, 1, 10, 127):
        want = np.float32(k * math.log(2.0))
        assert abs(int(f32bits(O.logf(2.0 ** k))) - int(f32bits(want))) <= 1


# ---------------------------------------------------------------------------
# the reference's unit tests (sampler.zig:171-213) in closed form
# ---------------------------------------------------------------------------
def test_reference_determinism_closed_form():
    p = Params(temperature=1.0, top_k=0, top_p=1.0, min_p=0.0, typical_p=1.0, **NO_REP)
    logits = np.zeros(4, np.float32)
    s1, s2 = O.Sampler(p, seed=1234), O.Sampler(p, seed=1234)
    seq1 = [s1.sample(logits) for _ in range(8)]
    seq2 = [s2.sample(logits) for _ in range(8)]
    assert seq1 == seq2
    # p = 0.25 exactly, total = 1 exactly: the walk returns ceil(4u) - 1
    u = O.uniforms(1234, 8)
    assert seq1 == [int(math.ceil(4.0 * float(v))) - 1 for v in u]


def test_reference_topk1_returns_argmax():
    p = Params(temperature=1.0, top_k=1, top_p=1.0, min_p=0.0, typical_p=1.0, **NO_REP)
    s = O.Sampler(p, seed=1)
    x = np.array([2.0, 1.9, 1.8], np.float32)
    assert [s.sample(x) for _ in range(16)] == [0] * 16


def test_seed_zero_falls_back_to_deadbeef():
    p = Params(temperature=1.0, top_p=1.0, **NO_REP)
    a, b = O.Sampler(p, seed=0), O.Sampler(p, seed=0xDEADBEEF)
    assert a.state == b.state


def test_rng_advances_only_on_draw():
    p = Params(temperature=0.8, top_p=0.9, **NO_REP)
    s = O.Sampler(p, seed=7)
    dom = np.full(64, -1.0, np.float32)
    dom[3] = 40.0   # p_max > top_p: empty kept set, no draw (sampler.zig:160)
    st0 = s.state
    assert s.sample(dom) == 3
    assert s.state == st0
    flat = np.zeros(64, np.float32)
    s.sample(flat)
    assert s.state != st0
    g = O.Sampler(Params(temperature=0.0, **NO_REP), seed=7)  # greedy: no draw (:50)
    st1 = g.state
    g.sample(flat)
    assert g.state == st1


# ---------------------------------------------------------------------------
# hand cases with exactly representable probabilities
# ---------------------------------------------------------------------------
QUARTERS = np.array([0.0, -np.inf, 0.0, 0.0, -np.inf, 0.0], np.float32)  # p = 0.25 on ids 0,2,3,5


def test_top_p_crossing_equality_keeps():
    # cum: 0.25, 0.5 (== top_p: kept), 0.75 (> top_p: dropped), ...
    o = O.sample_row(QUARTERS, Params(temperature=1.0, top_p=0.5, **NO_REP), 0.6)
    assert o.sum == 4.0 and o.kept_ids().tolist() == [0, 2]
    assert o.total == 0.5
    assert o.token == 2  # r = 0.3: 0.3 - 0.25 > 0, 0.05 - 0.25 <= 0
    o = O.sample_row(QUARTERS, Params(temperature=1.0, top_p=np.float32(0.4999), **NO_REP), 0.6)
    assert o.kept_ids().tolist() == [0]  # the crossing token is excluded


def test_min_p_is_strict():
    o = O.sample_row(QUARTERS, Params(temperature=1.0, top_p=1.0, min_p=1.0, **NO_REP), 0.3)
    assert o.kept_ids().tolist() == [0, 2, 3, 5]  # p == threshold is kept
    o = O.sample_row(QUARTERS, Params(temperature=1.0, top_p=1.0, min_p=np.float32(1.0000001), **NO_REP), 0.3)
    assert o.kept_count == 0 and o.consumed == 0 and o.token == 0


def test_typical_on_equal_probabilities():
    # every finite entry has the same deviation: stable order keeps the lowest ids
    o = O.sample_row(QUARTERS, Params(temperature=1.0, top_p=1.0, typical_p=0.6, **NO_REP), 0.3)
    assert o.kept_ids().tolist() == [0, 2]


def test_greedy_and_sum_exits():
    x = np.array([1.0, 5.0, 5.0, -2.0], np.float32)
    o = O.sample_row(x, Params(temperature=0.0, **NO_REP), 0.5)
    assert o.token == 1 and o.consumed == 0 and o.exit_path == O.EXIT_GREEDY
    # an all -inf row: (v - max) is NaN, so sum <= 0 is false (sampler.zig:89), every
    # comparison fails, and the walk ends at the fallback indices[0] after a draw
    o = O.sample_row(np.full(5, -np.inf, np.float32), Params(temperature=1.0, **NO_REP), 0.5)
    assert o.exit_path == O.EXIT_FALLBACK and o.token == 0 and o.consumed == 1
    assert np.isnan(o.sum)


def test_repetition_penalty_closed_form():
    x = np.array([2.0, -2.0, 1.0, 0.5], np.float32)
    p = Params(temperature=1.0, top_p=1.0, repetition_window=2, repetition_penalty=2.0)
    # window = the last two tokens {0, 1}: x0 -> 1.0, x1 -> -4.0; id 9 >= n never matches
    o = O.sample_row(x, p, 0.5, prev_tokens=np.array([2, 9, 0, 1], np.uint32))
    e = O.expf_array(np.array([1.0, -4.0, 1.0, 0.5], np.float32) - np.float32(1.0))
    assert f32bits(o.sum) == f32bits(np.cumsum(e, dtype=np.float32)[-1])


# ---------------------------------------------------------------------------
# invariants on seeded rows, computed independently with numpy
# ---------------------------------------------------------------------------
def _numpy_chain(x, p):
    """The chain's sets from numpy primitives: index-order float32 cumsum for
    the normaliser, lexsort for the order, cumsum over the order for top-p."""
    x = x.astype(np.float32)
    m = x.max()
    d = (x - m).astype(np.float32)
    if p.temperature != 1.0:
        d = (d / np.float32(p.temperature)).astype(np.float32)
    e = O.expf_array(d)
    s = np.cumsum(e, dtype=np.float32)[-1]
    probs = (e / s).astype(np.float32)
    order = np.lexsort((np.arange(x.size), -probs))
    sel = np.ones(x.size, bool)
    if 0 < p.top_k < x.size:
        sel[order[p.top_k:]] = False
    if 0 < p.top_p < 1:
        cand = order[sel[order]]
        cum = np.cumsum(probs[cand], dtype=np.float32)
        sel[cand[cum > np.float32(p.top_p)]] = False
    if p.min_p > 0:
        thr = np.float32(probs[order[0]] * np.float32(p.min_p))
        sel &= ~(probs < thr)
    return s, probs, order, sel


@pytest.mark.parametrize("name", ["c1", "c2", "c4", "headline"])
def test_chain_matches_numpy_primitives(name):
    w = WORKLOADS[name]
    gen = np.random.default_rng([w.data_seed, 77])
    for r in range(2):
        x = w.gen_row(gen, 20000, r)
        u = np.float32(0.25 + 0.5 * r)
        o = O.sample_row(x, w.params, u)
        s, probs, order, sel = _numpy_chain(x, w.params)
        assert f32bits(o.sum) == f32bits(s)
        assert np.array_equal(f32bits(o.probs), f32bits(probs))
        assert np.array_equal(o.order, order)
        assert np.array_equal(o.selected.astype(bool), sel)
        kept = order[sel[order]]
        assert o.kept_count == kept.size
        if kept.size:
            tot = np.cumsum(probs[kept], dtype=np.float32)[-1]
            assert f32bits(o.total) == f32bits(tot)
            r0 = np.float32(u * tot)
            walk = r0 - np.cumsum(probs[kept], dtype=np.float32)  # not the f32 chain; locate only
            # the f32 chain r -= p: replay it exactly
            rr = r0
            tok = int(order[0])
            for i in kept:
                rr = np.float32(rr - probs[i])
                if rr <= 0:
                    tok = int(i)
                    break
            assert o.token == tok
            assert walk.size == kept.size


def test_typical_matches_numpy_primitives():
    w = WORKLOADS["c3"]
    gen = np.random.default_rng([w.data_seed, 5])
    x = w.gen_row(gen, 8000, 0)
    p = w.params
    o = O.sample_row(x, p, 0.5)
    s, probs, order, sel = _numpy_chain(x, p)
    lg = O.logf_array(probs)
    ent = np.float32(0.0)
    for pi, li in zip(probs, lg):  # index order, sequential f32 (sampler.zig:129-132)
        if pi > 0:
            ent = np.float32(ent - np.float32(pi * li))
    assert f32bits(o.entropy) == f32bits(ent)
    surprise = np.where(probs > 0, -lg, np.float32(np.inf)).astype(np.float32)
    dev = np.abs((surprise - ent).astype(np.float32))
    torder = np.lexsort((np.arange(x.size), dev))
    cand = torder[sel[torder]]
    cum = np.cumsum(probs[cand], dtype=np.float32)
    sel[cand[cum > np.float32(p.typical_p)]] = False
    assert np.array_equal(o.selected.astype(bool), sel)


def test_batched_driver_matches_single_rows():
    w = WORKLOADS["c5"]
    x = np.stack([w.gen_row(np.random.default_rng([w.data_seed, 9, r]), 3000, r) for r in range(6)])
    u = O.uniforms(3, 6)
    tok, con, kept = O.sample_rows(x, w.params, u, threads=3)
    for r in range(6):
        o = O.sample_row(x[r], w.params, u[r])
        assert (tok[r], con[r], kept[r]) == (o.token, o.consumed, o.kept_count)


# ---------------------------------------------------------------------------
# the committed golden vectors
# ---------------------------------------------------------------------------
def _golden():
    return np.load(GOLDEN, allow_pickle=False)


def _params(row) -> Params:
    t, k, tp, mp, typ, win, rp = row
    return Params(temperature=float(t), top_k=int(k), top_p=float(tp), min_p=float(mp),
                  typical_p=float(typ), repetition_window=int(win), repetition_penalty=float(rp))


def test_oracle_reproduces_golden_vectors():
    g = _golden()
    for i, name in enumerate(g["name"]):
        n, off = int(g["n"][i]), int(g["offset"][i])
        x = g["logits"][off:off + n]
        prev = None
        if g["n_prev"][i]:
            po = int(g["prev_offset"][i])
            prev = g["prev_tokens"][po:po + int(g["n_prev"][i])]
        o = O.sample_row(x, _params(g["params"][i]), g["u"][i], prev_tokens=prev)
        assert o.token == g["token"][i], name
        assert o.consumed == g["consumed"][i], name
        assert o.kept_count == g["kept_count"][i], name
        assert o.exit_path == g["exit_path"][i], name
        assert np.array_equal(f32bits([o.max_logit, o.sum, o.entropy, o.total]), g["stats_bits"][i]), name
        if o.exit_path != O.EXIT_GREEDY:
            k = min(int(o.kept_count), g["kept_ids"].shape[1])
            assert np.array_equal(o.kept_ids()[:k], g["kept_ids"][i, :k]), name


def test_oracle_reproduces_golden_config1_full_vocab():
    g = _golden()
    w = WORKLOADS["c1"]
    x = w.logits(1)[0]
    assert hashlib.sha256(x.tobytes()).hexdigest() == str(g["c1_sha256"]), "workload generator drifted"
    o = O.sample_row(x, w.params, g["c1_u"])
    assert (o.token, o.consumed, o.kept_count) == (g["c1_token"], g["c1_consumed"], g["c1_kept"])
    assert np.array_equal(f32bits([o.max_logit, o.sum, o.entropy, o.total]), g["c1_stats_bits"])
    assert np.array_equal(o.kept_ids()[: g["c1_kept_ids"].size], g["c1_kept_ids"])


def test_planted_oracle_mistake_is_caught():
    """A plausible mistake (a parallel, more accurate normaliser) fails the
    sequential-f32 invariant the tests above rely on."""
    w = WORKLOADS["c2"]
    x = w.gen_row(np.random.default_rng([w.data_seed, 3]), 128256, 0)
    e = O.expf_array((x - x.max()).astype(np.float32))
    seq = np.cumsum(e, dtype=np.float32)[-1]
    pairwise = np.float32(np.sum(e.astype(np.float64)))
    o = O.sample_row(x, w.params, 0.5)
    assert f32bits(o.sum) == f32bits(seq)
    assert f32bits(pairwise) != f32bits(seq)


# ---------------------------------------------------------------------------
# expm1f / tanhf (musl expm1f.c / tanhf.c, the functions behind Zig's f32
# std.math.expm1 / tanh) and main.zig:653-666's post-processing.  The bit
# patterns Zig produces cannot be compared here (no Zig toolchain); what
# pins the restatement: musl's documented accuracy (< 1 ulp for expm1f,
# measured <= 2.05 ulp for tanhf over the sweeps), the branch structure
# (odd symmetry, saturation, the small-|x| identity), and a planted mistake
# that the accuracy check catches.
# ---------------------------------------------------------------------------
def _sweep(lo, hi, step):
    return np.arange(lo, hi, step, dtype=np.uint64).astype(np.uint32).view(np.float32)


def test_expm1f_within_one_ulp():
    x = np.concatenate([_sweep(0x80000000, 0xC18AA123, 89),    # -0 .. -17.3 (below: -1)
                        _sweep(0x00000000, 0x42B17180, 89)])    # 0 .. 88.72 (above: overflow)
    got = O.expm1f_array(x)
    want = np.expm1(x.astype(np.float64))
    ok = np.abs(want) >= np.finfo(np.float32).tiny
    err = _ulp_err(got[ok], want[ok])
    assert err.max() < 1.0, f"max error {err.max():.3f} ulp"


def test_expm1f_special_values():
    L = O.lib()
    assert L.llz_oracle_expm1f(0.0) == 0.0
    assert math.copysign(1.0, L.llz_oracle_expm1f(-0.0)) == -1.0
    assert L.llz_oracle_expm1f(-np.inf) == -1.0 and L.llz_oracle_expm1f(-30.0) == -1.0
    assert L.llz_oracle_expm1f(np.inf) == np.inf and L.llz_oracle_expm1f(89.0) == np.inf
    assert np.isnan(L.llz_oracle_expm1f(np.nan))
    t = np.float32(2.0 ** -26)  # |x| < 2^-25 returns x
    assert L.llz_oracle_expm1f(float(t)) == t


def test_tanhf_accuracy_and_structure():
    x = np.concatenate([_sweep(0x00800000, 0x41300000, 53),    # normal .. 11
                        _sweep(0x3E700000, 0x3F200000, 3)])    # the two branch edges, dense
    got = O.tanhf_array(x)
    want = np.tanh(x.astype(np.float64))
    err = _ulp_err(got, want)
    assert err.max() <= 2.5, f"max error {err.max():.3f} ulp"
    assert np.mean(err <= 0.5) > 0.85          # mostly correctly rounded
    # odd: tanh(-x) == -tanh(x) bit for bit
    assert np.array_equal(O.tanhf_array(-x).view(np.uint32), (-got).view(np.uint32))
    # saturation: exactly 1 for |x| > 10 and where tanh rounds to 1
    big = _sweep(0x41200001, 0x7F800001, 997)
    assert np.all(O.tanhf_array(big) == 1.0) and np.all(O.tanhf_array(-big) == -1.0)
    assert O.tanhf_array(np.float32([9.5]))[0] == 1.0
    # tiny arguments: tanh(x) == x (subnormals returned as they are)
    tiny = np.float32([1e-40, 2.0 ** -126, 1e-10, -3e-9])
    assert np.array_equal(O.tanhf_array(tiny), tiny)
    assert O.tanhf_array(np.float32([0.0]))[0] == 0.0
    assert np.isnan(O.tanhf_array(np.float32([np.nan]))[0])


def test_tanhf_planted_mistake_is_caught():
    """A tanh built on an expm1 with a wrong coefficient (Q1 off by 10%)
    violates the accuracy bound the test above enforces."""
    x = _sweep(0x3E900000, 0x3F800000, 101).astype(np.float64)
    q1, q2 = -3.3333212137e-2 * 1.1, 1.5807170421e-3

    def expm1_bad(v):  # k == 0 branch of the algorithm, in float64
        hfx = 0.5 * v
        hxs = v * hfx
        r1 = 1.0 + hxs * (q1 + hxs * q2)
        t = 3.0 - r1 * hfx
        e = hxs * ((r1 - t) / (6.0 - v * t))
        return v - (v * e - hxs)

    bad = np.array([expm1_bad(2 * v) / (expm1_bad(2 * v) + 2) for v in x], np.float32)
    assert _ulp_err(bad, np.tanh(x)).max() > 2.5


def test_logit_post_closed_forms():
    x = np.float32([-3.0, -0.5, 0.0, 0.25, 7.0, 100.0])
    # the scale: v * RN(1/scale); 1/0.5 == 2 exactly
    assert np.array_equal(O.logit_post(x, 0.0, 0.5), x * np.float32(2.0))
    # scale 1 and 0 (and a non-positive cap) leave the logits alone
    for s in (1.0, 0.0):
        assert np.array_equal(O.logit_post(x, -2.0, s), x)
    # the soft-cap: tanh(v / s) * s with f32 operations; bounded by s, odd, monotone
    y = O.logit_post(x, 30.0, 1.0)
    want = O.tanhf_array(x / np.float32(30.0)) * np.float32(30.0)
    assert np.array_equal(y, want)
    assert np.all(np.abs(y) <= 30.0) and np.all(np.diff(y) >= 0)
    assert np.array_equal(O.logit_post(-x, 30.0, 1.0), -y)
    # both: cap first, then the scale (main.zig:653-666's order)
    both = O.logit_post(x, 30.0, 0.5)
    assert np.array_equal(both, y * np.float32(2.0))


def test_libm_switch_changes_results_and_restores():
    """The sensitivity switch (oracle/libm_sensitivity.py): with the C
    library's expf/logf some probabilities of a headline row change, and the
    default (the msun restatement) comes back bit for bit."""
    w = WORKLOADS["headline"]
    x = w.logits(4)
    u = O.uniforms(w.uniform_seed, 4)
    base = [O.sample_row(x[r], w.params, u[r]).probs.copy() for r in range(4)]
    O.lib().llz_oracle_use_libm(1)
    try:
        alt = [O.sample_row(x[r], w.params, u[r]).probs.copy() for r in range(4)]
    finally:
        O.lib().llz_oracle_use_libm(0)
    again = [O.sample_row(x[r], w.params, u[r]).probs.copy() for r in range(4)]
    assert any(not np.array_equal(a.view(np.uint32), b.view(np.uint32)) for a, b in zip(base, alt))
    assert all(np.array_equal(a.view(np.uint32), b.view(np.uint32)) for a, b in zip(base, again))
