"""The C ABI without a GPU: the library loads, exports every function that
include/llz_sampler.h declares, and its host-only logic (the reference's
PRNG, SamplerConfig defaults, workspace sizing, argument validation that
returns before any HIP call) behaves as documented."""
from __future__ import annotations

import ctypes as C
import os
import re

import numpy as np

import llz
import oracle_lib as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER_DIR = os.path.join(ROOT, "include")


def declared_functions():
    names = set()
    for fn in os.listdir(HEADER_DIR):
        if not fn.endswith(".h"):
            continue
        text = open(os.path.join(HEADER_DIR, fn)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"\b(llz_[a-z0-9_]+)\s*\(", text):
            names.add(m.group(1))
    return names


def test_library_exports_every_declared_function():
    names = declared_functions()
    assert "llz_sample_rows" in names and "llz_argmax_rows" in names
    lib = llz.library()
    missing = [n for n in sorted(names) if not hasattr(lib, n)]
    assert not missing, f"declared but not exported: {missing}"
    assert set(names) <= set(llz.EXPORTED) | set(names)


def test_binding_lists_every_declared_function():
    assert declared_functions() == set(llz.EXPORTED)


def test_config_defaults_match_sampler_config():
    c = llz.CConfig()
    llz.library().llz_sampler_config_default(C.byref(c))
    d = llz.SamplerConfig()
    # SamplerConfig defaults (sampler.zig:4-13)
    assert np.float32(c.temperature) == np.float32(0.8) == np.float32(d.temperature)
    assert c.top_k == 0 == d.top_k
    assert np.float32(c.top_p) == np.float32(0.9)
    assert c.min_p == 0.0 and c.typical_p == 1.0
    assert c.repetition_window == 32 and np.float32(c.repetition_penalty) == np.float32(1.1)
    assert c.seed == 0 and c.reserved == 0


def test_host_prng_matches_oracle():
    for seed in (0, 1, 1234, 0xDEADBEEF, 2**64 - 1):
        a = llz.rng_uniforms(seed, 5000)
        b = O.uniforms(seed, 5000)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), seed
        p = llz.Prng(seed)
        s = (C.c_uint64 * 4)()
        O.lib().llz_oracle_xoshiro_seed(s, seed)
        assert [p.next_u64() for _ in range(4)] == [O.lib().llz_oracle_xoshiro_next(s) for _ in range(4)]


def test_workspace_bytes():
    cfg = llz.SamplerConfig(temperature=1.0, top_k=40, top_p=0.95, min_p=0.05)
    ws = llz.workspace_bytes(256, 128256, cfg)
    assert ws > 0 and ws % 256 == 0
    assert llz.workspace_bytes(512, 128256, cfg) > ws
    L = llz.library()
    c = cfg.to_c()
    assert L.llz_sample_workspace_bytes(0, 10, C.byref(c), 0) == 0
    assert L.llz_sample_workspace_bytes(1, 0, C.byref(c), 0) == 0
    assert L.llz_sample_workspace_bytes(1, 10, None, 0) == 0
    assert L.llz_sample_workspace_bytes(1, 10, C.byref(c), -1) == 0


def test_workspace_split_section():
    """Calls of at most 64 rows carry the split rows' records, 34,880 B per row
    (64 chunk records of 32 B, the election word and its padding, 64 x 64 list
    words of 8 B), last in the workspace; larger calls do not."""
    cfg = llz.SamplerConfig(temperature=1.0, top_k=40, top_p=0.95, min_p=0.05)
    per_row = 64 * 32 + 64 + 64 * 64 * 8
    assert per_row == 34880

    def step(rows):  # the bytes one more row adds
        return llz.workspace_bytes(rows + 1, 128256, cfg) - llz.workspace_bytes(rows, 128256, cfg)

    # every other section grows by the same bytes per row below and above 64
    # rows (up to 256), so one more row costs the split record more below 64
    # (sections are 256-byte aligned)
    assert abs((step(10) - step(100)) - per_row) <= 512
    # and the 65th row drops the whole section
    assert llz.workspace_bytes(65, 128256, cfg) < llz.workspace_bytes(64, 128256, cfg) + step(100) - 63 * per_row


def test_split_hook_modes():
    """llz_debug_set_split takes 0, 1, 2, 4 and 8 only (host-side, no GPU call)."""
    L = llz.library()
    for ok in (0, 1, 2, 4, 8):
        assert L.llz_debug_set_split(ok) == llz.LLZ_OK, ok
    for bad in (3, 5, 16, -1, 0x102, 0x200):
        assert L.llz_debug_set_split(bad) == llz.LLZ_E_INVALID_ARG, bad
    assert L.llz_debug_set_split(0) == llz.LLZ_OK


def test_argument_validation_without_gpu():
    """Invalid calls return an error code before any HIP call is made."""
    L = llz.library()
    fake = C.c_void_p(0x1000)  # never dereferenced: validation fails first
    cfg = llz.SamplerConfig(temperature=1.0).to_c()

    def call(logits=fake, stride=16, rows=1, vocab=16, c=C.byref(cfg), prev=None, n_prev=0, pstride=0,
             u=fake, tok=fake, con=None, ws=fake, wsb=1 << 30):
        return L.llz_sample_rows(logits, stride, rows, vocab, c, None, prev, n_prev, pstride, u, tok, con,
                                 None, ws, wsb, None)

    assert call(logits=None) == llz.LLZ_E_INVALID_ARG
    assert call(rows=0) == llz.LLZ_E_INVALID_ARG
    assert call(vocab=0) == llz.LLZ_E_INVALID_ARG
    assert call(stride=8) == llz.LLZ_E_INVALID_ARG          # row_stride < vocab
    assert call(c=None) == llz.LLZ_E_INVALID_ARG
    assert call(tok=None) == llz.LLZ_E_INVALID_ARG
    assert call(n_prev=3) == llz.LLZ_E_INVALID_ARG          # history length without a pointer
    assert call(n_prev=-1) == llz.LLZ_E_INVALID_ARG
    assert call(u=None) == llz.LLZ_E_INVALID_ARG            # sampling rows need uniforms
    nan_cfg = llz.SamplerConfig(temperature=float("nan")).to_c()
    assert call(c=C.byref(nan_cfg)) == llz.LLZ_E_INVALID_ARG
    assert call(ws=None) == llz.LLZ_E_WORKSPACE
    assert call(wsb=16) == llz.LLZ_E_WORKSPACE
    assert L.llz_argmax_rows(None, 16, 1, 16, None, fake, None) == llz.LLZ_E_INVALID_ARG
    assert L.llz_argmax_rows(fake, 16, 1, 16, None, None, None) == llz.LLZ_E_INVALID_ARG
    assert L.llz_debug_math(None, None, None, None, None, 4, None) == llz.LLZ_E_INVALID_ARG
    assert L.llz_debug_hw_error(0, 0, 16, None, None) == llz.LLZ_E_INVALID_ARG
    assert L.llz_debug_hw_error(4, 0, 16, fake, None) == llz.LLZ_E_INVALID_ARG
    assert L.llz_debug_hw_error(0, 0, 0, fake, None) == llz.LLZ_E_INVALID_ARG
    for code in (0, -1, -2, -3, -4, -5, -99):
        assert L.llz_strerror(code)


def test_sampler_create_rejects_bad_config():
    L = llz.library()
    h = C.c_void_p()
    bad = llz.SamplerConfig(temperature=float("nan")).to_c()
    assert L.llz_sampler_create(C.byref(bad), 0, C.byref(h)) == llz.LLZ_E_INVALID_ARG
    assert L.llz_sampler_create(None, 0, C.byref(h)) == llz.LLZ_E_INVALID_ARG
    L.llz_sampler_destroy(None)  # a no-op
