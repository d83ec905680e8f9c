"""ctypes binding of the CPU oracle (oracle/liboracle.so).

Test infrastructure: only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg import this module, and only as the checker.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from dataclasses import dataclass

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_DIR = os.path.join(ROOT, "oracle")
ORACLE_SO = os.path.join(ORACLE_DIR, "liboracle.so")

EXIT_GREEDY, EXIT_SUM_LE0, EXIT_EMPTY, EXIT_DRAW, EXIT_FALLBACK = range(5)


class OracleCfg(C.Structure):
    _fields_ = [
        ("temperature", C.c_float),
        ("top_k", C.c_uint32),
        ("top_p", C.c_float),
        ("min_p", C.c_float),
        ("typical_p", C.c_float),
        ("repetition_window", C.c_uint32),
        ("repetition_penalty", C.c_float),
        ("_pad", C.c_uint32),
        ("seed", C.c_uint64),
    ]


class OracleOut(C.Structure):
    _fields_ = [
        ("token", C.c_uint32),
        ("consumed", C.c_uint32),
        ("exit_path", C.c_uint32),
        ("kept_count", C.c_uint32),
        ("max_logit", C.c_float),
        ("sum", C.c_float),
        ("entropy", C.c_float),
        ("total", C.c_float),
        ("r0", C.c_float),
        ("p_max", C.c_float),
        ("probs", C.POINTER(C.c_float)),
        ("order", C.POINTER(C.c_uint32)),
        ("selected", C.POINTER(C.c_uint8)),
    ]


class OracleSampler(C.Structure):
    _fields_ = [("cfg", OracleCfg), ("prng", C.c_uint64 * 4)]


_lib = None


def build() -> None:
    subprocess.run(["make", "-s", "-C", ORACLE_DIR], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(ORACLE_SO):
            build()
        L = C.CDLL(ORACLE_SO)
        fp, u32, u64, i64 = C.POINTER(C.c_float), C.c_uint32, C.c_uint64, C.c_int64
        L.llz_oracle_expf.restype = C.c_float
        L.llz_oracle_expf.argtypes = [C.c_float]
        L.llz_oracle_logf.restype = C.c_float
        L.llz_oracle_logf.argtypes = [C.c_float]
        L.llz_oracle_expf_array.argtypes = [fp, fp, i64]
        L.llz_oracle_expf_array.restype = None
        L.llz_oracle_logf_array.argtypes = [fp, fp, i64]
        L.llz_oracle_logf_array.restype = None
        for name in ("llz_oracle_expm1f", "llz_oracle_tanhf"):
            getattr(L, name).restype = C.c_float
            getattr(L, name).argtypes = [C.c_float]
        for name in ("llz_oracle_expm1f_array", "llz_oracle_tanhf_array"):
            getattr(L, name).restype = None
            getattr(L, name).argtypes = [fp, fp, i64]
        L.llz_oracle_use_libm.restype = None
        L.llz_oracle_use_libm.argtypes = [C.c_int]
        L.llz_oracle_logit_post.restype = None
        L.llz_oracle_logit_post.argtypes = [fp, i64, C.c_float, C.c_float]
        L.llz_oracle_splitmix64_next.restype = u64
        L.llz_oracle_splitmix64_next.argtypes = [C.POINTER(u64)]
        L.llz_oracle_xoshiro_seed.argtypes = [C.POINTER(u64), u64]
        L.llz_oracle_xoshiro_next.restype = u64
        L.llz_oracle_xoshiro_next.argtypes = [C.POINTER(u64)]
        L.llz_oracle_random_f32.restype = C.c_float
        L.llz_oracle_random_f32.argtypes = [C.POINTER(u64)]
        L.llz_oracle_uniforms.argtypes = [C.POINTER(u64), fp, i64]
        L.llz_oracle_argmax.restype = u32
        L.llz_oracle_argmax.argtypes = [fp, i64]
        L.llz_oracle_sample_row.restype = C.c_int
        L.llz_oracle_sample_row.argtypes = [fp, i64, C.POINTER(OracleCfg), C.POINTER(u32), i64,
                                            C.c_float, C.POINTER(OracleOut)]
        L.llz_oracle_sample_rows.restype = C.c_int
        L.llz_oracle_sample_rows.argtypes = [fp, i64, i64, i64, C.POINTER(OracleCfg),
                                             C.POINTER(u32), i64, i64, fp, C.POINTER(u32),
                                             C.POINTER(C.c_uint8), C.POINTER(u32), C.c_int]
        L.llz_oracle_sample_rows_stats.restype = C.c_int
        L.llz_oracle_sample_rows_stats.argtypes = [fp, i64, i64, i64, C.POINTER(OracleCfg),
                                                   C.POINTER(u32), i64, i64, fp, C.POINTER(u32),
                                                   C.POINTER(C.c_uint8), C.POINTER(u32), fp, C.c_int]
        L.llz_oracle_sampler_init.argtypes = [C.POINTER(OracleSampler), C.POINTER(OracleCfg)]
        L.llz_oracle_sampler_sample.restype = C.c_int
        L.llz_oracle_sampler_sample.argtypes = [C.POINTER(OracleSampler), fp, i64, C.POINTER(u32),
                                                i64, C.POINTER(u32)]
        _lib = L
    return _lib


def _fptr(a: np.ndarray):
    return a.ctypes.data_as(C.POINTER(C.c_float))


def _uptr(a: np.ndarray):
    return a.ctypes.data_as(C.POINTER(C.c_uint32))


def make_cfg(params, seed: int = 0) -> OracleCfg:
    return OracleCfg(float(params.temperature), int(params.top_k), float(params.top_p),
                     float(params.min_p), float(params.typical_p),
                     int(params.repetition_window), float(params.repetition_penalty), 0,
                     int(seed))


@dataclass
class RowResult:
    token: int
    consumed: int
    exit_path: int
    kept_count: int
    max_logit: float
    sum: float
    entropy: float
    total: float
    r0: float
    p_max: float
    probs: np.ndarray | None = None
    order: np.ndarray | None = None
    selected: np.ndarray | None = None

    def kept_ids(self) -> np.ndarray:
        """Kept token ids in (p desc, idx asc) order."""
        return self.order[self.selected[self.order].astype(bool)]


def sample_row(logits: np.ndarray, params, u: float, prev_tokens=None, detail: bool = True) -> RowResult:
    L = lib()
    x = np.ascontiguousarray(logits, dtype=np.float32)
    n = x.shape[0]
    prev = np.ascontiguousarray(prev_tokens if prev_tokens is not None else [], dtype=np.uint32)
    out = OracleOut()
    probs = order = sel = None
    if detail:
        probs = np.empty(n, np.float32)
        order = np.empty(n, np.uint32)
        sel = np.empty(n, np.uint8)
        out.probs = _fptr(probs)
        out.order = _uptr(order)
        out.selected = sel.ctypes.data_as(C.POINTER(C.c_uint8))
    cfg = make_cfg(params)
    rc = L.llz_oracle_sample_row(_fptr(x), n, C.byref(cfg), _uptr(prev), prev.shape[0],
                                 C.c_float(np.float32(u)), C.byref(out))
    if rc != 0:
        raise MemoryError("oracle allocation failed")
    return RowResult(out.token, out.consumed, out.exit_path, out.kept_count, out.max_logit,
                     out.sum, out.entropy, out.total, out.r0, out.p_max, probs, order, sel)


def sample_rows(logits: np.ndarray, params, uniforms: np.ndarray, prev_tokens=None,
                threads: int = 1):
    """Token, consumed-flag and kept-count per row (no detail)."""
    L = lib()
    x = np.ascontiguousarray(logits, dtype=np.float32)
    rows, n = x.shape
    u = np.ascontiguousarray(uniforms, dtype=np.float32)
    assert u.shape[0] >= rows
    tokens = np.empty(rows, np.uint32)
    consumed = np.empty(rows, np.uint8)
    kept = np.empty(rows, np.uint32)
    if prev_tokens is None:
        prev = np.zeros(0, np.uint32)
        n_prev, stride = 0, 0
    else:
        prev = np.ascontiguousarray(prev_tokens, dtype=np.uint32)
        if prev.ndim == 1:
            n_prev, stride = prev.shape[0], 0
        else:
            n_prev, stride = prev.shape[1], prev.shape[1]
    cfg = make_cfg(params)
    rc = L.llz_oracle_sample_rows(_fptr(x), rows, n, n, C.byref(cfg), _uptr(prev), n_prev,
                                  stride, _fptr(u), _uptr(tokens),
                                  consumed.ctypes.data_as(C.POINTER(C.c_uint8)), _uptr(kept),
                                  int(threads))
    if rc != 0:
        raise MemoryError("oracle allocation failed")
    return tokens, consumed, kept


def sample_rows_stats(logits: np.ndarray, params, uniforms: np.ndarray, threads: int = 1):
    """Token, consumed flag, kept count and [max, normaliser, entropy, total]
    per row, no repetition history."""
    L = lib()
    x = np.ascontiguousarray(logits, dtype=np.float32)
    rows, n = x.shape
    u = np.ascontiguousarray(uniforms, dtype=np.float32)
    assert u.shape[0] >= rows
    tokens = np.empty(rows, np.uint32)
    consumed = np.empty(rows, np.uint8)
    kept = np.empty(rows, np.uint32)
    stats = np.empty((rows, 4), np.float32)
    prev = np.zeros(0, np.uint32)
    cfg = make_cfg(params)
    rc = L.llz_oracle_sample_rows_stats(_fptr(x), rows, n, n, C.byref(cfg), _uptr(prev), 0, 0, _fptr(u),
                                        _uptr(tokens), consumed.ctypes.data_as(C.POINTER(C.c_uint8)),
                                        _uptr(kept), _fptr(stats), int(threads))
    if rc != 0:
        raise MemoryError("oracle allocation failed")
    return tokens, consumed, kept, stats


def expf(x: float) -> np.float32:
    return np.float32(lib().llz_oracle_expf(C.c_float(np.float32(x))))


def logf(x: float) -> np.float32:
    return np.float32(lib().llz_oracle_logf(C.c_float(np.float32(x))))


def expf_array(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty_like(x)
    lib().llz_oracle_expf_array(_fptr(x), _fptr(out), x.size)
    return out


def logf_array(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty_like(x)
    lib().llz_oracle_logf_array(_fptr(x), _fptr(out), x.size)
    return out


def expm1f_array(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty_like(x)
    lib().llz_oracle_expm1f_array(_fptr(x), _fptr(out), x.size)
    return out


def tanhf_array(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty_like(x)
    lib().llz_oracle_tanhf_array(_fptr(x), _fptr(out), x.size)
    return out


def logit_post(x: np.ndarray, softcap: float = 0.0, logit_scale: float = 1.0) -> np.ndarray:
    """main.zig:653-666 on a copy of the logits (any shape)."""
    y = np.array(x, dtype=np.float32, order="C", copy=True)
    lib().llz_oracle_logit_post(_fptr(y), y.size, C.c_float(softcap), C.c_float(logit_scale))
    return y


def uniforms(seed: int, count: int) -> np.ndarray:
    """Successive Random.float(f32) draws from DefaultPrng.init(seed)."""
    L = lib()
    st = (C.c_uint64 * 4)()
    L.llz_oracle_xoshiro_seed(st, C.c_uint64(seed))
    out = np.empty(count, np.float32)
    L.llz_oracle_uniforms(st, _fptr(out), count)
    return out


class Sampler:
    """Oracle Sampler: init/sample with the reference's RNG lifecycle."""

    def __init__(self, params, seed: int):
        self._s = OracleSampler()
        cfg = make_cfg(params, seed)
        lib().llz_oracle_sampler_init(C.byref(self._s), C.byref(cfg))

    @property
    def state(self):
        return tuple(int(v) for v in self._s.prng)

    def sample(self, logits: np.ndarray, prev_tokens=None) -> int:
        x = np.ascontiguousarray(logits, dtype=np.float32)
        prev = np.ascontiguousarray(prev_tokens if prev_tokens is not None else [], dtype=np.uint32)
        tok = C.c_uint32()
        rc = lib().llz_oracle_sampler_sample(C.byref(self._s), _fptr(x), x.shape[0], _uptr(prev),
                                             prev.shape[0], C.byref(tok))
        if rc != 0:
            raise MemoryError("oracle allocation failed")
        return int(tok.value)
