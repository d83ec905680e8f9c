"""Python binding of libllzsample.so, the MI355X sampler for llama.zig.

The names mirror the reference's sampler API (src/sampler.zig):

* ``SamplerConfig``  -- SamplerConfig (sampler.zig:4-13), same defaults;
* ``Sampler``        -- Sampler.init / Sampler.sample (sampler.zig:15-28), with
  the reference's PRNG lifecycle (seed fallback 0xDEADBEEF, one stream, a
  draw consumed only when the row reaches sampler.zig:162);
* ``sample_argmax``  -- sampleArgmax (sampler.zig:31-41);
* ``sample_rows``    -- the batched device entry point behind them.

Device memory and streams come from PyTorch (plumbing only); every compute
call goes through the C ABI declared in include/llz_sampler.h.  There is no
CPU fallback: a missing or unloadable library raises.
"""
from __future__ import annotations

import ctypes as C
import dataclasses
import os
from typing import Optional, Tuple

import numpy as np

PKG_DIR = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
# LLZ_LIBRARY selects another build of the same library (the phase-stamp
# measurement build, libllzsample_stamp.so); by default the product build.
LIB_PATH = os.environ.get("LLZ_LIBRARY") or os.path.join(PKG_DIR, "libllzsample.so")

LLZ_OK = 0
LLZ_E_INVALID_ARG = -1
LLZ_E_WORKSPACE = -2
LLZ_E_HIP = -3
LLZ_E_OOM = -4
LLZ_E_NO_DEVICE = -5
LLZ_E_SCRATCH = -6

# Public symbols of include/llz_sampler.h.
EXPORTED = (
    "llz_sampler_config_default", "llz_sample_workspace_bytes", "llz_sample_rows", "llz_sample_rows_noalloc",
    "llz_argmax_rows", "llz_rng_seed", "llz_rng_next", "llz_rng_float", "llz_rng_uniforms",
    "llz_sampler_create", "llz_sampler_destroy", "llz_sampler_sample", "llz_sampler_sample_uniform",
    "llz_sampler_sample_config", "llz_sampler_get_state", "llz_sampler_set_state", "llz_debug_math",
    "llz_debug_hw_error", "llz_debug_kernel_events", "llz_debug_set_queue_cap", "llz_debug_set_split",
    "llz_strerror",
)


class LlzError(RuntimeError):
    def __init__(self, code: int, what: str = ""):
        self.code = code
        msg = _lib().llz_strerror(code).decode() if _LIB is not None else str(code)
        super().__init__(f"{what}: {msg} ({code})" if what else f"{msg} ({code})")


class CConfig(C.Structure):
    _fields_ = [
        ("temperature", C.c_float), ("top_k", C.c_uint32), ("top_p", C.c_float),
        ("min_p", C.c_float), ("typical_p", C.c_float), ("reserved", C.c_uint32),
        ("seed", C.c_uint64), ("repetition_window", C.c_uint32), ("repetition_penalty", C.c_float),
    ]


class CPost(C.Structure):
    _fields_ = [("final_logit_softcapping", C.c_float), ("logit_scale", C.c_float)]


@dataclasses.dataclass
class LogitPost:
    """The decode loop's final-logit post-processing (main.zig:653-666):
    soft-capping when final_logit_softcapping > 0, then v *= 1 / logit_scale
    when logit_scale is neither 1 nor 0."""

    final_logit_softcapping: float = 0.0
    logit_scale: float = 1.0

    def to_c(self) -> CPost:
        return CPost(float(self.final_logit_softcapping), float(self.logit_scale))


def _post_ref(post: Optional[LogitPost]):
    return C.byref(post.to_c()) if post is not None else None


class CExtras(C.Structure):
    _fields_ = [
        ("d_kept_count", C.c_void_p), ("d_kept_ids", C.c_void_p), ("d_kept_probs", C.c_void_p),
        ("kept_cap", C.c_int32), ("reserved", C.c_int32), ("d_row_stats", C.c_void_p),
        ("d_row_path", C.c_void_p),
    ]


@dataclasses.dataclass
class SamplerConfig:
    """SamplerConfig (src/sampler.zig:4-13), same field names and defaults."""

    temperature: float = 0.8
    top_k: int = 0
    top_p: float = 0.9
    min_p: float = 0.0
    typical_p: float = 1.0
    seed: int = 0
    repetition_window: int = 32
    repetition_penalty: float = 1.1

    def to_c(self) -> CConfig:
        return CConfig(float(self.temperature), int(self.top_k), float(self.top_p),
                       float(self.min_p), float(self.typical_p), 0, int(self.seed),
                       int(self.repetition_window), float(self.repetition_penalty))

    @classmethod
    def of(cls, params, seed: int = 0) -> "SamplerConfig":
        return cls(params.temperature, params.top_k, params.top_p, params.min_p, params.typical_p,
                   seed, params.repetition_window, params.repetition_penalty)


_LIB = None


def _lib():
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is not built (run __graft_entry__.build())")
        L = C.CDLL(LIB_PATH)
        vp, i32, i64, u64 = C.c_void_p, C.c_int32, C.c_int64, C.c_uint64
        L.llz_sampler_config_default.argtypes = [C.POINTER(CConfig)]
        L.llz_sampler_config_default.restype = None
        L.llz_sample_workspace_bytes.argtypes = [i32, i32, C.POINTER(CConfig), i32]
        L.llz_sample_workspace_bytes.restype = C.c_size_t
        L.llz_sample_rows.argtypes = [vp, i64, i32, i32, C.POINTER(CConfig), C.POINTER(CPost), vp, i32, i64,
                                      vp, vp, vp, C.POINTER(CExtras), vp, C.c_size_t, vp]
        L.llz_sample_rows.restype = C.c_int
        L.llz_sample_rows_noalloc.argtypes = [vp, i64, i32, i32, C.POINTER(CConfig), C.POINTER(CPost), vp, i32,
                                              i64, vp, vp, vp, C.POINTER(CExtras), vp]
        L.llz_sample_rows_noalloc.restype = C.c_int
        L.llz_argmax_rows.argtypes = [vp, i64, i32, i32, C.POINTER(CPost), vp, vp]
        L.llz_argmax_rows.restype = C.c_int
        L.llz_rng_seed.argtypes = [C.POINTER(u64), u64]
        L.llz_rng_seed.restype = None
        L.llz_rng_next.argtypes = [C.POINTER(u64)]
        L.llz_rng_next.restype = u64
        L.llz_rng_float.argtypes = [C.POINTER(u64)]
        L.llz_rng_float.restype = C.c_float
        L.llz_rng_uniforms.argtypes = [C.POINTER(u64), C.POINTER(C.c_float), i64]
        L.llz_rng_uniforms.restype = None
        L.llz_sampler_create.argtypes = [C.POINTER(CConfig), i32, C.POINTER(vp)]
        L.llz_sampler_create.restype = C.c_int
        L.llz_sampler_destroy.argtypes = [vp]
        L.llz_sampler_destroy.restype = None
        L.llz_sampler_sample.argtypes = [vp, vp, i32, C.POINTER(C.c_uint32), i32,
                                         C.POINTER(C.c_uint32)]
        L.llz_sampler_sample.restype = C.c_int
        L.llz_sampler_sample_uniform.argtypes = [vp, vp, i32, C.POINTER(C.c_uint32), i32, C.c_float,
                                                 C.POINTER(C.c_uint32), C.POINTER(C.c_uint8)]
        L.llz_sampler_sample_uniform.restype = C.c_int
        L.llz_sampler_sample_config.argtypes = [vp, C.POINTER(CConfig), vp, i32, C.POINTER(C.c_uint32), i32,
                                                C.c_float, C.POINTER(C.c_uint32), C.POINTER(C.c_uint8)]
        L.llz_sampler_sample_config.restype = C.c_int
        L.llz_sampler_get_state.argtypes = [vp, C.POINTER(u64)]
        L.llz_sampler_get_state.restype = None
        L.llz_sampler_set_state.argtypes = [vp, C.POINTER(u64)]
        L.llz_sampler_set_state.restype = None
        L.llz_debug_math.argtypes = [vp, vp, vp, vp, vp, i64, vp]
        L.llz_debug_math.restype = C.c_int
        L.llz_debug_hw_error.argtypes = [i32, C.c_uint32, C.c_uint32, vp, vp]
        L.llz_debug_hw_error.restype = C.c_int
        L.llz_debug_kernel_events.argtypes = [vp, vp]
        L.llz_debug_kernel_events.restype = C.c_int
        L.llz_debug_set_queue_cap.argtypes = [C.c_uint32]
        L.llz_debug_set_queue_cap.restype = C.c_int
        L.llz_debug_set_split.argtypes = [i32]
        L.llz_debug_set_split.restype = C.c_int
        L.llz_strerror.argtypes = [C.c_int]
        L.llz_strerror.restype = C.c_char_p
        _LIB = L
    return _LIB


def library():
    """The loaded ctypes library (raises if it is not built)."""
    return _lib()


def _check(rc: int, what: str) -> None:
    if rc != LLZ_OK:
        raise LlzError(rc, what)


# ---------------------------------------------------------------------------
# the reference's PRNG (std.Random.DefaultPrng + Random.float(f32))
# ---------------------------------------------------------------------------
class Prng:
    """Xoshiro256 seeded through SplitMix64 (sampler.zig:22)."""

    def __init__(self, seed: int):
        self.state = (C.c_uint64 * 4)()
        _lib().llz_rng_seed(self.state, C.c_uint64(seed))

    def next_u64(self) -> int:
        return int(_lib().llz_rng_next(self.state))

    def float32(self) -> np.float32:
        return np.float32(_lib().llz_rng_float(self.state))

    def uniforms(self, count: int) -> np.ndarray:
        out = np.empty(count, np.float32)
        _lib().llz_rng_uniforms(self.state, out.ctypes.data_as(C.POINTER(C.c_float)), count)
        return out


def rng_uniforms(seed: int, count: int) -> np.ndarray:
    """count successive Random.float(f32) draws from DefaultPrng.init(seed)."""
    return Prng(seed).uniforms(count)


# ---------------------------------------------------------------------------
# device entry points (torch tensors are only the memory holders)
# ---------------------------------------------------------------------------
def _torch():
    import torch  # noqa: PLC0415

    return torch


def _stream_ptr(stream) -> int:
    torch = _torch()
    s = stream if stream is not None else torch.cuda.current_stream()
    return int(s.cuda_stream)


def workspace_bytes(rows: int, vocab: int, cfg: SamplerConfig, n_prev: int = 0) -> int:
    return int(_lib().llz_sample_workspace_bytes(rows, vocab, C.byref(cfg.to_c()), n_prev))


@dataclasses.dataclass
class SampleResult:
    tokens: "object"                  # torch.uint32-as-int32 tensor [rows]
    consumed: "object"                # torch.uint8 [rows]
    kept_count: Optional[object] = None
    kept_ids: Optional[object] = None
    kept_probs: Optional[object] = None
    row_stats: Optional[object] = None
    row_path: Optional[object] = None  # torch.int32 [rows], LLZ_PATH_* bits


PATH_SUM_LE0, PATH_ENTROPY, PATH_FULL_SORT, PATH_STREAM_NORM = 1, 2, 4, 8
PATH_WALK_ROUNDS, PATH_RESOLVE_GENERIC = 16, 32  # diagnostics of the single pass's walk
PATH_BUCKETS = 64  # full row without a sort: kept prefix, total and draw from p-key buckets
PATH_TOKEN_ONLY = 128  # the token decided without the exact normaliser (calls asking for the token alone)
PATH_DECLINE_SHIFT = 8  # bits 8-15: why the bucket path declined a full-row row (a number, not flags)
PATH_RECOLLECT = 1 << 16  # a flooded candidate list collected again (its largest terms)
PATH_SPLIT = 1 << 17  # token-only row finished from chunks read by several workgroups (with PATH_TOKEN_ONLY)


def sample_rows(logits, cfg: SamplerConfig, uniforms, prev_tokens=None, *, post: Optional[LogitPost] = None,
                kept_cap: int = 0, probs: bool = True, stats: bool = False, path: bool = False, workspace=None,
                stream=None, out=None) -> SampleResult:
    """Batched Sampler.sample over device rows.

    logits: float32 CUDA tensor [rows, vocab] (rows may be strided);
    uniforms: float32 CUDA tensor [rows]; prev_tokens: int32 CUDA tensor
    [n_prev] (shared) or [rows, n_prev].  Returns device tensors; the call is
    asynchronous on ``stream`` (default: torch's current stream).  With
    kept_cap > 0 the kept ids (and, unless probs is False, their
    probabilities) are returned; a call that asks for neither probabilities nor
    row statistics may finish rows without the exact normaliser (the token,
    draw flag, kept count and ids are the same either way).
    """
    torch = _torch()
    if not (logits.is_cuda and logits.dtype == torch.float32 and logits.dim() == 2):
        raise ValueError("logits must be a 2-D float32 CUDA tensor")
    if logits.stride(1) != 1:
        raise ValueError("logits rows must be contiguous")
    rows, vocab = logits.shape
    dev = logits.device
    if (uniforms.dtype != torch.float32 or not uniforms.is_cuda or uniforms.numel() < rows
            or not uniforms.is_contiguous()):
        raise ValueError("uniforms must be a contiguous float32 CUDA tensor with one value per row")
    n_prev, prev_stride, prev_ptr = 0, 0, None
    if prev_tokens is not None and prev_tokens.numel() > 0:
        # token ids are u32 (tokenizer.zig:5): int32 / uint32 storage, on the device
        if not prev_tokens.is_cuda or prev_tokens.dtype not in (torch.int32, getattr(torch, "uint32", torch.int32)):
            raise ValueError("prev_tokens must be an int32 or uint32 CUDA tensor")
        if prev_tokens.dim() not in (1, 2) or prev_tokens.stride(-1) != 1:
            raise ValueError("prev_tokens must be 1-D or 2-D with contiguous rows")
        if prev_tokens.dim() == 1:
            n_prev, prev_stride = prev_tokens.shape[0], 0
        else:
            if prev_tokens.shape[0] != rows:
                raise ValueError("2-D prev_tokens needs one history row per logit row")
            n_prev, prev_stride = prev_tokens.shape[1], prev_tokens.stride(0)
        prev_ptr = prev_tokens.data_ptr()
    if out is None:
        tokens = torch.empty(rows, dtype=torch.int32, device=dev)
        consumed = torch.empty(rows, dtype=torch.uint8, device=dev)
    else:
        tokens, consumed = out
    res = SampleResult(tokens, consumed)
    ex = None
    if kept_cap > 0 or stats or path:
        ex = CExtras()
        if path:
            res.row_path = torch.empty(rows, dtype=torch.int32, device=dev)
            ex.d_row_path = res.row_path.data_ptr()
        res.kept_count = torch.empty(rows, dtype=torch.int32, device=dev)
        ex.d_kept_count = res.kept_count.data_ptr()
        if kept_cap > 0:
            res.kept_ids = torch.full((rows, kept_cap), -1, dtype=torch.int32, device=dev)
            ex.d_kept_ids = res.kept_ids.data_ptr()
            if probs:
                res.kept_probs = torch.full((rows, kept_cap), float("nan"), dtype=torch.float32, device=dev)
                ex.d_kept_probs = res.kept_probs.data_ptr()
            ex.kept_cap = kept_cap
        if stats:
            res.row_stats = torch.zeros((rows, 4), dtype=torch.float32, device=dev)
            ex.d_row_stats = res.row_stats.data_ptr()
    c = cfg.to_c()
    need = int(_lib().llz_sample_workspace_bytes(rows, vocab, C.byref(c), n_prev))
    if workspace is None:
        workspace = torch.empty(max(need, 1), dtype=torch.uint8, device=dev)
    rc = _lib().llz_sample_rows(
        logits.data_ptr(), logits.stride(0), rows, vocab, C.byref(c), _post_ref(post), prev_ptr, n_prev,
        prev_stride,
        uniforms.data_ptr(), tokens.data_ptr(), consumed.data_ptr(),
        C.byref(ex) if ex is not None else None, workspace.data_ptr(), workspace.numel(),
        _stream_ptr(stream))
    _check(rc, "llz_sample_rows")
    return res


class PreparedCall:
    """llz_sample_rows for a fixed shape and configuration with its outputs
    and workspace allocated once (serving loops, benchmarks): each call runs
    the C entry point on the given rows and uniforms and fills the same
    output tensors, with no allocation.  kept_cap > 0 asks for the kept ids
    (and with probs their probabilities); stats for the row statistics; path
    for the path bits.  A call asking for neither probabilities nor row
    statistics may finish rows without the exact normaliser."""

    def __init__(self, rows: int, vocab: int, cfg: SamplerConfig, device, *, kept_cap: int = 0,
                 probs: bool = False, stats: bool = False, path: bool = False, stream=None,
                 post: Optional[LogitPost] = None, prev_tokens=None):
        torch = _torch()
        self.rows, self.vocab = rows, vocab
        self._c = cfg.to_c()
        self._stream = _stream_ptr(stream)
        self._post = post.to_c() if post is not None else None
        # the repetition history: a [rows, n_prev] int32 device tensor, fixed for every call
        self._prev = prev_tokens
        self._n_prev = int(prev_tokens.shape[1]) if prev_tokens is not None else 0
        self.result = SampleResult(torch.empty(rows, dtype=torch.int32, device=device),
                                   torch.empty(rows, dtype=torch.uint8, device=device))
        self._ex = None
        if kept_cap > 0 or stats or path:
            ex = CExtras()
            r = self.result
            r.kept_count = torch.empty(rows, dtype=torch.int32, device=device)
            ex.d_kept_count = r.kept_count.data_ptr()
            if kept_cap > 0:
                r.kept_ids = torch.full((rows, kept_cap), -1, dtype=torch.int32, device=device)
                ex.d_kept_ids = r.kept_ids.data_ptr()
                if probs:
                    r.kept_probs = torch.full((rows, kept_cap), float("nan"), dtype=torch.float32, device=device)
                    ex.d_kept_probs = r.kept_probs.data_ptr()
                ex.kept_cap = kept_cap
            if stats:
                r.row_stats = torch.zeros((rows, 4), dtype=torch.float32, device=device)
                ex.d_row_stats = r.row_stats.data_ptr()
            if path:
                r.row_path = torch.empty(rows, dtype=torch.int32, device=device)
                ex.d_row_path = r.row_path.data_ptr()
            self._ex = ex
        need = int(_lib().llz_sample_workspace_bytes(rows, vocab, C.byref(self._c), self._n_prev))
        self.workspace = torch.empty(max(need, 1), dtype=torch.uint8, device=device)

    def __call__(self, logits, uniforms) -> SampleResult:
        if tuple(logits.shape) != (self.rows, self.vocab) or logits.stride(1) != 1:
            raise ValueError("logits must have the prepared shape with contiguous rows")
        r = self.result
        prev = self._prev
        rc = _lib().llz_sample_rows(
            logits.data_ptr(), logits.stride(0), self.rows, self.vocab, C.byref(self._c),
            C.byref(self._post) if self._post is not None else None,
            prev.data_ptr() if prev is not None else None, self._n_prev, prev.stride(0) if prev is not None else 0,
            uniforms.data_ptr(), r.tokens.data_ptr(), r.consumed.data_ptr(),
            C.byref(self._ex) if self._ex is not None else None, self.workspace.data_ptr(), self.workspace.numel(),
            self._stream)
        _check(rc, "llz_sample_rows")
        return r


def argmax_rows(logits, post: Optional[LogitPost] = None, stream=None):
    """sampleArgmax per row (sampler.zig:31-41) of the post-processed logits
    (main.zig:653-666) on a 2-D float32 CUDA tensor."""
    torch = _torch()
    if not (logits.is_cuda and logits.dtype == torch.float32 and logits.dim() == 2 and logits.stride(1) == 1):
        raise ValueError("logits must be a 2-D float32 CUDA tensor with contiguous rows")
    rows, vocab = logits.shape
    tokens = torch.empty(rows, dtype=torch.int32, device=logits.device)
    rc = _lib().llz_argmax_rows(logits.data_ptr(), logits.stride(0), rows, vocab, _post_ref(post),
                                tokens.data_ptr(), _stream_ptr(stream))
    _check(rc, "llz_argmax_rows")
    return tokens


def debug_math(x, extra: bool = False):
    """Device exp/log (and with extra, expm1/tanh) of a float32 CUDA tensor
    (parity tests of the math)."""
    torch = _torch()
    e = torch.empty_like(x)
    lg = torch.empty_like(x)
    em1 = torch.empty_like(x) if extra else None
    th = torch.empty_like(x) if extra else None
    rc = _lib().llz_debug_math(x.data_ptr(), e.data_ptr(), lg.data_ptr(),
                               em1.data_ptr() if extra else None, th.data_ptr() if extra else None,
                               x.numel(), _stream_ptr(None))
    _check(rc, "llz_debug_math")
    return (e, lg, em1, th) if extra else (e, lg)


def debug_hw_error(op: int, first_bits: int, count: int) -> float:
    """Largest relative error, in units of 2^-23, of the hardware exp2 (op 0),
    log2 (op 1) or reciprocal (op 2) over `count` float bit patterns from
    `first_bits`; op 3: the log2's error relative to max(1, |log2 x|)."""
    torch = _torch()
    out = torch.zeros(1, dtype=torch.int32, device="cuda")
    rc = _lib().llz_debug_hw_error(op, first_bits, count, out.data_ptr(), _stream_ptr(None))
    _check(rc, "llz_debug_hw_error")
    return float(int(out.cpu().numpy().view("uint32")[0])) / 2.0 ** 20


def debug_set_queue_cap(cap: int) -> None:
    """The single pass's special-queue chunk for following calls (0: the
    kernel's own); a test hook, results do not depend on it."""
    _check(_lib().llz_debug_set_queue_cap(int(cap)), "llz_debug_set_queue_cap")


def debug_set_split(mode) -> None:
    """Split rows for following calls (token-only calls of at most 64 plain
    rows read each row with several workgroups, one chunk of 2048 nv logits
    each): True or 1 turns them off, False or 0 restores the library's
    choice, 2, 4 or 8 asks for nv at least that.  A test hook; results do
    not depend on it."""
    _check(_lib().llz_debug_set_split(int(mode)), "llz_debug_set_split")


def set_kernel_events(begin=None, end=None) -> None:
    """Record torch.cuda.Event objects around the sampling kernel of every
    following sample_rows call (None, None clears)."""
    b = C.c_void_p(begin.cuda_event) if begin is not None else None
    e = C.c_void_p(end.cuda_event) if end is not None else None
    _check(_lib().llz_debug_kernel_events(b, e), "llz_debug_kernel_events")


class Sampler:
    """Sampler.init / Sampler.sample (src/sampler.zig:15-28) on one GPU."""

    def __init__(self, cfg: SamplerConfig, device: int = 0):
        self.cfg = cfg
        self._h = C.c_void_p()
        _check(_lib().llz_sampler_create(C.byref(cfg.to_c()), device, C.byref(self._h)),
               "llz_sampler_create")

    def sample(self, logits, prev_tokens=()) -> int:
        """logits: host numpy float32 [n] or a float32 CUDA tensor [n]."""
        prev = np.ascontiguousarray(np.asarray(prev_tokens, dtype=np.uint32))
        if isinstance(logits, np.ndarray):
            x = np.ascontiguousarray(logits, dtype=np.float32)
            ptr, n = x.ctypes.data, x.shape[0]
        else:
            ptr, n = logits.data_ptr(), logits.numel()
        tok = C.c_uint32()
        rc = _lib().llz_sampler_sample(self._h, ptr, n, prev.ctypes.data_as(C.POINTER(C.c_uint32)),
                                       prev.shape[0], C.byref(tok))
        _check(rc, "llz_sampler_sample")
        return int(tok.value)

    def sample_uniform(self, logits, u: float, prev_tokens=()) -> Tuple[int, bool]:
        """One row with the caller's uniform: (token, consumed-draw flag)."""
        prev = np.ascontiguousarray(np.asarray(prev_tokens, dtype=np.uint32))
        if isinstance(logits, np.ndarray):
            x = np.ascontiguousarray(logits, dtype=np.float32)
            ptr, n = x.ctypes.data, x.shape[0]
        else:
            ptr, n = logits.data_ptr(), logits.numel()
        tok, con = C.c_uint32(), C.c_uint8()
        rc = _lib().llz_sampler_sample_uniform(self._h, ptr, n, prev.ctypes.data_as(C.POINTER(C.c_uint32)),
                                               prev.shape[0], C.c_float(u), C.byref(tok), C.byref(con))
        _check(rc, "llz_sampler_sample_uniform")
        return int(tok.value), bool(con.value)

    def sample_config(self, cfg: SamplerConfig, logits, u: float, prev_tokens=()) -> Tuple[int, bool]:
        """One row with the caller's configuration and uniform (the handle's own
        configuration is not used): (token, consumed-draw flag)."""
        prev = np.ascontiguousarray(np.asarray(prev_tokens, dtype=np.uint32))
        x = np.ascontiguousarray(logits, dtype=np.float32)
        c = cfg.to_c()
        tok, con = C.c_uint32(), C.c_uint8()
        rc = _lib().llz_sampler_sample_config(self._h, C.byref(c), x.ctypes.data, x.shape[0],
                                              prev.ctypes.data_as(C.POINTER(C.c_uint32)), prev.shape[0],
                                              C.c_float(u), C.byref(tok), C.byref(con))
        _check(rc, "llz_sampler_sample_config")
        return int(tok.value), bool(con.value)

    @property
    def state(self) -> Tuple[int, int, int, int]:
        st = (C.c_uint64 * 4)()
        _lib().llz_sampler_get_state(self._h, st)
        return tuple(int(v) for v in st)

    @state.setter
    def state(self, value) -> None:
        st = (C.c_uint64 * 4)(*[int(v) for v in value])
        _lib().llz_sampler_set_state(self._h, st)

    def close(self) -> None:
        if self._h:
            _lib().llz_sampler_destroy(self._h)
            self._h = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:  # noqa: BLE001 - interpreter shutdown
            pass


def sample_argmax(logits) -> int:
    """sampleArgmax (sampler.zig:31-41) of one row (host array or CUDA tensor)."""
    torch = _torch()
    if isinstance(logits, np.ndarray):
        t = torch.from_numpy(np.ascontiguousarray(logits, dtype=np.float32)).cuda()
    else:
        t = logits
    return int(argmax_rows(t.view(1, -1))[0].item())
