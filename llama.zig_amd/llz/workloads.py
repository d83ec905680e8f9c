"""Synthetic logit workloads for the sampling chain.

Each workload is one of the five configurations the headline metric and the
parity suite are quoted on, plus the headline batch itself.  Logits are drawn
row by row from ``numpy.random.default_rng([seed, row])`` so that any prefix
of rows can be regenerated on its own (tests use the first few rows of the
large configurations).  Sampling parameters mirror ``SamplerConfig``
(src/sampler.zig:4-13 of the reference).

Readings of the configuration text that the generator pins:

* ``N(0, s)`` means standard deviation ``s``.
* A "Zipf(s=1.1) offset on a random permutation of ranks" is the log-prob
  offset ``-1.1 * ln(rank)`` with ``rank`` a random permutation of 1..V.
* "Boosted" tokens are distinct positions chosen uniformly at random.
"""
from __future__ import annotations

import dataclasses
from typing import Callable, Dict

import numpy as np


@dataclasses.dataclass(frozen=True)
class Params:
    """Mirror of SamplerConfig (src/sampler.zig:4-13) minus the seed."""

    temperature: float = 0.8
    top_k: int = 0
    top_p: float = 0.9
    min_p: float = 0.0
    typical_p: float = 1.0
    repetition_window: int = 32
    repetition_penalty: float = 1.1


@dataclasses.dataclass(frozen=True)
class Workload:
    name: str
    rows: int
    vocab: int
    params: Params
    data_seed: int
    uniform_seed: int
    gen_row: Callable[[np.random.Generator, int, int], np.ndarray]
    text: str

    def logits(self, rows: int | None = None, first_row: int = 0) -> np.ndarray:
        """float32 [rows, vocab] logits for rows first_row .. first_row+rows-1."""
        rows = self.rows if rows is None else rows
        out = np.empty((rows, self.vocab), dtype=np.float32)
        for r in range(rows):
            g = np.random.default_rng([self.data_seed, first_row + r])
            out[r] = self.gen_row(g, self.vocab, first_row + r)
        return out


# Repetition penalty is disabled in every configuration, as in the reference's
# decode loop (src/main.zig:508-517).
_NO_REP = dict(repetition_window=0, repetition_penalty=1.0)


def _c1_row(g: np.random.Generator, v: int, row: int) -> np.ndarray:
    x = g.normal(0.0, 2.0, v).astype(np.float32)
    hot = g.choice(v, 8, replace=False)
    x[hot] += np.float32(12.0)
    return x


def _zipf_row(g: np.random.Generator, v: int, row: int) -> np.ndarray:
    base = g.normal(0.0, 2.5, v)
    rank = g.permutation(v) + 1
    return (base - 1.1 * np.log(rank)).astype(np.float32)


def _c3_row(g: np.random.Generator, v: int, row: int) -> np.ndarray:
    x = g.gumbel(0.0, 1.5, v).astype(np.float32)
    hot = g.choice(v, 20, replace=False)
    x[hot] += np.float32(8.0)
    return x


def _c4_row(g: np.random.Generator, v: int, row: int) -> np.ndarray:
    return g.normal(0.0, 0.3, v).astype(np.float32)


def _c5_row(g: np.random.Generator, v: int, row: int) -> np.ndarray:
    x = g.normal(0.0, 2.0, v).astype(np.float32)
    if row % 2 == 1:
        x[int(g.integers(0, v))] += np.float32(20.0)
    return x


WORKLOADS: Dict[str, Workload] = {
    "c1": Workload(
        "c1", 1, 128256,
        Params(temperature=0.8, top_k=0, top_p=0.9, min_p=0.0, typical_p=1.0, **_NO_REP),
        # sampler seed 0: Sampler.init seeds DefaultPrng with 0xDEADBEEF
        # instead (sampler.zig:22)
        data_seed=0, uniform_seed=0xDEADBEEF, gen_row=_c1_row,
        text="1 x 128256, N(0,2) + 8 tokens at +12; T 0.8, top-p 0.9 (sampler.zig defaults)"),
    "c2": Workload(
        "c2", 64, 128256,
        Params(temperature=1.0, top_k=40, top_p=0.95, min_p=0.05, typical_p=1.0, **_NO_REP),
        data_seed=2, uniform_seed=2, gen_row=_zipf_row,
        text="64 x 128256, N(0,2.5) - 1.1 ln(rank); T 1.0, k 40, p 0.95, min-p 0.05"),
    "c3": Workload(
        "c3", 256, 151936,
        Params(temperature=0.7, top_k=0, top_p=1.0, min_p=0.0, typical_p=0.95, **_NO_REP),
        data_seed=3, uniform_seed=3, gen_row=_c3_row,
        text="256 x 151936, Gumbel(0,1.5) + 20 tokens at +8; T 0.7, typical 0.95"),
    "c4": Workload(
        "c4", 1024, 256000,
        Params(temperature=1.2, top_k=0, top_p=0.9, min_p=0.0, typical_p=1.0, **_NO_REP),
        data_seed=4, uniform_seed=4, gen_row=_c4_row,
        text="1024 x 256000, N(0,0.3); T 1.2, top-p 0.9"),
    "c5": Workload(
        "c5", 4096, 128256,
        Params(temperature=0.8, top_k=50, top_p=0.9, min_p=0.02, typical_p=0.98, **_NO_REP),
        data_seed=5, uniform_seed=5, gen_row=_c5_row,
        text="4096 x 128256, N(0,2) / N(0,2)+20 peak; T 0.8, k 50, p 0.9, min-p 0.02, typical 0.98"),
    # The headline metric's batch: 256 x 128256 with top-k/top-p/min-p, using
    # configuration 2's logit family and chain.
    "headline": Workload(
        "headline", 256, 128256,
        Params(temperature=1.0, top_k=40, top_p=0.95, min_p=0.05, typical_p=1.0, **_NO_REP),
        data_seed=7, uniform_seed=7, gen_row=_zipf_row,
        text="256 x 128256, configuration 2's logits and chain (T 1.0, k 40, p 0.95, min-p 0.05)"),
    # The headline's logits with the reference's default chain (SamplerConfig
    # defaults, sampler.zig:4-13, without the repetition penalty).
    "headline-default": Workload(
        "headline-default", 256, 128256,
        Params(temperature=0.8, top_k=0, top_p=0.9, min_p=0.0, typical_p=1.0, **_NO_REP),
        data_seed=7, uniform_seed=7, gen_row=_zipf_row,
        text="256 x 128256, the headline's logits with the reference's default chain (T 0.8, top-p 0.9)"),
}


def algorithmic_bytes(rows: int, vocab: int) -> int:
    """One read of every logit, one uniform in, one token out per row."""
    return rows * (4 * vocab + 4 + 4)
