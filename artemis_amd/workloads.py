"""Synthetic inputs for the five benchmark configurations (deterministic from a seed).

Logits are N(0, 2.5^2) in f64 from numpy's PCG64, plus the configuration's bump, rounded once to
f32. A Zipf(s) bump adds A * (r + 1)^-s to the id at rank r of a seeded permutation (A = 8). A
Zipf(s) history draws ids by inverse CDF over the same ranks and maps them through the same
permutation, so frequently repeated ids are the bumped ones. `digest` hashes a workload's arrays
so a run can say which inputs it saw.
"""
from __future__ import annotations

import hashlib
from dataclasses import dataclass, field
from typing import List, Optional

import numpy as np

VOCAB = 248_320
SIGMA = 2.5
ZIPF_AMPLITUDE = 8.0


@dataclass
class Row:
    temp: float
    top_k: int
    top_p: float
    min_p: float
    presence: float = 0.0
    frequency: float = 0.0
    repetition: float = 1.0


@dataclass
class Workload:
    name: str
    logits: np.ndarray                 # [rows, vocab] f32 (or [1, vocab] shared by every draw)
    params: List[Row]
    seeds: List[int]
    histories: List[np.ndarray] = field(default_factory=list)  # per row, u32 ids (may be empty)
    drafts: Optional[np.ndarray] = None  # config 4
    shared_row: bool = False           # every draw reads logits[0]

    def hist_csr(self):
        """(offsets [rows+1], ids) int32 arrays of the per-row histories."""
        hs = self.histories or [np.zeros(0, np.uint32)] * len(self.params)
        off = np.zeros(len(hs) + 1, np.int64)
        for i, h in enumerate(hs):
            off[i + 1] = off[i] + len(h)
        ids = np.concatenate(hs) if off[-1] else np.zeros(0, np.uint32)
        return off.astype(np.int32), ids.astype(np.int32)

    def sha256(self) -> str:
        """SHA-256 of the logits, then each history, then the drafts (u32), as raw bytes."""
        h = hashlib.sha256()
        h.update(np.ascontiguousarray(self.logits).tobytes())
        for x in self.histories:
            h.update(np.ascontiguousarray(x, dtype=np.uint32).tobytes())
        if self.drafts is not None:
            h.update(np.ascontiguousarray(self.drafts, dtype=np.uint32).tobytes())
        return h.hexdigest()

    def digest(self) -> str:
        return self.sha256()[:16]


def _zipf_weights(n: int, s: float) -> np.ndarray:
    return (np.arange(1, n + 1, dtype=np.float64)) ** (-s)


def _bumped_row(rng: np.random.Generator, n: int, s: float):
    perm = rng.permutation(n)
    x = rng.standard_normal(n) * SIGMA
    x[perm] += ZIPF_AMPLITUDE * _zipf_weights(n, s)
    return x.astype(np.float32), perm


def _zipf_history(rng: np.random.Generator, perm: np.ndarray, count: int, s: float) -> np.ndarray:
    cdf = np.cumsum(_zipf_weights(len(perm), s))
    ranks = np.searchsorted(cdf, rng.random(count) * cdf[-1], side="right")
    ranks = np.minimum(ranks, len(perm) - 1)
    return perm[ranks].astype(np.uint32)


def config1(n: int = VOCAB, seed: int = 1) -> Workload:
    """Greedy argmax: N(0, 2.5^2) with one seeded id boosted by +8."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal(n) * SIGMA
    x[rng.integers(n)] += 8.0
    return Workload("greedy", x.astype(np.float32)[None, :], [Row(0.0, 0, 1.0, 0.0)], [0])


def config2(n: int = VOCAB, seed: int = 2, draws: int = 1000) -> Workload:
    """Zipf(1.1) bump; T 0.6, top-k 20, top-p 0.95; seeds 0..draws-1, one draw each."""
    rng = np.random.default_rng(seed)
    x, _ = _bumped_row(rng, n, 1.1)
    return Workload("stochastic", x[None, :], [Row(0.6, 20, 0.95, 0.0)] * draws, list(range(draws)),
                    shared_row=True)


def config3(n: int = VOCAB, seed: int = 3, draws: int = 1, hist: int = 4096) -> Workload:
    """Config 2's distribution plus a Zipf(1.2) history of 4,096 ids; rep 1.05, presence 0.5,
    frequency 0.3; T 0.7, top-k 40, top-p 0.9, min-p 0.05."""
    rng = np.random.default_rng(seed)
    x, perm = _bumped_row(rng, n, 1.1)
    h = _zipf_history(rng, perm, hist, 1.2)
    p = Row(0.7, 40, 0.9, 0.05, presence=0.5, frequency=0.3, repetition=1.05)
    return Workload("penalised", x[None, :], [p] * draws, list(range(draws)), [h] * draws, shared_row=True)


def config4(n: int = VOCAB, seed: int = 4, k: int = 5) -> Workload:
    """k drafts checked against k+1 rows of N(0, 2.5^2) with +6 on one id per row; each draft is,
    with probability 1/2, the argmax of the row that verifies it (draft j <-> row j)."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((k + 1, n)) * SIGMA
    x[np.arange(k + 1), rng.integers(n, size=k + 1)] += 6.0
    x = x.astype(np.float32)
    drafts = rng.integers(n, size=k).astype(np.uint32)
    force = rng.random(k) < 0.5
    for j in range(k):
        if force[j]:
            drafts[j] = int(np.argmax(x[j]))
    return Workload("verify", x, [Row(0.6, 0, 0.95, 0.0)], [1234], drafts=drafts)


def config5(n: int = VOCAB, seed: int = 5, rows: int = 256, hist: int = 2048) -> Workload:
    """Independent rows with their own seed, Zipf(1.1) bump, 2,048-id Zipf(1.2) history and
    parameters: T in [0.3, 1], top-k in {0, 20, 50}, top-p in [0.8, 1], min-p in [0, 0.1];
    repetition 1.05, presence 0.5, frequency 0.3."""
    rng = np.random.default_rng(seed)
    logits = np.empty((rows, n), np.float32)
    params, histories = [], []
    for r in range(rows):
        x, perm = _bumped_row(rng, n, 1.1)
        logits[r] = x
        histories.append(_zipf_history(rng, perm, hist, 1.2))
        params.append(Row(
            temp=float(np.float32(rng.uniform(0.3, 1.0))),
            top_k=int(rng.choice([0, 20, 50])),
            top_p=float(np.float32(rng.uniform(0.8, 1.0))),
            min_p=float(np.float32(rng.uniform(0.0, 0.1))),
            presence=0.5, frequency=0.3, repetition=1.05))
    return Workload("batched", logits, params, [1000 + r for r in range(rows)], histories)
