"""Seeded synthetic sampling workloads at the Qwen3.5-family vocabulary size (V = 248,320).

Five workloads, each fully determined by its seed (numpy PCG64 streams; normals drawn in float64 and rounded
once to float32), so that the CPU checker and the GPU path read identical bytes:

* ``greedy``    — 1 row of N(0,1) logits with a planted maximum 6.0 at a seeded id plus seeded exact ties at
                  6.0 (some ids below, some above it): greedy decoding (temperature 0) must return the lowest.
* ``topk_topp`` — 1 row of N(0,1.5) plus 50 distinct "head" ids at N(8,2); temperature 0.7, top-k 20,
                  top-p 0.8, one uniform.
* ``penalties`` — the ``topk_topp`` logits with a 4,096-id history drawn Zipf(s=1.1) over the vocabulary
                  (ranks mapped to ids by a seeded permutation); repetition 1.1, presence 0.5, frequency 0.2,
                  then temperature 1.0, top-k 40, top-p 0.95, min-p 0.05.
* ``verify``    — the speculative-decoding verify step: 4 rows (1 main + 3 draft positions), each N(0,1.5) with
                  its own 50 heads; draft i+1 is drawn from row i's head set with probability 0.8, otherwise
                  uniformly over the vocabulary; temperature 0.6, top-k 20, top-p 0.95, 4 uniforms.
* ``batched``   — 64 independent rows distributed as in ``verify``, per-row histories of 16,384 Zipf(1.1) ids,
                  the ``penalties`` penalty settings, top-k 64, top-p 0.9, temperature 1.0, 64 uniforms.

Sampling parameters follow klein's SamplerParams (src/sampler.h:13-22); fields not named keep its defaults.
"""
from __future__ import annotations

import hashlib
from dataclasses import dataclass, field, asdict

import numpy as np

VOCAB = 248_320


@dataclass
class Params:
    """klein's SamplerParams (src/sampler.h:13-22), same field names and defaults."""
    temperature: float = 1.0
    top_k: int = 20
    top_p: float = 0.95
    min_p: float = 0.0
    presence_penalty: float = 0.0
    frequency_penalty: float = 0.0
    repetition_penalty: float = 1.0
    seed: int = 0

    def as_dict(self):
        return asdict(self)


@dataclass
class Workload:
    name: str
    logits: np.ndarray                      # float32 [rows, V], C-contiguous
    params: Params
    u: np.ndarray                           # float64 [rows], the draw's uniform per row
    histories: list = field(default_factory=list)   # per-row int32 arrays of history token ids ([] = none)
    drafts: np.ndarray | None = None        # int32 [rows-1] for the verify step
    expected_greedy: int | None = None      # closed-form answer of the greedy workload

    @property
    def rows(self) -> int:
        return self.logits.shape[0]

    @property
    def vocab(self) -> int:
        return self.logits.shape[1]

    def digest(self) -> str:
        """sha256 of the logits bytes (guards the generator in the committed fixtures)."""
        return hashlib.sha256(self.logits.tobytes()).hexdigest()


def _rng(seed: int, purpose: int) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64([seed, purpose]))


def _normal_f32(rng, n, mean, std):
    return (rng.standard_normal(n) * std + mean).astype(np.float32)


def _heads(rng, row: np.ndarray, n_heads=50, mean=8.0, std=2.0):
    ids = rng.choice(row.shape[0], size=n_heads, replace=False).astype(np.int64)
    row[ids] = _normal_f32(rng, n_heads, mean, std)
    return ids


_zipf_cache: dict = {}


def zipf_ids(rng, n: int, vocab: int, s: float = 1.1, perm: np.ndarray | None = None) -> np.ndarray:
    """n ids from a bounded Zipf(s) over ranks 1..vocab (inverse CDF over the harmonic table), ranks mapped to
    ids through `perm` (a permutation of the vocabulary)."""
    key = (vocab, s)
    if key not in _zipf_cache:
        w = np.arange(1, vocab + 1, dtype=np.float64) ** (-s)
        c = np.cumsum(w)
        _zipf_cache[key] = c / c[-1]
    cdf = _zipf_cache[key]
    ranks = np.searchsorted(cdf, rng.random(n), side="right")
    ranks = np.minimum(ranks, vocab - 1)
    if perm is None:
        perm = np.arange(vocab)
    return perm[ranks].astype(np.int32)


def uniforms(rng, n: int) -> np.ndarray:
    """53-bit uniforms in [0, 1)."""
    return rng.random(n).astype(np.float64)


def greedy(seed: int = 1, vocab: int = VOCAB, n_ties: int = 4) -> Workload:
    r = _rng(seed, 1)
    row = _normal_f32(r, vocab, 0.0, 1.0)
    row = np.minimum(row, np.float32(5.5))        # keep the background strictly below the planted maximum
    m = int(r.integers(vocab // 4, 3 * vocab // 4))
    row[m] = np.float32(6.0)
    below = r.choice(m, size=n_ties // 2, replace=False)
    above = m + 1 + r.choice(vocab - m - 1, size=n_ties - n_ties // 2, replace=False)
    row[below] = np.float32(6.0)
    row[above] = np.float32(6.0)
    expected = int(min(m, below.min()))
    return Workload("greedy", row[None, :].copy(), Params(temperature=0.0), np.zeros(1), expected_greedy=expected)


def topk_topp(seed: int = 2, vocab: int = VOCAB) -> Workload:
    r = _rng(seed, 2)
    row = _normal_f32(r, vocab, 0.0, 1.5)
    _heads(r, row)
    return Workload("topk_topp", row[None, :].copy(), Params(temperature=0.7, top_k=20, top_p=0.8),
                    uniforms(r, 1))


def penalties(seed: int = 3, vocab: int = VOCAB, n_hist: int = 4096) -> Workload:
    base = topk_topp(seed, vocab)
    r = _rng(seed, 3)
    perm = r.permutation(vocab)
    hist = zipf_ids(r, n_hist, vocab, 1.1, perm)
    p = Params(temperature=1.0, top_k=40, top_p=0.95, min_p=0.05, presence_penalty=0.5, frequency_penalty=0.2,
               repetition_penalty=1.1)
    return Workload("penalties", base.logits, p, uniforms(r, 1), histories=[hist])


def _head_rows(r, rows, vocab):
    logits = np.empty((rows, vocab), dtype=np.float32)
    heads = []
    for i in range(rows):
        logits[i] = _normal_f32(r, vocab, 0.0, 1.5)
        heads.append(_heads(r, logits[i]))
    return logits, heads


def verify(seed: int = 4, vocab: int = VOCAB, rows: int = 4) -> Workload:
    r = _rng(seed, 4)
    logits, heads = _head_rows(r, rows, vocab)
    drafts = np.empty(rows - 1, dtype=np.int32)
    for i in range(rows - 1):
        drafts[i] = heads[i][r.integers(len(heads[i]))] if r.random() < 0.8 else r.integers(vocab)
    return Workload("verify", logits, Params(temperature=0.6, top_k=20, top_p=0.95), uniforms(r, rows),
                    drafts=drafts)


def batched(seed: int = 5, vocab: int = VOCAB, rows: int = 64, n_hist: int = 16384) -> Workload:
    r = _rng(seed, 5)
    logits, _ = _head_rows(r, rows, vocab)
    perm = r.permutation(vocab)
    hist = [zipf_ids(r, n_hist, vocab, 1.1, perm) for _ in range(rows)]
    p = Params(temperature=1.0, top_k=64, top_p=0.9, presence_penalty=0.5, frequency_penalty=0.2,
               repetition_penalty=1.1)
    return Workload("batched", logits, p, uniforms(r, rows), histories=hist)


BUILDERS = {"greedy": greedy, "topk_topp": topk_topp, "penalties": penalties, "verify": verify, "batched": batched}


def counts_of(hist: np.ndarray, vocab: int) -> np.ndarray:
    """Dense per-id history counts (what klein's accept() builds, src/sampler.cpp:15)."""
    return np.bincount(np.asarray(hist, dtype=np.int64), minlength=vocab).astype(np.int32)
