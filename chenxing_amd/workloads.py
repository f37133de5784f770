"""Seeded synthetic inputs for the five sampling workloads.

Each generator is a pure function of its seed.  "N(0, s)" means standard
deviation s.  Sizes:

  small_batch     B=4,    V=32000,  fp32, T 0.8, top-k 50, top-p 0.9, rep 1.1,
                  64-id uniform histories, +8 spikes on 5 ids/row
  nucleus         B=64,   V=128256, fp32 N(0,3) + Zipf-shaped bias
                  -1.5*log(rank+1) over a random id permutation; top-p 0.95
                  (T 1.0) or greedy, no penalties
  full_penalty    B=256,  V=128256, fp32 as small_batch; 2048-id Zipf(1.1)
                  histories (ids >= V become -1); rep 1.1, presence 0.5,
                  frequency 0.3; T 0.7, top-k 40, top-p 0.9
  spec_verify     B=32, gamma=8, V=128256: target N(0,2) [B, 9, V], draft =
                  target[:, :8] + N(0, 0.5); draft ids drawn from the draft
                  softmax; T 1.0 or greedy
  typical         the nucleus logits, T 1.0, typical-p 0.95 (the exact
                  multi-pass path)
  hetero_bf16     B=1024, V=256000, bf16 of N(0,2) + 10 on 3 ids/row; per-row
                  T ~ U[0.3, 1.5], top-k in {0, 20, 100, 1000},
                  top-p ~ U[0.5, 1.0], 25% of rows greedy
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

from .params import RowParams


@dataclass
class SampleWorkload:
    name: str
    logits: np.ndarray                 # [B, V] fp32, or uint16 bf16 bits
    dtype: str                         # "f32" | "bf16"
    params: list                       # [B] RowParams
    hist: np.ndarray                   # [B, H] int32 (H may be 0)
    hist_len: np.ndarray               # [B] int32
    u: np.ndarray                      # [B] fp64 uniforms
    meta: dict = field(default_factory=dict)

    @property
    def B(self) -> int:
        return self.logits.shape[0]

    @property
    def V(self) -> int:
        return self.logits.shape[1]


@dataclass
class VerifyWorkload:
    name: str
    target: np.ndarray                 # [B, gamma+1, V] fp32
    draft: np.ndarray                  # [B, gamma, V] fp32
    draft_ids: np.ndarray              # [B, gamma] int32
    u: np.ndarray                      # [B, gamma+1] fp64
    temperature: np.ndarray            # [B] fp32 (0 = greedy)


def _normal_f32(rng: np.random.Generator, shape, std: float) -> np.ndarray:
    x = rng.standard_normal(shape, dtype=np.float32)
    x *= np.float32(std)
    return x


def _spike(rng: np.random.Generator, x: np.ndarray, n: int, amount: float) -> None:
    V = x.shape[1]
    for b in range(x.shape[0]):
        x[b, rng.choice(V, n, replace=False)] += np.float32(amount)


def small_batch(seed: int = 0, B: int = 4, V: int = 32000) -> SampleWorkload:
    rng = np.random.default_rng(seed)
    x = _normal_f32(rng, (B, V), 2.0)
    _spike(rng, x, 5, 8.0)
    hist = rng.integers(0, V, (B, 64)).astype(np.int32)
    prm = RowParams(temperature=0.8, top_k=50, top_p=0.9, repetition_penalty=1.1)
    u = np.random.default_rng(seed).random(B)
    return SampleWorkload("small_batch", x, "f32", [prm] * B, hist,
                          np.full(B, 64, np.int32), u)


def nucleus(seed: int = 0, B: int = 64, V: int = 128256, greedy: bool = False) -> SampleWorkload:
    rng = np.random.default_rng(seed)
    x = _normal_f32(rng, (B, V), 3.0)
    bias = (-1.5 * np.log(np.arange(V, dtype=np.float64) + 1.0)).astype(np.float32)
    for b in range(B):
        x[b, rng.permutation(V)] += bias
    prm = RowParams(temperature=0.0 if greedy else 1.0, top_p=0.95)
    u = np.random.default_rng(seed + 1).random(B)
    return SampleWorkload("nucleus_greedy" if greedy else "nucleus", x, "f32", [prm] * B,
                          np.zeros((B, 0), np.int32), np.zeros(B, np.int32), u)


def typical(seed: int = 0, B: int = 64, V: int = 128256, typical_p: float = 0.95) -> SampleWorkload:
    """The nucleus logits with typical-p sampling (sampler.py:95-105): T 1.0,
    typical_p 0.95, no other filter, no penalties."""
    w = nucleus(seed, B, V)
    prm = RowParams(temperature=1.0, typical_p=typical_p)
    return SampleWorkload("typical", w.logits, "f32", [prm] * B, w.hist, w.hist_len, w.u)


def zipf_history(rng: np.random.Generator, B: int, H: int, V: int) -> np.ndarray:
    z = rng.zipf(1.1, (B, H))
    ids = z - 1
    return np.where(ids < V, ids, -1).astype(np.int32)


def full_penalty(seed: int = 0, B: int = 256, V: int = 128256, H: int = 2048) -> SampleWorkload:
    rng = np.random.default_rng(seed)
    x = _normal_f32(rng, (B, V), 2.0)
    _spike(rng, x, 5, 8.0)
    hist = zipf_history(rng, B, H, V)
    prm = RowParams(temperature=0.7, top_k=40, top_p=0.9, repetition_penalty=1.1,
                    presence_penalty=0.5, frequency_penalty=0.3)
    u = np.random.default_rng(seed + 1).random(B)
    return SampleWorkload("full_penalty", x, "f32", [prm] * B, hist,
                          np.full(B, H, np.int32), u)


def spec_verify(seed: int = 0, B: int = 32, gamma: int = 8, V: int = 128256,
                greedy: bool = False) -> VerifyWorkload:
    rng = np.random.default_rng(seed)
    tgt = _normal_f32(rng, (B, gamma + 1, V), 2.0)
    drf = tgt[:, :gamma] + _normal_f32(rng, (B, gamma, V), 0.5)
    ids = np.empty((B, gamma), np.int32)
    ud = rng.random((B, gamma))
    for b in range(B):
        for i in range(gamma):
            z = drf[b, i].astype(np.float64)
            e = np.exp(z - z.max())
            cdf = np.cumsum(e)
            cdf /= cdf[-1]
            ids[b, i] = min(int(np.searchsorted(cdf, ud[b, i], side="right")), V - 1)
    u = rng.random((B, gamma + 1))
    T = np.full(B, 0.0 if greedy else 1.0, np.float32)
    return VerifyWorkload("spec_verify_greedy" if greedy else "spec_verify",
                          tgt, drf, ids, u, T)


def hetero_bf16(seed: int = 0, B: int = 1024, V: int = 256000) -> SampleWorkload:
    """Logits are returned as bf16 bit patterns (uint16), rounded to nearest even."""
    rng = np.random.default_rng(seed)
    bits = np.empty((B, V), np.uint16)
    for b in range(B):
        row = _normal_f32(rng, (1, V), 2.0)
        row[0, rng.choice(V, 3, replace=False)] += np.float32(10.0)
        bits[b] = f32_to_bf16_rne(row[0])
    prms = []
    for b in range(B):
        if rng.random() < 0.25:
            prms.append(RowParams(temperature=0.0))
            continue
        prms.append(RowParams(temperature=float(rng.uniform(0.3, 1.5)),
                              top_k=int(rng.choice([0, 20, 100, 1000])),
                              top_p=float(rng.uniform(0.5, 1.0))))
    u = np.random.default_rng(seed + 1).random(B)
    return SampleWorkload("hetero_bf16", bits, "bf16", prms, np.zeros((B, 0), np.int32),
                          np.zeros(B, np.int32), u)


def f32_to_bf16_rne(x: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bits, round to nearest even (finite inputs)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def algorithmic_bytes(w: SampleWorkload) -> int:
    """One read of every logit, the history ids actually used, the per-row
    parameter block, the uniform, the output id and the row status."""
    el = 2 if w.dtype == "bf16" else 4
    hist = int(np.minimum(w.hist_len, w.hist.shape[1]).sum()) * 4 if w.hist.size else 0
    return w.B * w.V * el + hist + w.B * (64 + 8 + 4 + 4 + (4 if w.hist.size else 0))


def verify_algorithmic_bytes(w: VerifyWorkload) -> int:
    B, g1, V = w.target.shape
    gamma = g1 - 1
    greedy = bool(np.all(w.temperature == 0))
    rows = B * g1 if greedy else B * (2 * gamma + 1)
    return rows * V * 4 + B * gamma * 4 + B * (gamma + 1) * 8 + B * 4 + B * 12
