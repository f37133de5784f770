"""Seeded bf16 (and deep fp32) test workloads shared by the GPU parity tests
and by the tie-order measurement (tests/golden/tie_order_rates.py).

bf16 logits tie constantly (256 mantissa values per octave), so these are
the rows where a group of equal probabilities can straddle the top-p cut and
numpy's argsort order (sampler.py:82) decides which of its ids survive.
Each builder is a pure function of its arguments.
"""
from __future__ import annotations

import numpy as np

from chenxing_amd import workloads as W
from chenxing_amd.params import RowParams


def deep_workload(dtype: str, B: int, V: int, seed: int) -> W.SampleWorkload:
    """Top-p / min-p rows without top-k or penalties: nuclei deeper than any
    region."""
    rng = np.random.default_rng(seed)
    x = rng.normal(0, 1.5 if dtype == "f32" else 2.0, (B, V)).astype(np.float32)
    for b in range(B):
        x[b, rng.choice(V, 3, replace=False)] += np.float32(8.0)
    prm = [RowParams(temperature=float(rng.uniform(0.8, 1.5)), top_p=float(rng.uniform(0.6, 0.995)),
                     min_p=float(rng.choice([0.0, 0.0, 0.001, 0.02]))) for _ in range(B)]
    logits = W.f32_to_bf16_rne(x) if dtype == "bf16" else x
    return W.SampleWorkload(f"deep_{dtype}", logits, dtype, prm, np.zeros((B, 0), np.int32),
                            np.zeros(B, np.int32), rng.random(B))


def counted_bf16() -> W.SampleWorkload:
    """Eight V=256000 rows through each branch of the counted deep-nucleus
    path: a value repeated 70000 times, 100000 masked (-inf) ids, signed
    zeros, a nucleus wider than the copied window, one through zero, and
    min-p alone."""
    rng = np.random.default_rng(77)
    B, V = 8, 256000
    x = rng.normal(0, 2.0, (B, V)).astype(np.float32)
    for b in range(B):
        x[b, rng.choice(V, 3, replace=False)] += np.float32(8.0)
    xb = W.f32_to_bf16_rne(x)
    xb[0, rng.choice(V, 70000, replace=False)] = W.f32_to_bf16_rne(np.float32([0.5]))[0]
    xb[1, rng.choice(V, 100000, replace=False)] = 0xFF80
    xb[2, :3000] = 0x0000
    xb[2, 3000:6000] = 0x8000
    prm = [RowParams(temperature=1.0, top_p=0.9), RowParams(temperature=1.0, top_p=0.9),
           RowParams(temperature=2.0, top_p=0.8), RowParams(temperature=3.0, top_p=0.995),
           RowParams(temperature=6.0, top_p=0.999), RowParams(temperature=1.0, top_p=1.0, min_p=0.01),
           RowParams(temperature=0.7, top_p=0.95, min_p=0.001), RowParams(temperature=1.2, top_p=0.6)]
    return W.SampleWorkload("counted_bf16", xb, "bf16", prm, np.zeros((B, 0), np.int32),
                            np.zeros(B, np.int32), rng.random(B))


def counted_mixed() -> W.SampleWorkload:
    """1100 V=16384 bf16 rows mixing greedy, top-k 20, top-k 100, top-k 1000
    and top-p-only rows (more rows than a workgroup has threads)."""
    rng = np.random.default_rng(91)
    B, V = 1100, 16384
    x = rng.normal(0, 2.0, (B, V)).astype(np.float32)
    x[np.arange(B), rng.integers(0, V, B)] += np.float32(6.0)
    kinds = [dict(temperature=0.0), dict(temperature=0.8, top_k=20, top_p=0.9),
             dict(temperature=1.0, top_k=100, top_p=0.95), dict(temperature=1.1, top_k=1000, top_p=0.9),
             dict(temperature=1.3, top_p=0.9), dict(temperature=0.9, top_p=0.97, min_p=0.01)]
    prm = [RowParams(**kinds[int(k)]) for k in rng.integers(0, len(kinds), B)]
    return W.SampleWorkload("counted_mixed", W.f32_to_bf16_rne(x), "bf16", prm,
                            np.zeros((B, 0), np.int32), np.zeros(B, np.int32), rng.random(B))


# label (as the GPU tests report it) -> builder, for every bf16 workload whose
# draws are compared with numpy's tie order
TIE_WORKLOADS = {
    "hetero_bf16": lambda: W.hetero_bf16(),
    "hetero_bf16[B=96]+probs": lambda: W.hetero_bf16(B=96),
    "deep_bf16[B=32]": lambda: deep_workload("bf16", 32, 256000, seed=32 + 256000),
    "counted_bf16[B=8]": counted_bf16,
    "counted_mixed[B=1100]": counted_mixed,
}
