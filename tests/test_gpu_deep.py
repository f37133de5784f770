"""Rows whose nucleus is deeper than any region (top-p / min-p without top-k,
no penalties) at full vocabulary sizes: the device against the oracle, and
the three-pass deep-nucleus path (CX_ROW_FLAG_DEEP) is the one that decided
them."""
from __future__ import annotations

import sys

import numpy as np
import pytest

from chenxing_amd import workloads as W
from chenxing_amd._lib import FLAG_DEEP, sample_host
from chenxing_amd.params import RowParams
from oracle_pool import oracle_rows_parallel
from parity import compare_rows

pytestmark = pytest.mark.gpu


def _deep_workload(dtype: str, B: int, V: int, seed: int) -> W.SampleWorkload:
    rng = np.random.default_rng(seed)
    x = rng.normal(0, 1.5 if dtype == "f32" else 2.0, (B, V)).astype(np.float32)
    for b in range(B):
        x[b, rng.choice(V, 3, replace=False)] += np.float32(8.0)
    prm = [RowParams(temperature=float(rng.uniform(0.8, 1.5)), top_p=float(rng.uniform(0.6, 0.995)),
                     min_p=float(rng.choice([0.0, 0.0, 0.001, 0.02]))) for _ in range(B)]
    logits = W.f32_to_bf16_rne(x) if dtype == "bf16" else x
    return W.SampleWorkload(f"deep_{dtype}", logits, dtype, prm, np.zeros((B, 0), np.int32),
                            np.zeros(B, np.int32), rng.random(B))


@pytest.mark.parametrize("dtype,B,V", [("f32", 32, 128256), ("f32", 256, 128256),
                                       ("bf16", 32, 256000)])
def test_deep_nucleus_rows(dtype, B, V):
    w = _deep_workload(dtype, B, V, seed=B + V)
    print(f"[gpu] deep-nucleus rows {dtype} B={B} V={V}", flush=True)
    sys.stdout.flush()
    ids, st, _ = sample_host(w.logits, w.params, None, None, w.u, bf16=(dtype == "bf16"))
    pairs = oracle_rows_parallel(w, ties=("stable", "numpy"))
    t = compare_rows(ids, st, None, [p[0] for p in pairs], f"deep_{dtype}[B={B}]",
                     ref_rows=[p[1] for p in pairs])
    assert not t.mismatches, t.mismatches[:5]
    assert t.draws == B and t.boundary == 0
    deep = int(np.sum((st & FLAG_DEEP) != 0))
    print(f"    {deep} of {B} rows by the deep-nucleus path", flush=True)
    assert deep >= (9 * B) // 10
