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


def test_counted_bf16_rows_and_hand_backs():
    """bf16 rows through each branch of the counted deep-nucleus path
    (cx_deep16.hpp): a value repeated 70000 times (its 16-bit counter wraps:
    the row is handed back to the later paths), a mask of 100000 -inf ids
    (counted apart), signed zeros (one value), a nucleus wider than the
    copied window (a second pass over the row) and one through zero (the
    three part tables), and min-p alone."""
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
    w = W.SampleWorkload("counted_bf16", xb, "bf16", prm, np.zeros((B, 0), np.int32),
                         np.zeros(B, np.int32), rng.random(B))
    print("[gpu] counted bf16 rows B=8 V=256000", flush=True)
    ids, st, _ = sample_host(w.logits, w.params, None, None, w.u, bf16=True)
    print("    status flags per row:", [hex(int(v) & 0xF00) for v in st], flush=True)
    pairs = oracle_rows_parallel(w, ties=("stable", "numpy"))
    t = compare_rows(ids, st, None, [p[0] for p in pairs], "counted_bf16[B=8]",
                     ref_rows=[p[1] for p in pairs])
    assert not t.mismatches, t.mismatches[:5]
    assert t.draws == B and t.boundary == 0


def test_counted_rows_in_a_batch_beyond_one_workgroup():
    """A bf16 batch of 1100 single-slice rows (more rows than a workgroup
    has threads, so finish16_kernel's work list is built over two chunks of
    rows), mixing greedy rows, top-k 20 rows (one-wave finish), top-k 100
    rows (regions and the finisher), and top-k 1000 and top-p-only rows
    (streamed for their maximum only, then counted): every row sampled as
    the oracle samples it."""
    rng = np.random.default_rng(91)
    B, V = 1100, 16384
    x = rng.normal(0, 2.0, (B, V)).astype(np.float32)
    x[np.arange(B), rng.integers(0, V, B)] += np.float32(6.0)
    kinds = [dict(temperature=0.0), dict(temperature=0.8, top_k=20, top_p=0.9),
             dict(temperature=1.0, top_k=100, top_p=0.95), dict(temperature=1.1, top_k=1000, top_p=0.9),
             dict(temperature=1.3, top_p=0.9), dict(temperature=0.9, top_p=0.97, min_p=0.01)]
    prm = [RowParams(**kinds[int(k)]) for k in rng.integers(0, len(kinds), B)]
    w = W.SampleWorkload("counted_mixed", W.f32_to_bf16_rne(x), "bf16", prm,
                         np.zeros((B, 0), np.int32), np.zeros(B, np.int32), rng.random(B))
    print(f"[gpu] counted rows in a mixed bf16 batch B={B} V={V}", flush=True)
    ids, st, _ = sample_host(w.logits, w.params, None, None, w.u, bf16=True)
    pairs = oracle_rows_parallel(w, ties=("stable", "numpy"))
    t = compare_rows(ids, st, None, [p[0] for p in pairs], "counted_mixed[B=1100]",
                     ref_rows=[p[1] for p in pairs])
    assert not t.mismatches, t.mismatches[:5]
    assert t.boundary == 0
