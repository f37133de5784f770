"""Rows whose nucleus is deeper than any region (top-p / min-p without top-k,
no penalties) at full vocabulary sizes: the device against the oracle, and
the three-pass deep-nucleus path (CX_ROW_FLAG_DEEP) is the one that decided
them."""
from __future__ import annotations

import sys

import numpy as np
import pytest

from bf16_workloads import counted_bf16, counted_mixed, deep_workload
from chenxing_amd._lib import FLAG_DEEP, sample_host
from oracle_pool import oracle_rows_parallel
from parity import compare_rows

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype,B,V", [("f32", 32, 128256), ("f32", 256, 128256),
                                       ("bf16", 32, 256000)])
def test_deep_nucleus_rows(dtype, B, V):
    w = deep_workload(dtype, B, V, seed=B + V)
    print(f"[gpu] deep-nucleus rows {dtype} B={B} V={V}", flush=True)
    sys.stdout.flush()
    ids, st, _ = sample_host(w.logits, w.params, None, None, w.u, bf16=(dtype == "bf16"))
    pairs = oracle_rows_parallel(w, ties=("spread", "numpy"))
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
    w = counted_bf16()
    B = w.B
    print("[gpu] counted bf16 rows B=8 V=256000", flush=True)
    ids, st, _ = sample_host(w.logits, w.params, None, None, w.u, bf16=True)
    print("    status flags per row:", [hex(int(v) & 0xF00) for v in st], flush=True)
    pairs = oracle_rows_parallel(w, ties=("spread", "numpy"))
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
    w = counted_mixed()
    B, V = w.B, w.V
    print(f"[gpu] counted rows in a mixed bf16 batch B={B} V={V}", flush=True)
    ids, st, _ = sample_host(w.logits, w.params, None, None, w.u, bf16=True)
    pairs = oracle_rows_parallel(w, ties=("spread", "numpy"))
    t = compare_rows(ids, st, None, [p[0] for p in pairs], "counted_mixed[B=1100]",
                     ref_rows=[p[1] for p in pairs])
    assert not t.mismatches, t.mismatches[:5]
    assert t.boundary == 0
