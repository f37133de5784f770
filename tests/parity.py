"""Parity accounting between the device library and the oracle.

Rules (stated once, used by every GPU test):
  * greedy ids, argmax fall-backs, outcome codes and top-k id sets: bit-exact;
  * post-filter probabilities: within 1e-5 relative on entries above 1e-30
    (fp32 output vs fp64 oracle), identical support;
  * sampled ids: equal, except boundary cases -- the oracle's u lies within
    1e-6 of a CDF step, a top-p running sum lies within 1e-6 of p, or tied
    probabilities straddle the top-p cut.  Boundary cases are counted; the
    caller bounds their rate.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

from oracle import sampler_ref as R

PROB_RTOL = 1e-5
PROB_FLOOR = 1e-30
BOUNDARY = 1e-6


@dataclass
class Tally:
    rows: int = 0
    draws: int = 0
    boundary: int = 0
    mismatches: list = field(default_factory=list)

    def merge(self, o: "Tally") -> None:
        self.rows += o.rows
        self.draws += o.draws
        self.boundary += o.boundary
        self.mismatches += o.mismatches


def is_boundary(res: R.RowResult) -> bool:
    d = res.diag
    return (d.get("draw_margin", 1.0) < BOUNDARY or d.get("top_p_margin", 1.0) < BOUNDARY or
            d.get("typical_margin", 1.0) < BOUNDARY or d.get("top_p_tie_straddle", False) or
            d.get("typical_tie_straddle", False))


def compare_rows(ids, status, probs, oracle_rows: list, label: str = "") -> Tally:
    """Compare device outputs with oracle RowResults (oracle run with tie='stable')."""
    t = Tally()
    for b, res in enumerate(oracle_rows):
        t.rows += 1
        got_st = int(status[b]) & 0xFF
        if got_st != res.status:
            t.mismatches.append((label, b, "status", got_st, res.status))
            continue
        if res.status == R.STATUS_ERROR:
            continue
        if res.status == R.STATUS_OK:
            t.draws += 1
        if int(ids[b]) != res.token:
            if res.status == R.STATUS_OK and is_boundary(res):
                t.boundary += 1
            else:
                t.mismatches.append((label, b, "token", int(ids[b]), res.token, res.diag))
            continue
        if probs is not None and res.probs is not None:
            want = res.probs
            got = probs[b].astype(np.float64)
            if not np.array_equal(want > 0, got > 0):
                if not is_boundary(res):
                    t.mismatches.append((label, b, "support",
                                         int((want > 0).sum()), int((got > 0).sum())))
                continue
            big = want > PROB_FLOOR
            rel = np.abs(got[big] - want[big]) / want[big]
            if rel.size and rel.max() > PROB_RTOL:
                t.mismatches.append((label, b, "probs", float(rel.max())))
    return t


def oracle_rows(w, rows=None, keep_probs=True) -> list:
    """Oracle results for the rows of a SampleWorkload (stable tie order)."""
    from oracle.bf16 import bf16_bits_to_f32
    rows = range(w.B) if rows is None else rows
    hl = R.hist_rows_to_lists(w.hist, w.hist_len) if w.hist.size else None
    out = []
    for b in rows:
        x = bf16_bits_to_f32(w.logits[b]) if w.dtype == "bf16" else w.logits[b]
        out.append(R.sample_row(x, w.params[b], None if hl is None else hl[b], float(w.u[b]),
                                tie="stable", keep_probs=keep_probs))
    return out
