"""Parity accounting between the device library and the oracle.

Rules (stated once, used by every GPU test):
  * greedy ids, argmax fall-backs, outcome codes and top-k id sets: bit-exact;
  * post-filter probabilities: within 1e-5 relative on entries above 1e-30
    (fp32 output vs fp64 oracle), identical support;
  * sampled ids, against the oracle run with the device's documented tie
    rule (``tie="spread"``: of a group of equal probabilities straddling the
    top-p or typical cut, the survivors are spread evenly over the group's
    ids): equal, except margin cases -- the oracle's u lies within 1e-6 of a
    CDF step, or a running sum lies within 1e-6 of p.  Margin cases are
    counted and must stay at or below 1e-4 of the draws.
  * sampled ids, against the oracle run with numpy's own argsort
    (``tie="numpy"``, what the reference computes on this host;
    sampler.py:82,103): every difference must be a tie straddle (tied
    probabilities on both sides of the top-p or typical cut, where numpy's
    unstable sort leaves the order unspecified) or a margin case.  Budgets:
      - margin-case differences: at most 1e-4 of the draws;
      - tie-straddle differences: at most 1e-4 of the draws on every
        workload not listed in tests/golden/tie_order_rates.json (every fp32
        workload: 0 at their sizes); on the bf16 workloads listed there, at
        most the largest number of draws on which two of numpy's own SIMD
        dispatch levels (AVX-512, AVX2, baseline) disagree for the same rows
        -- how often the reference disagrees with itself across hosts.
    The counts per workload are recorded in ``REF_RATES`` and printed at the
    end of the run (tests/conftest.py).
"""
from __future__ import annotations

import json
import os
from dataclasses import dataclass, field

import numpy as np

from oracle import sampler_ref as R

PROB_RTOL = 1e-5
PROB_FLOOR = 1e-30
BOUNDARY = 1e-6
REF_BUDGET = 1e-4          # boundary draws allowed per draw

_RATES_FILE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden",
                           "tie_order_rates.json")


def tie_bounds() -> dict:
    """label -> the most draws on which two numpy dispatch levels disagree
    (tests/golden/tie_order_rates.json, written by tie_order_rates.py)."""
    with open(_RATES_FILE) as f:
        rep = json.load(f)
    return {k: int(v["max_numpy_cross_level"]) for k, v in rep["workloads"].items()}

# label -> dict of reference-order counts, filled by compare_rows(ref_rows=...)
REF_RATES: dict = {}


@dataclass
class Tally:
    rows: int = 0
    draws: int = 0
    boundary: int = 0              # margin cases against the spread-order oracle
    ref_draws: int = 0
    ref_diff: int = 0              # drawing rows whose id differs from numpy's order
    ref_diff_tie: int = 0          # ... of which a tie straddles the cut
    ref_straddle: int = 0          # drawing rows with a tie straddling the cut
    mismatches: list = field(default_factory=list)

    def merge(self, o: "Tally") -> None:
        for k in ("rows", "draws", "boundary", "ref_draws", "ref_diff", "ref_diff_tie",
                  "ref_straddle"):
            setattr(self, k, getattr(self, k) + getattr(o, k))
        self.mismatches += o.mismatches


def is_margin(res: R.RowResult) -> bool:
    d = res.diag
    return (d.get("draw_margin", 1.0) < BOUNDARY or d.get("top_p_margin", 1.0) < BOUNDARY or
            d.get("typical_margin", 1.0) < BOUNDARY)


def is_tie_straddle(res: R.RowResult) -> bool:
    d = res.diag
    return bool(d.get("top_p_tie_straddle", False) or d.get("typical_tie_straddle", False))


def is_boundary(res: R.RowResult) -> bool:
    """A margin case or a tie straddle (the reference's own order unspecified)."""
    return is_margin(res) or is_tie_straddle(res)


def compare_rows(ids, status, probs, oracle_rows: list, label: str = "",
                 ref_rows: list | None = None) -> Tally:
    """Compare device outputs with oracle RowResults run with tie='spread'
    (``oracle_rows``) and, when given, with tie='numpy' (``ref_rows``); the
    budgets against numpy's order are checked here (violations are added to
    ``mismatches``)."""
    t = Tally()
    for b, res in enumerate(oracle_rows):
        t.rows += 1
        got_st = int(status[b]) & 0xFF
        if ref_rows is not None and got_st == R.STATUS_OK:
            ref = ref_rows[b]
            t.ref_draws += 1
            straddle = is_tie_straddle(ref) or is_tie_straddle(res)
            t.ref_straddle += int(straddle)
            if int(ids[b]) != ref.token:
                t.ref_diff += 1
                if straddle:
                    t.ref_diff_tie += 1
                elif not (is_margin(ref) or is_margin(res)):
                    t.mismatches.append((label, b, "ref-token", int(ids[b]), ref.token, ref.diag))
        if got_st != res.status:
            t.mismatches.append((label, b, "status", got_st, res.status))
            continue
        if res.status == R.STATUS_ERROR:
            continue
        if res.status == R.STATUS_OK:
            t.draws += 1
        if int(ids[b]) != res.token:
            if res.status == R.STATUS_OK and is_margin(res):
                t.boundary += 1
            else:
                t.mismatches.append((label, b, "token", int(ids[b]), res.token, res.diag))
            continue
        if probs is not None and res.probs is not None:
            want = res.probs
            got = probs[b].astype(np.float64)
            if not np.array_equal(want > 0, got > 0):
                if not is_margin(res):
                    t.mismatches.append((label, b, "support",
                                         int((want > 0).sum()), int((got > 0).sum())))
                continue
            big = want > PROB_FLOOR
            rel = np.abs(got[big] - want[big]) / want[big]
            if rel.size and rel.max() > PROB_RTOL:
                t.mismatches.append((label, b, "probs", float(rel.max())))
    if ref_rows is not None:
        record_ref_rate(label, t)
        t.mismatches += ref_budget_violations(label, t)
    return t


def ref_budget_violations(label: str, t: Tally) -> list:
    """The budgets of the draws that differ from numpy's order (see the
    module docstring)."""
    out = []
    margin = t.ref_diff - t.ref_diff_tie
    if margin > REF_BUDGET * t.ref_draws:
        out.append((label, "margin budget", margin, t.ref_draws))
    bound = tie_bounds().get(label)
    if bound is None:
        if t.ref_diff_tie > REF_BUDGET * t.ref_draws:
            out.append((label, "tie budget (1e-4)", t.ref_diff_tie, t.ref_draws))
    elif t.ref_diff_tie > bound:
        out.append((label, "tie budget (numpy cross-level)", t.ref_diff_tie, bound))
    return out


def record_ref_rate(label: str, t: Tally) -> None:
    """Keep the reference-order counts of one workload for the run summary."""
    REF_RATES[label] = {"draws": t.ref_draws, "diff": t.ref_diff, "diff_tie": t.ref_diff_tie,
                        "straddle": t.ref_straddle, "margin_vs_spread": t.boundary,
                        "bound": tie_bounds().get(label)}


def oracle_rows(w, rows=None, keep_probs=True, tie="spread") -> list:
    """Oracle results for the rows of a SampleWorkload."""
    from oracle.bf16 import bf16_bits_to_f32
    rows = range(w.B) if rows is None else rows
    hl = R.hist_rows_to_lists(w.hist, w.hist_len) if w.hist.size else None
    out = []
    for b in rows:
        x = bf16_bits_to_f32(w.logits[b]) if w.dtype == "bf16" else w.logits[b]
        out.append(R.sample_row(x, w.params[b], None if hl is None else hl[b], float(w.u[b]),
                                tie=tie, keep_probs=keep_probs))
    return out
