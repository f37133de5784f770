"""Rows whose top-p cut lies within the fused normaliser's error bound: the
exact kernel recomputes the normaliser in fp64 and finishes the row's region
again (CX_ROW_FLAG_EXACT) instead of running the multi-pass path
(CX_ROW_FLAG_SLOW).  Each constructed row puts top_p 1e-9 (relative) from
one of the oracle's cumulative sums, so only an exact normaliser decides it;
the device's token must equal the oracle's exactly."""
from __future__ import annotations

import sys

import numpy as np
import pytest

from chenxing_amd import workloads as W
from chenxing_amd._lib import FLAG_EXACT, FLAG_SLOW, sample_host
from chenxing_amd.params import RowParams
from oracle import sampler_ref as R
from parity import compare_rows, oracle_rows

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _near_cut_rows(rng, x, hist, kw, m_lo, m_hi, rel=1e-9):
    """Per row, top_p just below (even rows) or just above (odd rows) the
    oracle's cumulative sum at a random rank m of the post-top-k vector."""
    prms = []
    for b in range(x.shape[0]):
        base = RowParams(**kw)
        h = None if hist is None else [int(t) for t in hist[b]]
        P = R.tempered_probs(R.penalize(x[b], h, base), base.temperature)
        if base.top_k > 0:
            P = R.truncate(P, base, tie="spread")
        run = np.cumsum(P[np.argsort(-P, kind="stable")])
        m = int(rng.integers(m_lo, m_hi))
        side = 1.0 if b % 2 else -1.0
        prms.append(RowParams(**kw, top_p=float(run[m] * (1.0 + side * rel))))
    return prms


def _check_exact(x, prms, hist, u, want_probs, label):
    B = x.shape[0]
    hl = None if hist is None else np.full(B, hist.shape[1], np.int32)
    _say(f"[gpu] refine {label} B={B} V={x.shape[1]} probs={want_probs}")
    ids, st, probs = sample_host(x, prms, hist, hl, u, want_probs=want_probs)
    orc = [R.sample_row(x[b], prms[b], None if hist is None else [int(t) for t in hist[b]],
                        float(u[b]), tie="spread", keep_probs=want_probs) for b in range(B)]
    t = compare_rows(ids, st, probs, orc, label)
    assert not t.mismatches, t.mismatches[:5]
    want = np.array([o.token for o in orc])
    assert np.array_equal(ids, want), np.flatnonzero(ids != want)[:8]
    assert not np.any(st & FLAG_SLOW), np.flatnonzero(st & FLAG_SLOW)[:8]
    assert np.all(st & FLAG_EXACT), np.flatnonzero((st & FLAG_EXACT) == 0)[:8]


@pytest.mark.parametrize("want_probs", [False, True])
def test_near_cut_top_k_rows_with_penalties(want_probs):
    """One slice per row (B = 256): without probabilities out the one-wave
    top-k finish hands the row over, with them the block finisher does."""
    rng = np.random.default_rng(21)
    B, V, H = 256, 32000, 256
    x = rng.normal(0, 2, (B, V)).astype(np.float32)
    hist = W.zipf_history(rng, B, H, V).astype(np.int32)
    kw = dict(temperature=0.8, top_k=40, repetition_penalty=1.1, presence_penalty=0.5,
              frequency_penalty=0.3)
    prms = _near_cut_rows(rng, x, hist, kw, 3, 30)
    _check_exact(x, prms, hist, rng.random(B), want_probs, "top-k near cut")


@pytest.mark.parametrize("want_probs", [False, True])
def test_near_cut_nucleus_rows_in_slices(want_probs):
    """Several slices per row (B = 8): the region finisher hands the row over."""
    rng = np.random.default_rng(22)
    B, V = 8, 128256
    x = rng.normal(0, 2, (B, V)).astype(np.float32)
    prms = _near_cut_rows(rng, x, None, dict(temperature=1.0), 100, 1000)
    _check_exact(x, prms, None, rng.random(B), want_probs, "nucleus near cut")


@pytest.mark.parametrize("want_probs", [False, True])
def test_near_cut_sliced_rows_with_penalties(want_probs):
    """Sliced rows (B = 8) with 512-id Zipf histories and repetition,
    presence and frequency penalties: the exact normaliser applies the
    penalties as the stream did."""
    rng = np.random.default_rng(24)
    B, V, H = 8, 128256, 512
    x = rng.normal(0, 2, (B, V)).astype(np.float32)
    hist = W.zipf_history(rng, B, H, V).astype(np.int32)
    kw = dict(temperature=0.9, repetition_penalty=1.3, presence_penalty=0.4,
              frequency_penalty=0.2)
    prms = _near_cut_rows(rng, x, hist, kw, 100, 800)
    _check_exact(x, prms, hist, rng.random(B), want_probs, "sliced near cut, penalties")


def test_nucleus_config_avoids_multipass_path():
    """B = 64 top-p 0.95 rows: every nucleus fits the sliced region and the
    rows near the cut are refined, so no row takes the multi-pass path."""
    w = W.nucleus()
    _say(f"[gpu] refine {w.name} B={w.B} V={w.V}")
    ids, st, probs = sample_host(w.logits, w.params, None, w.hist_len, w.u, want_probs=True)
    t = compare_rows(ids, st, probs, oracle_rows(w), w.name)
    assert not t.mismatches, t.mismatches[:5]
    assert not np.any(st & FLAG_SLOW), np.flatnonzero(st & FLAG_SLOW)


@pytest.mark.parametrize("want_probs", [False, True])
def test_tied_group_at_the_cut_takes_the_sorting_finisher(want_probs):
    """200 ids share one value around rank 300 and top_p falls inside that
    group: the cut's bucket holds more than 64 entries, so the region
    finisher sorts the region instead (ties in ascending id order)."""
    rng = np.random.default_rng(23)
    B, V = 4, 32000
    x = rng.normal(0, 1, (B, V)).astype(np.float32)
    prms = []
    for b in range(B):
        order = np.argsort(-x[b], kind="stable")
        tied = rng.choice(order[250:2000], 200, replace=False)
        x[b, tied] = x[b, order[300]]
        base = RowParams(temperature=1.0)
        P = R.tempered_probs(R.penalize(x[b], None, base), 1.0)
        o = np.argsort(-P, kind="stable")
        run = np.cumsum(P[o])
        first = int(np.flatnonzero(P[o] == P[tied[0]])[0])
        m = first + 60 + 20 * b                      # inside the tied group
        prms.append(RowParams(temperature=1.0, top_p=float(0.5 * (run[m] + run[m + 1]))))
    u = rng.random(B)
    _say(f"[gpu] refine tied group B={B} V={V} probs={want_probs}")
    ids, st, probs = sample_host(x, prms, None, None, u, want_probs=want_probs)
    orc = [R.sample_row(x[b], prms[b], None, float(u[b]), tie="spread", keep_probs=want_probs)
           for b in range(B)]
    t = compare_rows(ids, st, probs, orc, "tied group")
    assert not t.mismatches, t.mismatches[:5]
    assert np.array_equal(ids, [o.token for o in orc])
    assert not np.any(st & FLAG_SLOW), np.flatnonzero(st & FLAG_SLOW)


def test_sliced_nucleus_rows_decided_by_the_split_normaliser():
    """The config-2 rows (B = 64, four slices) with top_p 3e-7 (relative)
    from one of the oracle's cumulative sums: within the streamed fp32
    normaliser's bound (4e-6), outside the split one's (exact fp64 terms for
    the buffered entries, the fp32 bound only on the small mass below the
    wave thresholds).  The region finisher decides them without the exact
    re-read, and the token equals the oracle's."""
    w = W.nucleus()
    rng = np.random.default_rng(25)
    prms = _near_cut_rows(rng, w.logits, None, dict(temperature=1.0), 100, 1000, rel=3e-7)
    u = rng.random(w.B)
    _say(f"[gpu] split normaliser B={w.B} V={w.V}")
    ids, st, probs = sample_host(w.logits, prms, None, None, u)
    orc = [R.sample_row(w.logits[b], prms[b], None, float(u[b]), tie="spread")
           for b in range(w.B)]
    want = np.array([o.token for o in orc])
    assert np.array_equal(ids, want), np.flatnonzero(ids != want)[:8]
    assert not np.any(st & FLAG_SLOW), np.flatnonzero(st & FLAG_SLOW)
    refined = int(np.count_nonzero(st & FLAG_EXACT))
    _say(f"[gpu] split normaliser: {refined} of {w.B} rows re-read")
    assert refined == 0, np.flatnonzero(st & FLAG_EXACT)
