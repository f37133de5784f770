"""Oracle for the per-row sampler (reference ``chenxing/core/sampler.py``).

TEST INFRASTRUCTURE ONLY -- see ``oracle/__init__.py``.

Restated steps, with the uniform ``u`` passed in instead of drawn:

  S1   x = float64(logits)                                    sampler.py:65
  S2   repetition penalty on the unique in-range ids of the
       penalty window (last max(64, n_keep) ids if n_keep,
       else all)                                              sampler.py:66-72
  S2'  presence / frequency penalty (build-defined; absent in
       the reference): x[t] -= freq*count[t]; x[t] -= pres
       for every in-range id t of the same window           (none)
  S3   T == 0  ->  argmax(x)                                  sampler.py:114-115
  S4   P = exp(x - max x); P /= sum P                         sampler.py:117-118
  S5   T != 1  ->  P = P ** (1/T); P /= sum P                 sampler.py:119-121
  S6   top-k: keep P >= k-th largest (ties kept)              sampler.py:76-79
  S7   top-p: keep argsort(-P)[:searchsorted(cumsum, p)+1]    sampler.py:81-89
  S8   min-p, typical-p                                       sampler.py:91-105
  S9   Z = sum P; Z <= 0 -> argmax(x)                          sampler.py:123-125
  S10  Generator.choice(V, p=P/Z) with one uniform u
       == searchsorted(cumsum(P/Z)/cdf[-1], u, 'right')       sampler.py:126-127

Every numpy reduction is called on the same arrays, in the same order, as the
reference calls it, so the fp64 bits (pairwise ``sum``, sequential ``cumsum``)
are the reference's bits.

The one freedom is ``argsort`` tie order in S7/S8: numpy's default sort is
unstable and its tie order depends on the SIMD sort numpy dispatches to on
the CPU at hand, so ``tie="numpy"`` reproduces the reference on this
machine.  Where a group of equal keys straddles a cut, the order decides
which members of the group survive; every order keeps the same number of
them.  ``tie="spread"`` is the device's rule, which follows how numpy's
SIMD argsort treats ties: a row of at most TIE_NET (256) entries is sorted
by a compare-exchange network that leaves equal keys mostly in index order,
so there the group's lowest ids survive; on a longer row, which numpy
partitions first, the survivors spread evenly over the group's ids -- of a
group of n members (in ascending id order) of which j survive, the first R
members hold K(R) = floor((2 R j + n - 1) / (2 n)) survivors, i.e. member r
survives iff K(r + 1) > K(r).  ``tie="stable"`` (lower id first on every
row) is kept for comparison.

Pins (tests/test_oracle_sampler.py):
  * the reference's own known answers, test_sampler.py:7-69;
  * golden vectors written by importing the reference in the build container
    (tests/golden/make_golden.py): penalties, _truncate, sample() with seeds;
  * numpy behaviour pins: choice == inverse CDF with one draw, random() is the
    top 53 bits of PCG64, argmax ties/NaN, partition multiplicity;
  * brute force on V <= 12 (enumerate the exact top-k / nucleus sets);
  * presence/frequency (S2'): closed form on hand-made rows and the reduction
    to S2 when both are 0 -- "parity unpinned" against the reference, which
    has no such penalty.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Optional, Sequence

import numpy as np

# Row outcome codes; they match the device library's CX_ROW_* codes.
STATUS_OK = 0       # stochastic draw, consumed one uniform
STATUS_GREEDY = 1   # T == 0: argmax, consumes nothing
STATUS_ARGMAX = 2   # filtered mass Z <= 0: argmax(x), consumes nothing
STATUS_ERROR = 3    # the reference raises ValueError (NaN probabilities)


@dataclass(frozen=True)
class RowParams:
    """Per-row knobs (``SamplingParams``, sampler.py:23-35, plus pres/freq)."""
    temperature: float = 1.0
    top_k: int = 0
    top_p: float = 1.0
    min_p: float = 0.0
    typical_p: float = 1.0
    repetition_penalty: float = 1.0
    presence_penalty: float = 0.0
    frequency_penalty: float = 0.0
    n_keep: int = 0


@dataclass
class RowResult:
    token: int
    status: int
    probs: Optional[np.ndarray] = None      # post-filter, normalised (fp64, [V])
    diag: dict = field(default_factory=dict)


# --------------------------------------------------------------------- S1-S2'
def penalty_window(hist: Sequence[int] | None, n_keep: int) -> list[int]:
    """The ids the penalties look at (sampler.py:67)."""
    h = [] if hist is None else [int(t) for t in hist]
    if not h:
        return []
    return h[-max(64, n_keep):] if n_keep else h


def penalize(logits: np.ndarray, hist: Sequence[int] | None,
             prm: RowParams) -> np.ndarray:
    """S1-S2': fp64 copy of the row with the penalties applied (sampler.py:63-73)."""
    x = np.asarray(logits).astype(np.float64, copy=True)
    V = x.size
    win = penalty_window(hist, prm.n_keep)
    if not win:
        return x
    in_range = [t for t in win if 0 <= t < V]                  # sampler.py:68
    if prm.repetition_penalty != 1.0:
        uniq = np.fromiter(sorted(set(in_range)), dtype=np.int64)
        if uniq.size:
            v = x[uniq]
            rp = prm.repetition_penalty
            x[uniq] = np.where(v > 0, v / rp, v * rp)           # sampler.py:70-72
    if (prm.presence_penalty != 0.0 or prm.frequency_penalty != 0.0) and in_range:
        ids, cnt = np.unique(np.asarray(in_range, dtype=np.int64), return_counts=True)
        x[ids] = x[ids] - prm.frequency_penalty * cnt.astype(np.float64)
        x[ids] = x[ids] - prm.presence_penalty
    return x


# --------------------------------------------------------------------- S4-S5
def tempered_probs(x: np.ndarray, temperature: float) -> np.ndarray:
    """S4-S5 (sampler.py:117-121): softmax, then the P**(1/T) re-weighting."""
    P = np.exp(x - x.max())
    P /= P.sum()
    if temperature != 1.0:
        P = P ** (1.0 / temperature)
        P /= P.sum()
    return P


# --------------------------------------------------------------------- S6-S8
TIES = ("numpy", "stable", "spread")
TIE_NET = 256        # rows up to this length keep a split group's lowest ids


def _argsort(keys: np.ndarray, tie: str) -> np.ndarray:
    if tie not in TIES:
        raise ValueError(f"tie must be one of {TIES}")
    return np.argsort(keys) if tie == "numpy" else np.argsort(keys, kind="stable")


def spread_kept(R, j: int, n: int):
    """Survivors among the first R members (ascending id) of a tie group of
    n members of which j survive a cut: floor((2 R j + n - 1) / (2 n)).
    Works elementwise on integer arrays."""
    if j <= 0 or n <= 0:
        return R * 0
    if j >= n:
        return R
    return (2 * R * j + n - 1) // (2 * n)


def spread_mask(n: int, j: int) -> np.ndarray:
    """Which of the n members (ascending id) of a tie group survive when j do."""
    r = np.arange(n, dtype=np.int64)
    return spread_kept(r + 1, j, n) > spread_kept(r, j, n)


def _keep_prefix(P: np.ndarray, order: np.ndarray, mass: float, diag: dict,
                 name: str, keys: np.ndarray | None = None,
                 tie: str = "numpy") -> np.ndarray:
    """Zero everything outside the shortest prefix of ``order`` whose running
    sum reaches ``mass`` (searchsorted 'left' + 1, sampler.py:84-89).

    With ``tie="spread"`` (``order`` the stable order of ``keys``) on a row
    longer than TIE_NET, the group of elements whose key equals the last kept
    element's keeps its survivors by :func:`spread_mask` instead of its
    lowest ids."""
    run = np.cumsum(P[order])
    m = int(np.searchsorted(run, mass))                       # first run[m] >= mass
    keep = np.zeros(P.shape, dtype=bool)
    keep[order[:m + 1]] = True
    if m < P.size:
        lo = abs(run[m - 1] - mass) if m > 0 else np.inf
        diag[name + "_margin"] = float(min(abs(run[m] - mass), lo))
        if m + 1 < P.size:
            a, b = P[order[m]], P[order[m + 1]]
            diag[name + "_tie_straddle"] = bool(a == b and a > 0)
        if tie == "spread" and m + 1 < P.size and P.size > TIE_NET:
            ko = keys[order]
            kc = ko[m]
            g0 = int(np.searchsorted(ko, kc, side="left"))     # the group's first position
            g1 = int(np.searchsorted(ko, kc, side="right"))
            if g1 > m + 1:                                      # the cut splits the group
                G = order[g0:g1]                                # ascending ids (stable order)
                keep[G] = spread_mask(g1 - g0, m + 1 - g0)
    return np.where(keep, P, 0.0)


def truncate(P: np.ndarray, prm: RowParams, tie: str = "numpy",
             diag: dict | None = None) -> np.ndarray:
    """S6-S8: ``Sampler._truncate`` (sampler.py:75-106)."""
    diag = {} if diag is None else diag
    out = P
    if prm.top_k > 0:                                          # :76-79
        k = min(prm.top_k, out.size)
        kth = np.partition(out, -k)[-k]
        out = np.where(out >= kth, out, 0.0)
    if prm.top_p < 1.0:                                        # :81-89
        key = -out
        out = _keep_prefix(out, _argsort(key, tie), prm.top_p, diag, "top_p", key, tie)
    if prm.min_p > 0.0:                                        # :91-93
        floor = prm.min_p * out.max()
        out = np.where(out >= floor, out, 0.0)
    if prm.typical_p < 1.0:                                    # :95-105
        logp = np.log(np.maximum(out, 1e-38))
        h = -(out * logp).sum()
        dist = np.abs(logp + h)
        out = _keep_prefix(out, _argsort(dist, tie), prm.typical_p, diag, "typical", dist, tie)
    return out


# --------------------------------------------------------------------- S9-S10
def inverse_cdf(P: np.ndarray, u: float, diag: dict | None = None) -> int:
    """``Generator.choice(len(P), p=P)`` with its single uniform ``u``:
    cdf = cumsum(P); cdf /= cdf[-1]; first i with cdf[i] > u."""
    cdf = np.cumsum(P)
    cdf /= cdf[-1]
    i = int(np.searchsorted(cdf, u, side="right"))
    if diag is not None:
        lo = cdf[i - 1] if i > 0 else 0.0
        diag["draw_margin"] = float(min(abs(cdf[i] - u), abs(u - lo)))
    return i


def sample_row(logits: np.ndarray, prm: RowParams, hist: Sequence[int] | None = None,
               u: float | None = None, tie: str = "numpy",
               keep_probs: bool = False) -> RowResult:
    """``Sampler.sample`` (sampler.py:108-127) with the uniform made explicit."""
    x = penalize(logits, hist, prm)
    if prm.temperature == 0.0:                                 # :114-115
        return RowResult(int(np.argmax(x)), STATUS_GREEDY)
    diag: dict = {}
    with np.errstate(all="ignore"):
        P = tempered_probs(x, prm.temperature)
        P = truncate(P, prm, tie, diag)
        Z = P.sum()
        if Z <= 0:                                             # :123-125
            return RowResult(int(np.argmax(x)), STATUS_ARGMAX, diag=diag)
        P = P / Z
    if np.isnan(P).any():            # Generator.choice: "probabilities contain NaN"
        return RowResult(-1, STATUS_ERROR, diag=diag)
    if u is None:
        raise ValueError("a stochastic row needs its uniform")
    tok = inverse_cdf(P, float(u), diag)
    return RowResult(tok, STATUS_OK, P if keep_probs else None, diag)


def sample_batch(logits: np.ndarray, params: Sequence[RowParams] | RowParams,
                 hists: Sequence[Sequence[int]] | None = None,
                 u: np.ndarray | None = None, tie: str = "numpy",
                 keep_probs: bool = False) -> list[RowResult]:
    """Row loop over :func:`sample_row` (the reference has no batch entry)."""
    B = logits.shape[0]
    prms = [params] * B if isinstance(params, RowParams) else list(params)
    out = []
    for b in range(B):
        h = None if hists is None else hists[b]
        ub = None if u is None else float(u[b])
        out.append(sample_row(logits[b], prms[b], h, ub, tie, keep_probs))
    return out


def hist_rows_to_lists(hist: np.ndarray, hist_len: np.ndarray | None = None) -> list[list[int]]:
    """[B, H] int32 history matrix (+ per-row lengths) -> per-row id lists.

    Padding and out-of-range ids stay in the list; ``penalize`` drops them
    exactly as sampler.py:68 does."""
    B, H = hist.shape
    lens = np.full(B, H) if hist_len is None else hist_len
    return [[int(t) for t in hist[b, :int(lens[b])]] for b in range(B)]
