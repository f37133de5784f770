"""Oracle for the speculative-decoding verify step
(reference ``chenxing/engine/speculative.py:67-69`` and ``:145-171``).

TEST INFRASTRUCTURE ONLY -- see ``oracle/__init__.py``.

One verify round for one sequence, with the round's uniforms passed in.
The reference draws them from one ``default_rng(params.seed)`` per
``generate()`` (speculative.py:111): one ``random()`` per accept test
(:158) and one more inside the residual ``choice`` (:166).  A round that
rejects at position r therefore uses u[0..r] for the tests and u[r+1] for
the residual, so ``gamma + 1`` uniforms always suffice.

Restated semantics:
  * greedy (T == 0, :150-155): accept iff tok == argmax(raw fp32 row);
    first mismatch -> next = argmax(row).
  * stochastic (:156-167): p = softmax64(row / T), q = softmax64(q_row / T)
    where ``row / T`` is an fp32 array divided by an fp32 T (NEP 50 keeps
    the Python float weak), and softmax64 exponentiates in fp64 (:67-69).
    accept iff u < min(1, p[tok] / max(q[tok], 1e-12)) with Python's
    min/max (a NaN ratio therefore accepts); on reject r = max(p - q, 0),
    R = sum r; R <= 0 -> argmax(row) else choice(V, r / R).
  * all gamma accepted (:168-171): greedy -> argmax(row gamma); stochastic
    -> the full sampler on row gamma with the sampler's own generator,
    which is outside the verify step (reported as BONUS).

Pins (tests/test_oracle_speculative.py): golden rounds recorded by driving
the reference ``SpeculativeDecoder.generate`` with a scripted engine in the
build container (tests/golden/make_golden.py); the reference invariants
(identical draft always accepts, greedy == target argmax chain); the NEP 50
fp32-division pin; and a Monte-Carlo check of Leviathan's theorem (the
accepted-or-resampled token is distributed as p).
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

BONUS = -1   # next_tok value when every draft token was accepted (stochastic)


@dataclass
class VerifyResult:
    accepted: int          # number of accepted draft tokens
    next_tok: int          # correction / bonus token; BONUS if the sampler must draw it
    uniforms_used: int     # how many of u[0..gamma] the reference consumed
    diag: dict = field(default_factory=dict)


def softmax64(z: np.ndarray) -> np.ndarray:
    """speculative.py:67-69: exp in fp64 after subtracting the fp32 max."""
    e = np.exp(z.astype(np.float64) - z.max())
    return e / e.sum()


def scale_by_temperature(row: np.ndarray, temperature: float) -> np.ndarray:
    """``row / params.temperature`` for an fp32 row (fp32 IEEE division)."""
    return np.asarray(row, dtype=np.float32) / np.float32(temperature)


def _py_max(a, b):
    return b if b > a else a


def _py_min(a, b):
    return b if b < a else a


def verify_round(target: np.ndarray, draft: np.ndarray, draft_ids, u: np.ndarray,
                 temperature: float) -> VerifyResult:
    """target: [gamma+1, V] fp32, draft: [gamma, V] fp32, draft_ids: [gamma],
    u: [gamma+1] fp64 (only the consumed prefix matters)."""
    gamma = len(draft_ids)
    greedy = temperature == 0.0
    used = 0
    diag: dict = {"accept_margin": np.inf}
    for i in range(gamma):
        tok = int(draft_ids[i])
        row = target[i]
        if greedy:
            best = int(np.argmax(row))
            if tok == best:
                continue
            return VerifyResult(i, best, 0, diag)
        with np.errstate(all="ignore"):
            p = softmax64(scale_by_temperature(row, temperature))
            q = softmax64(scale_by_temperature(draft[i], temperature))
            thr = _py_min(1.0, p[tok] / _py_max(q[tok], 1e-12))
        ui = float(u[used])
        used += 1
        if thr == thr:
            diag["accept_margin"] = min(diag["accept_margin"], abs(ui - float(thr)))
        if ui < thr:
            continue
        with np.errstate(all="ignore"):
            r = np.maximum(p - q, 0.0)
            R = r.sum()
        if R <= 0:
            return VerifyResult(i, int(np.argmax(row)), used, diag)
        cdf = np.cumsum(r / R)
        cdf /= cdf[-1]
        ur = float(u[used])
        used += 1
        j = int(np.searchsorted(cdf, ur, side="right"))
        lo = cdf[j - 1] if j > 0 else 0.0
        diag["draw_margin"] = float(min(abs(cdf[j] - ur), abs(ur - lo)))
        return VerifyResult(i, j, used, diag)
    if greedy:
        return VerifyResult(gamma, int(np.argmax(target[gamma])), 0, diag)
    return VerifyResult(gamma, BONUS, used, diag)


def verify_batch(target: np.ndarray, draft: np.ndarray, draft_ids: np.ndarray,
                 u: np.ndarray, temperature) -> list[VerifyResult]:
    """target [B, gamma+1, V], draft [B, gamma, V], draft_ids [B, gamma],
    u [B, gamma+1]; temperature scalar or [B]."""
    B = target.shape[0]
    T = np.broadcast_to(np.asarray(temperature, dtype=np.float64), (B,))
    return [verify_round(target[b], draft[b], draft_ids[b], u[b], float(T[b]))
            for b in range(B)]
