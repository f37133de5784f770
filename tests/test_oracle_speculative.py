"""Pins for the verify oracle and the host-side speculative loop (CPU only).

The reference's verify block (chenxing/engine/speculative.py:145-171) is
inline in ``generate``; the golden fixture records whole ``generate`` runs of
the reference driven by a scripted engine.  Replaying them through this
repo's ``SpeculativeDecoder`` with the oracle as the verify step must give
the same tokens, stop reason, statistics and forward calls.
"""
from __future__ import annotations

import json

import numpy as np
import pytest

import cases
from chenxing_amd.params import SamplingParams
from chenxing_amd.speculative import SpeculativeDecoder
from oracle import sampler_ref as R
from oracle import speculative_ref as S
from oracle_api import OracleSampler

with open(cases.__file__.replace("cases.py", "spec_golden.json")) as f:
    GOLD = json.load(f)


def oracle_verifier(target, draft, ids, u, T):
    r = S.verify_round(target, draft, ids, u, T)
    return r.accepted, r.next_tok, r.uniforms_used


@pytest.mark.parametrize("sc", cases.spec_cases(), ids=lambda s: s["name"])
def test_golden_generate(sc):
    gold = {c["name"]: c for c in GOLD["cases"]}[sc["name"]]
    V = sc["V"]
    tgt = cases.ScriptedEngine(V, sc["base_seed"], 0.0, 0, OracleSampler(V))
    drf = cases.ScriptedEngine(V, sc["base_seed"], sc["noise"], sc["noise_seed"],
                               OracleSampler(V))
    sd = SpeculativeDecoder(tgt, drf, num_speculative_tokens=sc["gamma"],
                            verifier=oracle_verifier)
    prm = SamplingParams(max_tokens=sc["max_tokens"], temperature=sc["temperature"],
                         seed=sc["seed"])
    toks, reason = sd.generate(sc["prompt"], prm)
    assert toks == gold["tokens"]
    assert reason == gold["reason"]
    assert sd.stats.as_dict() == gold["stats"]
    assert [list(map(list, [[a], b])) for a, b in tgt.forward_log] == \
        [list(map(list, [[a], b])) for a, b in gold["target_forwards"]]
    assert [list(map(list, [[a], b])) for a, b in drf.forward_log] == \
        [list(map(list, [[a], b])) for a, b in gold["draft_forwards"]]


def test_golden_exercises_rejections_and_residuals():
    """The fixture holds rounds that reject (stochastic and greedy)."""
    rej = [c for c in GOLD["cases"] if c["stats"]["accepted"] < c["stats"]["drafted"]]
    assert any("T0.0" not in c["name"] for c in rej)
    assert any("T0.0" in c["name"] for c in rej)


def test_identical_draft_always_accepts():             # test_speculative.py:24-48
    rng = np.random.default_rng(0)
    for t in range(20):
        V, g = 50, 4
        tgt = rng.normal(0, 2, (g + 1, V)).astype(np.float32)
        ids = rng.integers(0, V, g)
        r = S.verify_round(tgt, tgt[:g].copy(), ids, rng.random(g + 1), 1.0)
        assert r.accepted == g and r.next_tok == S.BONUS and r.uniforms_used == g


def test_greedy_round_is_target_argmax_chain():          # test_speculative.py:14-21
    rng = np.random.default_rng(1)
    V, g = 40, 6
    tgt = rng.normal(0, 2, (g + 1, V)).astype(np.float32)
    best = tgt.argmax(axis=1)
    for r_at in range(g + 1):
        ids = best[:g].copy()
        if r_at < g:
            ids[r_at] = (ids[r_at] + 1) % V
        r = S.verify_round(tgt, tgt[:g], ids, np.zeros(g + 1), 0.0)
        assert r.accepted == r_at and r.next_tok == best[r_at] and r.uniforms_used == 0


def test_leviathan_marginal_is_target():
    """Accept-or-resample yields a token distributed as p (Leviathan Thm 3.5)."""
    rng = np.random.default_rng(5)
    V = 6
    zt = rng.normal(0, 1, V).astype(np.float32)
    zd = rng.normal(0, 1, V).astype(np.float32)
    p = S.softmax64(zt)
    q = S.softmax64(zd)
    n = 60000
    toks = rng.choice(V, n, p=q)
    us = rng.random((n, 2))
    tgt = np.stack([zt, zt])
    out = np.empty(n, int)
    for j in range(n):
        r = S.verify_round(tgt, zd[None], [toks[j]], us[j], 1.0)
        out[j] = toks[j] if r.accepted == 1 else r.next_tok
    freq = np.bincount(out, minlength=V) / n
    assert np.abs(freq - p).max() < 4 * np.sqrt(p.max() / n)


def test_nan_ratio_accepts_like_python_min():
    """min(1.0, nan) is 1.0 in Python, so a NaN row accepts (speculative.py:158)."""
    V, g = 8, 2
    tgt = np.zeros((g + 1, V), np.float32)
    tgt[0, 3] = np.nan
    r = S.verify_round(tgt, np.zeros((g, V), np.float32), [1, 2], np.full(g + 1, 0.999), 1.0)
    assert r.accepted == 2 and r.next_tok == S.BONUS


def test_invalid_gamma_rejected():                       # test_speculative.py:59-62
    with pytest.raises(ValueError):
        SpeculativeDecoder(None, None, num_speculative_tokens=0, verifier=oracle_verifier)
