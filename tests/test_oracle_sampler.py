"""Pins for the sampler oracle (CPU only).

The oracle must equal the reference before anything is compared with it:
  * the reference's own known answers (chenxing tests/test_sampler.py:7-69),
  * golden vectors written by the reference itself (tests/golden/),
  * numpy behaviour the restatement relies on,
  * brute force on tiny vocabularies and closed forms.
"""
from __future__ import annotations

import itertools

import numpy as np
import pytest

import cases
from oracle import sampler_ref as R
from oracle.bf16 import bf16_bits_to_f32, f32_to_bf16_bits

GOLD = np.load(cases.__file__.replace("cases.py", "sampler_golden.npz"))


def _prm(d: dict) -> R.RowParams:
    return R.RowParams(temperature=d["temperature"], top_k=d["top_k"], top_p=d["top_p"],
                       min_p=d["min_p"], typical_p=d["typical_p"],
                       repetition_penalty=d["repetition_penalty"], n_keep=d["n_keep"])


# ------------------------------------------------ reference known answers
def test_greedy_is_argmax():                                   # test_sampler.py:7-10
    x = np.array([0.1, 5.0, 0.2, 0.0, -1, 0, 0, 0])
    assert R.sample_row(x, R.RowParams(temperature=0.0)).token == 1


def test_temperature_zero_consumes_nothing():                   # test_sampler.py:13-16
    r = R.sample_row(np.array([1.0, 3.0, 2.0, 0.0]), R.RowParams(temperature=0.0))
    assert r.token == 1 and r.status == R.STATUS_GREEDY


def test_seed_reproducible():                                  # test_sampler.py:19-26
    u = np.random.default_rng(99).random()
    g = np.random.default_rng(0)
    rows = [g.standard_normal(16) for _ in range(4)]
    a = [R.sample_row(x, R.RowParams(), u=u).token for x in rows]
    b = [R.sample_row(x, R.RowParams(), u=u).token for x in rows]
    assert a == b


def test_top_k_one_keeps_only_the_max():                       # test_sampler.py:29-33
    x = np.array([5.0, 4.9, 0.1, 0.0, 0, 0, 0, 0])
    for u in np.linspace(0, 0.999, 17):
        assert R.sample_row(x, R.RowParams(top_k=1), u=u).token == 0


def test_top_p_mass_cutoff():                                  # test_sampler.py:36-44
    logits = np.log(np.array([0.9, 0.09, 0.009, 0.001]))
    probs = R.truncate(np.exp(logits - logits.max()), R.RowParams(top_p=0.95))
    probs = probs / probs.sum()
    assert probs[2] == 0 and probs[3] == 0
    assert probs[0] + probs[1] > 0.99


def test_repetition_penalty_downweights_seen():                # test_sampler.py:47-52
    pen = R.penalize(np.array([4.0, 4.0, 0.0, 0.0]), [0],
                     R.RowParams(temperature=0.0, repetition_penalty=10.0))
    assert pen[0] < pen[1]


def test_min_p_relative_floor():                               # test_sampler.py:55-61
    logits = np.log(np.array([0.8, 0.15, 0.04, 0.01]))
    probs = R.truncate(np.exp(logits - logits.max()), R.RowParams(min_p=0.15))
    assert probs[3] == 0 and probs[2] == 0
    assert probs[0] > 0 and probs[1] > 0


def test_invalid_params_raise():                               # test_sampler.py:64-69
    from chenxing_amd.params import SamplingParams
    with pytest.raises(ValueError):
        SamplingParams(top_p=1.5)
    with pytest.raises(ValueError):
        SamplingParams(temperature=-1)
    with pytest.raises(ValueError):
        SamplingParams(min_p=-0.1)


# ------------------------------------------------ golden vectors from the reference
ALL_CASES = cases.small_sampler_cases() + cases.medium_sampler_cases()


def test_golden_inputs_unchanged():
    assert list(GOLD["names"]) == [c.name for c in ALL_CASES]
    assert list(GOLD["logit_digest"]) == [cases.digest(c.logits) for c in ALL_CASES]


@pytest.mark.parametrize("i", range(len(ALL_CASES)))
def test_golden_case(i):
    c = ALL_CASES[i]
    prm = _prm(c.params)
    pen = R.penalize(c.logits, c.hist, prm)
    assert cases.digest(pen) == GOLD["pen_digest"][i], "penalties differ bitwise"
    P_in = cases.truncate_input(c)
    assert cases.digest(P_in) == GOLD["trunc_in_digest"][i]
    with np.errstate(all="ignore"):
        tr = R.truncate(P_in.copy(), prm)
    assert cases.digest(tr) == GOLD["trunc_digest"][i], "_truncate differs bitwise"
    u = np.random.default_rng(c.params["seed"]).random()
    res = R.sample_row(c.logits, prm, c.hist, u)
    want = int(GOLD["sample"][i])
    if want == -9:
        assert res.status == R.STATUS_ERROR
    else:
        assert res.status != R.STATUS_ERROR and res.token == want


def test_golden_cover_every_outcome():
    """The fixture exercises greedy, stochastic, argmax fallback and errors."""
    seen = set()
    for c in ALL_CASES:
        u = np.random.default_rng(c.params["seed"]).random()
        seen.add(R.sample_row(c.logits, _prm(c.params), c.hist, u).status)
    assert seen == {R.STATUS_OK, R.STATUS_GREEDY, R.STATUS_ARGMAX, R.STATUS_ERROR}


# ------------------------------------------------ numpy behaviour pins
def test_choice_is_inverse_cdf_with_one_draw():
    for t in range(400):
        r = np.random.default_rng(5000 + t)
        V = int(r.integers(1, 300))
        P = r.random(V)
        P[r.random(V) < 0.5] = 0
        if P.sum() == 0:
            P[0] = 1
        P /= P.sum()
        seed = int(r.integers(0, 2**31))
        g = np.random.default_rng(seed)
        want = int(g.choice(V, p=P))
        nxt = g.random()
        h = np.random.default_rng(seed)
        u = h.random()
        assert R.inverse_cdf(P, u) == want
        assert h.random() == nxt          # choice consumed exactly one variate


def test_random_is_top_53_bits_of_pcg64():
    for s in range(50):
        raw = np.random.PCG64(s).random_raw()
        assert np.random.default_rng(s).random() == (raw >> 11) * 2.0**-53


def test_argmax_ties_and_nan():
    assert np.argmax([1.0, np.nan, 5.0, np.nan]) == 1
    assert np.argmax([3.0, 1.0, 3.0]) == 0
    assert np.argmax([-np.inf, -np.inf]) == 0


def test_partition_counts_multiplicity():
    P = np.array([0.3, 0.3, 0.3, 0.1])
    kept = R.truncate(P, R.RowParams(top_k=2))
    assert np.count_nonzero(kept) == 3


def test_fp32_row_over_python_float_is_fp32_division():
    r = np.random.default_rng(0).normal(0, 2, 10000).astype(np.float32)
    for T in (0.7, 0.3, 1.3):
        a = r / T
        assert a.dtype == np.float32
        assert np.array_equal(a, r / np.float32(T))


# ------------------------------------------------ brute force on tiny vocabularies
def _brute_topk(P, k):
    return {i for i in range(P.size) if sum(P > P[i]) < k}


def _brute_nucleus_stable(P, p):
    order = sorted(range(P.size), key=lambda i: (-P[i], i))
    run = 0.0
    for m, i in enumerate(order):
        run += P[i]
        if run >= p:
            return set(order[:m + 1])
    return set(range(P.size))


def test_brute_force_topk_and_nucleus():
    rng = np.random.default_rng(7)
    for t in range(300):
        V = int(rng.integers(1, 10))
        P = np.round(rng.random(V), 1) + 0.05           # ties on purpose
        P /= P.sum()
        k = int(rng.integers(1, V + 2))
        got = set(np.flatnonzero(R.truncate(P, R.RowParams(top_k=k))))
        assert got == _brute_topk(P, k)
        p = float(rng.choice([0.0, 0.3, 0.5, 0.9, 0.999]))
        got = set(np.flatnonzero(R.truncate(P, R.RowParams(top_p=p), tie="stable")))
        assert got == _brute_nucleus_stable(P, p)


def test_spread_rule_counts_and_evenness():
    """spread_mask(n, j) keeps exactly j members, every prefix of R members
    holds R j / n survivors to within 1/2 (the closest an integer count can
    be), and j = n / j = 0 keep all / none."""
    for n in range(1, 40):
        for j in range(0, n + 1):
            m = R.spread_mask(n, j)
            assert int(m.sum()) == j
            pref = np.concatenate([[0], np.cumsum(m)])
            R_ = np.arange(n + 1)
            assert np.all(np.abs(pref - R_ * j / n) <= 0.5 + 1e-12), (n, j)
            assert np.array_equal(pref, R.spread_kept(R_, j, n))
    assert R.spread_mask(5, 5).all() and not R.spread_mask(5, 0).any()
    assert list(np.flatnonzero(R.spread_mask(3, 1))) == [1]        # the middle one
    assert list(np.flatnonzero(R.spread_mask(4, 2))) == [1, 3]


def test_spread_nucleus_against_brute_force():
    """On rows longer than TIE_NET the spread nucleus keeps every value
    above the cut value, none below, as many as the stable nucleus, and of
    the tie group at the cut exactly the spread_mask members (in ascending
    id order); on rows of at most TIE_NET it is the stable nucleus."""
    rng = np.random.default_rng(11)
    straddles = 0
    for t in range(120):
        V = int(rng.choice([5, 40, R.TIE_NET, R.TIE_NET + 1, 300, 700]))
        P = np.round(rng.random(V), 1) + 0.05           # ties on purpose
        P /= P.sum()
        p = float(rng.choice([0.0, 0.3, 0.5, 0.7, 0.9, 0.999]))
        ref = _brute_nucleus_stable(P, p)
        got = set(np.flatnonzero(R.truncate(P, R.RowParams(top_p=p), tie="spread")))
        if V <= R.TIE_NET:
            assert got == ref
            continue
        assert len(got) == len(ref)
        vcut = min(P[i] for i in ref)
        assert {i for i in range(V) if P[i] > vcut} <= got
        assert not {i for i in got if P[i] < vcut}
        G = [i for i in range(V) if P[i] == vcut]
        j = sum(1 for i in ref if P[i] == vcut)
        assert {G[r] for r in np.flatnonzero(R.spread_mask(len(G), j))} == {i for i in got if P[i] == vcut}
        straddles += int(j < len(G))
    assert straddles > 20


def test_spread_typical_keeps_the_stable_count():
    """Typical-p in spread order keeps as many ids, and the same mass, as in
    the stable order (a flat group straddling the typical cut)."""
    P = np.array([0.1] * 6 + [0.2, 0.2] + [0.0] * 300, dtype=np.float64)
    for q in (0.15, 0.35, 0.55, 0.75):
        a = R.truncate(P.copy(), R.RowParams(typical_p=q), tie="stable")
        b = R.truncate(P.copy(), R.RowParams(typical_p=q), tie="spread")
        assert (a > 0).sum() == (b > 0).sum() and np.isclose(a.sum(), b.sum())


def test_brute_force_draw_distribution():
    """Each id is drawn for exactly the u-interval of width P_i (V <= 6)."""
    rng = np.random.default_rng(3)
    for t in range(50):
        V = int(rng.integers(1, 7))
        x = rng.normal(0, 1, V)
        prm = R.RowParams(temperature=float(rng.choice([0.5, 1.0, 2.0])))
        P = R.tempered_probs(x, prm.temperature)
        us = (np.arange(20000) + 0.5) / 20000
        hits = np.bincount([R.sample_row(x, prm, u=u).token for u in us], minlength=V)
        assert np.allclose(hits / us.size, P, atol=1.0 / 20000 * 2)


# ------------------------------------------------ closed forms
def test_tempered_probs_is_softmax_over_t():
    rng = np.random.default_rng(11)
    for T in (0.3, 0.7, 1.0, 1.5):
        x = rng.normal(0, 2, 5000)
        z = (x - x.max()) / T
        want = np.exp(z) / np.exp(z).sum()
        np.testing.assert_allclose(R.tempered_probs(x, T), want, rtol=1e-12, atol=0)


def test_presence_frequency_closed_form():
    x = np.array([1.0, -2.0, 3.0, 0.5], dtype=np.float32)
    hist = [0, 0, 2, 2, 2, 7, -1]
    prm = R.RowParams(repetition_penalty=1.0, presence_penalty=0.5, frequency_penalty=0.3)
    pen = R.penalize(x, hist, prm)
    assert pen[0] == (1.0 - 0.3 * 2.0) - 0.5
    assert pen[2] == (3.0 - 0.3 * 3.0) - 0.5
    assert pen[1] == -2.0 and pen[3] == 0.5
    # with the repetition penalty first: 3.0/1.1, -2 untouched, 1.0/1.1
    prm = R.RowParams(repetition_penalty=1.1, presence_penalty=0.5, frequency_penalty=0.3)
    pen = R.penalize(x, hist, prm)
    assert pen[0] == (1.0 / 1.1 - 0.3 * 2.0) - 0.5
    assert pen[2] == (3.0 / 1.1 - 0.3 * 3.0) - 0.5


def test_presence_frequency_zero_reduces_to_reference():
    rng = np.random.default_rng(2)
    for t in range(50):
        x = rng.normal(0, 2, 200).astype(np.float32)
        hist = list(rng.integers(-3, 205, 90))
        base = R.RowParams(repetition_penalty=1.3, n_keep=int(rng.choice([0, 70])))
        a = R.penalize(x, hist, base)
        b = R.penalize(x, hist, R.RowParams(repetition_penalty=1.3, n_keep=base.n_keep,
                                            presence_penalty=0.0, frequency_penalty=0.0))
        assert np.array_equal(a, b)


def test_penalty_window_n_keep():
    assert R.penalty_window(list(range(100)), 0) == list(range(100))
    assert R.penalty_window(list(range(100)), 10) == list(range(36, 100))
    assert R.penalty_window(list(range(100)), 80) == list(range(20, 100))


def test_degenerate_rows_follow_the_filter_cascade():
    """NaN/+inf/underflowed rows: argmax(x) when top-k or min-p is on, else error."""
    bad = np.array([0.5, np.nan, 2.0], dtype=np.float32)
    assert R.sample_row(bad, R.RowParams(), u=0.5).status == R.STATUS_ERROR
    assert R.sample_row(bad, R.RowParams(top_k=1), u=0.5).token == 1
    assert R.sample_row(bad, R.RowParams(min_p=0.1), u=0.5).status == R.STATUS_ARGMAX
    assert R.sample_row(bad, R.RowParams(top_p=0.5), u=0.5).status == R.STATUS_ERROR
    assert R.sample_row(bad, R.RowParams(top_p=0.5, min_p=0.1), u=0.5).status == R.STATUS_ARGMAX


# ------------------------------------------------ bf16
def test_bf16_matches_torch_rne():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.normal(0, 3, 20000), rng.normal(0, 1e-30, 100),
                        [0.0, -0.0, 1e38, -1e38, 3.3895314e38]]).astype(np.float32)
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(f32_to_bf16_bits(x), want)
    assert np.array_equal(bf16_bits_to_f32(want), torch.from_numpy(x).to(torch.bfloat16)
                          .to(torch.float32).numpy())


def test_workload_bf16_helper_matches_oracle():
    from chenxing_amd.workloads import f32_to_bf16_rne
    x = np.random.default_rng(1).normal(0, 2, 50000).astype(np.float32)
    assert np.array_equal(f32_to_bf16_rne(x), f32_to_bf16_bits(x))


def test_tie_order_fixture_covers_the_bf16_workloads():
    """tests/golden/tie_order_rates.json (tie_order_rates.py): one entry per
    bf16 workload the GPU tests bound, and on each the device's order
    (spread) disagrees with every numpy dispatch level on no more draws than
    two numpy levels disagree with each other."""
    import json
    import os
    from bf16_workloads import TIE_WORKLOADS
    path = os.path.join(os.path.dirname(cases.__file__), "tie_order_rates.json")
    rep = json.load(open(path))
    assert set(rep["workloads"]) == set(TIE_WORKLOADS)
    for label, r in rep["workloads"].items():
        assert r["max_spread_vs_numpy"] <= r["max_numpy_cross_level"], label
        assert r["draws"] > 0 and r["straddling_rows"] > 0, label
