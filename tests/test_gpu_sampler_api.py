"""The drop-in Sampler on the GPU: the reference's own tests
(chenxing tests/test_sampler.py), the golden vectors the reference wrote for
apply_penalties, _truncate and sample, and the generator bookkeeping."""
from __future__ import annotations

import sys

import numpy as np
import pytest

import cases
from chenxing_amd import Sampler, SamplingParams
from oracle import sampler_ref as R
from parity import is_margin, is_tie_straddle

pytestmark = pytest.mark.gpu

GOLD = np.load(cases.__file__.replace("cases.py", "sampler_golden.npz"))
ALL_CASES = cases.small_sampler_cases() + cases.medium_sampler_cases()


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _ref_params(d: dict) -> SamplingParams:
    return SamplingParams(**d)


def _orc_params(d: dict) -> R.RowParams:
    return R.RowParams(temperature=d["temperature"], top_k=d["top_k"], top_p=d["top_p"],
                       min_p=d["min_p"], typical_p=d["typical_p"],
                       repetition_penalty=d["repetition_penalty"], n_keep=d["n_keep"])


# ---------------------------------------------- chenxing tests/test_sampler.py
def test_greedy_is_argmax():                                       # :7-10
    _say("[gpu] Sampler greedy")
    s = Sampler(8)
    logits = np.array([0.1, 5.0, 0.2, 0.0, -1, 0, 0, 0])
    assert s.sample(logits, SamplingParams(temperature=0.0)) == 1


def test_temperature_zero_ignores_seed():                          # :13-16
    s = Sampler(4)
    logits = np.array([1.0, 3.0, 2.0, 0.0])
    assert all(s.sample(logits, SamplingParams(temperature=0.0)) == 1 for _ in range(5))


def test_seed_reproducible():                                      # :19-26
    s = Sampler(16)
    p = SamplingParams(temperature=1.0, seed=99)
    rng = np.random.default_rng(0)
    a = [s.sample(rng.standard_normal(16), p) for _ in range(4)]
    rng = np.random.default_rng(0)
    b = [s.sample(rng.standard_normal(16), p) for _ in range(4)]
    assert a == b


def test_top_k_zeroes_tail():                                      # :29-33
    s = Sampler(8)
    logits = np.array([5.0, 4.9, 0.1, 0.0, 0, 0, 0, 0])
    p = SamplingParams(temperature=1.0, top_k=1, seed=0)
    assert all(s.sample(logits, p) in (0, 1) for _ in range(10))


def test_top_p_mass_cutoff():                                      # :36-44
    s = Sampler(4)
    logits = np.log(np.array([0.9, 0.09, 0.009, 0.001]))
    p = SamplingParams(temperature=1.0, top_p=0.95, seed=0)
    probs = s._truncate(np.exp(logits - logits.max()), p)
    probs = probs / probs.sum()
    assert probs[2] == 0 and probs[3] == 0
    assert probs[0] + probs[1] > 0.99


def test_repetition_penalty_downweights_seen():                    # :47-52
    s = Sampler(4)
    logits = np.array([4.0, 4.0, 0.0, 0.0])
    p = SamplingParams(temperature=0.0, repetition_penalty=10.0)
    penalized = s.apply_penalties(logits.copy(), p, generated_ids=[0])
    assert penalized[0] < penalized[1]
    assert penalized.dtype == np.float64 and penalized[0] == 0.4


def test_min_p_relative_floor():                                   # :55-61
    s = Sampler(4)
    logits = np.log(np.array([0.8, 0.15, 0.04, 0.01]))
    p = SamplingParams(temperature=1.0, min_p=0.15, seed=0)
    probs = s._truncate(np.exp(logits - logits.max()), p)
    assert probs[3] == 0 and probs[2] == 0
    assert probs[0] > 0 and probs[1] > 0


# ---------------------------------------------- golden vectors of the reference
def test_golden_apply_penalties_bitwise():
    _say(f"[gpu] Sampler.apply_penalties on {len(ALL_CASES)} golden cases")
    for i, c in enumerate(ALL_CASES):
        s = Sampler(c.logits.size)
        pen = s.apply_penalties(c.logits, _ref_params(c.params), list(c.hist))
        assert cases.digest(pen) == GOLD["pen_digest"][i], c.name
        # fp64 input of the same values: the same fp64 result
        pen64 = s.apply_penalties(c.logits.astype(np.float64), _ref_params(c.params),
                                  list(c.hist))
        assert np.array_equal(pen64, pen, equal_nan=True), c.name


def test_golden_truncate():
    """Bitwise equal to the oracle in the device's tie order (tie="spread");
    a row that differs must be a margin case (a running sum within 1e-6 of
    the cut, where the summation order decides).  Against the reference's
    own _truncate output (numpy's argsort order on the host that wrote the
    fixture), every difference must be a tie straddle: tied probabilities
    on both sides of the top-p or typical cut.  Each exception is named."""
    _say(f"[gpu] Sampler._truncate on {len(ALL_CASES)} golden cases")
    tie_cases, margin_cases = [], []
    for i, c in enumerate(ALL_CASES):
        s = Sampler(c.logits.size)
        P_in = cases.truncate_input(c)
        got = s._truncate(P_in.copy(), _ref_params(c.params))
        diag: dict = {}
        with np.errstate(all="ignore"):
            want = R.truncate(P_in.copy(), _orc_params(c.params), tie="spread", diag=diag)
        margin = min(diag.get("top_p_margin", 1.0), diag.get("typical_margin", 1.0)) < 1e-6
        if not np.array_equal(got, want):
            assert margin, (c.name, "differs from the spread-order oracle outside a margin case")
            margin_cases.append(c.name)
            continue
        if cases.digest(got) != GOLD["trunc_digest"][i]:
            straddle = diag.get("top_p_tie_straddle") or diag.get("typical_tie_straddle")
            assert straddle, (c.name, "differs from the reference without a tie straddle")
            tie_cases.append(c.name)
    _say(f"    tie straddles {len(tie_cases)} {tie_cases}")
    _say(f"    margin cases {len(margin_cases)} {margin_cases}")


def test_golden_sample():
    """Sampled ids equal to the oracle in the device's tie order, except
    margin cases (u within 1e-6 of a CDF step, or a running sum within 1e-6
    of a cut) the oracle itself flags; against the ids the reference drew
    when it wrote the fixture, every other difference must be a tie
    straddle.  Each exception is named."""
    _say(f"[gpu] Sampler.sample on {len(ALL_CASES)} golden cases")
    tie_cases, margin_cases = [], []
    for i, c in enumerate(ALL_CASES):
        s = Sampler(c.logits.size)
        want = int(GOLD["sample"][i])
        prm = _ref_params(c.params)
        if want == -9:
            with pytest.raises(ValueError):
                s.sample(c.logits, prm, list(c.hist))
            continue
        got = s.sample(c.logits, prm, list(c.hist))
        u = np.random.default_rng(c.params["seed"]).random()
        res = R.sample_row(c.logits, _orc_params(c.params), c.hist, u, tie="spread")
        if got != res.token:
            assert is_margin(res), (c.name, got, res.token, res.diag)
            margin_cases.append(c.name)
        elif got != want:
            assert is_tie_straddle(res), (c.name, got, want, res.diag)
            tie_cases.append(c.name)
    _say(f"    tie straddles {len(tie_cases)} {tie_cases}")
    _say(f"    margin cases {len(margin_cases)} {margin_cases}")


def test_fp64_rows_take_the_exact_path():
    """fp64 logits (any float row is accepted by the reference) give the
    token the fp32 row of the same values gives, and the oracle's token for
    values fp32 cannot hold."""
    _say("[gpu] Sampler.sample with fp64 rows")
    for c in ALL_CASES[:60] + ALL_CASES[-12:]:
        s = Sampler(c.logits.size)
        prm = _ref_params(c.params)
        try:
            a = s.sample(c.logits, prm, list(c.hist))
        except ValueError:
            with pytest.raises(ValueError):
                s.sample(c.logits.astype(np.float64), prm, list(c.hist))
            continue
        b = s.sample(c.logits.astype(np.float64), prm, list(c.hist))
        if b != a:
            u = np.random.default_rng(c.params["seed"]).random()
            res = R.sample_row(c.logits, _orc_params(c.params), c.hist, u, tie="spread")
            assert is_margin(res), (c.name, a, b, res.token)
    rng = np.random.default_rng(5)
    for j in range(20):
        x = rng.normal(0, 2, 3000)                       # not representable in fp32
        d = dict(temperature=[0.0, 0.7, 1.0, 1.3][j % 4], top_k=[0, 40][j % 2],
                 top_p=[1.0, 0.9, 0.5][j % 3], min_p=0.0, typical_p=1.0,
                 repetition_penalty=1.2, n_keep=0, seed=j)
        hist = [int(t) for t in rng.integers(0, 3000, 100)]
        got = Sampler(3000).sample(x, _ref_params(d), hist)
        u = np.random.default_rng(j).random()
        res = R.sample_row(x, _orc_params(d), hist, u, tie="spread")
        assert got == res.token or is_margin(res), (j, got, res.token)


# ---------------------------------------------- generator bookkeeping
def test_unseeded_generator_advances_like_the_reference():
    """The shared generator advances by one variate per drawing row only
    (sampler.py:56,127): greedy rows and argmax fall-backs draw nothing."""
    _say("[gpu] Sampler generator bookkeeping")
    V = 300
    rng = np.random.default_rng(3)
    stoch = rng.normal(0, 1, V).astype(np.float32)
    flat = rng.normal(0, 0.1, V).astype(np.float32)
    s = Sampler(V)
    s._rng = np.random.default_rng(123)
    shadow = np.random.default_rng(123)
    s.sample(stoch, SamplingParams(temperature=0.0))
    assert s._rng.bit_generator.state == shadow.bit_generator.state
    s.sample(stoch, SamplingParams(temperature=0.9))
    shadow.random()
    assert s._rng.bit_generator.state == shadow.bit_generator.state
    # a seeded row leaves the shared generator alone
    s.sample(stoch, SamplingParams(temperature=0.9, seed=4))
    assert s._rng.bit_generator.state == shadow.bit_generator.state
    # P**(1/T) underflows to 0/0; top-k zeroes the NaNs and argmax(x) follows
    # (sampler.py:123-125) without a draw
    tok = s.sample(flat, SamplingParams(temperature=0.001, top_k=5))
    assert tok == int(np.argmax(flat))
    assert s._rng.bit_generator.state == shadow.bit_generator.state
    # without a filter numpy's choice raises on the NaNs, also without a draw
    with pytest.raises(ValueError):
        s.sample(flat, SamplingParams(temperature=0.001))
    assert s._rng.bit_generator.state == shadow.bit_generator.state


@pytest.mark.parametrize("on_device", [False, True])
def test_sample_batch_equals_sequential_calls(on_device):
    """Row 9 falls back to argmax without a draw, so the unseeded rows after
    it take the shared generator's variates one place earlier than the first
    launch gave them, and are sampled again."""
    import torch
    _say(f"[gpu] Sampler.sample_batch vs sequential sample (device tensor: {on_device})")
    V = 500
    rng = np.random.default_rng(11)
    X = rng.normal(0, 2, (24, V)).astype(np.float32)
    X[9] = rng.normal(0, 0.1, V)                         # argmax fall-back row below
    params = []
    for b in range(24):
        params.append(SamplingParams(temperature=[0.0, 0.8, 1.0][b % 3],
                                     top_k=[0, 20][b % 2], top_p=[1.0, 0.9][b % 2 == 0],
                                     repetition_penalty=1.1,
                                     seed=None if b % 4 else b))
    params[9] = SamplingParams(temperature=0.001, top_k=5)
    hists = [[int(t) for t in rng.integers(0, V, 30)] for _ in range(24)]
    a = Sampler(V)
    a._rng = np.random.default_rng(99)
    seq = [a.sample(X[b], params[b], hists[b]) for b in range(24)]
    b_ = Sampler(V)
    b_._rng = np.random.default_rng(99)
    bat = b_.sample_batch(torch.from_numpy(X).cuda() if on_device else X, params, hists)
    assert bat == seq
    assert a._rng.bit_generator.state == b_._rng.bit_generator.state


def test_device_tensor_input_matches_host_input():
    import torch
    _say("[gpu] Sampler.sample_batch on a device tensor")
    V = 1000
    rng = np.random.default_rng(12)
    X = rng.normal(0, 2, (8, V)).astype(np.float32)
    params = [SamplingParams(temperature=0.8, top_k=50, top_p=0.9, seed=b) for b in range(8)]
    host = Sampler(V).sample_batch(X, params)
    dev = Sampler(V).sample_batch(torch.from_numpy(X).cuda(), params)
    assert host == dev
    one = Sampler(V).sample(torch.from_numpy(X[3]).cuda(), params[3])
    assert one == host[3]


def test_bf16_device_tensor_matches_the_host_variant():
    """A torch.bfloat16 batch on the device (the large-vocabulary
    heterogeneous workload's rows: per-row temperature, top-k and top-p,
    greedy rows) gives the host variant's ids and statuses on the same bf16
    bits; the host variant is checked against the oracle elsewhere.  Only
    the outcome byte of the status is compared: the route flags (refined
    normaliser, exact multi-pass path) depend on how far each wave's region
    threshold had risen when the stream ended, which varies with the order
    the waves publish in; both routes give the exact token."""
    import torch
    from chenxing_amd import _lib, workloads as W
    from chenxing_amd.params import pack_rows
    w = W.hetero_bf16(B=64)
    _say(f"[gpu] bf16 device tensor {w.name} B={w.B} V={w.V}")
    ids_h, st_h, _ = _lib.sample_host(w.logits, w.params, None, None, w.u, bf16=True)
    dev = torch.device("cuda:0")
    x = torch.from_numpy(w.logits.view(np.int16)).to(dev).view(torch.bfloat16)
    prm = torch.from_numpy(pack_rows(w.params).view(np.uint8).copy()).to(dev)
    u = torch.from_numpy(np.ascontiguousarray(w.u, dtype=np.float64)).to(dev)
    ids_d, st_d = _lib.sample_device(x, prm, u)
    torch.cuda.synchronize()
    assert np.array_equal(ids_d.cpu().numpy(), ids_h)
    assert np.array_equal(st_d.cpu().numpy() & 0xFF, st_h & 0xFF)


def test_device_calls_on_two_streams_use_their_own_workspaces():
    """Two batches sampled alternately on two streams with no wait between
    the calls: each stream's results equal the host call on its batch (the
    device variant keeps one workspace per device and stream; the sliced
    top-p rows here fill it with regions and statistics)."""
    import torch
    from chenxing_amd import _lib
    from chenxing_amd.params import RowParams, pack_rows
    rng = np.random.default_rng(41)
    B, V = 32, 60000
    xs = [rng.normal(0, 2, (B, V)).astype(np.float32) for _ in range(2)]
    prm = [RowParams(temperature=1.0, top_p=0.9) for _ in range(B)]
    us = [rng.random(B) for _ in range(2)]
    want = [_lib.sample_host(x, prm, None, None, u)[:2] for x, u in zip(xs, us)]
    dev = torch.device("cuda:0")
    packed = torch.from_numpy(pack_rows(prm).view(np.uint8).copy()).to(dev)
    streams = [torch.cuda.Stream(device=dev), torch.cuda.Stream(device=dev)]
    xd = [torch.from_numpy(x).to(dev) for x in xs]
    ud = [torch.from_numpy(u).to(dev) for u in us]
    torch.cuda.synchronize()
    _say(f"[gpu] sample_device on two streams B={B} V={V}")
    outs = [[], []]
    for _ in range(3):
        for k in range(2):
            with torch.cuda.stream(streams[k]):
                outs[k].append(_lib.sample_device(xd[k], packed, ud[k]))
    torch.cuda.synchronize()
    for k in range(2):
        for ids, st in outs[k]:
            assert np.array_equal(ids.cpu().numpy(), want[k][0]), k
            assert np.array_equal(st.cpu().numpy() & 0xFF, want[k][1] & 0xFF), k


# ---------------------------------------------- batched row operations at full size
def test_apply_penalties_full_size_workload():
    """B=256, V=128256 rows with 2048-id Zipf histories, repetition,
    presence and frequency penalties: bitwise equal to the oracle."""
    from chenxing_amd import workloads as W
    from chenxing_amd._lib import ROW_OK, apply_penalties_host
    w = W.full_penalty()
    _say(f"[gpu] apply_penalties {w.name} B={w.B} V={w.V}")
    out, st = apply_penalties_host(w.logits, w.params, w.hist, w.hist_len)
    assert np.all(st == ROW_OK)
    hl = R.hist_rows_to_lists(w.hist, w.hist_len)
    for b in range(0, w.B, 17):
        want = R.penalize(w.logits[b], hl[b], w.params[b])
        assert np.array_equal(out[b], want), b


def test_truncate_full_vocab_rows():
    """_truncate on V=128256 probability rows (every filter, alone and
    combined): bitwise equal to the oracle (ties spread over their ids) except
    where a running sum lies within 1e-6 of a cut."""
    from chenxing_amd._lib import ROW_OK, truncate_host
    rng = np.random.default_rng(21)
    V = 128256
    B = 12
    x = rng.normal(0, 2, (B, V))
    x[:, :5] += 8.0
    P = np.exp(x - x.max(axis=1, keepdims=True))
    P /= P.sum(axis=1, keepdims=True)
    P[3] = np.round(P[3] * 1e5) / 1e5                   # many exact ties
    prms = [R.RowParams(top_k=40), R.RowParams(top_p=0.9), R.RowParams(top_k=40, top_p=0.9),
            R.RowParams(top_p=0.5), R.RowParams(min_p=0.05), R.RowParams(typical_p=0.9),
            R.RowParams(top_k=1000, typical_p=0.5), R.RowParams(top_p=0.0),
            R.RowParams(top_k=V + 5), R.RowParams(top_p=0.95, min_p=0.01),
            R.RowParams(top_k=3, top_p=0.99, min_p=0.1, typical_p=0.8), R.RowParams()]
    _say(f"[gpu] _truncate B={B} V={V}")
    out, st = truncate_host(P, prms)
    assert np.all(st == ROW_OK)
    boundary = 0
    for b in range(B):
        diag: dict = {}
        want = R.truncate(P[b].copy(), prms[b], tie="spread", diag=diag)
        if not np.array_equal(out[b], want):
            assert min(diag.get("top_p_margin", 1.0), diag.get("typical_margin", 1.0)) < 1e-6, b
            boundary += 1
    assert boundary <= 1
    bad = P[:2].copy()
    bad[0, 7] = np.nan
    bad[1, 9] = -1e-3
    _, st = truncate_host(bad, [R.RowParams(top_k=5)] * 2)
    assert list(st) == [3, 3]
