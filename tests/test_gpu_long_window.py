"""Penalty windows longer than one launch's penalty index (4095 ids) through
the drop-in ``Sampler`` (sampler.py:63-73, :108-127): the window is applied
on the device in groups of disjoint ids, and the penalised fp64 row sampled
on the exact path.  Every row must equal the oracle's, and the penalised row
the oracle's bit for bit."""
from __future__ import annotations

import sys

import numpy as np
import pytest

from chenxing_amd import Sampler, SamplingParams
from oracle import sampler_ref as R

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _batch(freq, seed):
    rng = np.random.default_rng(seed)
    B, V, H = 6, 128256, 10_000
    x = rng.standard_normal((B, V), dtype=np.float32) * np.float32(2.0)
    x[np.arange(B), rng.integers(0, V, B)] += np.float32(6.0)
    hists = [rng.integers(0, V, H).tolist() for _ in range(B)]
    hists[1][:6000] = rng.integers(0, 300, 6000).tolist()      # repeated ids
    hists[2] = hists[2][:3000]                                  # fits one launch
    hists[3][100:200] = [-1] * 50 + [V + 7] * 50                # ids the window drops
    kinds = [(0.0, 0, 1.0), (0.7, 40, 0.9), (1.0, 0, 0.9), (0.7, 0, 1.0), (1.0, 40, 1.0),
             (0.8, 0, 0.95)]
    params = [SamplingParams(temperature=t, top_k=k, top_p=p, repetition_penalty=1.3,
                             presence_penalty=0.4, frequency_penalty=freq, seed=1000 + b)
              for b, (t, k, p) in enumerate(kinds)]
    return x, hists, params


def _oracle(x, hists, params):
    out = []
    for b, p in enumerate(params):
        rp = R.RowParams(temperature=p.temperature, top_k=p.top_k, top_p=p.top_p,
                         repetition_penalty=p.repetition_penalty,
                         presence_penalty=p.presence_penalty,
                         frequency_penalty=p.frequency_penalty)
        u = np.random.default_rng(p.seed).random()
        out.append(R.sample_row(x[b], rp, hists[b], u, tie="spread").token)
    return out


@pytest.mark.parametrize("freq", [0.0, 0.3])
def test_windows_beyond_one_launch(freq):
    x, hists, params = _batch(freq, 41 + int(freq * 10))
    s = Sampler(x.shape[1])
    _say(f"[gpu] long windows freq={freq}: penalised rows")
    for b in (0, 1):
        got = s.apply_penalties(x[b], params[b], hists[b])
        rp = R.RowParams(repetition_penalty=params[b].repetition_penalty,
                         presence_penalty=params[b].presence_penalty,
                         frequency_penalty=params[b].frequency_penalty)
        assert np.array_equal(got.view(np.int64), R.penalize(x[b], hists[b], rp).view(np.int64))
    want = _oracle(x, hists, params)
    _say(f"[gpu] long windows freq={freq}: numpy batch")
    assert s.sample_batch(x, params, hists) == want
    import torch
    _say(f"[gpu] long windows freq={freq}: device tensor batch")
    assert s.sample_batch(torch.from_numpy(x).cuda(), params, hists) == want


def test_windows_beyond_one_launch_bf16_device_rows():
    import torch
    x, hists, params = _batch(0.3, 77)
    xb = torch.from_numpy(x).cuda().to(torch.bfloat16)
    want = _oracle(xb.float().cpu().numpy(), hists, params)
    _say("[gpu] long windows: bf16 device tensor batch")
    assert Sampler(x.shape[1]).sample_batch(xb, params, hists) == want


def test_unseeded_rows_after_a_long_window_and_an_argmax_row():
    """Unseeded rows share the sampler's generator: a row that falls back to
    argmax (a NaN logit under top-k, sampler.py:123-125) draws nothing, a
    long-window row takes the separate fp64 launch, and the rows after them
    take the next variates in order.  Tokens and the generator state after
    the batch equal the reference's sequential calls."""
    from oracle_api import OracleSampler
    rng = np.random.default_rng(5)
    B, V = 5, 128256
    x = rng.standard_normal((B, V), dtype=np.float32) * np.float32(2.0)
    x[0, 17] = np.nan
    hists = [[], rng.integers(0, V, 10_000).tolist(), [], rng.integers(0, V, 300).tolist(), []]
    params = [SamplingParams(temperature=1.0, top_k=40),
              SamplingParams(temperature=0.8, top_p=0.9, repetition_penalty=1.2),
              SamplingParams(temperature=1.0),
              SamplingParams(temperature=0.7, top_k=40, repetition_penalty=1.1),
              SamplingParams(temperature=1.2, top_p=0.95)]
    dev, ref = Sampler(V), OracleSampler(V, tie="spread")
    dev._rng = np.random.default_rng(2024)
    ref._rng = np.random.default_rng(2024)
    want = [ref.sample(x[b], params[b], hists[b]) for b in range(B)]
    _say("[gpu] unseeded rows after a long window and an argmax row")
    got = dev.sample_batch(x, params, hists)
    assert got == want
    assert dev._rng.bit_generator.state == ref._rng.bit_generator.state
