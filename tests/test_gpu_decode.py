"""Batched decode step on the device: decode_step_batched (one sample_batch
launch per step) against the reference's per-sequence decode loop with the
drop-in Sampler -- the same tokens and the same generator state."""
from __future__ import annotations

import copy

import numpy as np
import pytest

from chenxing_amd import Sampler, SamplingParams
from chenxing_amd.decode import decode_step_batched
from decode_stub import Engine, Seq

pytestmark = pytest.mark.gpu

V = 32000


def _params(i):
    kinds = [
        SamplingParams(temperature=0.0),
        SamplingParams(temperature=0.7, top_k=40, top_p=0.9, repetition_penalty=1.1),
        SamplingParams(temperature=1.0, top_p=0.9, seed=17 + i),
        SamplingParams(temperature=0.8, top_k=50, presence_penalty=0.5, frequency_penalty=0.3),
        SamplingParams(temperature=1.2, min_p=0.05),
    ]
    return kinds[i % len(kinds)]


def test_batched_decode_matches_per_sequence_loop():
    print("[gpu] batched decode vs per-sequence loop", flush=True)
    sr, sb = Sampler(V), Sampler(V)
    sr._rng = np.random.default_rng(123)
    sb._rng = np.random.default_rng(123)
    er, eb = Engine(sr, V, eos=-1), Engine(sb, V, eos=-1)
    seqs_r = [Seq(i, list(range(3 + i)), _params(i)) for i in range(12)]
    seqs_b = copy.deepcopy(seqs_r)
    for s in seqs_r:
        er.prefill(s)
    for s in seqs_b:
        eb.prefill(s)
    for step in range(6):
        tr = [er.decode_step(s) for s in seqs_r]
        tb = decode_step_batched(eb, seqs_b)
        assert tr == tb, (step, tr, tb)
    assert [s.generated for s in seqs_r] == [s.generated for s in seqs_b]
    assert sr._rng.random() == sb._rng.random()
