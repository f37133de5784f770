"""Batched decode on the device against the oracle: ``decode_step_batched``
and ``scheduler_step_batched`` (one ``Sampler.sample_batch`` launch per step)
with the device ``Sampler``, against the reference's per-sequence loop
(engine.py:160-167, scheduler.py:39-76, restated in tests/decode_stub.py)
whose sampler is the oracle (``OracleSampler``, tie order "stable") with the
same generator seed.  Tokens, finished sequences, stop reasons and the
generator state afterwards must be equal."""
from __future__ import annotations

import copy

import numpy as np
import pytest

from chenxing_amd import Sampler, SamplingParams
from chenxing_amd.decode import decode_step_batched, scheduler_step_batched
from decode_stub import Engine, Scheduler, Seq
from oracle_api import OracleSampler

pytestmark = pytest.mark.gpu

V = 32000


def _params(i):
    kinds = [
        SamplingParams(temperature=0.0),
        SamplingParams(temperature=0.7, top_k=40, top_p=0.9, repetition_penalty=1.1),
        SamplingParams(temperature=1.0, top_p=0.9, seed=17 + i),
        SamplingParams(temperature=0.8, top_k=50, presence_penalty=0.5, frequency_penalty=0.3),
        SamplingParams(temperature=1.2, min_p=0.05),
        SamplingParams(temperature=0.9, top_k=20, top_p=0.8, n_keep=70, repetition_penalty=1.3),
    ]
    p = copy.deepcopy(kinds[i % len(kinds)])
    p.max_tokens = 3 + i % 5
    return p


def _samplers(seed):
    ref, dev = OracleSampler(V, tie="spread"), Sampler(V)
    ref._rng = np.random.default_rng(seed)
    dev._rng = np.random.default_rng(seed)
    return ref, dev


def test_batched_decode_matches_the_oracle_loop():
    print("[gpu] batched decode vs the oracle's per-sequence loop", flush=True)
    sr, sb = _samplers(123)
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


def _state(s):
    seqs = list(s._running) + list(s._finished) + list(s._waiting)
    return sorted((q.seq_id, q.status, tuple(q.generated), q.stop_reason, q.n_tokens)
                  for q in seqs)


def test_batched_scheduler_matches_the_oracle_loop():
    print("[gpu] batched scheduler step vs the oracle's per-sequence loop", flush=True)
    sr, sb = _samplers(7)
    ref = Scheduler(Engine(sr, V, eos=11, oom={(2, 6)}), max_running=6)
    bat = Scheduler(Engine(sb, V, eos=11, oom={(2, 6)}), max_running=6)
    for i in range(10):
        p = _params(i)
        ref.submit(Seq(i, [1, 2, 3 + i], copy.deepcopy(p)))
        bat.submit(Seq(i, [1, 2, 3 + i], copy.deepcopy(p)))
    for _ in range(14):
        fr = [q.seq_id for q in ref.step()]
        fb = [q.seq_id for q in scheduler_step_batched(bat)]
        assert fr == fb
        assert _state(ref) == _state(bat)
    assert not ref._running and not ref._waiting
    assert sr._rng.random() == sb._rng.random()
