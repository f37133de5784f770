"""Batched decode step for the reference's engine and scheduler.

The reference advances each running sequence on its own
(``engine.py:160-167``, ``scheduler.py:55-75``): a forward of the next
uncommitted token, then ``Sampler.sample`` on that sequence's last logits
row, then the finish bookkeeping.  Here the forwards run as before, the rows
are stacked into one ``[B, V]`` batch and sampled with a single
``Sampler.sample_batch`` launch, and the bookkeeping follows in the same
sequence order.

Equivalence.  ``sample_batch`` draws from the sampler's generator in row
order, exactly as the per-sequence calls do, so the tokens, the sequences'
``generated`` lists and the generator's state match the per-sequence loop.
When a row raises (NaN probabilities, ...), the rows before it keep their
tokens, as in the loop, and the exception propagates.

One ordering differs from ``ContinuousBatchingScheduler.step``: there a
sequence that finishes releases its KV blocks before the next sequence's
forward runs; here every forward of the step runs first.  Under KV pressure a
forward may therefore hit ``OutOfKVCacheError`` where the reference's would
not; it is handled as the reference handles it (preempt the oldest other
sequence, retry on the next step).

The engine and scheduler are used through the attributes the reference's
classes have (``forward_ids``, ``sampler``, ``cfg.eos_token_id``, ``kv``,
``_publish_prefix``, ``_release_seq``, ``_preempt_oldest``, ``prefill``;
``engine``, ``_waiting``, ``_running``, ``_finished``, ``max_running``), so
this module does not import the reference.
"""
from __future__ import annotations

from typing import Sequence as Seq

import numpy as np

__all__ = ["decode_step_batched", "scheduler_step_batched"]

_RUNNING = "running"
_FINISHED = "finished"


def _is_kv_full(e: BaseException) -> bool:
    return type(e).__name__ == "OutOfKVCacheError"


def _stack(rows):
    first = rows[0]
    try:
        import torch
        if isinstance(first, torch.Tensor):
            return torch.stack([r.reshape(-1) for r in rows])
    except ImportError:
        pass
    return np.stack([np.asarray(r).reshape(-1) for r in rows])


def _forward(engine, seq) -> None:
    """The forward half of ``LLMEngine.decode_step`` (engine.py:162-164)."""
    if seq.n_tokens < len(seq.total_tokens):
        logits = engine.forward_ids(seq, seq.total_tokens[seq.n_tokens:seq.n_tokens + 1])
        seq.last_logits = logits[-1]


def _sample(engine, seqs) -> list[int]:
    """The sampling half of ``decode_step`` for every sequence, one launch;
    appends each token to its sequence (engine.py:165-166)."""
    if not seqs:
        return []
    x = _stack([s.last_logits for s in seqs])
    try:
        toks = engine.sampler.sample_batch(x, [s.params for s in seqs],
                                           [s.generated for s in seqs])
    except ValueError as e:
        for seq, tok in zip(seqs, getattr(e, "tokens_before", ())):
            seq.generated.append(tok)
        raise
    for seq, tok in zip(seqs, toks):
        seq.generated.append(tok)
    return toks


def decode_step_batched(engine, seqs: Seq) -> list[int]:
    """``[engine.decode_step(s) for s in seqs]`` with one sampling launch."""
    seqs = list(seqs)
    for seq in seqs:
        _forward(engine, seq)
    return _sample(engine, seqs)


def scheduler_step_batched(sched) -> list:
    """``ContinuousBatchingScheduler.step`` (scheduler.py:39-76) with the
    running sequences' tokens sampled in one launch.  Returns the sequences
    that finished during this step."""
    eng = sched.engine
    # admission, as the reference (scheduler.py:44-53)
    while sched._waiting and len(sched._running) < sched.max_running:
        seq = sched._waiting.popleft()
        try:
            eng.prefill(seq)
            sched._running.append(seq)
        except Exception as e:
            if not _is_kv_full(e):
                raise
            eng.kv.evict(1)
            sched._waiting.appendleft(seq)
            break

    # forwards; a sequence whose forward runs out of KV blocks preempts the
    # oldest other sequence and retries on the next step (scheduler.py:71-74)
    ready, retry = [], set()
    for seq in sched._running:
        try:
            _forward(eng, seq)
            ready.append(seq)
        except Exception as e:
            if not _is_kv_full(e):
                raise
            eng._preempt_oldest()
            retry.add(id(seq))

    toks = dict(zip((id(s) for s in ready), _sample(eng, ready)))

    # bookkeeping in sequence order (scheduler.py:62-70)
    eos = eng.cfg.eos_token_id
    finished_now, still_running = [], []
    for seq in sched._running:
        if id(seq) in retry:
            still_running.append(seq)
            continue
        tok = toks[id(seq)]
        done = tok == eos or len(seq.generated) >= seq.params.max_tokens
        if done:
            seq.stop_reason = "eos" if tok == eos else "length"
            seq.status = _FINISHED
            eng._publish_prefix(seq)
            eng._release_seq(seq)
            finished_now.append(seq)
        else:
            still_running.append(seq)
    sched._running = [s for s in still_running if s.status == _RUNNING]
    sched._finished.extend(finished_now)
    return finished_now
