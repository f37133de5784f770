"""Stand-ins for the reference's engine and scheduler objects (the
attributes ``chenxing_amd.decode`` uses), and the reference's per-sequence
decode loop restated (engine.py:160-167, scheduler.py:39-76) to compare
against."""
from __future__ import annotations

from collections import deque
from dataclasses import dataclass, field

import numpy as np


class OutOfKVCacheError(RuntimeError):
    pass


@dataclass
class Seq:
    seq_id: int
    prompt_tokens: list
    params: object
    status: str = "running"
    generated: list = field(default_factory=list)
    n_tokens: int = 0
    last_logits: object = None
    stop_reason: str = ""

    @property
    def total_tokens(self):
        return self.prompt_tokens + self.generated


class Cfg:
    def __init__(self, eos):
        self.eos_token_id = eos


class KV:
    def __init__(self):
        self.evicted = 0

    def evict(self, n):
        self.evicted += n


class Engine:
    """forward_ids returns a row that depends only on (seq_id, position);
    ``oom`` holds (seq_id, position) pairs whose forward runs out of KV."""

    def __init__(self, sampler, V, eos, oom=(), nan=()):
        self.sampler, self.V, self.cfg, self.kv = sampler, V, Cfg(eos), KV()
        self.oom, self.nan = set(oom), set(nan)
        self.log = []

    def forward_ids(self, seq, ids):
        key = (seq.seq_id, seq.n_tokens)
        if key in self.oom:
            self.oom.discard(key)               # succeeds on the retry
            raise OutOfKVCacheError("kv full")
        self.log.append(("fwd",) + key)
        seq.n_tokens += len(ids)
        rng = np.random.default_rng(1000 * seq.seq_id + seq.n_tokens)
        row = rng.normal(0, 2, self.V).astype(np.float32)
        row[rng.integers(0, self.V, 3)] += 6.0
        if key in self.nan:
            row[5] = np.nan
        return row[None]

    def prefill(self, seq):
        seq.last_logits = self.forward_ids(seq, seq.prompt_tokens)[-1]
        seq.status = "running"

    def _publish_prefix(self, seq):
        self.log.append(("publish", seq.seq_id))

    def _release_seq(self, seq):
        self.log.append(("release", seq.seq_id))

    def _preempt_oldest(self):
        self.log.append(("preempt",))

    # engine.py:160-167
    def decode_step(self, seq):
        if seq.n_tokens < len(seq.total_tokens):
            logits = self.forward_ids(seq, seq.total_tokens[seq.n_tokens:seq.n_tokens + 1])
            seq.last_logits = logits[-1]
        tok = self.sampler.sample(seq.last_logits, seq.params, seq.generated)
        seq.generated.append(tok)
        return tok


class Scheduler:
    def __init__(self, engine, max_running=64):
        self.engine, self.max_running = engine, max_running
        self._waiting, self._running, self._finished = deque(), [], []

    def submit(self, seq):
        seq.status = "waiting"
        self._waiting.append(seq)

    # scheduler.py:39-76
    def step(self):
        while self._waiting and len(self._running) < self.max_running:
            seq = self._waiting.popleft()
            try:
                self.engine.prefill(seq)
                self._running.append(seq)
            except OutOfKVCacheError:
                self.engine.kv.evict(1)
                self._waiting.appendleft(seq)
                break
        eos = self.engine.cfg.eos_token_id
        finished_now, still_running = [], []
        for seq in self._running:
            try:
                tok = self.engine.decode_step(seq)
                done = tok == eos or len(seq.generated) >= seq.params.max_tokens
                if done:
                    seq.stop_reason = "eos" if tok == eos else "length"
                    seq.status = "finished"
                    self.engine._publish_prefix(seq)
                    self.engine._release_seq(seq)
                    finished_now.append(seq)
                else:
                    still_running.append(seq)
            except OutOfKVCacheError:
                self.engine._preempt_oldest()
                still_running.append(seq)
        self._running = [s for s in still_running if s.status == "running"]
        self._finished.extend(finished_now)
        return finished_now
