"""Speculative decoding with the verify step on the device.

``SpeculativeDecoder`` keeps the reference's constructor, ``generate``
signature, statistics and round structure (``chenxing/engine/speculative.py``
:72-200).  The round loop (drafting, the target forward, commit and KV
rollback) stays host Python because it drives the engines; the verify block
(:145-171) is one call into the HIP library, which evaluates every draft
position in parallel and reports the first rejection.

Uniforms: the reference draws from one ``default_rng(params.seed)`` per
``generate`` -- one variate per accept test and one inside the residual
``choice``.  Each round pre-draws ``gamma + 1`` variates, lets the device
consume what the reference would have, and then rewinds the generator to
exactly that many draws, so the stream stays aligned with the reference.
"""
from __future__ import annotations

import numpy as np

from .params import SamplingParams

__all__ = ["SpeculativeDecoder", "SpeculativeStats", "DeviceVerifier"]

BONUS = -1


class SpeculativeStats:
    """Counters of speculative.py:43-64."""

    def __init__(self) -> None:
        self.drafted = 0
        self.accepted = 0
        self.steps = 0

    @property
    def acceptance_rate(self) -> float:
        return self.accepted / max(self.drafted, 1)

    @property
    def mean_accepted_per_step(self) -> float:
        return self.accepted / max(self.steps, 1)

    def as_dict(self) -> dict:
        return {
            "steps": self.steps,
            "drafted": self.drafted,
            "accepted": self.accepted,
            "acceptance_rate": round(self.acceptance_rate, 4),
            "mean_accepted_per_step": round(self.mean_accepted_per_step, 3),
        }


# Greedy draft proposals are ``int(np.argmax(q_row))`` (speculative.py:125):
# the draft engine's sampler at T = 0 with no history computes exactly that.
_GREEDY = SamplingParams(temperature=0.0)


class DeviceVerifier:
    """One verify round through ``cx_spec_verify_f32_host``."""

    def __init__(self) -> None:
        from . import _lib
        self._lib = _lib.load()

    def __call__(self, target: np.ndarray, draft: np.ndarray, draft_ids, u: np.ndarray,
                 temperature: float) -> tuple[int, int, int]:
        from ._lib import spec_verify_host
        acc, nxt, used, status = spec_verify_host(
            target[None], draft[None], np.asarray(draft_ids, np.int32)[None],
            np.asarray(u, np.float64)[None], np.array([temperature], np.float32))
        return int(acc[0]), int(nxt[0]), int(used[0])


class SpeculativeDecoder:
    """Draft gamma tokens with a small model; verify with the target in one pass."""

    def __init__(self, engine, draft_engine, *, num_speculative_tokens: int = 4,
                 verifier=None) -> None:
        if num_speculative_tokens < 1:
            raise ValueError("need at least 1 speculative token")
        self.engine = engine
        self.draft = draft_engine
        self.k_draft = num_speculative_tokens
        self.stats = SpeculativeStats()
        self._verify = verifier if verifier is not None else DeviceVerifier()

    def _sync_to(self, seq, eng, n_target: int) -> None:
        """Set a sequence's committed KV length to ``n_target`` (speculative.py:86-92)."""
        if seq.n_tokens > n_target:
            seq.n_tokens = n_target
        elif seq.n_tokens < n_target:
            eng.forward_ids(seq, seq.total_tokens[seq.n_tokens:n_target],
                            allow_unconfirmed=True)

    def _propose(self, dseq, confirmed: list, params, greedy: bool) -> tuple[list, list]:
        """Draft gamma tokens autoregressively (speculative.py:117-132)."""
        n_start = len(confirmed) - 1
        self._sync_to(dseq, self.draft, n_start)
        q_rows, proposed = [], []
        q_rows.append(self.draft.forward_ids(dseq, [confirmed[n_start]],
                                             allow_unconfirmed=True)[-1])
        for i in range(self.k_draft):
            row = q_rows[-1]
            if greedy and isinstance(row, np.ndarray):
                # a host row: the reference's own argmax (speculative.py:125),
                # no device round trip for one id
                tok = int(np.argmax(row))
            elif greedy:
                tok = self.draft.sampler.sample(row, _GREEDY)
            else:
                tok = self.draft.sampler.sample(row, params, confirmed)
            proposed.append(tok)
            self.stats.drafted += 1
            if i < self.k_draft - 1:
                q_rows.append(self.draft.forward_ids(dseq, [tok],
                                                     allow_unconfirmed=True)[-1])
        return q_rows, proposed

    def generate(self, prompt_tokens: list[int], params: SamplingParams | None = None,
                 *, stop_ids: set[int] | None = None) -> tuple[list[int], str]:
        params = params or SamplingParams()
        eos = self.engine.cfg.eos_token_id
        stops = set(stop_ids or ()) | {eos}

        tseq = self.engine.create_sequence(prompt_tokens, params)
        dseq = self.draft.create_sequence(prompt_tokens, params)
        try:
            self.engine.prefill(tseq)
            self.draft.prefill(dseq)
            confirmed = list(prompt_tokens)
            tseq.n_tokens -= 1
            dseq.n_tokens -= 1
            rng = np.random.default_rng(params.seed)
            greedy = params.temperature == 0.0
            gamma = self.k_draft

            while len(confirmed) - len(prompt_tokens) < params.max_tokens:
                n_start = len(confirmed) - 1
                q_rows, proposed = self._propose(dseq, confirmed, params, greedy)

                self._sync_to(tseq, self.engine, n_start)
                logits_t = self.engine.forward_ids(tseq, [confirmed[n_start]] + proposed,
                                                   allow_unconfirmed=True)

                if greedy:
                    u = np.zeros(gamma + 1)
                else:
                    state = rng.bit_generator.state
                    u = rng.random(gamma + 1)
                accepted_n, next_tok, used = self._verify(
                    np.ascontiguousarray(logits_t, dtype=np.float32),
                    np.ascontiguousarray(np.stack(q_rows), dtype=np.float32),
                    proposed, u, float(params.temperature))
                if not greedy:
                    rng.bit_generator.state = state
                    if used:
                        rng.random(used)
                if next_tok == BONUS:
                    next_tok = self.engine.sampler.sample(logits_t[-1], params, confirmed)

                self.stats.accepted += accepted_n
                self.stats.steps += 1

                confirmed.extend(proposed[:accepted_n])
                confirmed.append(int(next_tok))
                if accepted_n < self.k_draft:
                    target_len = len(confirmed) - 1
                    self._sync_to(dseq, self.draft, target_len)
                    self._sync_to(tseq, self.engine, target_len)

                tseq.generated = confirmed[len(prompt_tokens):]
                dseq.generated = tseq.generated
                tseq.last_logits = logits_t[-1] if len(logits_t) else None

                if any(t in stops for t in confirmed[len(prompt_tokens):]):
                    break

            out = confirmed[len(prompt_tokens):][:params.max_tokens]
            reason = "eos" if any(t == eos for t in out) else "length"
            self.engine._publish_prefix(tseq)
            return out, reason
        finally:
            self.engine._release_seq(tseq)
            self.draft._release_seq(dseq)
