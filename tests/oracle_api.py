"""``Sampler.sample`` semantics (sampler.py:54-61,108-127) on the oracle, for
tests that drive a whole engine loop with a CPU checker: the same generator
bookkeeping as the reference (a seeded call uses a fresh
``default_rng(seed)``, an unseeded one the sampler's own generator; a row
that draws nothing consumes no variate) and the same exception."""
from __future__ import annotations

import numpy as np

from oracle import sampler_ref as R


class OracleSampler:
    def __init__(self, vocab_size: int, tie: str = "numpy"):
        self.vocab_size = vocab_size
        self.tie = tie
        self._rng = np.random.default_rng()

    def sample(self, logits, params, generated_ids=None):
        prm = R.RowParams(temperature=params.temperature, top_k=params.top_k,
                          top_p=params.top_p, min_p=params.min_p, typical_p=params.typical_p,
                          repetition_penalty=params.repetition_penalty,
                          presence_penalty=getattr(params, "presence_penalty", 0.0),
                          frequency_penalty=getattr(params, "frequency_penalty", 0.0),
                          n_keep=params.n_keep)
        g = self._rng if params.seed is None else np.random.default_rng(params.seed)
        st = g.bit_generator.state
        res = R.sample_row(np.asarray(logits), prm, generated_ids or [], g.random(),
                           tie=self.tie)
        if res.status != R.STATUS_OK:
            g.bit_generator.state = st
        if res.status == R.STATUS_ERROR:
            raise ValueError("probabilities contain NaN")
        return res.token
