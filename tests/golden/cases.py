"""Deterministic inputs for the golden vectors.

Shared by ``make_golden.py`` (which feeds them to the reference in the build
container) and by the tests (which feed them to the oracle and the device
library).  Everything here is a pure function of its seed, so the fixtures
only hold seeds, input digests and the reference's outputs.
"""
from __future__ import annotations

import hashlib
from dataclasses import dataclass, field
from types import SimpleNamespace

import numpy as np


def digest(a: np.ndarray) -> str:
    a = np.ascontiguousarray(a)
    return hashlib.sha256(a.tobytes() + str(a.dtype).encode()).hexdigest()[:16]


# ----------------------------------------------------------------- sampler cases
@dataclass
class SamplerCase:
    name: str
    logits: np.ndarray                       # [V] fp32
    params: dict                             # SamplingParams fields (reference names)
    hist: list = field(default_factory=list)


_T = [0.0, 0.3, 0.7, 1.0, 1.5]
_K = [0, 0, 1, 3, 8, 50]
_P = [1.0, 1.0, 0.9, 0.5, 0.0, 0.95]
_MINP = [0.0, 0.0, 0.0, 0.05, 0.3]
_TYP = [1.0, 1.0, 1.0, 0.9, 0.5]
_RP = [1.0, 1.0, 1.1, 0.8, 2.0]


def _row(rng: np.random.Generator, V: int, kind: str) -> np.ndarray:
    if kind == "normal":
        x = rng.normal(0.0, 2.0, V)
    elif kind == "spiky":
        x = rng.normal(0.0, 1.0, V)
        x[rng.choice(V, min(3, V), replace=False)] += 6.0
    elif kind == "quantized":          # many exact ties, like bf16 logits
        x = np.round(rng.normal(0.0, 2.0, V) * 2.0) / 2.0
    elif kind == "flat":
        x = np.zeros(V)
    elif kind == "neginf":
        x = rng.normal(0.0, 2.0, V)
        x[rng.choice(V, max(1, V // 4), replace=False)] = -np.inf
    else:
        raise ValueError(kind)
    return x.astype(np.float32)


def small_sampler_cases(n: int = 240) -> list[SamplerCase]:
    """Small-V cases covering every knob, the tie and -inf edge cases."""
    out = []
    kinds = ["normal", "spiky", "quantized", "normal", "flat", "neginf"]
    for i in range(n):
        rng = np.random.default_rng(10_000 + i)
        V = int(rng.choice([2, 5, 12, 40, 257]))
        kind = kinds[i % len(kinds)]
        x = _row(rng, V, kind)
        prm = dict(temperature=float(rng.choice(_T)), top_k=int(rng.choice(_K)),
                   top_p=float(rng.choice(_P)), min_p=float(rng.choice(_MINP)),
                   typical_p=float(rng.choice(_TYP)),
                   repetition_penalty=float(rng.choice(_RP)),
                   n_keep=int(rng.choice([0, 0, 70])), seed=int(rng.integers(0, 2**31)))
        H = int(rng.choice([0, 3, 80]))
        hist = [int(t) for t in rng.integers(-2, V + 2, H)]
        out.append(SamplerCase(f"small{i}_{kind}_V{V}", x, prm, hist))
    # hand-made edge rows
    nan_row = np.array([0.5, np.nan, 2.0, 1.0], dtype=np.float32)
    inf_row = np.array([0.5, np.inf, 2.0, 1.0], dtype=np.float32)
    for j, (row, extra) in enumerate([(nan_row, {}), (nan_row, {"top_k": 2}),
                                      (inf_row, {}), (inf_row, {"min_p": 0.1}),
                                      (nan_row, {"temperature": 0.0})]):
        prm = dict(temperature=1.0, top_k=0, top_p=1.0, min_p=0.0, typical_p=1.0,
                   repetition_penalty=1.0, n_keep=0, seed=7)
        prm.update(extra)
        out.append(SamplerCase(f"edge_bad{j}", row.copy(), prm, []))
    # temperature underflow: flat-ish row, tiny T
    rng = np.random.default_rng(77)
    flat = rng.normal(0.0, 0.1, 300).astype(np.float32)
    for j, extra in enumerate([{}, {"top_k": 5}, {"top_p": 0.5}, {"min_p": 0.2},
                               {"top_p": 0.5, "min_p": 0.2}]):
        prm = dict(temperature=0.001, top_k=0, top_p=1.0, min_p=0.0, typical_p=1.0,
                   repetition_penalty=1.0, n_keep=0, seed=3)
        prm.update(extra)
        out.append(SamplerCase(f"edge_underflow{j}", flat.copy(), prm, []))
    return out


def medium_sampler_cases() -> list[SamplerCase]:
    """Config-1-sized rows (V = 32000): spikes, penalties, k/p/T mixes."""
    out = []
    for i in range(12):
        rng = np.random.default_rng(20_000 + i)
        V = 32000
        x = rng.normal(0.0, 2.0, V)
        x[rng.choice(V, 5, replace=False)] += 8.0
        prm = dict(temperature=[0.8, 1.0, 0.5, 0.0][i % 4], top_k=[50, 0, 40, 0][i % 4],
                   top_p=[0.9, 0.95, 0.9, 1.0][i % 4], min_p=0.0, typical_p=1.0,
                   repetition_penalty=[1.1, 1.0, 1.3, 1.1][i % 4], n_keep=0,
                   seed=int(rng.integers(0, 2**31)))
        hist = [int(t) for t in rng.integers(0, V, 64)]
        out.append(SamplerCase(f"medium{i}", x.astype(np.float32), prm, hist))
    return out


def truncate_input(case: SamplerCase) -> np.ndarray:
    """A probability vector to feed ``_truncate`` directly (tests call it so)."""
    rng = np.random.default_rng(int(digest(case.logits)[:8], 16))
    x = case.logits.astype(np.float64)
    with np.errstate(all="ignore"):
        e = np.exp(x - np.max(x))
        P = e / e.sum()
    if not np.all(np.isfinite(P)):
        P = rng.random(case.logits.size)
        P /= P.sum()
    return P


# ----------------------------------------------------------------- speculative
@dataclass
class ScriptedSeq:
    seq_id: int
    prompt_tokens: list
    params: object
    generated: list = field(default_factory=list)
    n_tokens: int = 0
    last_logits: object = None
    radix_node: object = None
    status: str = "waiting"
    stop_reason: str = ""

    @property
    def total_tokens(self) -> list:
        return self.prompt_tokens + self.generated


class ScriptedEngine:
    """Duck-typed stand-in for ``LLMEngine`` as ``SpeculativeDecoder`` uses it.

    The next-token logits depend only on (last token, position), so a target
    and a draft built from the same ``base_seed`` see correlated rows; the
    draft adds N(0, noise) per element.
    """

    def __init__(self, V: int, base_seed: int, noise: float, noise_seed: int,
                 sampler, eos: int | None = None):
        self.V = V
        self.base_seed = base_seed
        self.noise = noise
        self.noise_seed = noise_seed
        self.sampler = sampler
        self.cfg = SimpleNamespace(eos_token_id=(V - 1 if eos is None else eos),
                                   vocab_size=V)
        self._next = 0
        self.forward_log: list = []

    def row(self, last_tok: int, pos: int) -> np.ndarray:
        r = np.random.default_rng([self.base_seed, last_tok + 7, pos])
        x = r.normal(0.0, 2.0, self.V)
        x[int(r.integers(0, self.V))] += 3.0
        if self.noise:
            n = np.random.default_rng([self.noise_seed, last_tok + 7, pos])
            x = x + n.normal(0.0, self.noise, self.V)
        return x.astype(np.float32)

    def create_sequence(self, prompt_tokens, params=None):
        self._next += 1
        return ScriptedSeq(self._next, list(prompt_tokens), params)

    def prefill(self, seq):
        seq.n_tokens = len(seq.prompt_tokens)
        seq.last_logits = self.row(seq.prompt_tokens[-1], seq.n_tokens - 1)
        return seq.last_logits

    def forward_ids(self, seq, new_ids, *, allow_unconfirmed=False):
        n0 = seq.n_tokens
        rows = np.stack([self.row(int(t), n0 + j) for j, t in enumerate(new_ids)])
        seq.n_tokens += len(new_ids)
        self.forward_log.append((n0, list(map(int, new_ids))))
        return rows

    def _publish_prefix(self, seq):
        return None

    def _release_seq(self, seq):
        return None


def spec_cases() -> list[dict]:
    """Speculative generate() configurations (gamma, T, seeds, vocab)."""
    out = []
    i = 0
    for gamma in (1, 2, 4, 8):
        for T in (0.0, 0.7, 1.0, 1.3):
            for noise in (0.0, 0.6, 2.0):
                i += 1
                out.append(dict(name=f"spec{i}_g{gamma}_T{T}_n{noise}", gamma=gamma,
                                temperature=T, noise=noise, V=96, base_seed=300 + i,
                                noise_seed=900 + i, seed=40 + i, max_tokens=20,
                                prompt=[int(t) for t in
                                        np.random.default_rng(i).integers(0, 90, 6)]))
    return out
