"""Sampling parameters: the reference's ``SamplingParams`` and the packed
per-row block the device library reads.

``SamplingParams`` keeps the reference's fields, defaults and validation
(``chenxing/core/sampler.py:23-43``) and adds ``presence_penalty`` and
``frequency_penalty`` (OpenAI-style, default 0 = off).

``RowParams`` is the device subset; ``ROW_DTYPE`` is its 64-byte packed
layout, identical to ``cx_row_params`` in ``include/cx_sampler.h``.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Iterable

import numpy as np

__all__ = ["SamplingParams", "RowParams", "ROW_DTYPE", "pack_rows"]


@dataclass
class SamplingParams:
    """Per-request sampling configuration (sampler.py:23-35 + pres/freq)."""
    temperature: float = 1.0
    top_k: int = 0                 # 0 = off
    top_p: float = 1.0             # 1.0 = off
    min_p: float = 0.0
    typical_p: float = 1.0
    repetition_penalty: float = 1.0
    max_tokens: int = 64
    seed: int | None = None
    stop: list[str] = field(default_factory=list)
    n_keep: int = 0                # prompt length: penalty window is the last max(64, n_keep) ids
    presence_penalty: float = 0.0  # subtracted once from every id seen in the window
    frequency_penalty: float = 0.0 # subtracted once per occurrence in the window

    def __post_init__(self) -> None:          # sampler.py:37-43
        if not 0.0 <= self.top_p <= 1.0:
            raise ValueError("top_p must be in [0, 1]")
        if not 0.0 <= self.min_p <= 1.0:
            raise ValueError("min_p must be in [0, 1]")
        if self.temperature < 0:
            raise ValueError("temperature must be >= 0")


@dataclass(frozen=True)
class RowParams:
    """What the device needs for one row."""
    temperature: float = 1.0
    top_k: int = 0
    top_p: float = 1.0
    min_p: float = 0.0
    typical_p: float = 1.0
    repetition_penalty: float = 1.0
    presence_penalty: float = 0.0
    frequency_penalty: float = 0.0
    n_keep: int = 0

    @classmethod
    def of(cls, p) -> "RowParams":
        if isinstance(p, RowParams):
            return p
        return cls(temperature=float(p.temperature), top_k=int(p.top_k),
                   top_p=float(p.top_p), min_p=float(p.min_p),
                   typical_p=float(p.typical_p),
                   repetition_penalty=float(p.repetition_penalty),
                   presence_penalty=float(getattr(p, "presence_penalty", 0.0)),
                   frequency_penalty=float(getattr(p, "frequency_penalty", 0.0)),
                   n_keep=int(getattr(p, "n_keep", 0)))


ROW_DTYPE = np.dtype([
    ("temperature", "<f8"), ("top_p", "<f8"), ("min_p", "<f8"), ("typical_p", "<f8"),
    ("repetition_penalty", "<f8"), ("presence_penalty", "<f8"),
    ("frequency_penalty", "<f8"), ("top_k", "<i4"), ("n_keep", "<i4")])
assert ROW_DTYPE.itemsize == 64


def pack_rows(params: Iterable) -> np.ndarray:
    rows = [RowParams.of(p) for p in params]
    out = np.zeros(len(rows), dtype=ROW_DTYPE)
    for i, r in enumerate(rows):
        out[i] = (r.temperature, r.top_p, r.min_p, r.typical_p, r.repetition_penalty,
                  r.presence_penalty, r.frequency_penalty, r.top_k, r.n_keep)
    return out
