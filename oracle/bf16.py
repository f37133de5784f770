"""Exact bf16 <-> fp32 conversion for the oracle.

TEST INFRASTRUCTURE ONLY -- see ``oracle/__init__.py``.

bf16 is the top 16 bits of an IEEE fp32.  fp32 -> bf16 rounds to nearest,
ties to even; NaNs stay quiet NaNs.  Pinned against torch's CPU
``Tensor.to(torch.bfloat16)`` (tests/test_oracle_sampler.py).
"""
from __future__ import annotations

import numpy as np


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    lsb = (u >> 16) & 1
    r = ((u + 0x7FFF + lsb) >> 16).astype(np.uint16)
    nan = np.isnan(np.asarray(x, dtype=np.float32))
    if nan.any():
        r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)
