"""CPU restatement of the LM head's greedy step: the checker of the device's
fused projection + argmax (cx_lmhead_argmax_bf16).  Test infrastructure:
only tests/, __graft_entry__.smoke() and bench.py's CPU leg use it.

Reference:
  chenxing/model/transformer.py:102-104
      x = rms_norm(x, self.output_norm, c.rms_norm_eps)
      out_w = self.output if self.output is not None else self.tok_emb
      return x @ out_w.T
  chenxing/core/sampler.py:114-115  T == 0: argmax of the penalised row,
      which with no penalty is the row itself (:66, only a repetition
      penalty != 1 changes it).

The device takes the normed hidden states x and the head weights out_w as
bf16 and accumulates in fp32.  This restatement takes the same bf16 bits:
a product of two bf16 values has at most 16 significant bits, so the fp64
products are exact and their fp64 sum is within D * 2^-53 (relative to the
sum of magnitudes) of the exact dot product -- the logits the device
approximates.  ``head_tolerance`` bounds the device's fp32 accumulation
error per logit; a row whose best logit is not clear of every other by
both their bounds is a margin case, where either id is a faithful argmax.

Pins (tests/test_oracle_lmhead.py): brute-force dot products on small
shapes, numpy's fp32 matmul within the bound, argmax ties and NaN as
np.argmax (first maximum, first NaN), vocab permutation invariance.
"""
from __future__ import annotations

import numpy as np

from .bf16 import bf16_bits_to_f32

# MFMA k-slices of 32 are summed into the fp32 accumulator one after
# another; each slice's 32 products are added inside the instruction.  A
# bound with a factor of 2 to spare: (D / 32 + 32) roundings of 2^-24
# relative to the running sum of magnitudes.
def _acc_bound(D: int) -> float:
    return 2.0 * (D / 32.0 + 32.0) * 2.0 ** -24


def head_logits(h_bits: np.ndarray, w_bits: np.ndarray, chunk: int = 8192) -> np.ndarray:
    """Exact-product fp64 logits [B, V] of bf16 hidden [B, D] and weights
    [V, D] (transformer.py:104, ``x @ out_w.T``), in vocab chunks."""
    h = bf16_bits_to_f32(np.asarray(h_bits, np.uint16)).astype(np.float64)
    V = w_bits.shape[0]
    out = np.empty((h.shape[0], V), np.float64)
    for v0 in range(0, V, chunk):
        w = bf16_bits_to_f32(np.asarray(w_bits[v0:v0 + chunk], np.uint16)).astype(np.float64)
        out[:, v0:v0 + chunk] = h @ w.T
    return out


def head_tolerance(h_bits: np.ndarray, w_bits: np.ndarray, chunk: int = 8192) -> np.ndarray:
    """[B, V]: a bound on |device fp32 logit - exact logit|."""
    h = np.abs(bf16_bits_to_f32(np.asarray(h_bits, np.uint16)).astype(np.float64))
    D = h.shape[1]
    V = w_bits.shape[0]
    out = np.empty((h.shape[0], V), np.float64)
    for v0 in range(0, V, chunk):
        w = np.abs(bf16_bits_to_f32(np.asarray(w_bits[v0:v0 + chunk], np.uint16))
                   .astype(np.float64))
        out[:, v0:v0 + chunk] = h @ w.T
    return _acc_bound(D) * out + 1e-300


def greedy_ids(logits: np.ndarray) -> np.ndarray:
    """sampler.py:114-115: np.argmax per row (first maximum; a NaN row
    gives its first NaN)."""
    return np.argmax(logits, axis=1)


def margin_rows(logits: np.ndarray, tol: np.ndarray) -> np.ndarray:
    """Rows whose argmax the device's rounding may move: some other logit
    lies within the two bounds of the best one.  NaN rows are never margin
    cases (the first NaN is exact)."""
    best = greedy_ids(logits)
    out = np.zeros(logits.shape[0], bool)
    for b in range(logits.shape[0]):
        row = logits[b]
        if np.isnan(row).any():
            continue
        v = best[b]
        near = row >= row[v] - (tol[b, v] + tol[b])
        near[v] = False
        out[b] = bool(near.any())
    return out
