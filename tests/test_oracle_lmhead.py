"""Pins of oracle/lmhead_ref.py: the LM head's projection
(transformer.py:102-104) and the greedy argmax (sampler.py:114-115) on
bf16 operands.  CPU only."""
from __future__ import annotations

import numpy as np
import pytest

from oracle import lmhead_ref as H
from oracle.bf16 import bf16_bits_to_f32, f32_to_bf16_bits


def _bits(rng, shape, scale):
    return f32_to_bf16_bits(rng.normal(0, scale, shape).astype(np.float32))


def test_logits_equal_brute_force_dot_products():
    rng = np.random.default_rng(1)
    h, w = _bits(rng, (3, 256), 1.0), _bits(rng, (50, 256), 0.05)
    got = H.head_logits(h, w, chunk=16)
    hf, wf = bf16_bits_to_f32(h), bf16_bits_to_f32(w)
    for b in range(3):
        for v in range(50):
            exact = sum(float(hf[b, k]) * float(wf[v, k]) for k in range(256))
            assert abs(got[b, v] - exact) <= 1e-12 * (1 + abs(exact))


def test_fp32_matmul_lies_within_the_bound():
    # numpy's fp32 matmul is one faithful fp32 accumulation: within the bound
    rng = np.random.default_rng(2)
    h, w = _bits(rng, (4, 1024), 1.0), _bits(rng, (300, 1024), 0.02)
    exact = H.head_logits(h, w)
    tol = H.head_tolerance(h, w)
    f32 = bf16_bits_to_f32(h) @ bf16_bits_to_f32(w).T
    assert np.all(np.abs(f32 - exact) <= tol)
    # the bound is not vacuous: well below the spread of the logits
    assert tol.max() < 1e-3 * exact.std()


def test_argmax_ties_and_nan_follow_numpy():
    rng = np.random.default_rng(3)
    h, w = _bits(rng, (2, 128), 1.0), _bits(rng, (40, 128), 0.05)
    lg = H.head_logits(h, w)
    best = H.greedy_ids(lg)
    # a duplicate of the best row placed before it wins (first maximum)
    b0 = int(best[0])
    w2 = np.concatenate([w[b0:b0 + 1], w], axis=0)
    assert H.greedy_ids(H.head_logits(h, w2))[0] == 0
    # a NaN weight makes that logit NaN: the first NaN is the argmax
    w3 = w.copy()
    w3[[7, 20], 5] = 0x7FC0
    assert list(H.greedy_ids(H.head_logits(h, w3))) == [7, 7]
    assert not H.margin_rows(H.head_logits(h, w3), H.head_tolerance(h, w)).any()


def test_vocab_permutation_permutes_the_argmax():
    rng = np.random.default_rng(4)
    h, w = _bits(rng, (5, 256), 1.0), _bits(rng, (200, 256), 0.05)
    perm = rng.permutation(200)
    a = H.greedy_ids(H.head_logits(h, w))
    b = H.greedy_ids(H.head_logits(h, w[perm]))
    assert np.array_equal(perm[b], a)


def test_margin_rows_flag_near_ties_only():
    rng = np.random.default_rng(5)
    h, w = _bits(rng, (2, 128), 1.0), _bits(rng, (30, 128), 0.05)
    lg = H.head_logits(h, w)
    tol = H.head_tolerance(h, w)
    assert not H.margin_rows(lg, tol).any()
    lg2 = lg.copy()
    v = int(H.greedy_ids(lg)[1])
    other = (v + 1) % 30
    lg2[1, other] = lg2[1, v] - 0.5 * tol[1, v]        # inside the bound
    assert list(H.margin_rows(lg2, tol)) == [False, True]
