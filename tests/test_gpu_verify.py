"""Speculative verify parity on the GPU against the oracle: accept/reject
decisions and accepted counts bit-exact; correction tokens equal except
boundary draws (tests/parity.py rules)."""
from __future__ import annotations

import numpy as np
import pytest

from chenxing_amd import workloads as W
from chenxing_amd._lib import spec_verify_host
from oracle import speculative_ref as S

pytestmark = pytest.mark.gpu


def _compare(w, acc, nxt, used):
    boundary = 0
    for b in range(w.target.shape[0]):
        r = S.verify_round(w.target[b], w.draft[b], w.draft_ids[b], w.u[b],
                           float(w.temperature[b]))
        assert acc[b] == r.accepted, (b, acc[b], r.accepted)
        assert used[b] == r.uniforms_used, (b, used[b], r.uniforms_used)
        if nxt[b] != r.next_tok:
            assert r.diag.get("draw_margin", 1.0) < 1e-6, (b, nxt[b], r.next_tok, r.diag)
            boundary += 1
    return boundary


@pytest.mark.parametrize("greedy", [False, True])
def test_spec_verify_config(greedy):
    w = W.spec_verify(greedy=greedy)
    print(f"[gpu] verify {w.name}", flush=True)
    acc, nxt, used, st = spec_verify_host(w.target, w.draft, w.draft_ids, w.u, w.temperature)
    assert _compare(w, acc, nxt, used) == 0


def test_spec_verify_small_mixed():
    """Mixed greedy / stochastic sequences, several temperatures, small V."""
    rng = np.random.default_rng(4)
    B, g, V = 48, 5, 3000
    tgt = rng.normal(0, 2, (B, g + 1, V)).astype(np.float32)
    drf = (tgt[:, :g] + rng.normal(0, 0.7, (B, g, V))).astype(np.float32)
    ids = np.empty((B, g), np.int32)
    T = rng.choice([0.0, 0.5, 1.0, 1.7], B).astype(np.float32)
    for b in range(B):
        for i in range(g):
            ids[b, i] = tgt[b, i].argmax() if rng.random() < 0.5 else rng.integers(0, V)
    u = rng.random((B, g + 1))
    w = W.VerifyWorkload("mixed", tgt, drf, ids, u, T)
    print("[gpu] verify mixed", flush=True)
    acc, nxt, used, st = spec_verify_host(tgt, drf, ids, u, T)
    # boundary draws within the 1e-4-of-draws budget: none at 48 sequences
    assert _compare(w, acc, nxt, used) <= 1e-4 * B


def test_identical_draft_accepts_everything():
    rng = np.random.default_rng(9)
    B, g, V = 8, 4, 5000
    tgt = rng.normal(0, 2, (B, g + 1, V)).astype(np.float32)
    ids = rng.integers(0, V, (B, g)).astype(np.int32)
    print("[gpu] verify identical draft", flush=True)
    acc, nxt, used, st = spec_verify_host(tgt, tgt[:, :g].copy(), ids, rng.random((B, g + 1)),
                                          np.ones(B, np.float32))
    assert np.all(acc == g) and np.all(nxt == -1) and np.all(used == g)


def test_device_variant_repeated_calls_reuse_the_workspace():
    """Three device calls in a row on one workspace, with different shapes,
    inputs and greedy / stochastic mixes (so each call finds the previous
    call's values in the workspace), each equal to the oracle."""
    import torch
    from chenxing_amd._lib import spec_verify_device
    dev = torch.device("cuda:0")
    for k, (B, g, V) in enumerate([(6, 3, 40000), (9, 7, 70001), (4, 2, 8192)]):
        rng = np.random.default_rng(100 + k)
        tgt = rng.normal(0, 2, (B, g + 1, V)).astype(np.float32)
        drf = (tgt[:, :g] + rng.normal(0, 0.6, (B, g, V))).astype(np.float32)
        ids = rng.integers(0, V, (B, g)).astype(np.int32)
        ids[:, 0] = tgt[:, 0].argmax(axis=1)
        T = rng.choice([0.0, 0.8, 1.0], B).astype(np.float32)
        u = rng.random((B, g + 1))
        print(f"[gpu] verify device call {k} B={B} g={g} V={V}", flush=True)
        outs = spec_verify_device(*(torch.from_numpy(a).to(dev) for a in (tgt, drf, ids, u, T)))
        acc, nxt, used, st = (o.cpu().numpy() for o in outs)
        assert _compare(W.VerifyWorkload(f"dev{k}", tgt, drf, ids, u, T), acc, nxt, used) <= 1e-4 * B


def test_rejections_at_every_position():
    """Drafts built so the first rejection falls at each position in turn
    (position gamma = all accepted)."""
    rng = np.random.default_rng(31)
    B, g, V = 10, 9, 20000
    tgt = rng.normal(0, 2, (B, g + 1, V)).astype(np.float32)
    drf = tgt[:, :g].copy()
    ids = np.empty((B, g), np.int32)
    u = rng.random((B, g + 1))
    for b in range(B):
        for i in range(g):
            ids[b, i] = tgt[b, i].argmax()
        r = b % (g + 1)
        if r < g:                                  # make position r reject for sure
            drf[b, r] = tgt[b, r]
            drf[b, r, ids[b, r]] += 12.0           # q[tok] >> p[tok]
            u[b, r] = 0.999
    T = np.ones(B, np.float32)
    print("[gpu] verify rejection positions", flush=True)
    acc, nxt, used, st = spec_verify_host(tgt, drf, ids, u, T)
    w = W.VerifyWorkload("positions", tgt, drf, ids, u, T)
    assert _compare(w, acc, nxt, used) <= 1e-4 * B
    assert [int(a) for a in acc] == [min(b % (g + 1), g) for b in range(B)]
