"""The fused LM head + greedy argmax (cx_lmhead_argmax_bf16) against the
oracle (oracle/lmhead_ref.py: transformer.py:102-104 then sampler.py:114-115)
through the C-ABI: logits within the fp32 accumulation bound, greedy ids
bit-exact except counted margin rows (another logit within the bound of the
best), ties to the lowest id, the first NaN."""
from __future__ import annotations

import numpy as np
import pytest

from oracle import lmhead_ref as H
from oracle.bf16 import f32_to_bf16_bits

pytestmark = pytest.mark.gpu


def _dev(bits):
    import torch
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).cuda().view(torch.bfloat16)


def _host(t):
    import torch
    return t.view(torch.int16).cpu().numpy().view(np.uint16)


def _run(h_bits, w_bits, want_logits=True):
    import torch
    from chenxing_amd._lib import lmhead_argmax_device
    h, w = _dev(h_bits), _dev(w_bits)
    lg = torch.empty((h.shape[0], w.shape[0]), dtype=torch.float32, device="cuda") \
        if want_logits else None
    ids, mx = lmhead_argmax_device(h, w, out_logits=lg)
    torch.cuda.synchronize()
    return ids.cpu().numpy(), mx.cpu().numpy(), None if lg is None else lg.cpu().numpy()


def _check(h_bits, w_bits, ids, mx, logits=None):
    exact = H.head_logits(h_bits, w_bits)
    tol = H.head_tolerance(h_bits, w_bits)
    if logits is not None:
        bad = np.abs(logits.astype(np.float64) - exact) > tol
        assert not bad.any(), (np.argwhere(bad)[:5], np.abs(logits - exact).max())
    want = H.greedy_ids(exact)
    margin = H.margin_rows(exact, tol)
    for b in range(len(ids)):
        v = int(want[b])
        if not margin[b]:
            assert ids[b] == v, (b, ids[b], v)
            assert abs(float(mx[b]) - exact[b, v]) <= tol[b, v]
        else:
            # another logit within the bounds of the best: the device's id
            # must be one of those near the top
            near = exact[b] >= exact[b, v] - (tol[b, v] + tol[b])
            assert near[ids[b]], (b, ids[b], v)
    return int(margin.sum())


@pytest.mark.parametrize("B,D,V", [(1, 128, 1000), (5, 256, 4099), (16, 1024, 2048),
                                   (33, 512, 3001), (64, 1024, 5000), (100, 256, 777)])
def test_small_shapes_logits_and_ids(B, D, V):
    print(f"[gpu] lm head B={B} D={D} V={V}", flush=True)
    rng = np.random.default_rng(B * 7 + D + V)
    h = f32_to_bf16_bits(rng.normal(0, 1, (B, D)).astype(np.float32))
    w = f32_to_bf16_bits(rng.normal(0, 0.05, (V, D)).astype(np.float32))
    ids, mx, lg = _run(h, w)
    _check(h, w, ids, mx, lg)


def test_ties_and_nan():
    print("[gpu] lm head ties and NaN", flush=True)
    rng = np.random.default_rng(9)
    B, D, V = 4, 256, 600
    h = f32_to_bf16_bits(rng.normal(0, 1, (B, D)).astype(np.float32))
    w = f32_to_bf16_bits(rng.normal(0, 0.05, (V, D)).astype(np.float32))
    best = H.greedy_ids(H.head_logits(h, w))
    # copies of row 0's best row at a lower id in the same tile, in another
    # tile and in another workgroup: the lowest copy wins
    w2 = w.copy()
    src = int(best[0])
    for dst in (src - 1, 3, 130, 599):
        if 0 <= dst < V and dst != src:
            w2[dst] = w[src]
    ids, _, _ = _run(h, w2, want_logits=False)
    want = H.greedy_ids(H.head_logits(h, w2))
    assert ids[0] == want[0] == min(d for d in (src - 1, 3, 130, 599, src) if 0 <= d < V)
    # NaN weights: the first NaN logit is the argmax of every row
    w3 = w.copy()
    w3[[400, 77], 9] = 0x7FC0
    ids, mx, _ = _run(h, w3, want_logits=False)
    assert list(ids) == [77] * B and np.isnan(mx).all()


def test_full_vocab_decode_batch():
    """A Llama-3-8B-sized head (D=4096, V=128256) at a decode batch of 16."""
    import torch
    print("[gpu] lm head B=16 D=4096 V=128256", flush=True)
    g = torch.Generator(device="cuda")
    g.manual_seed(1234)
    w = (torch.randn(128256, 4096, generator=g, device="cuda") * 0.02).to(torch.bfloat16)
    h = torch.randn(16, 4096, generator=g, device="cuda").to(torch.bfloat16)
    from chenxing_amd._lib import lmhead_argmax_device
    ids, mx = lmhead_argmax_device(h, w)
    torch.cuda.synchronize()
    ids, mx = ids.cpu().numpy(), mx.cpu().numpy()
    h_bits, w_bits = _host(h), _host(w)
    del w
    margin = _check(h_bits, w_bits, ids, mx)
    print(f"[gpu] lm head full vocab: margin rows {margin}", flush=True)


def test_argument_errors():
    import torch
    from chenxing_amd._lib import lmhead_argmax_device
    h = torch.zeros((2, 100), dtype=torch.bfloat16, device="cuda")
    w = torch.zeros((10, 100), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ValueError):
        lmhead_argmax_device(h, w)                     # D not a multiple of 128
    with pytest.raises(ValueError):
        lmhead_argmax_device(h.float(), w.float())
