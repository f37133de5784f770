"""The allocation-free entry point ``cx_sample_f32_noalloc`` against the
entry point it varies, ``cx_sample_f32``, through the C-ABI: identical ids
and outcomes on two calls in a row (the second with a smaller batch and a
shorter vocabulary, so the static scratch holds the first call's records).
A batch too large for the scratch is refused before any device work
(tests/test_lib_abi.py, on the CPU)."""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _batch(w):
    import torch
    from chenxing_amd.params import pack_rows
    dev = torch.device("cuda:0")
    x = torch.from_numpy(w.logits).to(dev)
    prm = torch.from_numpy(pack_rows(w.params).view(np.uint8).copy()).to(dev)
    u = torch.from_numpy(np.ascontiguousarray(w.u, np.float64)).to(dev)
    h = torch.from_numpy(w.hist).to(dev) if w.hist.size else None
    hl = torch.from_numpy(w.hist_len).to(dev) if w.hist.size else None
    return x, prm, u, h, hl


def test_noalloc_entry_point_matches_the_workspace_entry_point():
    import torch
    from chenxing_amd import _lib, workloads as W
    _lib.load()
    for w in (W.full_penalty(B=256), W.small_batch(B=32, V=30011)):
        print(f"[gpu] noalloc vs workspace entry point B={w.B} V={w.V}", flush=True)
        x, prm, u, h, hl = _batch(w)
        ids_a, st_a = _lib.sample_device(x, prm, u, h, hl)
        ids_b = torch.full((w.B,), -7, dtype=torch.int32, device=x.device)
        st_b = torch.full((w.B,), -7, dtype=torch.int32, device=x.device)
        _lib.sample_device_noalloc(x, prm, u, h, hl, ids_b, st_b)
        torch.cuda.synchronize()
        assert np.array_equal(ids_a.cpu().numpy(), ids_b.cpu().numpy())
        assert np.array_equal(st_a.cpu().numpy() & 0xFF, st_b.cpu().numpy() & 0xFF)


def test_noalloc_entry_point_allocates_nothing():
    """After a warm-up call, a call of the allocation-free entry point with
    preallocated outputs leaves both the device's free memory and torch's
    allocator untouched."""
    import torch
    from chenxing_amd import _lib, workloads as W
    _lib.load()
    w = W.full_penalty(B=64)
    print(f"[gpu] noalloc allocation check B={w.B} V={w.V}", flush=True)
    x, prm, u, h, hl = _batch(w)
    ids = torch.empty(w.B, dtype=torch.int32, device=x.device)
    st = torch.empty(w.B, dtype=torch.int32, device=x.device)
    _lib.sample_device_noalloc(x, prm, u, h, hl, ids, st)       # warm-up
    torch.cuda.synchronize()
    free0, _ = torch.cuda.mem_get_info()
    alloc0 = torch.cuda.memory_allocated()
    _lib.sample_device_noalloc(x, prm, u, h, hl, ids, st)
    torch.cuda.synchronize()
    free1, _ = torch.cuda.mem_get_info()
    assert torch.cuda.memory_allocated() == alloc0
    assert free1 == free0
