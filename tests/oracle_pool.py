"""The oracle over many large rows in a pool of worker processes.

The workers are started with the "spawn" method (a fresh interpreter each,
importing only numpy and the oracle), so a test process that already holds
the GPU forks nothing of its GPU state.  The logits reach them through a
temporary .npy file they memory-map; parameters, histories and uniforms are
small and are pickled.
"""
from __future__ import annotations

import multiprocessing as mp
import os
import tempfile

import numpy as np

_W = {}


def _init(path, dtype, params, hist_lists, u, ties, keep_probs, root):
    import sys
    if root not in sys.path:
        sys.path.insert(0, root)
    _W.update(x=np.load(path, mmap_mode="r"), dtype=dtype, params=params, hist=hist_lists,
              u=u, ties=ties, keep_probs=keep_probs)


def _rows(rng):
    from oracle import sampler_ref as R
    from oracle.bf16 import bf16_bits_to_f32
    out = []
    for b in range(*rng):
        row = np.asarray(_W["x"][b])
        x = bf16_bits_to_f32(row) if _W["dtype"] == "bf16" else row
        h = None if _W["hist"] is None else _W["hist"][b]
        out.append(tuple(R.sample_row(x, _W["params"][b], h, float(_W["u"][b]), tie=t,
                                      keep_probs=_W["keep_probs"]) for t in _W["ties"]))
    return out


def oracle_rows_parallel(w, ties=("spread", "numpy"), keep_probs=False, workers=16) -> list:
    """[(RowResult per tie order) for every row of SampleWorkload ``w``]."""
    from oracle import sampler_ref as R
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    hl = R.hist_rows_to_lists(w.hist, w.hist_len) if w.hist.size else None
    workers = max(1, min(workers, os.cpu_count() or 1, w.B))
    base = "/dev/shm" if os.path.isdir("/dev/shm") else None
    fd, path = tempfile.mkstemp(suffix=".npy", dir=base)
    os.close(fd)
    try:
        np.save(path, w.logits)
        per = (w.B + workers - 1) // workers
        spans = [(k, min(w.B, k + per)) for k in range(0, w.B, per)]
        ctx = mp.get_context("spawn")
        with ctx.Pool(workers, initializer=_init,
                      initargs=(path, w.dtype, list(w.params), hl, np.asarray(w.u), tuple(ties),
                                keep_probs, root)) as pool:
            parts = pool.map(_rows, spans)
    finally:
        os.unlink(path)
    return [r for part in parts for r in part]
