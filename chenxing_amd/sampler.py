"""Drop-in ``Sampler`` with every computation on the device.

Mirrors ``chenxing/core/sampler.py:46-127``: the same constructor, methods,
return types and exceptions, so a caller of the reference (``engine.py:165``,
``speculative.py:126,171``, ``scheduler.py:61``) can swap classes:

  Sampler(vocab_size)
  .sample(logits, params, generated_ids=None) -> int        sampler.py:108-127
  .apply_penalties(logits, params, generated_ids) -> fp64   sampler.py:63-73
  ._truncate(probs, params) -> fp64                         sampler.py:75-106
  ._rng, ._rng_for(seed)                                    sampler.py:54-61

plus ``sample_batch`` for a decode batch in one launch.  The arithmetic runs
in the HIP library (``include/cx_sampler.h``); this module only marshals
arguments, supplies the uniforms and maps row outcomes to the reference's
exceptions.  Without the built library every method raises.

Uniforms.  The reference draws exactly one variate, inside
``Generator.choice``, and only on rows that reach it: greedy rows, rows whose
filtered mass is zero (argmax fallback) and rows numpy rejects draw nothing.
A seeded call uses a fresh ``default_rng(seed)``; an unseeded one the
sampler's own generator.  Here the next variate is read before the launch
and the generator is rewound when the device reports that the row did not
draw, so the generator advances exactly as the reference's does.
"""
from __future__ import annotations

import array
import threading
from typing import Sequence

import numpy as np

from . import _lib

try:
    from . import _cxhist
except ImportError as e:          # built beside libcx_sampler.so by build.py
    raise ImportError("chenxing_amd._cxhist is not built: run chenxing_amd/build.py") from e
from .params import RowParams, SamplingParams, pack_rows

__all__ = ["Sampler", "SamplingParams"]

# Longest penalty window one launch of the device's penalty index holds
# (distinct ids when only the repetition and presence penalties are on).
WINDOW_MAX = 4095


class _Groups(list):
    """A penalty window longer than WINDOW_MAX, as groups of at most
    WINDOW_MAX ids with disjoint id sets (every occurrence of an id in one
    group).  The penalties act on each id alone, from its value and its count
    (sampler.py:70-72), so applying the groups one after another gives the
    row that one pass over the whole window would."""

_NUMPY_NAN = "probabilities contain NaN"          # numpy Generator.choice's message
_NUMPY_SIZE = "'a' and 'p' must have same size"


def _is_torch_cuda(x) -> bool:
    try:
        import torch
    except ImportError:
        return False
    return isinstance(x, torch.Tensor) and x.is_cuda


class Sampler:
    """Logits processor + sampler (sampler.py:46-127) on the GPU."""

    def __init__(self, vocab_size: int) -> None:
        self.vocab_size = vocab_size
        self._rng = np.random.default_rng()
        self._lock = threading.Lock()
        _lib.load()

    def _rng_for(self, seed: int | None) -> np.random.Generator:
        if seed is None:
            return self._rng
        return np.random.default_rng(seed)

    # ------------------------------------------------------------ arguments
    @staticmethod
    def _window_seq(params, generated_ids):
        """The slice of the history the penalties read (sampler.py:66-67), or
        None when no penalty is on."""
        rp = float(params.repetition_penalty)
        pres = float(getattr(params, "presence_penalty", 0.0))
        freq = float(getattr(params, "frequency_penalty", 0.0))
        if rp == 1.0 and pres == 0.0 and freq == 0.0:
            return None
        if generated_ids is None or len(generated_ids) == 0:
            return None
        n_keep = int(getattr(params, "n_keep", 0))
        return generated_ids[-max(64, n_keep):] if n_keep else generated_ids

    def _window(self, params, generated_ids, V: int):
        """The history handed to the device for one row: the reference's
        penalty window (sampler.py:67) with ids outside [0, vocab_size)
        replaced by -1 (:68).  None when no penalty is on."""
        seq = self._window_seq(params, generated_ids)
        if seq is None:
            return None
        rp = float(params.repetition_penalty)
        freq = float(getattr(params, "frequency_penalty", 0.0))
        if isinstance(seq, np.ndarray):
            h = seq.astype(np.int64)
        else:
            try:
                # array('q') unboxes a list of ints fastest
                h = np.frombuffer(array.array("q", seq), dtype=np.int64)
            except TypeError:
                h = np.fromiter(seq, dtype=np.int64, count=len(seq))
            except OverflowError:
                h = np.asarray([t if -1 <= t < 2**62 else -1 for t in seq], dtype=np.int64)
        if rp != 1.0 and V < self.vocab_size:
            bad = (h >= V) & (h < self.vocab_size)
            if bad.any():
                # the reference indexes the row with every in-range id
                raise IndexError(f"index {int(h[bad][0])} is out of bounds for axis 0 "
                                 f"with size {V}")
        h = np.where((h >= 0) & (h < min(V, self.vocab_size)), h, -1)
        if h.size > WINDOW_MAX:
            h = h[h >= 0]
        if h.size <= WINDOW_MAX:
            return h.astype(np.int32)
        ids, cnt = np.unique(h, return_counts=True)
        if freq == 0.0:
            # repetition and presence penalties depend on the set of ids only
            if ids.size <= WINDOW_MAX:
                return ids.astype(np.int32)
            return _Groups(ids[i:i + WINDOW_MAX].astype(np.int32)
                           for i in range(0, ids.size, WINDOW_MAX))
        if int(cnt.max()) > WINDOW_MAX:
            raise ValueError(f"frequency penalty over an id seen {int(cnt.max())} times in "
                             f"the window: the device counts at most {WINDOW_MAX}")
        # the ids with their counts, packed in id order into groups of at
        # most WINDOW_MAX occurrences
        groups, start, n = _Groups(), 0, 0
        for i, c in enumerate(cnt.tolist()):
            if n + c > WINDOW_MAX:
                groups.append(np.repeat(ids[start:i], cnt[start:i]).astype(np.int32))
                start, n = i, 0
            n += c
        groups.append(np.repeat(ids[start:], cnt[start:]).astype(np.int32))
        return groups

    def _windows(self, plist, hists, V: int):
        """Every row's penalty window: (wins, lists).  Plain lists (or tuples)
        of at most WINDOW_MAX ids are kept as they are, their rows listed in
        ``lists``, for _cxhist's C loop; every other window (numpy arrays,
        long windows, rows indexed beyond a short V) goes through _window."""
        fast = V >= self.vocab_size
        wins, lists = [], []
        for b, (p, h) in enumerate(zip(plist, hists)):
            seq = self._window_seq(p, h) if fast else None
            if fast and type(seq) in (list, tuple) and len(seq) <= WINDOW_MAX:
                wins.append(seq)
                lists.append(b)
            else:
                wins.append(self._window(p, [] if h is None else h, V))
        return wins, lists

    def _history_arrays(self, wins, lists, plist, hists, V: int):
        """The int32 [B, H] history and hist_len [B] the library takes (None,
        None when no row has a window).  Rows of ``lists`` are written by
        _cxhist.fill; a row it returns (an item that is not a plain int) gets
        numpy's conversion and errors through _window, as in ``sample``."""
        on_list = set(lists)
        H = max((len(w) if b in on_list else w.size for b, w in enumerate(wins)
                 if w is not None), default=0)
        if H == 0:
            return None, None
        B = len(wins)
        hist = np.full((B, H), -1, np.int32)
        hist_len = np.zeros(B, np.int32)
        if lists:
            for b in _cxhist.fill([wins[b] for b in lists], lists, hist, hist_len,
                                  self.vocab_size):
                wins[b] = self._window(plist[b], hists[b], V)
                on_list.discard(b)
                hist[b] = -1
        for b, w in enumerate(wins):
            if w is not None and b not in on_list:
                hist[b, :w.size] = w
                hist_len[b] = w.size
        return hist, hist_len

    @staticmethod
    def _penalise_groups(row, bf16: bool, params, groups: _Groups) -> np.ndarray:
        """The fp64 row with a long window's penalties applied, group by
        group, on the device (one apply_penalties launch per group)."""
        prm = [RowParams.of(params)]
        out = np.asarray(row)[None]
        for k, g in enumerate(groups):
            out, st = _lib.apply_penalties_host(out, prm, g[None], bf16=bf16 and k == 0)
            if st[0] != _lib.ROW_OK:
                raise ValueError(f"apply_penalties: device status {int(st[0])}")
        return out[0]

    @staticmethod
    def _as_row(logits) -> tuple[np.ndarray, bool]:
        x = np.asarray(logits)
        if x.ndim != 1:
            raise ValueError("logits must be a 1-D row")
        if x.dtype not in (np.float32, np.float64):
            x = x.astype(np.float64)            # the reference's first step (sampler.py:65)
        return np.ascontiguousarray(x), False

    # ------------------------------------------------------------ reference API
    def apply_penalties(self, logits: np.ndarray, params,
                        generated_ids: list[int]) -> np.ndarray:
        """fp64 copy of the row with the penalties applied (sampler.py:63-73)."""
        x, _ = self._as_row(logits)
        win = self._window(params, generated_ids, x.size)
        if isinstance(win, _Groups):
            return self._penalise_groups(x, False, params, win)
        hist = None if win is None else win[None]
        out, st = _lib.apply_penalties_host(x[None], [RowParams.of(params)], hist)
        if st[0] != _lib.ROW_OK:
            raise ValueError(f"apply_penalties: device status {int(st[0])}")
        return out[0]

    def _truncate(self, probs: np.ndarray, params) -> np.ndarray:
        """top-k / top-p / min-p / typical-p filter (sampler.py:75-106): the
        input values where kept, zero elsewhere; not renormalised."""
        p = np.asarray(probs, dtype=np.float64)
        if p.ndim != 1:
            raise ValueError("probs must be a 1-D row")
        out, st = _lib.truncate_host(p[None], [RowParams.of(params)])
        if st[0] != _lib.ROW_OK:
            raise ValueError("_truncate expects finite, non-negative probabilities")
        return out[0]

    def sample(self, logits: np.ndarray, params,
               generated_ids: list[int] | None = None) -> int:
        """Draw one token id from ``logits`` (1-D, vocab size) (sampler.py:108-127)."""
        if _is_torch_cuda(logits):
            return self.sample_batch(logits.reshape(1, -1), [params],
                                     [generated_ids or []])[0]
        x, _ = self._as_row(logits)
        return self.sample_batch(x[None], [params], [generated_ids or []])[0]

    # ------------------------------------------------------------ batched
    def sample_batch(self, logits, params: Sequence | object,
                     generated_ids: Sequence[Sequence[int]] | None = None) -> list[int]:
        """``sample`` for every row of ``logits`` [B, V] in one launch.

        Equivalent to ``[self.sample(logits[b], params[b], generated_ids[b])
        for b in range(B)]``, including the order in which rows draw from
        the sampler's generator and the exception the first failing row
        raises (its ``tokens_before`` attribute holds the tokens of the rows
        before it).  ``logits`` is a numpy array (float32 or float64) or a CUDA
        tensor (float32, bfloat16 or float64) that stays on the device.
        """
        on_dev = _is_torch_cuda(logits)
        if on_dev:
            import torch
            B, V = int(logits.shape[0]), int(logits.shape[1])
        else:
            x = np.asarray(logits)
            if x.ndim != 2:
                raise ValueError("logits must be [B, V]")
            if x.dtype not in (np.float32, np.float64):
                x = x.astype(np.float64)
            x = np.ascontiguousarray(x)
            B, V = x.shape
        plist = list(params) if isinstance(params, (list, tuple)) else [params] * B
        if len(plist) != B:
            raise ValueError("need one SamplingParams per row")
        hists = list(generated_ids) if generated_ids is not None else [[]] * B
        if len(hists) != B:
            raise ValueError("need one history per row")
        if B == 0:
            return []
        wins, lists = self._windows(plist, hists, V)
        # rows whose window one launch cannot hold: their penalised fp64 rows
        # (group by group), sampled with the penalties off on the exact fp64
        # path; the other rows take the batch launch
        longs = [b for b, w in enumerate(wins) if isinstance(w, _Groups)]
        pen = prm_long = None
        if longs:
            rows_l = []
            for b in longs:
                if on_dev:
                    r = logits[b]
                    bf = r.dtype == torch.bfloat16
                    r = (r.view(torch.int16).cpu().numpy().view(np.uint16) if bf
                         else r.cpu().numpy())
                else:
                    r, bf = x[b], False
                rows_l.append(self._penalise_groups(r, bf, plist[b], wins[b]))
                wins[b] = None
            pen = np.stack(rows_l)
            prm_long = pack_rows([plist[b] for b in longs])
            for f in ("presence_penalty", "frequency_penalty"):
                prm_long[f] = 0.0
            prm_long["repetition_penalty"] = 1.0
        hist, hist_len = self._history_arrays(wins, lists, plist, hists, V)
        prm = pack_rows(plist)
        stoch = [float(p.temperature) != 0.0 for p in plist]
        seeds = [getattr(p, "seed", None) for p in plist]

        def run(u, rows=None):
            """Sample every row, or the listed rows only (returned in that order)."""
            if not longs:
                return run_batch(u, rows)
            sel = list(range(B)) if rows is None else list(rows)
            at = {b: i for i, b in enumerate(longs)}
            ids = np.empty(len(sel), np.int32)
            st = np.empty(len(sel), np.int32)
            ia = [i for i, b in enumerate(sel) if b not in at]
            il = [i for i, b in enumerate(sel) if b in at]
            if ia:
                ids[ia], st[ia] = run_batch(u, [sel[i] for i in ia])
            if il:
                li = [at[sel[i]] for i in il]
                ids[il], st[il], _ = _lib.sample_host(pen[li], prm_long[li], None, None,
                                                      u[[sel[i] for i in il]])
            return ids, st

        def run_batch(u, rows=None):
            sel = slice(None) if rows is None else rows
            h = None if hist is None else hist[sel]
            hl = None if hist_len is None else hist_len[sel]
            if on_dev:
                xs = logits if rows is None else logits.index_select(
                    0, torch.as_tensor(rows, device=logits.device))
                return self._run_device(xs, prm[sel], u[sel], h, hl)
            ids, st, _ = _lib.sample_host(x if rows is None else x[rows], prm[sel], h, hl, u[sel])
            return ids, st

        with self._lock:
            state = self._rng.bit_generator.state
            u = self._uniforms(stoch, seeds, None)
            ids, st = run(u)
            draws = [(int(s) & 0xFF) == _lib.ROW_OK for s in st]
            if any(stoch[b] and seeds[b] is None and not draws[b] for b in range(B)):
                # a row that draws nothing must not take a variate from the
                # shared generator: the variates go to the drawing rows only,
                # and the rows whose variate moved are sampled again (whether
                # a row draws does not depend on its variate)
                self._rng.bit_generator.state = state
                u2 = self._uniforms(stoch, seeds, draws)
                redo = [b for b in range(B) if draws[b] and u2[b] != u[b]]
                if redo:
                    ids = np.array(ids)
                    st = np.array(st)
                    ids[redo], st[redo] = run(u2, redo)
            out = []
            self._rng.bit_generator.state = state
            for b in range(B):
                code = int(st[b]) & 0xFF
                err = None
                if code == _lib.ROW_OK and V != self.vocab_size:
                    err = ValueError(_NUMPY_SIZE)      # choice(vocab_size, p) (:127)
                elif code == _lib.ROW_ERROR:
                    err = ValueError(_NUMPY_NAN)
                elif code == _lib.ROW_UNSUPPORTED:
                    err = ValueError("row outside the sampler library's limits")
                if err is not None:
                    # the tokens of the rows before it, which the per-row
                    # loop would have returned before raising
                    err.tokens_before = out
                    raise err
                if code == _lib.ROW_OK and seeds[b] is None:
                    self._rng.random()                 # the variate this row drew
                out.append(int(ids[b]))
            return out

    def _uniforms(self, stoch, seeds, draws) -> np.ndarray:
        """One variate per row: fresh default_rng(seed) for seeded rows, the
        shared generator's next variate (in row order) for unseeded rows that
        draw (all stochastic rows when ``draws`` is None)."""
        u = np.zeros(len(stoch))
        for b, s in enumerate(stoch):
            if not s or (draws is not None and not draws[b]):
                continue
            u[b] = np.random.default_rng(seeds[b]).random() if seeds[b] is not None \
                else self._rng.random()
        return u

    @staticmethod
    def _run_device(logits, prm: np.ndarray, u: np.ndarray, hist, hist_len):
        import torch
        dev = logits.device
        prm_d = torch.from_numpy(prm.view(np.uint8).copy()).to(dev)
        u_d = torch.from_numpy(u).to(dev)
        h_d = hl_d = None
        if hist is not None:
            h_d = torch.from_numpy(hist).to(dev)
            hl_d = torch.from_numpy(hist_len).to(dev)
        ids, st = _lib.sample_device(logits, prm_d, u_d, h_d, hl_d)
        return ids.cpu().numpy(), st.cpu().numpy()
