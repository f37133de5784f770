"""ctypes binding of ``libcx_sampler.so`` (declared in ``include/cx_sampler.h``).

``load()`` raises if the library is missing: there is no CPU fallback.
Host entry points take numpy arrays; device entry points take torch tensors
that already live on the GPU and run on the current torch stream.
"""
from __future__ import annotations

import ctypes as C
import os
import threading

import numpy as np

from .params import ROW_DTYPE, pack_rows

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libcx_sampler.so")

CX_OK, CX_EINVAL, CX_EHIP, CX_ENOSPACE = 0, -1, -2, -3
ROW_OK, ROW_GREEDY, ROW_ARGMAX, ROW_ERROR, ROW_UNSUPPORTED = 0, 1, 2, 3, 4
FLAG_SLOW, FLAG_EXACT, FLAG_DEEP = 0x100, 0x200, 0x400

_lib = None
_lock = threading.Lock()

_P = C.c_void_p
_SIGS = {
    "cx_sample_f32": (C.c_int, [_P, C.c_int64, C.c_int32, C.c_int32, _P, _P, C.c_int64, _P, _P,
                                _P, _P, _P, _P, C.c_size_t, _P]),
    "cx_sample_bf16": (C.c_int, [_P, C.c_int64, C.c_int32, C.c_int32, _P, _P, C.c_int64, _P, _P,
                                 _P, _P, _P, _P, C.c_size_t, _P]),
    "cx_sample_f64": (C.c_int, [_P, C.c_int64, C.c_int32, C.c_int32, _P, _P, C.c_int64, _P, _P,
                                _P, _P, _P, _P, C.c_size_t, _P]),
    "cx_sample_workspace_bytes": (C.c_size_t, [C.c_int32, C.c_int32, C.c_int64]),
    "cx_sample_f32_noalloc": (C.c_int, [_P, C.c_int64, C.c_int32, C.c_int32, _P, _P, C.c_int64,
                                        _P, _P, _P, _P, _P, _P]),
    "cx_apply_penalties": (C.c_int, [_P, C.c_int32, C.c_int64, C.c_int32, C.c_int32, _P, _P,
                                     C.c_int64, _P, _P, C.c_int64, _P, _P]),
    "cx_apply_penalties_host": (C.c_int, [_P, C.c_int32, C.c_int64, C.c_int32, C.c_int32, _P,
                                          _P, C.c_int64, _P, _P, _P]),
    "cx_truncate_f64": (C.c_int, [_P, C.c_int64, C.c_int32, C.c_int32, _P, _P, C.c_int64, _P,
                                  _P]),
    "cx_truncate_host": (C.c_int, [_P, C.c_int64, C.c_int32, C.c_int32, _P, _P, _P]),
    "cx_sample_host": (C.c_int, [_P, C.c_int32, C.c_int64, C.c_int32, C.c_int32, _P, _P,
                                 C.c_int64, _P, _P, _P, _P, _P]),
    "cx_spec_verify_f32": (C.c_int, [_P, _P, _P, _P, _P, C.c_int32, C.c_int32, C.c_int32, _P, _P,
                                     _P, _P, _P, C.c_size_t, _P]),
    "cx_spec_verify_workspace_bytes": (C.c_size_t, [C.c_int32, C.c_int32, C.c_int32]),
    "cx_spec_verify_host": (C.c_int, [_P, _P, _P, _P, _P, C.c_int32, C.c_int32, C.c_int32, _P,
                                      _P, _P, _P]),
    "cx_lmhead_argmax_bf16": (C.c_int, [_P, C.c_int64, _P, C.c_int64, C.c_int32, C.c_int32,
                                        C.c_int32, _P, _P, _P, _P, C.c_size_t, _P]),
    "cx_lmhead_workspace_bytes": (C.c_size_t, [C.c_int32, C.c_int32]),
    "cx_timing_enable": (C.c_int, [C.c_int]),
    "cx_timing_read": (C.c_int, [C.c_int32, _P, _P]),
    "cx_last_error": (C.c_char_p, []),
    "cx_version": (C.c_char_p, []),
}


class CxError(RuntimeError):
    """A HIP or argument failure inside the library."""


def load(path: str | None = None):
    """Load the HIP library once; raise if it is not built."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        p = path or LIB_PATH
        if not os.path.exists(p):
            raise CxError(f"{p} is not built; run `python -m chenxing_amd.build` "
                          "(the sampler has no CPU fallback)")
        # One HIP runtime per process: torch bundles its own libamdhip64.so.7,
        # and the first copy loaded serves every later library with that
        # soname, so torch (when installed) is loaded first.
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
        lib = C.CDLL(p)
        for name, (res, args) in _SIGS.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
        return lib


def _check(rc: int) -> None:
    if rc != CX_OK:
        msg = _lib.cx_last_error().decode()
        if rc == CX_EINVAL:
            raise ValueError(msg)
        raise CxError(f"cx_sampler error {rc}: {msg}")


def _ptr(a: np.ndarray | None):
    return None if a is None else a.ctypes.data_as(_P)


def _prep_hist(hist, hist_len, B):
    if hist is None or np.asarray(hist).size == 0:
        return None, None, 0
    h = np.ascontiguousarray(hist, dtype=np.int32)
    if h.ndim != 2 or h.shape[0] != B:
        raise ValueError("hist must be [B, H]")
    hl = (np.full(B, h.shape[1], np.int32) if hist_len is None
          else np.ascontiguousarray(hist_len, dtype=np.int32))
    return h, hl, h.shape[1]


def _prep_params(params, B):
    prm = params if isinstance(params, np.ndarray) and params.dtype == ROW_DTYPE \
        else pack_rows(params if isinstance(params, (list, tuple)) else [params] * B)
    if prm.shape[0] != B:
        raise ValueError("need one parameter row per logits row")
    return np.ascontiguousarray(prm)


def _logits_dtype(logits, bf16: bool):
    """(contiguous array, dtype code): fp32 = 0, bf16 bits = 1, fp64 = 2."""
    if bf16:
        return np.ascontiguousarray(logits, dtype=np.uint16), 1
    a = np.asarray(logits)
    if a.dtype == np.float64:
        return np.ascontiguousarray(a), 2
    return np.ascontiguousarray(a, dtype=np.float32), 0


def sample_host(logits: np.ndarray, params, hist=None, hist_len=None, u=None,
                bf16: bool = False, want_probs: bool = False):
    """Numpy in / numpy out: (ids [B], status [B], probs [B, V] or None).

    ``logits`` is [B, V] float32 or float64 (float64 rows take the exact
    multi-pass path), or uint16 bf16 bit patterns with ``bf16=True``.
    """
    lib = load()
    x, code = _logits_dtype(logits, bf16)
    if x.ndim != 2:
        raise ValueError("logits must be [B, V]")
    B, V = x.shape
    prm = _prep_params(params, B)
    uu = np.zeros(B) if u is None else np.ascontiguousarray(u, dtype=np.float64)
    h, hl, ldh = _prep_hist(hist, hist_len, B)
    ids = np.empty(B, np.int32)
    st = np.empty(B, np.int32)
    probs = np.empty((B, V), np.float32) if want_probs else None
    _check(lib.cx_sample_host(_ptr(x), code, V, B, V, _ptr(h), _ptr(hl), ldh,
                              _ptr(prm), _ptr(uu), _ptr(ids), _ptr(st), _ptr(probs)))
    return ids, st, probs


def apply_penalties_host(logits: np.ndarray, params, hist=None, hist_len=None,
                         bf16: bool = False):
    """[B, V] logits (fp32, fp64 or bf16 bits) -> (fp64 [B, V], status [B])."""
    lib = load()
    x, code = _logits_dtype(logits, bf16)
    if x.ndim != 2:
        raise ValueError("logits must be [B, V]")
    B, V = x.shape
    prm = _prep_params(params, B)
    h, hl, ldh = _prep_hist(hist, hist_len, B)
    out = np.empty((B, V), np.float64)
    st = np.empty(B, np.int32)
    _check(lib.cx_apply_penalties_host(_ptr(x), code, V, B, V, _ptr(h), _ptr(hl), ldh,
                                       _ptr(prm), _ptr(out), _ptr(st)))
    return out, st


def truncate_host(probs: np.ndarray, params):
    """[B, V] fp64 probabilities -> (filtered fp64 [B, V], status [B])."""
    lib = load()
    p = np.ascontiguousarray(probs, dtype=np.float64)
    if p.ndim != 2:
        raise ValueError("probs must be [B, V]")
    B, V = p.shape
    prm = _prep_params(params, B)
    out = np.empty((B, V), np.float64)
    st = np.empty(B, np.int32)
    _check(lib.cx_truncate_host(_ptr(p), V, B, V, _ptr(prm), _ptr(out), _ptr(st)))
    return out, st


def spec_verify_host(target: np.ndarray, draft: np.ndarray | None, draft_ids: np.ndarray,
                     u: np.ndarray, temperature: np.ndarray):
    """target [B, g+1, V], draft [B, g, V], draft_ids [B, g], u [B, g+1], T [B]
    -> (accepted [B], next_tok [B], used [B], status [B])."""
    lib = load()
    t = np.ascontiguousarray(target, dtype=np.float32)
    B, g1, V = t.shape
    g = g1 - 1
    d = None if draft is None else np.ascontiguousarray(draft, dtype=np.float32)
    if d is not None and d.shape != (B, g, V):
        raise ValueError("draft must be [B, gamma, V]")
    ids = np.ascontiguousarray(draft_ids, dtype=np.int32).reshape(B, g)
    if np.any(ids < 0) or np.any(ids >= V):
        raise ValueError("draft ids must be in [0, V)")
    uu = np.ascontiguousarray(u, dtype=np.float64).reshape(B, g1)
    T = np.ascontiguousarray(np.broadcast_to(np.asarray(temperature, np.float32), (B,)))
    acc, nxt, used, st = (np.empty(B, np.int32) for _ in range(4))
    _check(lib.cx_spec_verify_host(_ptr(t), _ptr(d), _ptr(ids), _ptr(uu), _ptr(T), B, g, V,
                                   _ptr(acc), _ptr(nxt), _ptr(used), _ptr(st)))
    return acc, nxt, used, st


# ------------------------------------------------------------------ device entry points
class Workspace:
    """Zero-filled device scratch buffers, one per (device, stream), grown on
    demand.  The library's calls on one stream run in order and can share a
    buffer; calls on different streams (or from threads using different
    streams) must not, since each call's kernels use the buffer for the
    rows' regions and statistics.  A buffer is allocated on the stream it
    serves, so replacing it with a larger one is ordered after the calls
    already queued there."""

    def __init__(self):
        self.bufs: dict = {}
        self.lock = threading.Lock()

    def get(self, nbytes: int, device, stream_ptr: int):
        import torch
        key = (device.index, stream_ptr)
        with self.lock:
            buf = self.bufs.get(key)
            if buf is None or buf.numel() < nbytes:
                buf = torch.zeros(max(nbytes, 256), dtype=torch.uint8, device=device)
                self.bufs[key] = buf
            return buf


_ws_sample = Workspace()
_ws_verify = Workspace()
_ws_head = Workspace()


def _stream_ptr(device):
    import torch
    return C.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def sample_device(logits, prm, u, hist=None, hist_len=None, out_id=None, row_status=None,
                  out_probs=None):
    """Device-resident batch sample on the current stream (no synchronisation).

    logits: [B, V] cuda tensor, float32 or bfloat16 (row stride may exceed V);
    prm: cuda uint8 tensor holding [B] cx_row_params (see ``params.ROW_DTYPE``);
    u: [B] float64; hist: [B, H] int32 (+ hist_len [B] int32) or None.
    Returns (out_id, row_status) int32 tensors."""
    import torch
    lib = load()
    if logits.dim() != 2 or logits.stride(1) != 1:
        raise ValueError("logits must be a [B, V] tensor with unit column stride")
    B, V = logits.shape
    dev = logits.device
    if out_id is None:
        out_id = torch.empty(B, dtype=torch.int32, device=dev)
    if row_status is None:
        row_status = torch.empty(B, dtype=torch.int32, device=dev)
    ldh = 0 if hist is None else hist.shape[1]
    nbytes = lib.cx_sample_workspace_bytes(B, V, ldh)
    sp = _stream_ptr(dev)
    ws = _ws_sample.get(nbytes, dev, sp.value)
    fns = {torch.bfloat16: lib.cx_sample_bf16, torch.float32: lib.cx_sample_f32,
           torch.float64: lib.cx_sample_f64}
    if logits.dtype not in fns:
        raise ValueError("logits must be float32, bfloat16 or float64")
    fn = fns[logits.dtype]
    _check(fn(_P(logits.data_ptr()), logits.stride(0), B, V,
              _P(hist.data_ptr()) if hist is not None else None,
              _P(hist_len.data_ptr()) if hist_len is not None else None, ldh,
              _P(prm.data_ptr()), _P(u.data_ptr()), _P(out_id.data_ptr()),
              _P(row_status.data_ptr()),
              _P(out_probs.data_ptr()) if out_probs is not None else None,
              _P(ws.data_ptr()), ws.numel(), sp))
    return out_id, row_status


def sample_device_noalloc(logits, prm, u, hist=None, hist_len=None, out_id=None,
                          row_status=None, out_probs=None):
    """``sample_device`` for float32 logits through ``cx_sample_f32_noalloc``:
    the library's static per-GPU scratch serves as the workspace, so the call
    allocates no device memory (the caller passes ``out_id`` and
    ``row_status`` to allocate nothing at all).  Calls that overlap on one
    GPU race on that scratch."""
    import torch
    lib = load()
    if logits.dim() != 2 or logits.stride(1) != 1 or logits.dtype != torch.float32:
        raise ValueError("logits must be a float32 [B, V] tensor with unit column stride")
    B, V = logits.shape
    dev = logits.device
    if out_id is None:
        out_id = torch.empty(B, dtype=torch.int32, device=dev)
    if row_status is None:
        row_status = torch.empty(B, dtype=torch.int32, device=dev)
    ldh = 0 if hist is None else hist.shape[1]
    _check(lib.cx_sample_f32_noalloc(
        _P(logits.data_ptr()), logits.stride(0), B, V,
        _P(hist.data_ptr()) if hist is not None else None,
        _P(hist_len.data_ptr()) if hist_len is not None else None, ldh,
        _P(prm.data_ptr()), _P(u.data_ptr()), _P(out_id.data_ptr()), _P(row_status.data_ptr()),
        _P(out_probs.data_ptr()) if out_probs is not None else None, _stream_ptr(dev)))
    return out_id, row_status


def spec_verify_device(target, draft, draft_ids, u, temperature, accepted=None, next_tok=None,
                       used=None, row_status=None):
    """Device-resident verify on the current stream (no synchronisation)."""
    import torch
    lib = load()
    B, g1, V = target.shape
    g = g1 - 1
    dev = target.device
    outs = [x if x is not None else torch.empty(B, dtype=torch.int32, device=dev)
            for x in (accepted, next_tok, used, row_status)]
    nbytes = lib.cx_spec_verify_workspace_bytes(B, g, V)
    sp = _stream_ptr(dev)
    ws = _ws_verify.get(nbytes, dev, sp.value)
    _check(lib.cx_spec_verify_f32(
        _P(target.data_ptr()), _P(draft.data_ptr()) if draft is not None else None,
        _P(draft_ids.data_ptr()), _P(u.data_ptr()), _P(temperature.data_ptr()), B, g, V,
        *[_P(o.data_ptr()) for o in outs], _P(ws.data_ptr()), ws.numel(), sp))
    return tuple(outs)


def lmhead_argmax_device(hidden, weight, out_id=None, out_max=None, out_logits=None):
    """LM-head projection with the greedy argmax fused, on the current stream.

    hidden: [B, D] torch.bfloat16 cuda tensor (the final-normed hidden
    states); weight: [V, D] torch.bfloat16 (the head weights); D a multiple
    of 128, unit column stride.  Returns (out_id int32 [B], out_max float32
    [B]); ``out_logits`` ([B, V] float32) is filled when given (verification
    only)."""
    import torch
    lib = load()
    for name, t in (("hidden", hidden), ("weight", weight)):
        if t.dim() != 2 or t.stride(1) != 1 or t.dtype != torch.bfloat16 or not t.is_cuda:
            raise ValueError(f"{name} must be a bfloat16 cuda matrix with unit column stride")
    B, D = hidden.shape
    V = weight.shape[0]
    if weight.shape[1] != D:
        raise ValueError("hidden and weight differ in D")
    dev = hidden.device
    if out_id is None:
        out_id = torch.empty(B, dtype=torch.int32, device=dev)
    if out_max is None:
        out_max = torch.empty(B, dtype=torch.float32, device=dev)
    if out_logits is not None and (tuple(out_logits.shape) != (B, V) or
                                   out_logits.dtype != torch.float32 or
                                   not out_logits.is_contiguous()):
        raise ValueError("out_logits must be a contiguous float32 [B, V] tensor")
    sp = _stream_ptr(dev)
    ws = _ws_head.get(lib.cx_lmhead_workspace_bytes(B, V), dev, sp.value)
    _check(lib.cx_lmhead_argmax_bf16(
        _P(hidden.data_ptr()), hidden.stride(0), _P(weight.data_ptr()), weight.stride(0),
        B, D, V, _P(out_id.data_ptr()), _P(out_max.data_ptr()),
        _P(out_logits.data_ptr()) if out_logits is not None else None,
        _P(ws.data_ptr()), ws.numel(), sp))
    return out_id, out_max


def header_symbols() -> list[str]:
    """Function names declared in include/cx_sampler.h."""
    import re
    path = os.path.join(os.path.dirname(HERE), "include", "cx_sampler.h")
    text = open(path).read()
    return sorted(set(re.findall(r"^\s*(?:int|size_t|const char\*)\s+(cx_\w+)\s*\(", text,
                                 flags=re.M)))


(KERNEL_SAMPLE, KERNEL_SAMPLE_SLOW, KERNEL_VERIFY_STATS, KERNEL_VERIFY_REST,
 KERNEL_SAMPLE_FINISH, KERNEL_PENALTIES, KERNEL_TRUNCATE, KERNEL_LMHEAD,
 KERNEL_LMHEAD_MERGE) = range(9)
KERNEL_KINDS = 9


def timing_enable(on: bool = True) -> None:
    load().cx_timing_enable(1 if on else 0)


def timing_read(kernel: int) -> tuple[float, int]:
    """(summed milliseconds, launches) of one kernel since the last read."""
    lib = load()
    ms = C.c_double()
    n = C.c_int64()
    _check(lib.cx_timing_read(kernel, C.cast(C.byref(ms), _P), C.cast(C.byref(n), _P)))
    return ms.value, n.value
