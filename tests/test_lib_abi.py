"""The C-ABI library loads, exports what the header declares, and rejects bad
arguments on the host (CPU only: no call reaches the GPU)."""
from __future__ import annotations

import ctypes as C
import os

import numpy as np
import pytest

from chenxing_amd import _lib
from chenxing_amd.params import ROW_DTYPE, RowParams, SamplingParams, pack_rows

pytestmark = pytest.mark.skipif(not os.path.exists(_lib.LIB_PATH),
                                reason="libcx_sampler.so not built")


def test_exports_every_declared_symbol():
    lib = _lib.load()
    names = _lib.header_symbols()
    assert "cx_sample_f32" in names and "cx_spec_verify_f32" in names
    for n in names:
        assert hasattr(lib, n), n
    assert set(names) == set(_lib._SIGS)


def test_version_and_error_strings():
    lib = _lib.load()
    assert b"gfx950" in lib.cx_version()
    assert lib.cx_last_error() is not None


def test_row_params_layout_matches_header():
    assert ROW_DTYPE.itemsize == 64
    assert ROW_DTYPE.fields["top_k"][1] == 56 and ROW_DTYPE.fields["n_keep"][1] == 60
    p = pack_rows([SamplingParams(temperature=0.7, top_k=40, top_p=0.9, repetition_penalty=1.1,
                                  presence_penalty=0.5, frequency_penalty=0.3, n_keep=3)])
    assert p["temperature"][0] == 0.7 and p["top_k"][0] == 40 and p["n_keep"][0] == 3
    assert RowParams.of(SamplingParams()).top_p == 1.0


def test_workspace_sizes_are_host_only():
    lib = _lib.load()
    assert lib.cx_sample_workspace_bytes(256, 128256, 2048) > 0
    assert lib.cx_spec_verify_workspace_bytes(32, 8, 128256) > 0


def test_bad_arguments_fail_before_any_device_work():
    lib = _lib.load()
    x = np.zeros((2, 8), np.float32)
    prm = pack_rows([RowParams()] * 2)
    u = np.zeros(2)
    ids = np.zeros(2, np.int32)
    st = np.zeros(2, np.int32)
    P = C.c_void_p
    # ld < V
    rc = lib.cx_sample_f32(P(x.ctypes.data), 4, 2, 8, None, None, 0, P(prm.ctypes.data),
                           P(u.ctypes.data), P(ids.ctypes.data), P(st.ctypes.data), None,
                           P(1), 1 << 20, None)
    assert rc == _lib.CX_EINVAL and b"bad shape" in lib.cx_last_error()
    # vocabulary beyond the 2^20 id limit
    rc = lib.cx_sample_f32(P(x.ctypes.data), 1 << 20, 2, 1 << 20, None, None, 0,
                           P(prm.ctypes.data), P(u.ctypes.data), P(ids.ctypes.data),
                           P(st.ctypes.data), None, P(1), 1 << 40, None)
    assert rc == _lib.CX_EINVAL
    # workspace too small
    rc = lib.cx_sample_f32(P(x.ctypes.data), 8, 2, 8, None, None, 0, P(prm.ctypes.data),
                           P(u.ctypes.data), P(ids.ctypes.data), P(st.ctypes.data), None,
                           P(1), 16, None)
    assert rc == _lib.CX_ENOSPACE
    # gamma < 1 (speculative.py:77-78 raises for it too)
    rc = lib.cx_spec_verify_f32(P(x.ctypes.data), None, P(ids.ctypes.data), P(u.ctypes.data),
                                P(x.ctypes.data), 2, 0, 8, P(ids.ctypes.data),
                                P(ids.ctypes.data), P(ids.ctypes.data), P(st.ctypes.data),
                                P(1), 1 << 20, None)
    assert rc == _lib.CX_EINVAL
    # B == 0 is a no-op
    assert lib.cx_sample_f32(None, 8, 0, 8, None, None, 0, None, None, None, None, None, None,
                             0, None) == 0


def test_noalloc_refuses_a_batch_beyond_its_static_scratch():
    """cx_sample_f32_noalloc checks the workspace the batch needs against its
    64 MiB static scratch before any device call (null pointers: nothing is
    touched)."""
    lib = _lib.load()
    assert lib.cx_sample_workspace_bytes(1024, 256000, 0) > (64 << 20)
    rc = lib.cx_sample_f32_noalloc(None, 256000, 1024, 256000, None, None, 0, None, None, None,
                                   None, None, None)
    assert rc == _lib.CX_EINVAL and b"static scratch" in lib.cx_last_error()
    assert lib.cx_sample_f32_noalloc(None, 8, 0, 8, None, None, 0, None, None, None, None, None,
                                     None) == 0
