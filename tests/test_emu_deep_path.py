"""The deep-nucleus row paths (cx_deep.hpp ``deep_row``, value buckets, and
cx_deep16.hpp ``deep16_row``, counted bf16 values) compiled for the host and
run under AddressSanitizer: one OS thread per work-item, a std::barrier per
workgroup for __syncthreads, per-wave exchanges for ballots and shuffles
(tests/emu/hip_emu.h).  Every LDS and global buffer is an exact-size heap
allocation, so an out-of-bounds access fails the run.  On top-p / min-p rows
with deep nuclei (fp32 rows of odd length, so most rows start unaligned, and
bf16 rows full of ties) every row a path decides must sample the oracle's
id; a row it hands back (-2) is allowed only where the test expects it.
CPU only."""
from __future__ import annotations

import os
import re
import shutil
import struct
import subprocess
import tempfile

import numpy as np
import pytest

from chenxing_amd.params import RowParams, pack_rows
from chenxing_amd import workloads as W
from chenxing_amd.workloads import bf16_to_f32, f32_to_bf16_rne
from oracle import sampler_ref as R

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(ROOT, "chenxing_amd", "csrc")

pytestmark = pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")


def _build(tmp: str) -> str:
    src = os.path.join(tmp, "src")
    os.makedirs(os.path.join(tmp, "inc", "hip"))
    os.makedirs(src)
    shutil.copy(os.path.join(HERE, "emu", "hip_emu.h"), os.path.join(tmp, "inc", "hip", "hip_runtime.h"))
    for f in ("cx_device.hpp", "cx_deep.hpp", "cx_deep16.hpp", "cx_internal.hpp"):
        text = open(os.path.join(CSRC, f)).read()
        text = re.sub(r"^#define CX_LDS __attribute__\(\(address_space\(3\)\)\)", "#define CX_LDS",
                      text, flags=re.M)
        text = re.sub(r"^#define CX_CONST __attribute__\(\(address_space\(4\)\)\)", "#define CX_CONST",
                      text, flags=re.M)
        open(os.path.join(src, f), "w").write(text)
    shutil.copy(os.path.join(ROOT, "include", "cx_sampler.h"), src)
    exe = os.path.join(tmp, "deep_path_emu")
    cmd = ["g++", "-std=c++20", "-O1", "-g", "-fsanitize=address", "-fno-omit-frame-pointer",
           "-pthread", "-I", os.path.join(tmp, "inc"), "-I", src, "-include", "hip/hip_runtime.h",
           os.path.join(HERE, "emu", "deep_path_emu.cpp"), "-o", exe]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-3000:]
    return exe


def _groups():
    rng = np.random.default_rng(5)
    out = []
    # fp32, odd V: rows 1.. start unaligned
    V = 30011
    x = rng.normal(0, 1.0, (9, V)).astype(np.float32)
    x[:, rng.choice(V, 4, replace=False)] += np.float32(6.0)
    prm = [RowParams(temperature=0.7, top_p=0.9), RowParams(temperature=1.0, top_p=0.99),
           RowParams(temperature=1.3, top_p=0.5), RowParams(temperature=1.0, top_p=0.95, min_p=0.02),
           RowParams(temperature=0.9, top_p=1.0, min_p=0.001), RowParams(temperature=1.1, top_p=0.0),
           RowParams(temperature=1.0, top_p=0.999), RowParams(temperature=2.0, top_p=0.8),
           RowParams(temperature=1.0, top_p=0.9)]
    x[8, 123] = np.nan                                   # handed back: NaN
    x[0, rng.choice(V, 100, replace=False)] = -np.inf    # masked tokens
    out.append(("f32", x, prm, {8}, None))
    # bf16 with many equal values at the cut
    V = 40000
    xb = f32_to_bf16_rne(rng.normal(0, 2.0, (6, V)).astype(np.float32))
    xb[0, rng.choice(V, 100, replace=False)] = 0xFF80    # -inf: masked tokens
    prm = [RowParams(temperature=1.5, top_p=0.9), RowParams(temperature=1.0, top_p=0.7),
           RowParams(temperature=0.8, top_p=0.95, min_p=0.05), RowParams(temperature=1.2, top_p=0.6),
           RowParams(temperature=1.0, top_p=1.0, min_p=0.3), RowParams(temperature=1.4, top_p=0.97)]
    out.append(("bf16", xb, prm, set(), None))
    # rows of the B=1024 V=256000 bf16 heterogeneous workload whose cut
    # element holds ~5e-7 of the mass: too little for running sums kept to
    # 2^-42 of the total to place the cut robustly
    w = W.hetero_bf16()
    rows = [1, 227, 669, 677, 901]
    out.append(("bf16", np.ascontiguousarray(w.logits[rows]), [w.params[b] for b in rows], set(),
                w.u[rows]))
    return out


def _splits_a_tie(row: np.ndarray, prm: RowParams) -> bool:
    """Whether the top-p cut keeps only part of a group of equal values."""
    z = (row.astype(np.float64) - row.max()) / prm.temperature
    p = np.exp(z) / np.exp(z).sum()
    order = np.argsort(-p, kind="stable")
    cut = int(np.searchsorted(np.cumsum(p[order]), prm.top_p)) + 1
    v = p[order[min(cut, p.size) - 1]]
    return int(np.sum(p[order[:cut]] == v)) < int(np.sum(p == v))


def _run(groups, mode: int = 0):
    us = []
    with tempfile.TemporaryDirectory() as tmp:
        exe = _build(tmp)
        fin, fout = os.path.join(tmp, "in.bin"), os.path.join(tmp, "out.bin")
        with open(fin, "wb") as f:
            f.write(struct.pack("i", len(groups)))
            for kind, x, prm, _, ug in groups:
                B, V = x.shape
                u = ug if ug is not None else np.random.default_rng(B * 7 + V).random(B)
                us.append(u)
                f.write(struct.pack("iii", B, V, 1 if kind == "bf16" else 0))
                for a in (x, pack_rows(prm), u.astype(np.float64)):
                    f.write(np.ascontiguousarray(a).tobytes())
        r = subprocess.run([exe, fin, fout, str(mode)], capture_output=True, text=True, timeout=900)
        assert r.returncode == 0, r.stderr[-4000:]
        out = open(fout, "rb").read()
    return _check(groups, us, out)


def _check(groups, us, out) -> int:
    off = 0
    decided = 0
    for (kind, x, prm, back, _), u in zip(groups, us):
        B, V = x.shape
        ids = np.frombuffer(out, np.int32, B, off)
        off += 8 * B
        rows = bf16_to_f32(x) if kind == "bf16" else x
        for b in range(B):
            if b in back:
                assert ids[b] == -2, (kind, b)
                continue
            assert ids[b] != -2, (kind, b, "handed back")
            res = R.sample_row(rows[b], prm[b], None, u[b], tie="spread")
            assert res.status == R.STATUS_OK
            assert int(ids[b]) == res.token, (kind, b, int(ids[b]), res.token)
            decided += 1
    return decided


def test_deep_path_emulated_on_deep_nucleus_rows():
    groups = _groups()
    kind, xb, prm, _, _ = groups[1]
    assert any(_splits_a_tie(r, q) for r, q in zip(bf16_to_f32(xb), prm) if q.top_p < 1.0)
    assert _run(groups) == 19


def test_counted_deep_path_emulated_on_bf16_rows():
    """deep16_row: every bf16 row of the groups above decided by counting its
    values (ties straddling the cut included), plus a row whose mask holds
    more than 65535 ids (counted apart from the 16-bit counters), a row of
    many signed zeros (one value), and a row with a value repeated 70000
    times, whose counter would wrap: handed back."""
    groups = [g for g in _groups() if g[0] == "bf16"]
    rng = np.random.default_rng(11)
    V = 100000
    xb = f32_to_bf16_rne(rng.normal(0, 1.5, (3, V)).astype(np.float32))
    xb[0, rng.choice(V, 70000, replace=False)] = 0xFF80          # -inf
    xb[1, rng.choice(V, 3000, replace=False)] = 0x0000           # +0
    xb[1, rng.choice(V, 3000, replace=False)] = 0x8000           # -0
    xb[2, rng.choice(V, 70000, replace=False)] = f32_to_bf16_rne(np.float32([0.5]))[0]
    prm = [RowParams(temperature=1.0, top_p=0.9), RowParams(temperature=2.0, top_p=0.7),
           RowParams(temperature=1.0, top_p=0.9)]
    groups.append(("bf16", xb, prm, {2}, None))
    assert _run(groups, 16) == 11 + 2


def test_counted_deep_path_top_k_rows():
    """deep16_row on bf16 rows with a top-k bound (sampler.py:76-79: every
    value at or above the k-th largest kept, ties included), alone and with
    top-p cutting inside the top-k set or beyond it (then the whole set is
    kept), with min-p, with ties at the k-th value and with k above the
    number of finite values: every row sampled as the oracle samples it."""
    rng = np.random.default_rng(17)
    V = 40000
    xb = f32_to_bf16_rne(rng.normal(0, 2.0, (10, V)).astype(np.float32))
    xb[3, :] = f32_to_bf16_rne(np.round(rng.normal(0, 2.0, V) * 4).astype(np.float32) / 4)
    xb[9, rng.choice(V, V - 50, replace=False)] = 0xFF80          # 50 finite values
    prm = [RowParams(temperature=1.0, top_k=100),
           RowParams(temperature=0.8, top_k=1000, top_p=0.9),
           RowParams(temperature=1.2, top_k=1000, top_p=0.3),
           RowParams(temperature=1.0, top_k=77, top_p=0.95),        # ties at the k-th value
           RowParams(temperature=1.5, top_k=5000, top_p=0.99),
           RowParams(temperature=1.0, top_k=300, min_p=0.05),
           RowParams(temperature=2.0, top_k=2000, top_p=0.8, min_p=0.01),
           RowParams(temperature=0.7, top_k=65),
           RowParams(temperature=1.0, top_k=20000, top_p=0.97),
           RowParams(temperature=1.0, top_k=100, top_p=0.9)]
    rows = bf16_to_f32(xb)
    kth = np.sort(rows[3])[::-1][76]
    assert np.sum(rows[3] == kth) > 1 and np.sum(rows[3] > kth) < 77      # a tie at the k-th
    assert _run([("bf16", xb, prm, set(), None)], 16) == 10


def test_counted_deep_path_kept_range_through_zero():
    """deep16_row on kept ranges through zero, whose ~27K codes of values
    below 2^-20 in magnitude outgrow a term table by key (the three part
    tables of every bf16 code): rows of logits with such values and signed
    zeros kept, and a row of only tiny values: every row sampled as the
    oracle samples it."""
    rng = np.random.default_rng(23)
    V = 40000
    x = rng.normal(0, 2.0, (4, V)).astype(np.float32)
    for b in range(3):
        idx = rng.choice(V, 200, replace=False)
        x[b, idx[:60]] = rng.normal(0, 1e-7, 60).astype(np.float32)      # inside the gap
        x[b, idx[60:80]] = np.float32(0.0)
        x[b, idx[80:100]] = np.float32(-0.0)
        x[b, idx[100:]] = rng.normal(0, 1e-5, 100).astype(np.float32)    # just outside it
    x[3] = rng.normal(0, 1.0, V).astype(np.float32) * np.float32(1e-8)   # only tiny values
    xb = f32_to_bf16_rne(x)
    prm = [RowParams(temperature=2.0, top_p=0.95), RowParams(temperature=1.5, top_p=0.99),
           RowParams(temperature=3.0, top_p=0.9, min_p=0.001), RowParams(temperature=1.0, top_p=0.9)]
    rows = bf16_to_f32(xb)
    tiny = np.abs(rows) < 2.0 ** -20
    assert tiny[:3].sum(axis=1).min() >= 60 and tiny[3].all()
    assert _run([("bf16", xb, prm, set(), None)], 16) == 4
