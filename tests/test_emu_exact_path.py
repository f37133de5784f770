"""The exact multi-pass row path (cx_slow.hpp ``slow_row``) compiled for the
host and run under AddressSanitizer, on the golden small rows (V = 2 and 5,
and the rows of V = 12, 40 and 257 whose cut splits a tie group):
one OS thread per work-item, a std::barrier per workgroup for
__syncthreads, and per-wave exchanges for ballots, shuffles, readlane and
the DPP moves (tests/emu/hip_emu.h).  Every LDS and global buffer is an
exact-size heap allocation, so an out-of-bounds access fails the run; the
sampled ids and outcomes must equal the oracle's.  CPU only."""
from __future__ import annotations

import os
import re
import shutil
import struct
import subprocess
import tempfile

import numpy as np
import pytest

import cases
from chenxing_amd.params import RowParams, pack_rows
from oracle import sampler_ref as R
from parity import is_margin

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(ROOT, "chenxing_amd", "csrc")

pytestmark = pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")


def _build(tmp: str) -> str:
    """Copy the device headers with the address-space qualifiers removed
    (the host compiler has none) and build the emulated path with ASan."""
    src = os.path.join(tmp, "src")
    os.makedirs(os.path.join(tmp, "inc", "hip"))
    os.makedirs(src)
    shutil.copy(os.path.join(HERE, "emu", "hip_emu.h"), os.path.join(tmp, "inc", "hip", "hip_runtime.h"))
    for f in ("cx_device.hpp", "cx_slow.hpp", "cx_internal.hpp"):
        text = open(os.path.join(CSRC, f)).read()
        text = re.sub(r"^#define CX_LDS __attribute__\(\(address_space\(3\)\)\)", "#define CX_LDS",
                      text, flags=re.M)
        text = re.sub(r"^#define CX_CONST __attribute__\(\(address_space\(4\)\)\)", "#define CX_CONST",
                      text, flags=re.M)
        open(os.path.join(src, f), "w").write(text)
    shutil.copy(os.path.join(ROOT, "include", "cx_sampler.h"), src)
    exe = os.path.join(tmp, "exact_path_emu")
    cmd = ["g++", "-std=c++20", "-O1", "-g", "-fsanitize=address", "-fno-omit-frame-pointer",
           "-pthread", "-I", os.path.join(tmp, "inc"), "-I", src, "-include", "hip/hip_runtime.h",
           os.path.join(HERE, "emu", "exact_path_emu.cpp"), "-o", exe]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-3000:]
    return exe


def _straddles(c) -> bool:
    """The oracle's cut (top-p or typical) splits a group of equal values."""
    u = np.random.default_rng(c.params["seed"]).random()
    p = c.params
    r = R.sample_row(c.logits, R.RowParams(temperature=p["temperature"], top_k=p["top_k"],
                                           top_p=p["top_p"], min_p=p["min_p"],
                                           typical_p=p["typical_p"],
                                           repetition_penalty=p["repetition_penalty"],
                                           n_keep=p["n_keep"]), c.hist, u, tie="spread")
    return bool(r.diag.get("top_p_tie_straddle") or r.diag.get("typical_tie_straddle"))


@pytest.mark.parametrize("which", ["all V=2,5", "tie straddles V=12,40,257"])
def test_exact_path_emulated_on_golden_small_rows(which):
    """Every golden row of V = 2 and 5; and every golden row of V = 12, 40
    and 257 whose top-p or typical cut splits a group of equal values (the
    group's survivors spread over its ids: the wave-range ranks)."""
    by_v: dict = {}
    for c in cases.small_sampler_cases():
        if which.startswith("all") or _straddles(c):
            by_v.setdefault(c.logits.size, []).append(c)
    with tempfile.TemporaryDirectory() as tmp:
        exe = _build(tmp)
        groups = []
        fin, fout = os.path.join(tmp, "in.bin"), os.path.join(tmp, "out.bin")
        with open(fin, "wb") as f:
            vs = [2, 5] if which.startswith("all") else [12, 40, 257]
            f.write(struct.pack("i", len(vs)))
            for V in vs:
                cs = by_v[V]
                B = len(cs)
                x = np.stack([c.logits for c in cs]).astype(np.float32)
                prm = [RowParams(temperature=c.params["temperature"], top_k=c.params["top_k"],
                                 top_p=c.params["top_p"], min_p=c.params["min_p"],
                                 typical_p=c.params["typical_p"],
                                 repetition_penalty=c.params["repetition_penalty"],
                                 n_keep=c.params["n_keep"]) for c in cs]
                H = max(1, max(len(c.hist) for c in cs))
                hist = np.full((B, H), -1, np.int32)
                hl = np.zeros(B, np.int32)
                for b, c in enumerate(cs):
                    hist[b, :len(c.hist)] = c.hist
                    hl[b] = len(c.hist)
                u = np.array([np.random.default_rng(c.params["seed"]).random() for c in cs])
                f.write(struct.pack("iii", B, V, H))
                for a in (x, pack_rows(prm), hist, hl, u.astype(np.float64)):
                    f.write(np.ascontiguousarray(a).tobytes())
                groups.append((V, cs, prm, u))
        r = subprocess.run([exe, fin, fout], capture_output=True, text=True, timeout=900)
        assert r.returncode == 0, r.stderr[-4000:]
        out = open(fout, "rb").read()
    off = 0
    margins = []
    for V, cs, prm, u in groups:
        B = len(cs)
        ids = np.frombuffer(out, np.int32, B, off)
        off += 4 * B
        st = np.frombuffer(out, np.int32, B, off)
        off += 4 * B + 4 * B * V
        for b, (c, p) in enumerate(zip(cs, prm)):
            res = R.sample_row(c.logits, p, c.hist, u[b], tie="spread")
            assert int(st[b]) & 0xFF == res.status, (V, b)
            if res.status != R.STATUS_ERROR and int(ids[b]) != res.token:
                # a running sum within 1e-6 of its threshold (tests/parity.py)
                assert is_margin(res), (V, b, c.name, int(ids[b]), res.token, res.diag)
                margins.append(c.name)
    print("margin cases:", margins)


def test_spread_counts_on_the_host():
    """cx_device.hpp's survivor counts of a split tie group (fp64 quotients
    and the incremental remainder form) equal the exact integer formula for
    group sizes up to 2^20 (tests/emu/spread_check.cpp)."""
    with tempfile.TemporaryDirectory() as tmp:
        inc = os.path.join(tmp, "inc", "hip")
        os.makedirs(inc)
        shutil.copy(os.path.join(HERE, "emu", "hip_emu.h"), os.path.join(inc, "hip_runtime.h"))
        text = open(os.path.join(CSRC, "cx_device.hpp")).read()
        text = re.sub(r"^#define CX_LDS __attribute__\(\(address_space\(3\)\)\)", "#define CX_LDS",
                      text, flags=re.M)
        text = re.sub(r"^#define CX_CONST __attribute__\(\(address_space\(4\)\)\)", "#define CX_CONST",
                      text, flags=re.M)
        open(os.path.join(tmp, "cx_device.hpp"), "w").write(text)
        exe = os.path.join(tmp, "spread_check")
        r = subprocess.run(["g++", "-std=c++20", "-O1", "-pthread", "-I", os.path.join(tmp, "inc"),
                            "-I", tmp, "-include", "hip/hip_runtime.h",
                            os.path.join(HERE, "emu", "spread_check.cpp"), "-o", exe],
                           capture_output=True, text=True)
        assert r.returncode == 0, r.stderr[-3000:]
        r = subprocess.run([exe], capture_output=True, text=True, timeout=300)
        assert r.returncode == 0 and r.stdout.startswith("ok"), r.stdout + r.stderr
