"""What a cx_sample_f32 call runs on the GPU -- the fused kernel
(cx_sample.hip, sample_kernel), then slow_kernel (cx_slow.hip: the region
finisher of cx_finish.hpp, the refinement, the deep-nucleus and exact
multi-pass paths) -- compiled for the host and run under AddressSanitizer on
the golden small rows (V = 2 to 300, every knob), with the fused kernel's own
hand-off (row status words, hand-off marks, slice records, regions) feeding
slow_kernel (tests/emu/pipeline_emu.cpp).  Each launch's dynamic LDS is an
exact-size allocation of the bytes the launch requests and every static LDS
array its own object, so an LDS index past the launch's allocation fails
the run; the ids and outcomes must equal the oracle's (margin cases
counted).  CPU only."""
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
CLANG = "/opt/rocm/llvm/bin/clang++"

pytestmark = pytest.mark.skipif(not os.path.exists(CLANG), reason="needs ROCm's clang++")


def _host_source(text: str) -> str:
    """A device source for the host build: no address-space qualifiers, the
    dynamic LDS from the emulation, no launch code (timing, attributes)."""
    text = re.sub(r"^#define CX_LDS __attribute__\(\(address_space\(3\)\)\)", "#define CX_LDS",
                  text, flags=re.M)
    text = re.sub(r"^#define CX_CONST __attribute__\(\(address_space\(4\)\)\)", "#define CX_CONST",
                  text, flags=re.M)
    text = text.replace("extern __shared__ __align__(16) unsigned char dyn[];",
                        "unsigned char* dyn = emu::dyn_lds;")
    text = text.replace('#include "cx_timing.hpp"\n', "")
    # gfx950 inline assembly, restated: the three scalar loads of a row's
    # scalars, v_max3_f32, and the empty statements that pin a value to
    # VGPRs
    text = re.sub(r'asm volatile\(\s*"s_load_dwordx16.*?: "s"\(p\), "s"\(u\), "s"\(hl\)\);',
                  "v = *(const u32x16*)p; uu = *(const u32x2*)u; h = *(const uint32_t*)hl;",
                  text, flags=re.S)
    text = text.replace('asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));',
                        "r = fmaxf(fmaxf(a, b), c);")
    text = text.replace('"+v"', '"+m"')
    return text


def _build(tmp: str) -> str:
    src = os.path.join(tmp, "src")
    os.makedirs(os.path.join(tmp, "inc", "hip"))
    os.makedirs(src)
    shutil.copy(os.path.join(HERE, "emu", "hip_emu.h"), os.path.join(tmp, "inc", "hip", "hip_runtime.h"))
    for f in ("cx_device.hpp", "cx_internal.hpp", "cx_slow.hpp", "cx_deep.hpp", "cx_deep16.hpp",
              "cx_finish.hpp"):
        open(os.path.join(src, f), "w").write(_host_source(open(os.path.join(CSRC, f)).read()))
    shutil.copy(os.path.join(ROOT, "include", "cx_sampler.h"), src)
    # the kernels without their launch functions
    samp = _host_source(open(os.path.join(CSRC, "cx_sample.hip")).read())
    samp = samp[:samp.rindex("namespace cx {\nint launch_sample")]
    open(os.path.join(src, "sample_emu.cpp"), "w").write(samp)
    slow = _host_source(open(os.path.join(CSRC, "cx_slow.hip")).read())
    slow = slow[:slow.index("template <typename K>\nstatic int set_lds")] + "}  // namespace cx\n"
    open(os.path.join(src, "slow_emu.cpp"), "w").write(slow)
    exe = os.path.join(tmp, "pipeline_emu")
    cmd = [CLANG, "-std=c++20", "-O1", "-g", "-fsanitize=address", "-fno-omit-frame-pointer",
           "-pthread", "-Wno-unknown-attributes", "-I", os.path.join(tmp, "inc"), "-I", src,
           "-include", "hip/hip_runtime.h", os.path.join(HERE, "emu", "pipeline_emu.cpp"),
           os.path.join(src, "sample_emu.cpp"), os.path.join(src, "slow_emu.cpp"), "-o", exe]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-4000:]
    return exe


def _params(c) -> RowParams:
    p = c.params
    return RowParams(temperature=p["temperature"], top_k=p["top_k"], top_p=p["top_p"],
                     min_p=p["min_p"], typical_p=p["typical_p"],
                     repetition_penalty=p["repetition_penalty"], n_keep=p["n_keep"])


def run_pipeline(groups_in, tmp, env=None):
    """groups_in: list of case lists (one V each).  Returns [(ids, status)]."""
    exe = _build(tmp)
    fin, fout = os.path.join(tmp, "in.bin"), os.path.join(tmp, "out.bin")
    with open(fin, "wb") as f:
        f.write(struct.pack("i", len(groups_in)))
        for cs in groups_in:
            B, V = len(cs), cs[0].logits.size
            x = np.stack([c.logits for c in cs]).astype(np.float32)
            H = max(len(c.hist) for c in cs)
            f.write(struct.pack("iii", B, V, H))
            f.write(np.ascontiguousarray(x).tobytes())
            f.write(pack_rows([_params(c) for c in cs]).tobytes())
            if H > 0:
                hist = np.full((B, H), -1, np.int32)
                hl = np.zeros(B, np.int32)
                for b, c in enumerate(cs):
                    hist[b, :len(c.hist)] = c.hist
                    hl[b] = len(c.hist)
                f.write(hist.tobytes())
                f.write(hl.tobytes())
            u = np.array([np.random.default_rng(c.params["seed"]).random() for c in cs])
            f.write(u.astype(np.float64).tobytes())
    r = subprocess.run([exe, fin, fout], capture_output=True, text=True, timeout=1500,
                       env=dict(os.environ, **(env or {})))
    assert r.returncode == 0, r.stderr[-6000:]
    out = open(fout, "rb").read()
    res, off = [], 0
    for cs in groups_in:
        B = len(cs)
        ids = np.frombuffer(out, np.int32, B, off)
        st = np.frombuffer(out, np.int32, B, off + 4 * B)
        off += 8 * B
        res.append((ids, st))
    return res


# The golden group run by default: V = 2 (46 rows: the batch and vocabulary
# of the call that faulted on the GPU).  EMU_ALL_GROUPS=1 runs every group
# (V = 2 to 300, 250 rows; about 8 minutes).
DEFAULT_V = (2,)


def test_fused_and_slow_kernels_emulated_on_golden_small_rows():
    by_v: dict = {}
    for c in cases.small_sampler_cases():
        by_v.setdefault(c.logits.size, []).append(c)
    every = os.environ.get("EMU_ALL_GROUPS") == "1"
    groups = [by_v[v] for v in sorted(by_v) if every or v in DEFAULT_V]
    with tempfile.TemporaryDirectory() as tmp:
        outs = run_pipeline(groups, tmp)
    margins = []
    for cs, (ids, st) in zip(groups, outs):
        for b, c in enumerate(cs):
            u = np.random.default_rng(c.params["seed"]).random()
            res = R.sample_row(c.logits, _params(c), c.hist, u, tie="spread")
            assert int(st[b]) & 0xFF == res.status, (c.name, int(st[b]), res.status)
            if res.status != R.STATUS_ERROR and int(ids[b]) != res.token:
                assert is_margin(res), (c.name, int(ids[b]), res.token, res.diag)
                margins.append(c.name)
    assert len(margins) <= 2, margins


def _sliced_cases():
    """Rows of a sliced launch (V = 40000: two slices of the fused kernel's
    sliced variant): top-p rows without a penalty window or top-k (the split
    exact normaliser), one with a top-k and one with a penalty window (the
    full one), and a row whose large values all sit in its second slice."""
    V = 40000
    rng = np.random.default_rng(31)
    base = dict(temperature=1.0, top_k=0, top_p=0.9, min_p=0.0, typical_p=1.0,
                repetition_penalty=1.0, n_keep=0)
    rows = []
    for i, (kw, hist) in enumerate([
            (dict(), []),
            (dict(temperature=0.7, top_p=0.95), []),
            (dict(temperature=0.8, top_k=50, top_p=0.9), []),
            (dict(repetition_penalty=1.3), [int(t) for t in rng.integers(0, V, 200)]),
            (dict(top_p=0.99), [])]):
        x = rng.normal(0.0, 3.0, V).astype(np.float32)
        if i == 4:
            x[V // 2:] += 4.0
        prm = dict(base, **kw, seed=int(rng.integers(0, 2**31)))
        rows.append(cases.SamplerCase(f"sliced{i}", x, prm, hist))
    return rows


def test_sliced_top_p_rows_emulated():
    cs = _sliced_cases()
    with tempfile.TemporaryDirectory() as tmp:
        (ids, st), = run_pipeline([cs], tmp)
    for b, c in enumerate(cs):
        u = np.random.default_rng(c.params["seed"]).random()
        res = R.sample_row(c.logits, _params(c), c.hist, u, tie="spread")
        assert int(st[b]) & 0xFF == res.status, (c.name, int(st[b]), res.status)
        assert int(ids[b]) == res.token or is_margin(res), (c.name, int(ids[b]), res.token)
    # the split normaliser decides rows 0 and 1 in the region finisher (no
    # exact re-read, no multi-pass path); rows 2 and 3 keep the full one
    FLAG_SLOW, FLAG_EXACT = 0x100, 0x200
    assert all(int(st[b]) & (FLAG_SLOW | FLAG_EXACT) == 0 for b in (0, 1)), st
    assert all(int(st[b]) & FLAG_EXACT for b in (2, 3)), st


def test_long_single_slice_rows_emulated():
    """Single-slice rows of 50000 elements (49 chunks, so the LDS chunk
    counter hands out chunks past the first two per wave; the slice count is
    forced to 1, as a batch of 256 rows would give): a top-k + top-p row, a
    nucleus row and a penalised row."""
    V = 50000
    rng = np.random.default_rng(37)
    base = dict(temperature=0.8, top_k=0, top_p=0.9, min_p=0.0, typical_p=1.0,
                repetition_penalty=1.0, n_keep=0)
    rows = []
    for i, (kw, hist) in enumerate([
            (dict(top_k=40), []),
            (dict(top_p=0.95, temperature=1.0), []),
            (dict(top_k=50, repetition_penalty=1.2), [int(t) for t in rng.integers(0, V, 300)])]):
        x = rng.normal(0.0, 3.0, V).astype(np.float32)
        rows.append(cases.SamplerCase(f"long{i}", x, dict(base, **kw, seed=int(rng.integers(0, 2**31))),
                                      hist))
    with tempfile.TemporaryDirectory() as tmp:
        (ids, st), = run_pipeline([rows], tmp, env={"EMU_NSPLIT": "1"})
    for b, c in enumerate(rows):
        u = np.random.default_rng(c.params["seed"]).random()
        res = R.sample_row(c.logits, _params(c), c.hist, u, tie="spread")
        assert int(st[b]) & 0xFF == res.status, (c.name, int(st[b]), res.status)
        assert int(ids[b]) == res.token or is_margin(res), (c.name, int(ids[b]), res.token)
