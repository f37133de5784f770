"""Every HIP kernel of the library, compiled for gfx950, runs without a
scratch frame and without out-of-line calls (CPU only: device-only
compilation to assembly).

Two earlier builds of the exact multi-pass path faulted the GPU with an
aperture violation; both had slow_kernel call select functions out of line,
with a scratch frame and flat (generic) instructions reaching LDS, which no
passing build had.  The same shape reappears when a change tips the
inliner's budget (dynamic LDS then reached through
llvm.amdgcn.dynlds.offset.table), so every build is held to the shape that
has always run: private segment 0, no s_swappc except the fused kernel's
compaction, which is out of line on purpose (the stream's cold path) and
touches only the LDS pointers it is passed."""
from __future__ import annotations

import os
import re
import shutil
import subprocess
import tempfile

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "chenxing_amd", "csrc")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ALLOWED_CALLS = {"_ZN2cx17wave_compact_callEPU3AS3jPU3AS3iijibS1_"}

pytestmark = pytest.mark.skipif(not os.path.exists(HIPCC), reason="needs hipcc")


def _asm(src: str, out: str) -> str:
    from chenxing_amd.build import FLAGS
    flags = [f for f in FLAGS if f not in ("-fPIC", "-shared")]
    r = subprocess.run([HIPCC, *flags, "--cuda-device-only", "-S", "-I", os.path.join(ROOT, "include"),
                        "-I", CSRC, os.path.join(CSRC, src), "-o", out],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-3000:]
    return open(out).read()


@pytest.mark.parametrize("src", ["cx_sample.hip", "cx_slow.hip", "cx_verify.hip"])
def test_kernels_have_no_scratch_and_no_calls(src):
    with tempfile.TemporaryDirectory() as tmp:
        s = _asm(src, os.path.join(tmp, "k.s"))
    kernels = re.findall(r"\.amdhsa_kernel (\S+)(.*?)\.end_amdhsa_kernel", s, re.S)
    assert kernels
    for name, body in kernels:
        priv = int(re.search(r"\.amdhsa_private_segment_fixed_size\s+(\d+)", body).group(1))
        assert priv == 0, (name, "scratch frame", priv)
    # a call: a pc-relative reference to a symbol the assembly defines as a
    # function (data such as the exp table is referenced the same way)
    funcs = set(re.findall(r"\.type\s+(\S+),@function", s))
    calls = {r for r in re.findall(r"(\S+)@rel32@lo", s) if r in funcs}
    assert calls <= ALLOWED_CALLS, calls - ALLOWED_CALLS
    if src == "cx_sample.hip":
        assert calls == ALLOWED_CALLS          # the detection itself sees the one known call
    assert "dynlds.offset.table" not in s
