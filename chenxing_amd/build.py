"""Build the gfx950 HIP library ``libcx_sampler.so`` in-tree with hipcc."""
from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libcx_sampler.so")
SOURCES = ["cx_api.hip", "cx_sample.hip", "cx_slow.hip", "cx_verify.hip", "cx_head.hip"]

FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared",
    "-ffp-contract=off",                        # numpy never fuses multiply-adds
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result",
]


def build_hist(verbose: bool = False) -> str:
    """The CPython extension that writes a batch's penalty windows from Python
    lists (csrc/cx_hist.c), compiled with the host C compiler."""
    import sysconfig
    out = os.path.join(HERE, "_cxhist" + sysconfig.get_config_var("EXT_SUFFIX"))
    cmd = [os.environ.get("CC", "gcc"), "-O2", "-shared", "-fPIC", "-Wall",
           "-I", sysconfig.get_paths()["include"], "-o", out + ".tmp",
           os.path.join(CSRC, "cx_hist.c")]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError("gcc failed building _cxhist")
    os.replace(out + ".tmp", out)
    return out


def build(verbose: bool = False) -> str:
    hipcc = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
    cmd = [hipcc, *FLAGS, "-I", os.path.join(ROOT, "include"), "-I", CSRC, "-o", LIB + ".tmp",
           *[os.path.join(CSRC, s) for s in SOURCES]]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError("hipcc failed building libcx_sampler.so")
    os.replace(LIB + ".tmp", LIB)
    build_hist(verbose)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
