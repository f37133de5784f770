"""Measure how often the reference disagrees with itself on tied bf16 rows.

The reference orders the top-p candidates with ``np.argsort(-probs)``
(chenxing/core/sampler.py:82; typical-p at :103), numpy's default sort,
which is not stable.  numpy 2.2 dispatches that sort to a SIMD kernel chosen
at run time from the CPU's features, and each dispatch level orders equal
keys differently.  Where a group of equal probabilities straddles the top-p
cut, the level decides which ids of the group survive, so the same reference
code samples different ids for the same inputs and uniforms on different
hosts.

This script runs the oracle in numpy's order (``tie="numpy"``, which calls
that same ``np.argsort``) on every bf16 workload the GPU tests compare, once
per dispatch level, each in a child interpreter started with
``NPY_DISABLE_CPU_FEATURES`` (AVX-512, AVX2, and the SSE3 baseline); in the
order the device implements (``tie="spread"``: a straddling group's
survivors spread evenly over its ids); and in the lower-id-first stable
order for comparison.  For every pair of orders it counts the drawing rows
whose sampled id differs.  CPU only; it needs no GPU and no reference
checkout.

Writes ``tie_order_rates.json`` beside this file (data only).  The GPU tests
read the largest disagreement between two numpy levels per workload as the
bound on the device's disagreement with the host's numpy.

Usage:  python tests/golden/tie_order_rates.py [--workers N]
"""
from __future__ import annotations

import argparse
import itertools
import json
import os
import platform
import subprocess
import sys
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
TESTS = os.path.dirname(HERE)
ROOT = os.path.dirname(TESTS)
for p in (ROOT, TESTS, HERE):
    if p not in sys.path:
        sys.path.insert(0, p)

_AVX512 = "AVX512F AVX512CD AVX512_KNL AVX512_KNM AVX512_SKX AVX512_CLX AVX512_CNL AVX512_ICL AVX512_SPR"
LEVELS = {
    "avx512": "",
    "avx2": _AVX512,
    "baseline": _AVX512 + " AVX2 FMA3 F16C AVX SSE42 POPCNT SSE41 SSSE3",
}


def _child(level: str, out: str, workers: int) -> None:
    """Oracle ids in numpy's order for every workload, at this process's
    dispatch level (set by the parent through the environment)."""
    import numpy as np
    from numpy._core._multiarray_umath import __cpu_features__ as feats

    from bf16_workloads import TIE_WORKLOADS
    from oracle_pool import oracle_rows_parallel
    res = {"features": sorted(k for k, v in feats.items() if v)}
    arrays = {}
    for label, build in TIE_WORKLOADS.items():
        w = build()
        rows = oracle_rows_parallel(w, ties=("numpy",), keep_probs=False, workers=workers)
        arrays[label + ":id"] = np.array([r[0].token for r in rows], np.int64)
        arrays[label + ":st"] = np.array([r[0].status for r in rows], np.int64)
        arrays[label + ":tie"] = np.array([bool(r[0].diag.get("top_p_tie_straddle", False) or
                                                r[0].diag.get("typical_tie_straddle", False))
                                           for r in rows])
        print(f"  [{level}] {label}: {w.B} rows", flush=True)
    np.savez(out, **arrays)
    with open(out + ".json", "w") as f:
        json.dump(res, f)


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--workers", type=int, default=min(8, os.cpu_count() or 1))
    ap.add_argument("--child", default=None)
    ap.add_argument("--out", default=None)
    a = ap.parse_args()
    if a.child:
        _child(a.child, a.out, a.workers)
        return
    import numpy as np

    from bf16_workloads import TIE_WORKLOADS
    from oracle_pool import oracle_rows_parallel
    tmp = tempfile.mkdtemp()
    ids, feats = {}, {}
    for level, disable in LEVELS.items():
        env = dict(os.environ)
        env.pop("NPY_DISABLE_CPU_FEATURES", None)
        if disable:
            env["NPY_DISABLE_CPU_FEATURES"] = disable
        out = os.path.join(tmp, level + ".npz")
        print(f"[{level}] NPY_DISABLE_CPU_FEATURES={disable!r}", flush=True)
        subprocess.run([sys.executable, __file__, "--child", level, "--out", out,
                        "--workers", str(a.workers)], env=env, check=True)
        with np.load(out) as z:
            ids[level] = {k: z[k] for k in z.files}
        with open(out + ".json") as f:
            feats[level] = json.load(f)["features"]
    for tie in ("spread", "stable"):
        got = {}
        for label, build in TIE_WORKLOADS.items():
            w = build()
            rows = oracle_rows_parallel(w, ties=(tie,), keep_probs=False, workers=a.workers)
            got[label + ":id"] = np.array([r[0].token for r in rows], np.int64)
            got[label + ":st"] = np.array([r[0].status for r in rows], np.int64)
        ids[tie] = got
    orders = list(LEVELS) + ["spread", "stable"]
    report = {
        "about": "drawing rows whose sampled id differs between two argsort tie orders of the "
                 "reference's top-p/typical sort (sampler.py:82,103); numpy levels by "
                 "NPY_DISABLE_CPU_FEATURES, 'spread' = the device's rule (a straddling tie "
                 "group's survivors spread evenly over its ids), 'stable' = lower id first",
        "numpy": np.__version__,
        "python": platform.python_version(),
        "cpu": _cpu_name(),
        "levels": {lv: {"disabled": LEVELS[lv], "enabled_features": feats[lv]} for lv in LEVELS},
        "workloads": {},
    }
    for label in TIE_WORKLOADS:
        ok = np.ones_like(ids["spread"][label + ":st"], dtype=bool)
        for o in orders:
            ok &= ids[o][label + ":st"] == 0
        draws = int(ok.sum())
        pairs = {}
        for x, y in itertools.combinations(orders, 2):
            pairs[f"{x}/{y}"] = int((ids[x][label + ":id"][ok] != ids[y][label + ":id"][ok]).sum())
        cross = max(v for k, v in pairs.items() if "stable" not in k and "spread" not in k)
        spread = max(v for k, v in pairs.items() if "spread" in k and "stable" not in k)
        straddle = int(ids["avx512"][label + ":tie"][ok].sum())
        report["workloads"][label] = {"draws": draws, "straddling_rows": straddle,
                                      "differ": pairs, "max_numpy_cross_level": cross,
                                      "max_spread_vs_numpy": spread}
        print(f"{label}: draws {draws}, straddling {straddle}, " +
              ", ".join(f"{k} {v}" for k, v in pairs.items()), flush=True)
    with open(os.path.join(HERE, "tie_order_rates.json"), "w") as f:
        json.dump(report, f, indent=1, sort_keys=True)
        f.write("\n")


def _cpu_name() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor()


if __name__ == "__main__":
    main()
