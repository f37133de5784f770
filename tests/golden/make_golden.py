"""Write the golden fixtures by running the reference implementation.

Runs ONLY in the build container, where the reference checkout lives at
/root/reference (it never travels with this repository).  It imports the
reference's pure-NumPy modules and records, for the deterministic inputs of
``cases.py``:

* ``Sampler.apply_penalties``  (chenxing/core/sampler.py:63-73)
* ``Sampler._truncate``        (chenxing/core/sampler.py:75-106)
* ``Sampler.sample``           (chenxing/core/sampler.py:108-127), seeded
* ``SpeculativeDecoder.generate`` (chenxing/engine/speculative.py:94-200),
  driven by ``cases.ScriptedEngine`` -- the only way to reach the inline
  verify loop at :145-171.

Only data is written (``sampler_golden.npz``, ``spec_golden.json``): seeds,
input digests and the reference's outputs.

Usage:  python tests/golden/make_golden.py
"""
from __future__ import annotations

import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)
sys.path.insert(0, "/root/reference")

import cases  # noqa: E402
from chenxing.core.sampler import Sampler, SamplingParams  # noqa: E402
from chenxing.engine.speculative import SpeculativeDecoder  # noqa: E402


def _sample_or_error(s, x, prm, hist):
    try:
        return int(s.sample(x, prm, hist))
    except ValueError:
        return -9


def sampler_golden() -> dict:
    rec: dict = {"names": [], "pen_digest": [], "pen_sparse_idx": [], "pen_sparse_val": [],
                 "trunc_in_digest": [], "trunc_digest": [], "trunc_idx": [], "trunc_val": [], "sample": [],
                 "logit_digest": []}
    all_cases = cases.small_sampler_cases() + cases.medium_sampler_cases()
    for c in all_cases:
        V = c.logits.size
        s = Sampler(V)
        prm = SamplingParams(**c.params)
        pen = s.apply_penalties(c.logits, prm, list(c.hist))
        changed = np.flatnonzero(~((pen == c.logits.astype(np.float64)) |
                                   (np.isnan(pen) & np.isnan(c.logits))))
        P_in = cases.truncate_input(c)
        with np.errstate(all="ignore"):
            tr = s._truncate(P_in.copy(), prm)
        nz = np.flatnonzero(tr)
        rec["trunc_digest"].append(cases.digest(tr))
        if nz.size > 300:          # large outputs: the digest pins them bitwise
            nz = nz[:0]
        rec["names"].append(c.name)
        rec["logit_digest"].append(cases.digest(c.logits))
        rec["pen_digest"].append(cases.digest(pen))
        rec["pen_sparse_idx"].append(changed.astype(np.int64))
        rec["pen_sparse_val"].append(pen[changed])
        rec["trunc_in_digest"].append(cases.digest(P_in))
        rec["trunc_idx"].append(nz.astype(np.int64))
        rec["trunc_val"].append(tr[nz])
        with np.errstate(all="ignore"):
            rec["sample"].append(_sample_or_error(s, c.logits, prm, list(c.hist)))
    return rec


def spec_golden() -> list[dict]:
    out = []
    for sc in cases.spec_cases():
        V = sc["V"]
        tgt = cases.ScriptedEngine(V, sc["base_seed"], 0.0, 0, Sampler(V))
        drf = cases.ScriptedEngine(V, sc["base_seed"], sc["noise"], sc["noise_seed"],
                                   Sampler(V))
        sd = SpeculativeDecoder(tgt, drf, num_speculative_tokens=sc["gamma"])
        prm = SamplingParams(max_tokens=sc["max_tokens"], temperature=sc["temperature"],
                             seed=sc["seed"])
        toks, reason = sd.generate(sc["prompt"], prm)
        out.append(dict(name=sc["name"], tokens=[int(t) for t in toks], reason=reason,
                        stats=sd.stats.as_dict(),
                        target_forwards=tgt.forward_log, draft_forwards=drf.forward_log))
    return out


def main() -> None:
    rec = sampler_golden()
    n = len(rec["names"])

    def ragged(key, dtype):
        arrs = rec[key]
        offs = np.zeros(n + 1, dtype=np.int64)
        offs[1:] = np.cumsum([a.size for a in arrs])
        flat = np.concatenate(arrs).astype(dtype) if offs[-1] else np.zeros(0, dtype)
        return flat, offs

    pi, po = ragged("pen_sparse_idx", np.int64)
    pv, _ = ragged("pen_sparse_val", np.float64)
    ti, to = ragged("trunc_idx", np.int64)
    tv, _ = ragged("trunc_val", np.float64)
    np.savez_compressed(
        os.path.join(HERE, "sampler_golden.npz"),
        names=np.array(rec["names"]), logit_digest=np.array(rec["logit_digest"]),
        pen_digest=np.array(rec["pen_digest"]), pen_idx=pi, pen_val=pv, pen_off=po,
        trunc_in_digest=np.array(rec["trunc_in_digest"]),
        trunc_digest=np.array(rec["trunc_digest"]), trunc_idx=ti, trunc_val=tv,
        trunc_off=to, sample=np.array(rec["sample"], dtype=np.int64),
        numpy_version=np.array(np.__version__))
    with open(os.path.join(HERE, "spec_golden.json"), "w") as f:
        json.dump({"numpy_version": np.__version__, "cases": spec_golden()}, f)
    print(f"wrote {n} sampler cases and {len(cases.spec_cases())} speculative cases")


if __name__ == "__main__":
    main()
