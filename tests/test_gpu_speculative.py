"""The shipped ``SpeculativeDecoder`` on the GPU: the default
``DeviceVerifier`` for the verify block (speculative.py:145-171) and the
device ``Sampler`` for the draft proposals (:124-132) and the bonus token
(:168-171), replayed against the ``generate()`` runs the reference itself
recorded (tests/golden/spec_golden.json).  Tokens, stop reason, statistics
and every forward call of both engines must be the reference's."""
from __future__ import annotations

import json
import sys

import pytest

import cases
from chenxing_amd import Sampler
from chenxing_amd.params import SamplingParams
from chenxing_amd.speculative import DeviceVerifier, SpeculativeDecoder

pytestmark = pytest.mark.gpu

with open(cases.__file__.replace("cases.py", "spec_golden.json")) as f:
    GOLD = {c["name"]: c for c in json.load(f)["cases"]}


def _pairs(log):
    return [[[a], list(b)] for a, b in log]


@pytest.mark.parametrize("sc", cases.spec_cases(), ids=lambda s: s["name"])
def test_golden_generate_on_device(sc):
    print(f"[gpu] speculative generate {sc['name']}", flush=True)
    sys.stdout.flush()
    gold = GOLD[sc["name"]]
    V = sc["V"]
    tgt = cases.ScriptedEngine(V, sc["base_seed"], 0.0, 0, Sampler(V))
    drf = cases.ScriptedEngine(V, sc["base_seed"], sc["noise"], sc["noise_seed"], Sampler(V))
    sd = SpeculativeDecoder(tgt, drf, num_speculative_tokens=sc["gamma"])
    assert isinstance(sd._verify, DeviceVerifier)
    prm = SamplingParams(max_tokens=sc["max_tokens"], temperature=sc["temperature"],
                         seed=sc["seed"])
    toks, reason = sd.generate(sc["prompt"], prm)
    assert toks == gold["tokens"]
    assert reason == gold["reason"]
    assert sd.stats.as_dict() == gold["stats"]
    assert _pairs(tgt.forward_log) == _pairs(gold["target_forwards"])
    assert _pairs(drf.forward_log) == _pairs(gold["draft_forwards"])
