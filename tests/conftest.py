"""Shared test setup: the ``gpu`` marker, import paths and small helpers."""
from __future__ import annotations

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLDEN = os.path.join(ROOT, "tests", "golden")
for p in (ROOT, GOLDEN):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the HIP C-ABI)")


def gpu_available() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(scope="session")
def lib():
    """The device library, loaded once; GPU tests only."""
    from chenxing_amd import _lib
    return _lib.load()


def pytest_terminal_summary(terminalreporter, exitstatus, config):
    """Per workload: drawing rows whose sampled id differs from the oracle run
    in numpy's own tie order (the reference on this host), and how many of
    those are tie straddles at the top-p / typical cut."""
    parity = sys.modules.get("parity")
    rates = getattr(parity, "REF_RATES", None) if parity else None
    if not rates:
        return
    tr = terminalreporter
    tr.write_line("device vs numpy tie order (reference): label draws differ tie-straddle "
                  "rate straddling-rows margin-cases tie-bound")
    for label, r in sorted(rates.items()):
        d = max(r["draws"], 1)
        tr.write_line(f"  {label}: {r['draws']} {r['diff']} {r['diff_tie']} "
                      f"{r['diff'] / d:.2e} {r['straddle']} {r['margin_vs_spread']} "
                      f"{r['bound'] if r['bound'] is not None else '1e-4'}")
