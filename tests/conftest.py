"""Pytest configuration: the ``gpu`` marker and shared fixtures.

``-m "not gpu"`` runs the oracle-vs-golden checks, host-logic tests and the
C-ABI symbol check (no GPU needed).  ``-m gpu`` runs the parity tests, which
call the HIP library through its C ABI on ``cuda:0``.
"""

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
PKG = ROOT / "spconv-triton_amd"
for p in (str(ROOT), str(PKG), str(ROOT / "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP library)")


@pytest.fixture(scope="session")
def golden():
    import torch

    cache = {}

    def load(name):
        if name not in cache:
            cache[name] = torch.load(ROOT / "tests" / "golden" / name, map_location="cpu",
                                     weights_only=True)
        return cache[name]

    def case(name, case_id):
        for c in load(name)["cases"]:
            if c["id"] == case_id:
                return c
        raise KeyError(case_id)

    return case
