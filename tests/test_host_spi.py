"""Runs tests/host/spi_tests, the C++ tests of the Backend-SPI mirror
(aljabr_amd/host): provider and descriptor rules on any machine, and on a GPU
the ComputeBackend ops against the oracle (rel-L2 <= 1e-3). Built by
__graft_entry__.build() (tests/host/build_tests.py)."""
from __future__ import annotations

import os
import subprocess

import pytest

BIN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "host", "spi_tests")


def _cases():
    if not os.path.exists(BIN):
        return [("spi_tests binary missing (run __graft_entry__.build())", "cpu")]
    out = subprocess.run([BIN, "--list"], capture_output=True, text=True, timeout=60, check=True).stdout
    return [tuple(line.split()) for line in out.splitlines() if line.strip()]


CASES = _cases()


@pytest.mark.parametrize("name", [pytest.param(n, marks=pytest.mark.gpu) if k == "gpu" else n for n, k in CASES])
def test_spi(name):
    assert os.path.exists(BIN), "tests/host/spi_tests is not built"
    res = subprocess.run([BIN, name], capture_output=True, text=True, timeout=300)
    assert res.returncode == 0, res.stdout + res.stderr
    assert f"PASS {name}" in res.stdout
