"""Shared fixtures. GPU tests carry ``@pytest.mark.gpu``; everything else runs
on the CPU with no GPU calls."""
from __future__ import annotations

import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


def rel_l2(actual, expected) -> float:
    a = np.asarray(actual, dtype=np.float64).ravel()
    e = np.asarray(expected, dtype=np.float64).ravel()
    den = np.linalg.norm(e)
    return float(np.linalg.norm(a - e) / (den if den > 0 else 1.0))


@pytest.fixture(scope="session")
def oracle():
    import oracle as orc
    orc.lib()
    return orc


@pytest.fixture(scope="session")
def rocm():
    """Initialised C-ABI library on cuda:0 (GPU tests only)."""
    import torch
    from aljabr_amd import abi
    assert torch.cuda.is_available(), "GPU test needs a visible MI355X"
    lib = abi.load()
    abi.init(0)
    yield abi
    torch.cuda.synchronize()


@pytest.fixture(scope="session")
def dev():
    """Helpers to move numpy arrays to and from cuda:0 (torch is plumbing)."""
    import torch

    class Dev:
        @staticmethod
        def put(a: np.ndarray):
            t = torch.from_numpy(np.ascontiguousarray(a)).to("cuda:0")
            torch.cuda.synchronize()
            return t

        @staticmethod
        def empty(n: int, dtype=np.float32):
            tdt = {np.float32: torch.float32, np.int32: torch.int32, np.uint8: torch.uint8,
                   np.uint16: torch.int16, np.int16: torch.int16}[dtype]
            t = torch.empty(int(n), dtype=tdt, device="cuda:0")
            torch.cuda.synchronize()
            return t

        @staticmethod
        def get(t) -> np.ndarray:
            torch.cuda.synchronize()
            return t.cpu().numpy()

        @staticmethod
        def ptr(t) -> int:
            return t.data_ptr()

    return Dev
