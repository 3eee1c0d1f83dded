"""The C-ABI library loads, exports every symbol ``include/aljabr_rocm.h``
declares, and reports status codes without a GPU (CPU only: no compute
calls are made)."""
from __future__ import annotations

import ctypes
import os
import re
import subprocess
import sys

import pytest

from aljabr_amd import abi

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "aljabr_rocm.h")


def declared_functions() -> list[str]:
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(aljabr_rocm_\w+)\s*\(", text)))


def test_library_is_built_and_loads():
    assert os.path.exists(abi.LIB_PATH), "run __graft_entry__.build() first"
    abi.load()


def test_every_declared_symbol_is_exported_and_bound():
    lib = ctypes.CDLL(abi.LIB_PATH)
    names = declared_functions()
    assert len(names) >= 30
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    assert set(names) == set(abi.SIGNATURES), set(names) ^ set(abi.SIGNATURES)


def test_status_codes_match_the_metal_abi():
    text = open(HEADER).read()
    codes = dict(re.findall(r"#define (ALJABR_ROCM_\w+) \((-?\d+)\)", text))
    assert codes["ALJABR_ROCM_ERR_NOT_INITIALIZED"] == "-1"
    assert codes["ALJABR_ROCM_ERR_BAD_ARGUMENT"] == "-2"
    assert codes["ALJABR_ROCM_ERR_UNSUPPORTED"] == "-3"
    assert codes["ALJABR_ROCM_ERR_BUFFER"] == "-4"


_UNINIT_SCRIPT = r"""
import ctypes, sys
sys.path.insert(0, %r)
from aljabr_amd import abi
lib = abi.load()
assert lib.aljabr_rocm_is_initialized() == 0
# Compute before init: -1 and a message, like the Metal ABI's g_initialized gate.
rc = lib.aljabr_rocm_matvec_tb_q4_0(None, None, None, 32, 1)
assert rc == abi.ERR_NOT_INITIALIZED, rc
assert "init" in abi.last_error()
rc = lib.aljabr_rocm_alloc(16, ctypes.byref(ctypes.c_void_p()))
assert rc == abi.ERR_NOT_INITIALIZED, rc
# Null out-pointers are argument errors, checked before anything else.
assert lib.aljabr_rocm_device_count(None) == abi.ERR_BAD_ARGUMENT
assert lib.aljabr_rocm_version() == 100
print("ok")
"""


def test_calls_before_init_fail_with_not_initialized():
    out = subprocess.run([sys.executable, "-c", _UNINIT_SCRIPT % ROOT], capture_output=True, text=True, timeout=120)
    assert out.returncode == 0, out.stderr
    assert out.stdout.strip().endswith("ok")


_NO_GPU_SCRIPT = r"""
import sys
sys.path.insert(0, %r)
from aljabr_amd import abi
lib = abi.load()
n = abi.device_count()
if n == 0:
    rc = lib.aljabr_rocm_init(0)
    assert rc == abi.ERR_NOT_INITIALIZED, rc
    assert "no HIP device" in abi.last_error()
    print("no-gpu ok")
else:
    print("gpu present")
"""


def test_init_without_a_device_reports_not_initialized():
    out = subprocess.run([sys.executable, "-c", _NO_GPU_SCRIPT % ROOT], capture_output=True, text=True, timeout=120)
    assert out.returncode == 0, out.stderr
    if "gpu present" in out.stdout:
        pytest.skip("a GPU is visible; the no-device path is exercised on CPU-only hosts")
    assert "no-gpu ok" in out.stdout
