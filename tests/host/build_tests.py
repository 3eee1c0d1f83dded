"""Builds tests/host/spi_tests, the C++ test driver of the Backend-SPI mirror
(links aljabr_amd/libaljabr_rocm_spi.so and the oracle library, which is test
infrastructure). Called from __graft_entry__.build()."""
from __future__ import annotations

import os
import shutil
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
BIN = os.path.join(HERE, "spi_tests")


def build(verbose: bool = True) -> str:
    cxx = os.environ.get("CXX") or shutil.which("g++") or "g++"
    pkg, orc = os.path.join(ROOT, "aljabr_amd"), os.path.join(ROOT, "oracle")
    cmd = [cxx, "-O2", "-std=c++17", "-Wall", os.path.join(HERE, "spi_tests.cpp"),
           f"-L{pkg}", "-laljabr_rocm_spi", f"-L{orc}", "-laljabr_oracle",
           "-Wl,-rpath,$ORIGIN/../../aljabr_amd", "-Wl,-rpath,$ORIGIN/../../oracle", "-o", BIN + ".tmp"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"building spi_tests failed:\n{res.stderr}")
    os.replace(BIN + ".tmp", BIN)
    if verbose:
        print(f"built {BIN}")
    return BIN


if __name__ == "__main__":
    build()
