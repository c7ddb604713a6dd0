"""The kernels' integer index maps (specfold_amd/csrc/sf_index.h), checked on the
CPU: tests/cpp/index_check.cpp is compiled with the host C++ compiler against the
same header the HIP kernels include and run against the built library (for its
workspace-size queries).  It walks the stream-K GEMM plans, the GEMM output
columns and packed-weight fragments, the prefix attention's staged-chunk LDS
layout with its K and transposed V^T operand reads (emulated element by element,
with the bank-conflict properties of the swizzles), page-group addressing,
persistent-grid item walk, chunk ranges and partial slots over the shapes the entry points accept (see the checker's header
for the list of properties)."""

import shutil
import subprocess
from pathlib import Path

import pytest

from specfold_amd import _lib

ROOT = Path(__file__).resolve().parents[1]
SRC = ROOT / "tests" / "cpp" / "index_check.cpp"
CSRC = ROOT / "specfold_amd" / "csrc"


@pytest.fixture(scope="module")
def checker(tmp_path_factory):
    cxx = shutil.which("g++") or shutil.which("c++")
    if cxx is None:
        pytest.skip("no host C++ compiler")
    exe = tmp_path_factory.mktemp("index_check") / "index_check"
    subprocess.run([cxx, "-O2", "-std=c++17", "-Wall", "-Werror", f"-I{CSRC}", str(SRC), "-o",
                    str(exe), "-ldl"], check=True, capture_output=True, text=True)
    return exe


def test_index_maps(checker):
    lib = _lib.LIB_PATH
    assert lib.exists(), "build the library first (python -m specfold_amd.build)"
    r = subprocess.run([str(checker), str(lib)], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    out = r.stdout
    for family in ("gemm plans", "all-rows GEMM", "gemm columns", "operand reads", "page-group",
                   "attention grids"):
        assert family in out, out
    assert out.strip().splitlines()[-1].startswith("OK"), out


def test_header_builds_without_hip():
    """sf_index.h is plain C++ outside hipcc (no HIP header, no device code)."""
    text = (CSRC / "sf_index.h").read_text()
    assert "#include <hip" not in text and "__global__" not in text
