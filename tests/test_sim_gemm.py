"""The weight-streaming GEMM kernels' own source (specfold_amd/csrc/sf_ffn.hip,
sf_qkv.hip, sf_gemm_core.h) run on the CPU through the SIMT simulator of
tests/sim, called through the library's entry points: weight packing, FFN
gate/up (stream-K, SiLU epilogue from registers or in the fix-up), FFN down
(stream-K with partial slots, fix-up, row scatter), o_proj + residual (+ the
post-attention norm), the head (sf_head.hip: weights straight into registers,
rows through an LDS ring; one or two passes; unshifted, and with Fast-dLLM's
shift in the stores, across a pass boundary inside a block), and the QKV projection with bias, RoPE from
absolute-position tables, the optional q scale and the scatter by flat row, for
row counts of one row up to two passes of 128 rows, against float64 dot products
rounded as each epilogue specifies (tests/sim/gemm_sim.cpp states the
tolerance)."""

import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
SIM = ROOT / "tests" / "sim"
CSRC = ROOT / "specfold_amd" / "csrc"
CLANG = Path("/opt/rocm/llvm/bin/clang++")


def _build(tmp_path_factory, extra=()):
    cxx = str(CLANG) if CLANG.exists() else shutil.which("clang++")
    if cxx is None:
        pytest.skip("no clang++ (the simulator needs clang's vector extensions)")
    d = tmp_path_factory.mktemp("gemm_sim")
    # copies, so the sources' quoted includes of sf_common.h resolve to the
    # simulator's host header instead of the HIP one next to the originals
    for f in ("sf_ffn.hip", "sf_qkv.hip", "sf_head.hip", "sf_gemm_core.h", "sf_gemm_rows.h",
              "sf_compact.h"):
        (d / f).write_text((CSRC / f).read_text())
    flags = ["-std=c++20", "-O2", "-Wno-unknown-attributes", "-Wno-psabi", f"-I{SIM}",
             f"-I{ROOT / 'include'}", f"-I{CSRC}", *extra]
    objs = []
    for src, obj in ((d / "sf_ffn.hip", d / "ffn.o"), (d / "sf_qkv.hip", d / "qkv.o"),
                     (d / "sf_head.hip", d / "head.o"), (SIM / "gemm_sim.cpp", d / "drv.o")):
        lang = ["-x", "c++"] if src.suffix == ".hip" else []
        r = subprocess.run([cxx, *flags, *lang, "-c", str(src), "-o", str(obj)],
                           capture_output=True, text=True)
        assert r.returncode == 0, r.stderr[-4000:]
        objs.append(str(obj))
    exe = d / "gemm_sim"
    r = subprocess.run([cxx, *objs, "-o", str(exe), "-lpthread"], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-4000:]
    return exe


@pytest.fixture(scope="module")
def gemm_sim(tmp_path_factory):
    return _build(tmp_path_factory)


@pytest.fixture(scope="module")
def gemm_sim_grid3(tmp_path_factory):
    """The library with a 3-workgroup grid: small outputs then take the gate/up's
    column-spread plan (I/16 units over 3 workgroups, 2 to 8 each, uneven where
    3 does not divide them) that the 7B-14B intermediate widths take on the
    256-workgroup grid."""
    return _build(tmp_path_factory, ("-DSFG_GRID=3",))


@pytest.fixture(scope="module")
def gemm_sim_grid7(tmp_path_factory):
    """A 7-workgroup grid: 24 gate/up units take the spread plan over
    spread_workgroups(24, 7) = 6 workgroups (4 units each), fewer than the grid, as
    1184 units take 237 of 256 at the 7B shape."""
    return _build(tmp_path_factory, ("-DSFG_GRID=7",))


@pytest.mark.parametrize("case", [
    (256, 384, 39, 64, 40, 1),      # D, I, count, bucket, M, seed: one row block
    (384, 512, 100, 128, 70, 2),    # two row blocks
    (384, 512, 117, 128, 117, 7),   # the recomputed-row count of a trained 7B model
    (512, 640, 130, 256, 130, 3),   # three of four row blocks in use
    (256, 384, 1, 256, 1, 4),       # a single row
    (640, 768, 200, 256, 256, 5),   # four full row blocks for the static-M GEMMs
    (256, 384, 50, 64, 300, 8),     # all-rows GEMMs in two passes (256 + 44 rows)
    (1152, 384, 40, 64, 40, 9),     # o_proj over three K ranges
], ids=lambda c: "D%d_I%d_count%d_bucket%d_M%d" % c[:5])
def test_gemm_kernels_in_simulator(gemm_sim, case):
    r = subprocess.run([str(gemm_sim), *map(str, case)], capture_output=True, text=True,
                       timeout=600)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr


@pytest.mark.parametrize("case", [
    (256, 384, 39, 64, 40, 11),     # 24 units: 8 per workgroup
    (128, 256, 70, 128, 70, 12),    # 16 units: 5, 5, 6; two row blocks
    (256, 128, 5, 64, 5, 13),       # 8 units: 2, 3, 3
], ids=lambda c: "D%d_I%d_count%d_bucket%d_M%d" % c[:5])
def test_gemm_kernels_column_spread_plan(gemm_sim_grid3, case):
    r = subprocess.run([str(gemm_sim_grid3), *map(str, case)], capture_output=True, text=True,
                       timeout=600)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr


def test_gemm_kernels_spread_plan_on_part_of_the_grid(gemm_sim_grid7):
    r = subprocess.run([str(gemm_sim_grid7), "256", "384", "39", "64", "40", "14"],
                       capture_output=True, text=True, timeout=600)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
