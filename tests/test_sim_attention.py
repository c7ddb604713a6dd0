"""Kernel sources run on the CPU through the SIMT simulator of tests/sim: the
attention kernels (specfold_amd/csrc/sf_attn.hip) here, the GEMM kernels in
test_sim_gemm.py.

The attention kernels' own source runs in the simulator (fibers per work-item, barriers,
wave-collective MFMA and shuffles from the documented operand layouts), called
through the library's entry point sf_attn_prefix_block with its host checks and
launch arithmetic, and checked against a float64 restatement of the attention.

This pins the kernels' data movement and indexing (paged and shuffled prefix
pages, permuted key slots, swizzled V^T, chunk ranges with the flash rescale,
persistent-grid walk, partial slots, the per-row merge, folded rows, causal block)
on machines without a
GPU; the GPU tests pin the same kernels on the hardware."""

import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
SIM = ROOT / "tests" / "sim"
CSRC = ROOT / "specfold_amd" / "csrc"
CLANG = Path("/opt/rocm/llvm/bin/clang++")


def _build_sim(tmp_path_factory, defines=()):
    cxx = str(CLANG) if CLANG.exists() else shutil.which("clang++")
    if cxx is None:
        pytest.skip("no clang++ (the simulator needs clang's vector extensions)")
    d = tmp_path_factory.mktemp("attn_sim")
    # a copy of the kernel file, so its quoted include of sf_common.h resolves to the
    # simulator's host header (tests/sim) instead of the HIP one next to the original
    src = d / "sf_attn.hip"
    src.write_text((CSRC / "sf_attn.hip").read_text())
    exe = d / "attn_sim"
    r = subprocess.run([cxx, "-std=c++20", "-O2", "-Wno-unknown-attributes", *defines, f"-I{SIM}",
                        f"-I{ROOT / 'include'}", f"-I{CSRC}", f'-DKERNEL_SRC="{src}"',
                        str(SIM / "attn_sim.cpp"), "-o", str(exe), "-lpthread"],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-4000:]
    return exe


@pytest.fixture(scope="module")
def attn_sim(tmp_path_factory):
    return _build_sim(tmp_path_factory)


@pytest.fixture(scope="module")
def attn_sim_one_range(tmp_path_factory):
    # a work-item target of 1: every (query tile, kv head) item takes the whole
    # prefix as one chunk range, so the prefix kernel's LDS ring wraps many times
    return _build_sim(tmp_path_factory, ("-DSFA_ITEMS_TARGET=1",))


CASES = [
    # P, page size, B1, N, H, Hkv, R, causal, seed[, folded]
    (1, 16, 2, 8, 4, 2, 5, 0, 1),        # one prefix key
    (17, 16, 3, 8, 4, 2, 9, 0, 2),       # two pages, partial last
    (130, 32, 2, 16, 6, 2, 11, 1, 3),    # partial second chunk, causal block
    (300, 16, 3, 8, 8, 1, 7, 0, 4),      # G = 8
    (257, 128, 2, 8, 4, 4, 16, 0, 5),    # G = 1, 128-key pages
    (0, 16, 2, 8, 4, 2, 6, 1, 6),        # no prefix: block keys only
    (2112, 16, 8, 32, 28, 4, 39, 0, 11),  # the 7B verify shape
    (4096, 16, 8, 32, 16, 8, 256, 0, 12),  # two chunks per work item (flash rescale)
    # sf_attn_rows over a gate structure: every row, folded ones from their source's query
    (0, 16, 4, 8, 4, 2, 0, 0, 21, 1),    # no prefix
    (130, 32, 5, 16, 6, 2, 0, 0, 22, 1),  # partial chunk, G = 3
    (300, 16, 9, 8, 8, 1, 0, 0, 23, 1),  # G = 8, 9 branches (a wave takes 3 rows)
    (17, 16, 3, 64, 4, 2, 0, 0, 25, 1),  # N = 64: two 32-key blocks
    (520, 16, 8, 32, 28, 4, 0, 0, 24, 1),  # the 7B verify shape, shorter prefix
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "P%d_ps%d_B%d_N%d_H%d-%d_R%d_c%d%s" % (
    c[0], c[1], c[2], c[3], c[4], c[5], c[6], c[7], "_folded" if len(c) > 9 and c[9] else ""))
def test_attention_kernels_in_simulator(attn_sim, case):
    r = subprocess.run([str(attn_sim), *map(str, case)], capture_output=True, text=True,
                       timeout=600)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr


# Long chunk ranges (11 and 18 chunks per item, the ring of four slots wrapping, a
# partial last chunk) with prefix keys scaled up along the prefix (ramp 1), and
# their last keys more (ramp 2), so the softmax reference moves in later chunks and
# in the last: the deferred rescale and the P.V carried from one chunk's step into
# the next.
RANGE_CASES = [
    # P, page size, B1, N, H, Hkv, R, causal, seed, folded, ramp
    (700, 16, 2, 8, 4, 2, 6, 0, 31, 0, 1),
    (1100, 32, 3, 8, 8, 2, 0, 0, 32, 1, 2),
    (700, 16, 2, 8, 4, 2, 6, 0, 33, 0, 0),
    (1000, 16, 2, 8, 4, 2, 5, 0, 34, 0, 2),
]


@pytest.mark.parametrize("case", RANGE_CASES, ids=lambda c: "P%d_ps%d_R%d_folded%d_ramp%d" % (
    c[0], c[1], c[6], c[9], c[10]))
def test_attention_long_ranges_in_simulator(attn_sim_one_range, case):
    r = subprocess.run([str(attn_sim_one_range), *map(str, case)], capture_output=True,
                       text=True, timeout=600)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
