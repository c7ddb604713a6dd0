"""Builds the C-ABI library from the kernel sources for the CPU SIMT simulator of
tests/sim, and points specfold_amd._lib at it for the duration of a test, so
the library's own Python wrappers drive the kernels' own sources on CPU tensors.

Test infrastructure only: the product's _lib accepts GPU tensors alone and has
no CPU path; `use_sim_library` lifts that check inside the `with` block and
restores everything afterwards."""

import contextlib
import ctypes
import shutil
import subprocess
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
SIM = ROOT / "tests" / "sim"
CSRC = ROOT / "specfold_amd" / "csrc"
CLANG = Path("/opt/rocm/llvm/bin/clang++")
FLAGS = ["-std=c++20", "-O2", "-fPIC", "-Wno-unknown-attributes", "-Wno-psabi"]


def compiler():
    return str(CLANG) if CLANG.exists() else shutil.which("clang++")


def build_sim_library(out_dir: Path, sources: Path = CSRC) -> Path:
    """Compile every *.hip of `sources` (with its headers copied alongside, so quoted
    includes of sf_common.h resolve to the simulator's host header) into one shared
    library exporting the C ABI."""
    cxx = compiler()
    if cxx is None:
        raise RuntimeError("no clang++")
    out_dir.mkdir(parents=True, exist_ok=True)
    for f in list(sources.glob("*.hip")) + list(sources.glob("*.h")):
        if f.name != "sf_common.h":
            (out_dir / f.name).write_text(f.read_text())
    inc = [f"-I{SIM}", f"-I{ROOT / 'include'}", f"-I{CSRC}"]

    def compile_one(src: Path) -> Path:
        obj = src.with_suffix(".o")
        r = subprocess.run([cxx, *FLAGS, *inc, "-x", "c++", "-c", str(src), "-o", str(obj)],
                           capture_output=True, text=True)
        if r.returncode:
            raise RuntimeError(f"{src.name}: {r.stderr[-3000:]}")
        return obj

    with ThreadPoolExecutor(max_workers=8) as ex:
        objs = list(ex.map(compile_one, sorted(out_dir.glob("*.hip"))))
    lib = out_dir / "libspecfold_sim.so"
    r = subprocess.run([cxx, "-shared", *map(str, objs), "-o", str(lib), "-lpthread"],
                       capture_output=True, text=True)
    if r.returncode:
        raise RuntimeError(r.stderr[-3000:])
    return lib


@contextlib.contextmanager
def use_sim_library(path: Path):
    """specfold_amd._lib bound to the simulated library, CPU tensors accepted."""
    from specfold_amd import _lib
    lib = ctypes.CDLL(str(path))
    for name, (res, args) in _lib.SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    saved = (_lib._LIB, _lib._need, _lib._stream)
    real_need = _lib._need

    def need_any_device(t, name, dtype, numel=None, min_numel=None, align=16):
        if t is not None and t.device.type == "cpu":
            # every check but the device one
            if t.dtype != dtype:
                raise TypeError(f"{name}: expected {dtype}, got {t.dtype}")
            if not t.is_contiguous():
                raise ValueError(f"{name}: must be contiguous")
            # torch's CPU allocator aligns to 64 bytes (its GPU allocator to 256, the
            # workspaces' requirement); the simulated kernels' vector accesses need 16
            if t.data_ptr() % min(align, 64):
                raise ValueError(f"{name}: data pointer must be {min(align, 64)}-byte aligned")
            if numel is not None and t.numel() != numel:
                raise ValueError(f"{name}: expected {numel} elements, got {t.numel()}")
            if min_numel is not None and t.numel() < min_numel:
                raise ValueError(f"{name}: expected at least {min_numel} elements")
            return
        return real_need(t, name, dtype, numel, min_numel, align)

    _lib._LIB, _lib._need, _lib._stream = lib, need_any_device, (lambda stream=None: None)
    try:
        yield _lib
    finally:
        _lib._LIB, _lib._need, _lib._stream = saved
