"""Build the gfx950 C-ABI library ``specfold_amd/lib/libspecfold_amd.so`` in-tree.

    python -m specfold_amd.build            # compile every HIP source, link
    python -m specfold_amd.build --asm      # also dump gfx950 assembly to _build/

hipcc cross-compiles for gfx950 without a GPU.  Packed-fp32 instructions are
switched off for every device compile (``-Xclang -target-feature -Xclang
-packed-fp32-ops``); hipcc's host pass warns that it does not know the
feature, which is harmless.
"""

from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import re
import shutil
import subprocess
import sys
from pathlib import Path
from typing import Dict, List

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
INCLUDE = ROOT / "include"
BUILD = ROOT / "_build"
LIB_DIR = PKG / "lib"
LIB_PATH = LIB_DIR / "libspecfold_amd.so"
ARCH = "gfx950"

HIPCC = os.environ.get("HIPCC", shutil.which("hipcc") or "/opt/rocm/bin/hipcc")

DEVICE_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def sources():
    return sorted(CSRC.glob("*.hip"))


_REMARK = re.compile(r"remark:\s+(Function Name|ScratchSize \[bytes/lane\]|VGPRs Spill|SGPRs Spill"
                     r"|VGPRs|AGPRs):\s*(\S+)")


def kernel_resources(remarks: str) -> Dict[str, Dict[str, str]]:
    """Per kernel (mangled name) its VGPRs, AGPRs, ScratchSize and spill counts,
    from hipcc's -Rpass-analysis=kernel-resource-usage remarks."""
    out: Dict[str, Dict[str, str]] = {}
    cur = None
    for m in _REMARK.finditer(remarks):
        key, val = m.group(1), m.group(2)
        if key == "Function Name":
            cur = out.setdefault(val, {})
        elif cur is not None:
            cur[key] = val
    return out


def spilling_kernels(res: Dict[str, Dict[str, str]]) -> List[str]:
    """Kernels with private scratch or spilled vector registers.  The kernels
    read LDS with untracked inline-asm loads (sf_lds_read16 and kin) that are
    waited for by an explicit lgkmcnt wait: a spill or register copy of a
    destination placed between the read and its wait would store stale data
    silently, so the build refuses any kernel that spills a VGPR or uses scratch
    at all.  Scalar registers spilled into VGPR lanes (v_writelane, with no
    scratch) are accepted: they never hold a load's destination and touch no
    memory."""
    bad = []
    for name, r in res.items():
        if int(r.get("ScratchSize [bytes/lane]", "0")) or int(r.get("VGPRs Spill", "0")):
            bad.append(f"{name}: {r}")
    return bad


def _compile(src: Path, asm: bool) -> Path:
    obj = BUILD / (src.stem + ".o")
    cmd = [HIPCC, *DEVICE_FLAGS, f"-I{INCLUDE}", f"-I{CSRC}", "-c", str(src), "-o", str(obj),
           "-Rpass-analysis=kernel-resource-usage"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{r.stderr}")
    res = kernel_resources(r.stderr)
    if not res:
        raise RuntimeError(f"hipcc reported no kernel resource usage for {src.name}")
    bad = spilling_kernels(res)
    if bad:
        raise RuntimeError(f"{src.name}: kernels with scratch or register spills:\n" +
                           "\n".join(bad))
    (BUILD / (src.stem + ".resources.txt")).write_text(
        "".join(f"{k} {v}\n" for k, v in sorted(res.items())))
    if asm:
        s = BUILD / (src.stem + f"-{ARCH}.s")
        cmd = [HIPCC, *DEVICE_FLAGS, f"-I{INCLUDE}", f"-I{CSRC}", "--cuda-device-only", "-S",
               str(src), "-o", str(s)]
        subprocess.run(cmd, capture_output=True, text=True, check=True)
    return obj


def build(asm: bool = False, verbose: bool = True) -> Path:
    """Compile every csrc/*.hip for gfx950 and link the shared library."""
    BUILD.mkdir(exist_ok=True)
    LIB_DIR.mkdir(exist_ok=True)
    srcs = sources()
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(lambda s: _compile(s, asm), srcs))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH.relative_to(ROOT)} from {len(srcs)} sources for {ARCH}")
    return LIB_PATH


def main(argv=None) -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--asm", action="store_true")
    args = ap.parse_args(argv)
    build(asm=args.asm)
    return 0


if __name__ == "__main__":
    sys.exit(main())
