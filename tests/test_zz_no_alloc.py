"""sf_logit_stats_noalloc (the allocation-free variant of sf_logit_stats, whose
scratch is a fixed per-GPU array in the library) against sf_logit_stats on the
same logits: every output bit-identical, over consecutive calls of shrinking
size (the shared array keeps the previous call's contents), and rows beyond the
array's limit rejected with SF_ERR_SCRATCH before anything is launched."""

import ctypes

import pytest
import torch

from specfold_amd import _lib

pytestmark = pytest.mark.gpu

V = 152064  # Qwen2.5 vocabulary: the decode loop's row length


def _logits(M, seed, ties):
    g = torch.Generator(device="cuda").manual_seed(seed)
    x = torch.randn(M, V, generator=g, device="cuda") * 3.0
    if ties:
        # coarse values: thousands of tokens share each bf16 value, and some rows
        # share their maximum among more than 8 tokens
        x = torch.round(x * 2.0) / 2.0
        x[::3, 1000:1040] = x[::3].max(dim=1, keepdim=True).values
    return x.to(torch.bfloat16)


def _same(got, ref, M):
    for name in _lib.LogitStats.__slots__:
        ta, tb = getattr(got, name)[:M], getattr(ref, name)
        assert torch.equal(ta.view(torch.int32), tb.view(torch.int32)), name


@pytest.mark.parametrize("ties", [False, True])
def test_noalloc_matches_workspace_entry_point(ties):
    cap = _lib.load().sf_logit_stats_noalloc_max_rows()
    print(f"[no_alloc] max rows {cap}, ties={ties}", flush=True)
    assert cap == 64
    out = _lib.LogitStats(cap, "cuda")
    for i, M in enumerate([cap, 7, cap, 1]):
        x = _logits(M, 100 + i, ties)
        print(f"[no_alloc] call {i}: M={M} V={V}", flush=True)
        ref = _lib.logit_stats(x, top_p=0.9)
        got = _lib.logit_stats_noalloc(x, out, top_p=0.9)
        torch.cuda.synchronize()
        _same(got, ref, M)


def test_noalloc_rejects_rows_beyond_scratch():
    lib = _lib.load()
    cap = lib.sf_logit_stats_noalloc_max_rows()
    M = cap + 1
    x = torch.zeros(M, 64, dtype=torch.bfloat16, device="cuda")
    out = _lib.LogitStats(M, "cuda")
    p = [ctypes.c_void_p(getattr(out, n).data_ptr()) for n in _lib.LogitStats.__slots__]
    st = lib.sf_logit_stats_noalloc(ctypes.c_void_p(x.data_ptr()), M, 64, 64, 0.9, *p, None)
    assert st == 5, st
    assert "allocation-free" in lib.sf_status_string(st).decode()
    with pytest.raises(_lib.SpecFoldKernelError):
        _lib.logit_stats_noalloc(x, out)


_FIRST_CALL_UNDER_CAPTURE = r"""
import sys, torch
sys.path.insert(0, sys.argv[1])
from specfold_amd import _lib
V = 152064
x = (torch.randn(8, V, device="cuda") * 3).to(torch.bfloat16)
out = _lib.LogitStats(8, "cuda")
g = torch.cuda.CUDAGraph()
print("[child] first call under capture", flush=True)
try:
    with torch.cuda.graph(g):
        _lib.logit_stats_noalloc(x, out, top_p=0.9)
except _lib.SpecFoldKernelError as e:
    print("[child] refused:", e, flush=True)
    assert "capture" in str(e)
else:
    raise AssertionError("a first call under capture must be refused")
torch.cuda.synchronize()
print("[child] eager call, then a captured one", flush=True)
ref = _lib.logit_stats(x, top_p=0.9)
_lib.logit_stats_noalloc(x, out, top_p=0.9)
g2 = torch.cuda.CUDAGraph()
out2 = _lib.LogitStats(8, "cuda")
with torch.cuda.graph(g2):
    _lib.logit_stats_noalloc(x, out2, top_p=0.9)
for rep in range(3):
    for n in _lib.LogitStats.__slots__:
        getattr(out2, n).zero_()
    g2.replay()
    torch.cuda.synchronize()
    for n in _lib.LogitStats.__slots__:
        assert torch.equal(getattr(out2, n).view(torch.int32), getattr(ref, n).view(torch.int32)), n
    _ = (x.float().sum()).item()          # eager work between replays
print("[child] ok", flush=True)
"""


def test_noalloc_first_call_under_capture_is_refused():
    """A process's first call on a device sets the scratch array up (symbol
    lookup, a clear it waits for): under stream capture it is refused with
    SF_ERR_CAPTURE and nothing is launched; after one eager call, captured calls
    replay with the workspace entry point's results.  Runs in a fresh child
    process, since this process has set its array up already."""
    import subprocess
    import sys
    from pathlib import Path
    root = str(Path(__file__).resolve().parents[1])
    r = subprocess.run([sys.executable, "-c", _FIRST_CALL_UNDER_CAPTURE, root],
                       capture_output=True, text=True, timeout=300)
    print(r.stdout[-2000:], r.stderr[-2000:], flush=True)
    assert r.returncode == 0 and "[child] ok" in r.stdout
