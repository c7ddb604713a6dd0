"""ctypes binding of the gfx950 C-ABI library (include/specfold_amd.h).

The library is built in-tree by ``python -m specfold_amd.build``.  There is no
fallback: if the shared library is missing, every call raises
``SpecFoldLibraryMissing``.  Wrappers validate dtype, device, contiguity,
alignment and shape of every tensor before launching, then pass raw device
pointers and the current HIP stream.
"""

from __future__ import annotations

import ctypes
from pathlib import Path
from typing import Optional

import torch

LIB_PATH = Path(__file__).resolve().parent / "lib" / "libspecfold_amd.so"

SF_OK = 0
SF_GATE_MODEL_DTYPE = 0
SF_GATE_FP32_SQUARED = 1
SF_GATE_ALL = 2
SF_GATE_ROOTS_BY_PARENT = 16  # flag: roots are the branches with par[b] == b
SF_GATE_DEFER_COMPACT = 32  # flag: the compaction runs in sf_qkv_rope_gated

_vp = ctypes.c_void_p
_i = ctypes.c_int
_f = ctypes.c_float
_ll = ctypes.c_longlong
_sz = ctypes.c_size_t

# name -> (restype, argtypes); mirrors include/specfold_amd.h
SIGNATURES = {
    "sf_status_string": (ctypes.c_char_p, [_i]),
    "sf_abi_version": (_i, []),
    "sf_fold_gate": (_i, [_vp, _vp, _vp, _i, _i, _i, _i, _f, _f, _i,
                          _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "sf_fold_gate_residual": (_i, [_vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _f, _f, _i, _vp,
                                   _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "sf_residual_rmsnorm": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _f, _vp, _vp, _vp]),
    "sf_qkv_workspace_bytes": (_sz, [_i, _i, _i]),
    "sf_qkv_rope": (_i, [_vp, _vp, _vp, _i, _i, _vp, _vp, _vp, _vp, _vp, _i, _vp,
                         _i, _i, _i, _i, _i, _vp, _vp, _vp, _sz, _vp]),
    "sf_qkv_rope_branches": (_i, [_vp, _vp, _vp, _i, _i, _vp, _vp, _vp, _vp, _vp, _i, _vp,
                                  _i, _i, _i, _i, _i, _vp, _vp, _vp, _sz, _vp]),
    "sf_qkv_rope_gated": (_i, [_vp, _vp, _vp, _i, _i, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                               _vp, _vp, _vp, _vp, _vp, _i, _i, _vp, _i, _i, _i, _i, _vp, _vp,
                               _vp, _sz, _vp]),
    "sf_attn_workspace_bytes": (_sz, [_i, _i, _i]),
    "sf_attn_prefix_block": (_i, [_vp, _vp, _vp, _vp, _vp, _i, _i, _ll, _ll, _vp, _vp, _vp,
                                  _i, _i, _i, _i, _i, _i, _f, _vp, _i, _vp, _vp, _vp, _vp, _vp,
                                  _sz, _vp]),
    "sf_attn_rows": (_i, [_vp, _vp, _vp, _vp, _vp, _i, _i, _ll, _ll, _vp, _vp, _vp,
                          _i, _i, _i, _i, _i, _i, _i, _i, _f, _vp, _vp, _vp, _vp, _vp, _vp,
                          _sz, _vp]),
    "sf_chain_correct": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _f,
                              _vp, _vp, _vp, _vp, _vp]),
    "sf_kv_append": (_i, [_vp, _i, _i, _i, _i, _vp, _vp, _vp, _i, _ll, _ll, _i, _vp]),
    "sf_gemm_workspace_bytes": (_sz, [_i, _i, _i]),
    "sf_ffn_gate_up_workspace_bytes": (_sz, [_i, _i, _i]),
    "sf_pack_weight": (_i, [_vp, _i, _i, _vp, _vp]),
    "sf_o_proj_workspace_bytes": (_sz, [_i, _i, _i]),
    "sf_o_proj_residual": (_i, [_vp, _vp, _vp, _i, _i, _i, _vp, _vp, _sz, _vp]),
    "sf_o_proj_post_norm": (_i, [_vp, _vp, _vp, _i, _i, _i, _vp, _vp, _f, _vp, _vp, _vp, _sz,
                                 _vp]),
    "sf_residual_post_norm": (_i, [_vp, _vp, _vp, _i, _i, _vp, _f, _vp, _vp, _vp]),
    "sf_rows_rmsnorm": (_i, [_vp, _vp, _vp, _i, _vp, _i, _f, _vp, _vp]),
    "sf_ffn_gate_up": (_i, [_vp, _vp, _i, _vp, _vp, _i, _i, _vp, _vp, _sz, _vp]),
    "sf_ffn_down_scatter": (_i, [_vp, _vp, _i, _vp, _vp, _i, _i, _vp, _vp, _sz, _vp]),
    "sf_residual_gather_add": (_i, [_vp, _vp, _vp, _i, _i, _i, _vp, _vp]),
    "sf_lm_head": (_i, [_vp, _i, _vp, _i, _i, _vp, _vp]),
    "sf_head_logits": (_i, [_vp, _i, _vp, _i, _i, _i, _vp, _ll, _vp]),
    "sf_head_logits_rows": (_i, [_vp, _i, _vp, _i, _i, _i, _i, _i, _i, _vp, _ll, _vp]),
    "sf_decode_facts": (_i, [_vp, _i, _i, _i, _i, _i, _ll, _ll, _vp, _vp, _f, _vp, _i, _vp, _vp,
                             _vp]),
    "sf_logit_stats_workspace_bytes": (ctypes.c_size_t, [_i]),
    "sf_parent_map": (_i, [_vp, _i, _i, _vp, _vp, _vp]),
    "sf_logit_stats": (_i, [_vp, _i, _i, _ll, _f] + [_vp] * 7 + [_vp, ctypes.c_size_t, _vp]),
    "sf_logit_stats_noalloc_max_rows": (_i, []),
    "sf_logit_stats_noalloc": (_i, [_vp, _i, _i, _ll, _f] + [_vp] * 7 + [_vp]),
}


class SpecFoldLibraryMissing(RuntimeError):
    pass


class SpecFoldKernelError(RuntimeError):
    pass


_LIB: Optional[ctypes.CDLL] = None


def load() -> ctypes.CDLL:
    """Load (once) and type the shared library; raise if it is not built."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not LIB_PATH.exists():
        raise SpecFoldLibraryMissing(
            f"{LIB_PATH} is not built; run `python -m specfold_amd.build` "
            "(the HIP path has no CPU fallback)")
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _LIB = lib
    return lib


def _check(status: int, name: str) -> None:
    if status != SF_OK:
        msg = load().sf_status_string(status).decode()
        raise SpecFoldKernelError(f"{name} returned {status}: {msg}")


def _ptr(t: Optional[torch.Tensor]):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(stream=None):
    s = torch.cuda.current_stream() if stream is None else stream
    return ctypes.c_void_p(s.cuda_stream)


def _need(t: torch.Tensor, name: str, dtype: torch.dtype, numel: Optional[int] = None,
          min_numel: Optional[int] = None, align: int = 16) -> None:
    if t is None:
        raise ValueError(f"{name} is required")
    if t.dtype != dtype:
        raise TypeError(f"{name}: expected {dtype}, got {t.dtype}")
    if t.device.type != "cuda":
        raise ValueError(f"{name}: expected a GPU tensor, got {t.device}")
    if not t.is_contiguous():
        raise ValueError(f"{name}: must be contiguous")
    if t.data_ptr() % align:
        raise ValueError(f"{name}: data pointer must be {align}-byte aligned")
    if numel is not None and t.numel() != numel:
        raise ValueError(f"{name}: expected {numel} elements, got {t.numel()}")
    if min_numel is not None and t.numel() < min_numel:
        raise ValueError(f"{name}: expected at least {min_numel} elements, got {t.numel()}")


# ---------------------------------------------------------------------------
# typed wrappers
# ---------------------------------------------------------------------------

def _need_gate_outputs(B1, N, bucket, D, rec, f, src, rows, count, seg, segcnt, slot, rstd, xn):
    BN = B1 * N
    _need(rec, "rec", torch.int8, min_numel=BN, align=4)
    for nm, t, n in (("f", f, BN), ("src", src, BN), ("rows", rows, bucket), ("count", count, 1),
                     ("seg", seg, BN), ("segcnt", segcnt, B1)):
        _need(t, nm, torch.int32, min_numel=n, align=4)
    if slot is not None:
        _need(slot, "slot", torch.int32, min_numel=BN, align=4)
    _need(rstd, "rstd", torch.float32, min_numel=BN, align=4)
    _need(xn, "xn", torch.bfloat16, min_numel=BN * D)


def fold_gate(hidden, par, ln_w, B1, N, bucket, delta, eps, gate_mode,
              rec, f, src, rows, count, seg, segcnt, rstd, xn, stream=None, slot=None) -> None:
    D = hidden.shape[-1]
    BN = B1 * N
    _need(hidden, "hidden", torch.bfloat16, numel=BN * D)
    _need(par, "par", torch.int32, numel=B1, align=4)
    _need(ln_w, "ln_w", torch.bfloat16, numel=D)
    _need_gate_outputs(B1, N, bucket, D, rec, f, src, rows, count, seg, segcnt, slot, rstd, xn)
    st = load().sf_fold_gate(_ptr(hidden), _ptr(par), _ptr(ln_w), B1, N, D, bucket, float(delta),
                             float(eps), int(gate_mode), _ptr(rec), _ptr(f), _ptr(src), _ptr(rows),
                             _ptr(count), _ptr(seg), _ptr(segcnt), _ptr(slot), _ptr(rstd),
                             _ptr(xn), _stream(stream))
    _check(st, "sf_fold_gate")


def fold_gate_residual(hp, ffn, src_prev, par, ln_w, B1, N, D, bucket, delta, eps, gate_mode,
                       hidden_out, rec, f, src, rows, count, seg, segcnt, slot, rstd, xn,
                       stream=None) -> None:
    """The gate of a layer after the first, with the previous layer's residual
    update x = bf16(hp + ffn[src_prev*N + n]) fused in (written to hidden_out)."""
    BN = B1 * N
    _need(hp, "hp", torch.bfloat16, min_numel=BN * D)
    _need(ffn, "ffn", torch.bfloat16, min_numel=BN * D)
    _need(src_prev, "src_prev", torch.int32, min_numel=BN, align=4)
    _need(par, "par", torch.int32, numel=B1, align=4)
    _need(ln_w, "ln_w", torch.bfloat16, numel=D)
    _need(hidden_out, "hidden_out", torch.bfloat16, min_numel=BN * D)
    _need_gate_outputs(B1, N, bucket, D, rec, f, src, rows, count, seg, segcnt, slot, rstd, xn)
    st = load().sf_fold_gate_residual(
        _ptr(hp), _ptr(ffn), _ptr(src_prev), _ptr(par), _ptr(ln_w), B1, N, D, bucket,
        float(delta), float(eps), int(gate_mode), _ptr(hidden_out), _ptr(rec), _ptr(f),
        _ptr(src), _ptr(rows), _ptr(count), _ptr(seg), _ptr(segcnt), _ptr(slot), _ptr(rstd),
        _ptr(xn), _stream(stream))
    _check(st, "sf_fold_gate_residual")


def residual_rmsnorm(hp, ffn, src, w, B1, N, D, eps, hidden_out, out, stream=None) -> None:
    """hidden_out = bf16(hp + ffn[src*N + n]) and out = RMSNorm(hidden_out), every row."""
    BN = B1 * N
    _need(hp, "hp", torch.bfloat16, min_numel=BN * D)
    _need(ffn, "ffn", torch.bfloat16, min_numel=BN * D)
    _need(src, "src", torch.int32, min_numel=BN, align=4)
    _need(w, "w", torch.bfloat16, numel=D)
    _need(hidden_out, "hidden_out", torch.bfloat16, min_numel=BN * D)
    _need(out, "out", torch.bfloat16, min_numel=BN * D)
    st = load().sf_residual_rmsnorm(_ptr(hp), _ptr(ffn), _ptr(src), _ptr(w), B1, N, D, float(eps),
                                    _ptr(hidden_out), _ptr(out), _stream(stream))
    _check(st, "sf_residual_rmsnorm")


def qkv_workspace_bytes(bucket: int, D: int, n_qkv: int) -> int:
    return int(load().sf_qkv_workspace_bytes(bucket, D, n_qkv))


def qkv_rope(xn, rows, count, bucket, BN, w_qkv, b_qkv, cos, sin, q_scale, N, D, H, Hkv, hd,
             q_buf, kv_buf, workspace, stream=None, pos0=None) -> None:
    """cos/sin: [N, hd] block tables, or (with ``pos0``, an int32 device scalar
    holding the block's first position) [T, hd] tables over absolute positions."""
    nq = (H + 2 * Hkv) * hd
    _need(xn, "xn", torch.bfloat16, min_numel=BN * D)
    _need(rows, "rows", torch.int32, min_numel=bucket, align=4)
    _need(count, "count", torch.int32, min_numel=1, align=4)
    _need(w_qkv, "w_qkv", torch.bfloat16, numel=nq * D)
    if b_qkv is not None:
        _need(b_qkv, "b_qkv", torch.bfloat16, numel=nq, align=4)
    if pos0 is None:
        _need(cos, "cos", torch.bfloat16, numel=N * hd, align=4)
        table_rows = N
    else:
        _need(pos0, "pos0", torch.int32, min_numel=1, align=4)
        table_rows = cos.numel() // hd
        _need(cos, "cos", torch.bfloat16, numel=table_rows * hd, align=4)
    _need(sin, "sin", torch.bfloat16, numel=cos.numel(), align=4)
    if q_scale is not None:
        _need(q_scale, "q_scale", torch.float32, numel=N, align=4)
    _need(q_buf, "q_buf", torch.bfloat16, min_numel=(BN + 1) * H * hd)
    _need(kv_buf, "kv_buf", torch.bfloat16, min_numel=(BN + 1) * 2 * Hkv * hd)
    _need(workspace, "workspace", torch.uint8, min_numel=qkv_workspace_bytes(bucket, D, nq),
          align=256)
    st = load().sf_qkv_rope(_ptr(xn), _ptr(rows), _ptr(count), bucket, BN, _ptr(w_qkv),
                            _ptr(b_qkv), _ptr(cos), _ptr(sin), _ptr(pos0), table_rows,
                            _ptr(q_scale), N, D, H, Hkv, hd,
                            _ptr(q_buf), _ptr(kv_buf), _ptr(workspace), workspace.numel(),
                            _stream(stream))
    _check(st, "sf_qkv_rope")


def qkv_rope_branches(xn, rows, count, bucket, BN, w_qkv, b_qkv, cos, sin, q_scale_rows, N, D,
                      H, Hkv, hd, q_buf, kv_buf, workspace, pos0_branch, stream=None) -> None:
    """qkv_rope over a batched step's branches: ``pos0_branch`` int32 [BN/N] (each
    branch's first absolute position), cos/sin [T, hd] tables over absolute
    positions, ``q_scale_rows`` optional fp32 [BN]."""
    nq = (H + 2 * Hkv) * hd
    if BN % N:
        raise ValueError(f"BN={BN} is not a multiple of N={N}")
    _need(xn, "xn", torch.bfloat16, min_numel=BN * D)
    _need(rows, "rows", torch.int32, min_numel=bucket, align=4)
    _need(count, "count", torch.int32, min_numel=1, align=4)
    _need(w_qkv, "w_qkv", torch.bfloat16, numel=nq * D)
    if b_qkv is not None:
        _need(b_qkv, "b_qkv", torch.bfloat16, numel=nq, align=4)
    _need(pos0_branch, "pos0_branch", torch.int32, numel=BN // N, align=4)
    table_rows = cos.numel() // hd
    _need(cos, "cos", torch.bfloat16, numel=table_rows * hd, align=4)
    _need(sin, "sin", torch.bfloat16, numel=cos.numel(), align=4)
    if q_scale_rows is not None:
        _need(q_scale_rows, "q_scale_rows", torch.float32, numel=BN, align=4)
    _need(q_buf, "q_buf", torch.bfloat16, min_numel=(BN + 1) * H * hd)
    _need(kv_buf, "kv_buf", torch.bfloat16, min_numel=(BN + 1) * 2 * Hkv * hd)
    _need(workspace, "workspace", torch.uint8, min_numel=qkv_workspace_bytes(bucket, D, nq),
          align=256)
    st = load().sf_qkv_rope_branches(_ptr(xn), _ptr(rows), _ptr(count), bucket, BN, _ptr(w_qkv),
                                     _ptr(b_qkv), _ptr(cos), _ptr(sin), _ptr(pos0_branch),
                                     table_rows, _ptr(q_scale_rows), N, D, H, Hkv, hd,
                                     _ptr(q_buf), _ptr(kv_buf), _ptr(workspace),
                                     workspace.numel(), _stream(stream))
    _check(st, "sf_qkv_rope_branches")


def qkv_rope_gated(xn, rec, par, B1, N, bucket, f, src, rows, count, seg, segcnt, slot, w_qkv,
                   b_qkv, cos, sin, q_scale, D, H, Hkv, hd, q_buf, kv_buf, workspace,
                   pos0=None, pos0_branch=None, stream=None) -> None:
    """The QKV projection with the fold gate's compaction in its GEMM's prologue,
    after a gate launched with SF_GATE_DEFER_COMPACT: writes f, src, rows, count,
    seg, segcnt and slot as fold_gate does, then q/kv as qkv_rope (``pos0``: an
    int32 device scalar, ``q_scale`` [N]) or qkv_rope_branches (``pos0_branch``
    int32 [B1], ``q_scale`` [B1*N])."""
    BN = B1 * N
    nq = (H + 2 * Hkv) * hd
    _need(xn, "xn", torch.bfloat16, min_numel=BN * D)
    _need(rec, "rec", torch.int8, min_numel=BN, align=4)
    _need(par, "par", torch.int32, numel=B1, align=4)
    for nm, t, n in (("f", f, BN), ("src", src, BN), ("rows", rows, bucket), ("count", count, 1),
                     ("seg", seg, BN), ("segcnt", segcnt, B1)):
        _need(t, nm, torch.int32, min_numel=n, align=4)
    if slot is not None:
        _need(slot, "slot", torch.int32, min_numel=BN, align=4)
    _need(w_qkv, "w_qkv", torch.bfloat16, numel=nq * D)
    if b_qkv is not None:
        _need(b_qkv, "b_qkv", torch.bfloat16, numel=nq, align=4)
    if pos0_branch is not None:
        _need(pos0_branch, "pos0_branch", torch.int32, numel=B1, align=4)
        pos, per_branch, nscale = pos0_branch, 1, BN
    else:
        if pos0 is not None:
            _need(pos0, "pos0", torch.int32, min_numel=1, align=4)
        pos, per_branch, nscale = pos0, 0, N
    table_rows = cos.numel() // hd if pos is not None else N
    _need(cos, "cos", torch.bfloat16, numel=table_rows * hd, align=4)
    _need(sin, "sin", torch.bfloat16, numel=cos.numel(), align=4)
    if q_scale is not None:
        _need(q_scale, "q_scale", torch.float32, numel=nscale, align=4)
    _need(q_buf, "q_buf", torch.bfloat16, min_numel=(BN + 1) * H * hd)
    _need(kv_buf, "kv_buf", torch.bfloat16, min_numel=(BN + 1) * 2 * Hkv * hd)
    _need(workspace, "workspace", torch.uint8, min_numel=qkv_workspace_bytes(bucket, D, nq),
          align=256)
    st = load().sf_qkv_rope_gated(
        _ptr(xn), _ptr(rec), _ptr(par), B1, N, bucket, _ptr(f), _ptr(src), _ptr(rows),
        _ptr(count), _ptr(seg), _ptr(segcnt), _ptr(slot), _ptr(w_qkv), _ptr(b_qkv), _ptr(cos),
        _ptr(sin), _ptr(pos), per_branch, table_rows, _ptr(q_scale), D, H, Hkv, hd, _ptr(q_buf),
        _ptr(kv_buf), _ptr(workspace), workspace.numel(), _stream(stream))
    _check(st, "sf_qkv_rope_gated")


def attn_workspace_bytes(bucket: int, H: int, P: int) -> int:
    return int(load().sf_attn_workspace_bytes(bucket, H, P))


def _need_attn_outputs(BN, H, hd, o32, o_bf, m_tab, z_tab):
    """o_bf is required; o32, m_tab and z_tab may be None (not written)."""
    if o32 is not None:
        _need(o32, "o32", torch.float32, min_numel=BN * H * hd)
    _need(o_bf, "o_bf", torch.bfloat16, min_numel=BN * H * hd)
    for nm, t in (("m_tab", m_tab), ("z_tab", z_tab)):
        if t is not None:
            _need(t, nm, torch.float32, min_numel=BN * H, align=4)


def attn_prefix_block(q_buf, kv_buf, prefix_k, prefix_v, page_table, P, page_size, page_stride,
                      head_stride, src, rows, count, bucket, B1, N, H, Hkv, hd, scaling,
                      o32, o_bf, m_tab, z_tab, workspace, prefix_len=None, stream=None,
                      block_causal: bool = False) -> None:
    """prefix_len: optional device int32[1] holding the prefix length; P is then
    the capacity (grid / workspace size).  block_causal: block position n sees the
    block keys j <= n only (a causal block commit; every row recomputed).  o32, m_tab
    and z_tab may be None (not written)."""
    BN = B1 * N
    _need(q_buf, "q_buf", torch.bfloat16, min_numel=(BN + 1) * H * hd)
    _need(kv_buf, "kv_buf", torch.bfloat16, min_numel=(BN + 1) * 2 * Hkv * hd)
    if P > 0:
        _need(prefix_k, "prefix_k", torch.bfloat16)
        _need(prefix_v, "prefix_v", torch.bfloat16)
        if page_table is not None:
            _need(page_table, "page_table", torch.int32, min_numel=(P + page_size - 1) // page_size,
                  align=4)
    _need(src, "src", torch.int32, min_numel=BN, align=4)
    _need(rows, "rows", torch.int32, min_numel=bucket, align=4)
    _need(count, "count", torch.int32, min_numel=1, align=4)
    _need_attn_outputs(BN, H, hd, o32, o_bf, m_tab, z_tab)
    _need(workspace, "workspace", torch.uint8, min_numel=attn_workspace_bytes(bucket, H, P),
          align=256)
    if prefix_len is not None:
        _need(prefix_len, "prefix_len", torch.int32, numel=1, align=4)
    st = load().sf_attn_prefix_block(
        _ptr(q_buf), _ptr(kv_buf), _ptr(prefix_k) if P > 0 else None,
        _ptr(prefix_v) if P > 0 else None, _ptr(page_table) if P > 0 else None, P,
        page_size, page_stride, head_stride, _ptr(src), _ptr(rows), _ptr(count), bucket, B1, N, H,
        Hkv, hd, float(scaling), _ptr(prefix_len) if P > 0 else None, 1 if block_causal else 0,
        _ptr(o32), _ptr(o_bf),
        _ptr(m_tab), _ptr(z_tab), _ptr(workspace), workspace.numel(), _stream(stream))
    _check(st, "sf_attn_prefix_block")


def attn_rows(q_buf, kv_buf, prefix_k, prefix_v, page_table, P, page_size, page_stride,
              head_stride, src, rows, count, bucket, B1, N, b_first, b_count, H, Hkv, hd,
              scaling, o32, o_bf, m_tab, z_tab, workspace, prefix_len=None, stream=None) -> None:
    """Attention of every row of branches [b_first, b_first + b_count): recomputed
    rows as attn_prefix_block, folded rows from their source row's query over the
    prefix and their own branch's block keys (sf_attn_rows: attention + chain
    correction in one call).  o32, m_tab and z_tab may be None (not written)."""
    BN = B1 * N
    _need(q_buf, "q_buf", torch.bfloat16, min_numel=(BN + 1) * H * hd)
    _need(kv_buf, "kv_buf", torch.bfloat16, min_numel=(BN + 1) * 2 * Hkv * hd)
    if P > 0:
        _need(prefix_k, "prefix_k", torch.bfloat16)
        _need(prefix_v, "prefix_v", torch.bfloat16)
        if page_table is not None:
            _need(page_table, "page_table", torch.int32, min_numel=(P + page_size - 1) // page_size,
                  align=4)
    _need(src, "src", torch.int32, min_numel=BN, align=4)
    _need(rows, "rows", torch.int32, min_numel=bucket, align=4)
    _need(count, "count", torch.int32, min_numel=1, align=4)
    _need_attn_outputs(BN, H, hd, o32, o_bf, m_tab, z_tab)
    _need(workspace, "workspace", torch.uint8, min_numel=attn_workspace_bytes(bucket, H, P),
          align=256)
    if prefix_len is not None:
        _need(prefix_len, "prefix_len", torch.int32, numel=1, align=4)
    st = load().sf_attn_rows(
        _ptr(q_buf), _ptr(kv_buf), _ptr(prefix_k) if P > 0 else None,
        _ptr(prefix_v) if P > 0 else None, _ptr(page_table) if P > 0 else None, P,
        page_size, page_stride, head_stride, _ptr(src), _ptr(rows), _ptr(count), bucket, B1, N,
        b_first, b_count, H, Hkv, hd, float(scaling), _ptr(prefix_len) if P > 0 else None,
        _ptr(o32), _ptr(o_bf), _ptr(m_tab), _ptr(z_tab), _ptr(workspace), workspace.numel(),
        _stream(stream))
    _check(st, "sf_attn_rows")


def chain_correct(q_buf, kv_buf, src, par, rec, seg, segcnt, B1, N, H, Hkv, hd, scaling,
                  o32, o_bf, m_tab, z_tab, stream=None) -> None:
    BN = B1 * N
    _need(q_buf, "q_buf", torch.bfloat16, min_numel=(BN + 1) * H * hd)
    _need(kv_buf, "kv_buf", torch.bfloat16, min_numel=(BN + 1) * 2 * Hkv * hd)
    for nm, t, n in (("src", src, BN), ("par", par, B1), ("seg", seg, BN), ("segcnt", segcnt, B1)):
        _need(t, nm, torch.int32, min_numel=n, align=4)
    _need(rec, "rec", torch.int8, min_numel=BN, align=4)
    _need(o32, "o32", torch.float32, min_numel=BN * H * hd)
    _need(o_bf, "o_bf", torch.bfloat16, min_numel=BN * H * hd)
    _need(m_tab, "m_tab", torch.float32, min_numel=BN * H, align=4)
    _need(z_tab, "z_tab", torch.float32, min_numel=BN * H, align=4)
    st = load().sf_chain_correct(_ptr(q_buf), _ptr(kv_buf), _ptr(src), _ptr(par), _ptr(rec),
                                 _ptr(seg), _ptr(segcnt), B1, N, H, Hkv, hd, float(scaling),
                                 _ptr(o32), _ptr(o_bf), _ptr(m_tab), _ptr(z_tab), _stream(stream))
    _check(st, "sf_chain_correct")


def kv_append(kv_buf, row0, n_tok, Hkv, hd, k_cache, v_cache, page_table, page_size,
              page_stride, head_stride, start_pos, stream=None) -> None:
    _need(kv_buf, "kv_buf", torch.bfloat16, min_numel=(row0 + n_tok) * 2 * Hkv * hd)
    _need(k_cache, "k_cache", torch.bfloat16)
    _need(v_cache, "v_cache", torch.bfloat16)
    if page_table is not None:
        _need(page_table, "page_table", torch.int32, align=4)
    st = load().sf_kv_append(_ptr(kv_buf), row0, n_tok, Hkv, hd, _ptr(k_cache), _ptr(v_cache),
                             _ptr(page_table), page_size, page_stride, head_stride, start_pos,
                             _stream(stream))
    _check(st, "sf_kv_append")


def gemm_workspace_bytes(mcap: int, N: int, K: int) -> int:
    """Bytes of the GEMM workspace (fp32 partial slots of the stream-K split)."""
    return int(load().sf_gemm_workspace_bytes(mcap, N, K))


def pack_weight(w: torch.Tensor, out: Optional[torch.Tensor] = None, stream=None) -> torch.Tensor:
    """Row-major bf16 [N, K] -> the packed fragment-major layout every GEMM entry
    point takes (same shape, same bytes, reordered).  Returns ``out``."""
    if w.dim() != 2:
        raise ValueError("pack_weight takes a 2-D [N, K] weight")
    N, K = w.shape
    _need(w, "w", torch.bfloat16, numel=N * K)
    if out is None:
        out = torch.empty_like(w)
    _need(out, "out", torch.bfloat16, numel=N * K)
    st = load().sf_pack_weight(_ptr(w), N, K, _ptr(out), _stream(stream))
    _check(st, "sf_pack_weight")
    return out


def o_proj_residual(o_bf, x, wo, M, K, N, hp, workspace, stream=None) -> None:
    _need(o_bf, "o_bf", torch.bfloat16, min_numel=M * K)
    _need(x, "x", torch.bfloat16, min_numel=M * N)
    _need(wo, "wo", torch.bfloat16, numel=N * K)
    _need(hp, "hp", torch.bfloat16, min_numel=M * N)
    _need(workspace, "workspace", torch.uint8, min_numel=o_proj_workspace_bytes(M, N, K),
          align=256)
    st = load().sf_o_proj_residual(_ptr(o_bf), _ptr(x), _ptr(wo), M, K, N, _ptr(hp),
                                   _ptr(workspace), workspace.numel(), _stream(stream))
    _check(st, "sf_o_proj_residual")


def o_proj_workspace_bytes(M: int, N: int, K: int) -> int:
    """Bytes of the all-rows o_proj workspace (fp32 sums of its K ranges)."""
    return int(load().sf_o_proj_workspace_bytes(M, N, K))


def o_proj_post_norm(o_bf, x, wo, BN, K, D, slot, w, eps, hp, zn, workspace, stream=None) -> None:
    """hp = bf16(x + bf16(o_bf . Wo^T)) for every row (Wo packed); zn[slot[r]] =
    RMSNorm(hp[r]) where slot[r] >= 0."""
    _need(o_bf, "o_bf", torch.bfloat16, min_numel=BN * K)
    _need(x, "x", torch.bfloat16, min_numel=BN * D)
    _need(wo, "wo", torch.bfloat16, numel=D * K)
    _need(slot, "slot", torch.int32, min_numel=BN, align=4)
    _need(w, "w", torch.bfloat16, numel=D)
    _need(hp, "hp", torch.bfloat16, min_numel=BN * D)
    _need(zn, "zn", torch.bfloat16)
    _need(workspace, "workspace", torch.uint8, min_numel=o_proj_workspace_bytes(BN, D, K),
          align=256)
    st = load().sf_o_proj_post_norm(_ptr(o_bf), _ptr(x), _ptr(wo), BN, K, D, _ptr(slot), _ptr(w),
                                    float(eps), _ptr(hp), _ptr(zn), _ptr(workspace),
                                    workspace.numel(), _stream(stream))
    _check(st, "sf_o_proj_post_norm")


def residual_post_norm(x, y, slot, BN, D, w, eps, hp, zn, stream=None) -> None:
    """hp = bf16(x + y) for every row; zn[slot[r]] = RMSNorm(hp[r]) where slot[r] >= 0."""
    _need(x, "x", torch.bfloat16, min_numel=BN * D)
    _need(y, "y", torch.bfloat16, min_numel=BN * D)
    _need(slot, "slot", torch.int32, min_numel=BN, align=4)
    _need(w, "w", torch.bfloat16, numel=D)
    _need(hp, "hp", torch.bfloat16, min_numel=BN * D)
    _need(zn, "zn", torch.bfloat16)
    st = load().sf_residual_post_norm(_ptr(x), _ptr(y), _ptr(slot), BN, D, _ptr(w), float(eps),
                                      _ptr(hp), _ptr(zn), _stream(stream))
    _check(st, "sf_residual_post_norm")


def rows_rmsnorm(x, rows, count, bucket, w, D, eps, out, stream=None) -> None:
    _need(x, "x", torch.bfloat16)
    _need(rows, "rows", torch.int32, min_numel=bucket, align=4)
    _need(count, "count", torch.int32, min_numel=1, align=4)
    _need(w, "w", torch.bfloat16, numel=D)
    _need(out, "out", torch.bfloat16, min_numel=bucket * D)
    st = load().sf_rows_rmsnorm(_ptr(x), _ptr(rows), _ptr(count), bucket, _ptr(w), D, float(eps),
                                _ptr(out), _stream(stream))
    _check(st, "sf_rows_rmsnorm")


def gate_up_workspace_bytes(bucket: int, D: int, I: int) -> int:
    """Bytes of the gate/up GEMM's partial-slot workspace (0 for invalid shapes)."""
    return int(load().sf_ffn_gate_up_workspace_bytes(bucket, D, I))


def ffn_gate_up(zn, count, bucket, wg, wu, D, I, act, workspace, stream=None) -> None:
    _need(zn, "zn", torch.bfloat16, min_numel=bucket * D)
    _need(count, "count", torch.int32, min_numel=1, align=4)
    _need(wg, "wg", torch.bfloat16, numel=I * D)
    _need(wu, "wu", torch.bfloat16, numel=I * D)
    _need(act, "act", torch.bfloat16, min_numel=bucket * I)
    _need(workspace, "workspace", torch.uint8, min_numel=gate_up_workspace_bytes(bucket, D, I),
          align=256)
    st = load().sf_ffn_gate_up(_ptr(zn), _ptr(count), bucket, _ptr(wg), _ptr(wu), D, I, _ptr(act),
                               _ptr(workspace), workspace.numel(), _stream(stream))
    _check(st, "sf_ffn_gate_up")


def ffn_down_scatter(act, count, bucket, rows, wd, I, D, ffn, workspace, stream=None) -> None:
    _need(act, "act", torch.bfloat16, min_numel=bucket * I)
    _need(count, "count", torch.int32, min_numel=1, align=4)
    _need(rows, "rows", torch.int32, min_numel=bucket, align=4)
    _need(wd, "wd", torch.bfloat16, numel=D * I)
    _need(ffn, "ffn", torch.bfloat16)
    _need(workspace, "workspace", torch.uint8, min_numel=gemm_workspace_bytes(bucket, D, I),
          align=256)
    st = load().sf_ffn_down_scatter(_ptr(act), _ptr(count), bucket, _ptr(rows), _ptr(wd), I, D,
                                    _ptr(ffn), _ptr(workspace), workspace.numel(), _stream(stream))
    _check(st, "sf_ffn_down_scatter")


def residual_gather_add(hp, ffn, src, B1, N, D, out, stream=None) -> None:
    _need(hp, "hp", torch.bfloat16, min_numel=B1 * N * D)
    _need(ffn, "ffn", torch.bfloat16, min_numel=B1 * N * D)
    _need(src, "src", torch.int32, min_numel=B1 * N, align=4)
    _need(out, "out", torch.bfloat16, min_numel=B1 * N * D)
    st = load().sf_residual_gather_add(_ptr(hp), _ptr(ffn), _ptr(src), B1, N, D, _ptr(out),
                                       _stream(stream))
    _check(st, "sf_residual_gather_add")


def lm_head(x, M, w, D, V, logits, stream=None) -> None:
    _need(x, "x", torch.bfloat16, min_numel=M * D)
    _need(w, "w", torch.bfloat16, numel=V * D)
    _need(logits, "logits", torch.bfloat16, min_numel=M * V)
    st = load().sf_lm_head(_ptr(x), M, _ptr(w), D, V, _ptr(logits), _stream(stream))
    _check(st, "sf_lm_head")


def head_logits(x, M, w, D, V, logits, shift_n: int = 0, stream=None) -> None:
    """logits [M, V] (row stride logits.stride(0)) = x [M, D] . W^T with W packed
    [V, D]; shift_n = N: Fast-dLLM's shift of N-row blocks in the stores
    (sf_head_logits)."""
    _need(x, "x", torch.bfloat16, min_numel=M * D)
    _need(w, "w", torch.bfloat16, numel=V * D)
    ld = logits.stride(0) if logits.dim() == 2 else V
    if logits.dtype != torch.bfloat16 or logits.stride(-1) != 1 or \
            logits.storage_offset() + (M - 1) * ld + V > logits.untyped_storage().nbytes() // 2:
        raise ValueError(f"logits must be bf16 rows of stride {ld} holding {M} x {V}")
    st = load().sf_head_logits(_ptr(x), M, _ptr(w), D, V, int(shift_n), _ptr(logits), ld,
                               _stream(stream))
    _check(st, "sf_head_logits")


def decode_facts(x_t, plen: int, bl: int, sbs: int, s0: int, mask_id: int, stop_id: int,
                 conf, x_1, threshold_bf16: float, states, unmask, facts, stream=None) -> int:
    """sf_decode_facts on the token state x_t (int64 [1, L] or [L], contiguous):
    with conf (bf16 [sbs]) the small block at block offset s0 is decided and
    written (x_1 int64 [sbs], unmask int8 [sbs] out), then the loop facts go to
    facts (int64, at least 4 + bl // sbs).  states: cached draft states (int64
    [bl] each, contiguous).  Returns the number of facts written."""
    _need(x_t, "x_t", torch.int64, align=8)
    L = x_t.numel()
    _need(facts, "facts", torch.int64, min_numel=4 + bl // sbs, align=8)
    if conf is not None:
        _need(conf, "conf", torch.bfloat16, min_numel=sbs, align=2)
        _need(x_1, "x_1", torch.int64, min_numel=sbs, align=8)
        _need(unmask, "unmask", torch.int8, min_numel=sbs, align=1)
    ptrs = (ctypes.c_void_p * max(1, len(states)))()
    for i, t in enumerate(states):
        _need(t, "state", torch.int64, min_numel=bl, align=8)
        ptrs[i] = t.data_ptr()
    st = load().sf_decode_facts(_ptr(x_t), L, plen, bl, sbs, s0, int(mask_id), int(stop_id),
                                _ptr(conf), _ptr(x_1), float(threshold_bf16),
                                ctypes.cast(ptrs, ctypes.c_void_p), len(states), _ptr(unmask),
                                _ptr(facts), _stream(stream))
    _check(st, "sf_decode_facts")
    return 2 + bl // sbs + (1 if states else 0) + (1 if conf is not None else 0)


def head_logits_rows(x, M, w, D, V, logits, N: int, shift: bool, row_lo: int, row_n: int,
                     stream=None) -> None:
    """The head for a row window: of every N-row block of x [M, D], the logits rows
    of positions [row_lo, row_lo + row_n) (Fast-dLLM's shift with ``shift``: row n
    from x row n - 1, row 0 from itself); the other rows of ``logits`` are not
    written (sf_head_logits_rows)."""
    _need(x, "x", torch.bfloat16, min_numel=M * D)
    _need(w, "w", torch.bfloat16, numel=V * D)
    ld = logits.stride(0) if logits.dim() == 2 else V
    if logits.dtype != torch.bfloat16 or logits.stride(-1) != 1 or \
            logits.storage_offset() + (M - 1) * ld + V > logits.untyped_storage().nbytes() // 2:
        raise ValueError(f"logits must be bf16 rows of stride {ld} holding {M} x {V}")
    st = load().sf_head_logits_rows(_ptr(x), M, _ptr(w), D, V, int(N), 1 if shift else 0,
                                    int(row_lo), int(row_n), _ptr(logits), ld, _stream(stream))
    _check(st, "sf_head_logits_rows")


class LogitStats:
    """Per-row greedy decoding statistics (see ``logit_stats``)."""

    __slots__ = ("top_idx", "top_val", "zfull", "znuc", "greedy_tok", "conf", "conf_full")

    def __init__(self, M: int, device):
        self.top_idx = torch.empty(M, 8, dtype=torch.int32, device=device)
        self.top_val = torch.empty(M, 8, dtype=torch.float32, device=device)
        self.zfull = torch.empty(M, dtype=torch.float32, device=device)
        self.znuc = torch.empty(M, dtype=torch.float32, device=device)
        self.greedy_tok = torch.empty(M, dtype=torch.int32, device=device)
        self.conf = torch.empty(M, dtype=torch.float32, device=device)
        self.conf_full = torch.empty(M, dtype=torch.float32, device=device)


_STATS_WS: dict = {}


def _stats_rows(logits: torch.Tensor):
    if logits.dtype != torch.bfloat16 or not logits.is_cuda:
        raise TypeError("logits must be a bf16 CUDA tensor")
    V = logits.shape[-1]
    x = logits.reshape(-1, V)
    if x.stride(1) != 1:
        x = x.contiguous()
    if x.stride(0) % 8 or x.data_ptr() % 16:
        x = x.contiguous()
    return x, x.shape[0], V, x.stride(0)


def logit_stats(logits: torch.Tensor, top_p: float = 0.95, stream=None) -> LogitStats:
    """Greedy statistics of the rows of ``logits`` ([..., V] bf16, rows contiguous
    along V): top-8 tokens, softmax / nucleus normalisers, greedy token and its
    bf16 probability (sf_logit_stats)."""
    x, M, V, ld = _stats_rows(logits)
    need = int(load().sf_logit_stats_workspace_bytes(M))
    key = (x.device.index, M)
    ws = _STATS_WS.get(key)
    if ws is None or ws.numel() < need:
        ws = torch.zeros(need, dtype=torch.uint8, device=x.device)  # kept zero by every call
        _STATS_WS[key] = ws
    out = LogitStats(M, x.device)
    st = load().sf_logit_stats(_ptr(x), M, V, ld, float(top_p), _ptr(out.top_idx),
                               _ptr(out.top_val), _ptr(out.zfull), _ptr(out.znuc),
                               _ptr(out.greedy_tok), _ptr(out.conf), _ptr(out.conf_full),
                               _ptr(ws), ws.numel(), _stream(stream))
    _check(st, "sf_logit_stats")
    return out


def logit_stats_noalloc(logits: torch.Tensor, out: LogitStats, top_p: float = 0.95,
                        stream=None) -> LogitStats:
    """``logit_stats`` into caller-owned outputs with no workspace: the library's
    fixed per-GPU scratch (sf_logit_stats_noalloc; at most
    sf_logit_stats_noalloc_max_rows() rows; calls that overlap on one GPU race).
    ``logits`` must already be bf16 with rows contiguous, 8-element aligned."""
    if logits.dtype != torch.bfloat16 or not logits.is_cuda:
        raise TypeError("logits must be a bf16 CUDA tensor")
    V = logits.shape[-1]
    x = logits.reshape(-1, V)
    M, ld = x.shape[0], x.stride(0)
    if x.stride(1) != 1 or ld % 8 or x.data_ptr() % 16:
        raise ValueError("logits rows must be contiguous, 16-byte aligned, stride % 8 == 0")
    for name in LogitStats.__slots__:
        t = getattr(out, name)
        if t.device != x.device or t.shape[0] < M or not t.is_contiguous():
            raise ValueError(f"out.{name} must hold {M} rows on {x.device}")
    st = load().sf_logit_stats_noalloc(_ptr(x), M, V, ld, float(top_p), _ptr(out.top_idx),
                                       _ptr(out.top_val), _ptr(out.zfull), _ptr(out.znuc),
                                       _ptr(out.greedy_tok), _ptr(out.conf), _ptr(out.conf_full),
                                       _stream(stream))
    _check(st, "sf_logit_stats_noalloc")
    return out


def parent_map(tokens: torch.Tensor, par: torch.Tensor, counts: Optional[torch.Tensor] = None,
               stream=None) -> None:
    """Branch parent map of a token block [B1, N] int64 into par [B1] int32
    (sf_parent_map)."""
    B1, N = tokens.shape
    _need(tokens, "tokens", torch.int64, numel=B1 * N, align=8)
    _need(par, "par", torch.int32, min_numel=B1, align=4)
    if counts is not None:
        _need(counts, "counts", torch.int32, min_numel=B1, align=4)
    st = load().sf_parent_map(_ptr(tokens), B1, N, _ptr(par),
                              _ptr(counts) if counts is not None else None, _stream(stream))
    _check(st, "sf_parent_map")
