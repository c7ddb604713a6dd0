"""The C-ABI library loads on a machine without a GPU and exports every
function include/specfold_amd.h declares, with the signatures the ctypes
binding uses; argument validation rejects bad shapes without launching."""

import ctypes
import re
from pathlib import Path

import pytest

from specfold_amd import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "specfold_amd.h"


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(sf_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_entry_points():
    names = declared_functions()
    for n in ("sf_fold_gate", "sf_qkv_rope", "sf_attn_prefix_block", "sf_chain_correct",
              "sf_kv_append", "sf_qkv_workspace_bytes", "sf_attn_workspace_bytes"):
        assert n in names


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    names = declared_functions()
    assert set(names) == set(_lib.SIGNATURES), "ctypes signatures out of sync with the header"
    for n in names:
        assert isinstance(getattr(lib, n), ctypes._CFuncPtr), n


def test_host_side_validation_without_gpu():
    lib = _lib.load()
    assert lib.sf_abi_version() == 14
    assert lib.sf_status_string(1).decode() == "shape outside kernel limits"
    # NULL pointers and bad shapes are rejected before any launch
    assert lib.sf_fold_gate(*([None] * 3), 8, 32, 64, 256, 0.1, 1e-6, 0, *([None] * 11)) == 2
    assert lib.sf_fold_gate_residual(*([None] * 5), 8, 32, 64, 256, 0.1, 1e-6, 0,
                                     *([None] * 12)) == 2
    assert lib.sf_residual_rmsnorm(*([None] * 4), 8, 32, 64, 1e-6, *([None] * 3)) == 2
    assert lib.sf_residual_post_norm(*([None] * 3), 256, 64, None, 1e-6, *([None] * 3)) == 2
    assert lib.sf_pack_weight(None, 16, 128, None, None) == 2
    fake = ctypes.c_void_p(256)   # never dereferenced: the shape check comes first
    assert lib.sf_pack_weight(fake, 15, 128, ctypes.c_void_p(512), None) == 1
    assert lib.sf_pack_weight(fake, 16, 100, ctypes.c_void_p(512), None) == 1
    assert lib.sf_chain_correct(*([None] * 7), 8, 32, 28, 4, 64, 0.1, *([None] * 5)) == 2
    assert lib.sf_qkv_workspace_bytes(256, 3584, 4608) > 0
    assert lib.sf_attn_workspace_bytes(256, 28, 0) > 0
    # logit statistics: null outputs, then a vocabulary that is not a multiple of 8
    assert lib.sf_logit_stats(fake, 8, 152064, 152064, 0.95, *([None] * 7), fake, 1 << 30,
                              None) == 2
    outs = [ctypes.c_void_p(4096 * (i + 1)) for i in range(7)]
    assert lib.sf_logit_stats(fake, 8, 152063, 152064, 0.95, *outs, fake, 1 << 30, None) == 1
    assert lib.sf_logit_stats_workspace_bytes(8) >= 8 * 65536 * 4
    assert lib.sf_parent_map(None, 8, 32, fake, None, None) == 2
    # the decode step's facts: the tail must lie inside the block (L - bl <= plen < L)
    assert lib.sf_decode_facts(fake, 64, 64, 32, 8, 0, 1, 2, None, None, 0.9, None, 0, None,
                               fake, None) == 1
    assert lib.sf_decode_facts(fake, 64, 40, 65, 5, 0, 1, 2, None, None, 0.9, None, 0, None,
                               fake, None) == 1
    assert lib.sf_decode_facts(None, 64, 40, 32, 8, 0, 1, 2, None, None, 0.9, None, 0, None,
                               fake, None) == 2
    assert lib.sf_parent_map(fake, 65, 32, fake, None, None) == 1
    # attention: the rows kernel stages src in a 1024-entry LDS table and finds a
    # row's branches with one 64-lane ballot, so a bucket or a step beyond 1024 rows,
    # or more than 64 branches, is a shape error, not an overrun
    p = [ctypes.c_void_p(4096 * (i + 1)) for i in range(9)]
    q, kv, src, rows, cnt, o32, obf, mt, zt = p

    def attn_rows(bucket, B1, N=32):
        return lib.sf_attn_rows(q, kv, None, None, None, 0, 16, 0, 0, src, rows, cnt, bucket, B1,
                                N, 0, B1, 28, 4, 128, 0.088, None, o32, obf, mt, zt, None, 0,
                                None)

    def attn_block(bucket, B1, N=32):
        return lib.sf_attn_prefix_block(q, kv, None, None, None, 0, 16, 0, 0, src, rows, cnt,
                                        bucket, B1, N, 28, 4, 128, 0.088, None, 0, o32, obf, mt,
                                        zt, None, 0, None)
    for fn in (attn_rows, attn_block):
        assert fn(1025, 33) == 1
        assert fn(1024, 33) == 1      # 33 * 32 rows > 1024
        assert fn(1025, 32) == 1      # bucket above B1 * N
        assert fn(100, 65, 8) == 1    # 65 branches


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(_lib, "LIB_PATH", tmp_path / "nope.so")
    monkeypatch.setattr(_lib, "_LIB", None)
    with pytest.raises(_lib.SpecFoldLibraryMissing):
        _lib.load()
