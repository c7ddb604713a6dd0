"""The fused entry points against the unfused compositions they replace, on the
same inputs, bit for bit:

* sf_fold_gate_residual  == sf_residual_gather_add then sf_fold_gate
* sf_residual_post_norm  == bf16 add (torch) then sf_rows_rmsnorm of the recomputed rows
* sf_residual_rmsnorm    == sf_residual_gather_add then sf_rows_rmsnorm of every row
* sf_fold_gate(SF_GATE_DEFER_COMPACT) + sf_qkv_rope_gated
                         == sf_fold_gate then sf_qkv_rope (or sf_qkv_rope_branches):
                            every compaction output and the q/kv tables

(each unfused step is itself checked against the reference semantics in
test_gpu_gate.py / test_gpu_gemm.py)."""

import pytest
import torch

from specfold_amd import _lib
from specfold_amd.synthetic import TREE_PARENTS, perturbed_hidden

pytestmark = pytest.mark.gpu

I32 = dict(dtype=torch.int32, device="cuda")


def gate_buffers(B1, N, D, bucket):
    BN = B1 * N
    return dict(rec=torch.zeros(BN, dtype=torch.int8, device="cuda"), f=torch.zeros(BN, **I32),
                src=torch.zeros(BN, **I32), rows=torch.full((bucket,), -7, **I32),
                count=torch.zeros(1, **I32), seg=torch.full((BN,), -1, **I32),
                segcnt=torch.zeros(B1, **I32), slot=torch.full((BN,), -9, **I32),
                rstd=torch.zeros(BN, dtype=torch.float32, device="cuda"),
                xn=torch.zeros(BN, D, dtype=torch.bfloat16, device="cuda"))


@pytest.mark.parametrize("D,bucket,seed", [(3584, 256, 0), (1536, 40, 1), (5120, 256, 2)])
def test_fold_gate_residual_matches_unfused(D, bucket, seed):
    g = torch.Generator().manual_seed(seed)
    parents = TREE_PARENTS
    B1, N = len(parents), 32
    BN = B1 * N
    hp = torch.zeros(BN + 1, D, dtype=torch.bfloat16)
    hp[:BN] = perturbed_hidden(parents, N, D, g).reshape(BN, D)
    ffn = (0.02 * torch.randn(BN + 1, D, generator=g)).to(torch.bfloat16)
    src_prev = torch.randint(0, B1, (BN,), generator=g, dtype=torch.int32)
    hp, ffn, src_prev = hp.cuda(), ffn.cuda(), src_prev.cuda()
    par = torch.tensor([0] + [int(p) for p in parents[1:]], **I32)
    ln_w = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16).cuda()
    mode, delta = _lib.SF_GATE_MODEL_DTYPE, 0.1

    h = torch.empty(BN, D, dtype=torch.bfloat16, device="cuda")
    _lib.residual_gather_add(hp, ffn, src_prev, B1, N, D, h)
    u = gate_buffers(B1, N, D, bucket)
    _lib.fold_gate(h, par, ln_w, B1, N, bucket, delta, 1e-6, mode, u["rec"], u["f"], u["src"],
                   u["rows"], u["count"], u["seg"], u["segcnt"], u["rstd"], u["xn"],
                   slot=u["slot"])
    # fused, with src written over src_prev in place (the engine's use)
    fz = gate_buffers(B1, N, D, bucket)
    fz["src"].copy_(src_prev)
    h2 = torch.empty(BN, D, dtype=torch.bfloat16, device="cuda")
    _lib.fold_gate_residual(hp, ffn, fz["src"], par, ln_w, B1, N, D, bucket, delta, 1e-6, mode, h2,
                            fz["rec"], fz["f"], fz["src"], fz["rows"], fz["count"], fz["seg"],
                            fz["segcnt"], fz["slot"], fz["rstd"], fz["xn"])
    torch.cuda.synchronize()
    assert torch.equal(h2, h)
    for k in ("rec", "f", "src", "rows", "count", "segcnt", "slot", "rstd"):
        assert torch.equal(fz[k], u[k]), k
    for b in range(B1):
        c = int(u["segcnt"][b])
        assert torch.equal(fz["seg"][b * N:b * N + c], u["seg"][b * N:b * N + c])
    rows = u["rows"][:min(int(u["count"][0]), bucket)].long()
    assert torch.equal(fz["xn"][rows], u["xn"][rows])
    # the mask is a mixture, and slot inverts rows
    n_rec = int(u["rec"].sum())
    assert N < n_rec < BN
    slot = u["slot"].cpu()
    for m, r in enumerate(rows.cpu().tolist()):
        assert int(slot[r]) == m
    assert int((slot >= 0).sum()) == rows.numel()


@pytest.mark.parametrize("D,seed", [(3584, 0), (1536, 1)])
def test_residual_post_norm_matches_unfused(D, seed):
    g = torch.Generator().manual_seed(seed)
    BN, bucket = 256, 256
    x = torch.randn(BN, D, generator=g).to(torch.bfloat16).cuda()
    y = (0.3 * torch.randn(BN, D, generator=g)).to(torch.bfloat16).cuda()
    w = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16).cuda()
    rec = torch.rand(BN, generator=g) < 0.4
    rows_l = rec.nonzero().flatten().to(torch.int32)
    cnt = rows_l.numel()
    rows = torch.full((bucket,), BN, dtype=torch.int32)
    rows[:cnt] = rows_l
    slot = torch.full((BN,), -1, dtype=torch.int32)
    slot[rows_l.long()] = torch.arange(cnt, dtype=torch.int32)
    rows, slot, count = rows.cuda(), slot.cuda(), torch.tensor([cnt], **I32)

    hp_ref = torch.zeros(BN + 1, D, dtype=torch.bfloat16, device="cuda")
    torch.add(x, y, out=hp_ref[:BN])
    zn_ref = torch.zeros(bucket, D, dtype=torch.bfloat16, device="cuda")
    _lib.rows_rmsnorm(hp_ref, rows, count, bucket, w, D, 1e-6, zn_ref)
    hp = torch.zeros(BN + 1, D, dtype=torch.bfloat16, device="cuda")
    zn = torch.zeros(bucket, D, dtype=torch.bfloat16, device="cuda")
    _lib.residual_post_norm(x, y, slot, BN, D, w, 1e-6, hp, zn)
    torch.cuda.synchronize()
    assert torch.equal(hp, hp_ref)
    assert torch.equal(zn[:cnt], zn_ref[:cnt])


@pytest.mark.parametrize("D,seed", [(3584, 3), (4096, 4)])
def test_residual_rmsnorm_matches_unfused(D, seed):
    g = torch.Generator().manual_seed(seed)
    B1, N = 8, 32
    BN = B1 * N
    hp = torch.randn(BN + 1, D, generator=g).to(torch.bfloat16).cuda()
    ffn = (0.3 * torch.randn(BN + 1, D, generator=g)).to(torch.bfloat16).cuda()
    src = torch.randint(0, B1, (BN,), generator=g, dtype=torch.int32).cuda()
    w = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16).cuda()
    h_ref = torch.empty(BN, D, dtype=torch.bfloat16, device="cuda")
    _lib.residual_gather_add(hp, ffn, src, B1, N, D, h_ref)
    out_ref = torch.empty(BN, D, dtype=torch.bfloat16, device="cuda")
    _lib.rows_rmsnorm(h_ref, torch.arange(BN, **I32), torch.tensor([BN], **I32), BN, w, D, 1e-6,
                      out_ref)
    h = torch.empty(BN, D, dtype=torch.bfloat16, device="cuda")
    out = torch.empty(BN, D, dtype=torch.bfloat16, device="cuda")
    _lib.residual_rmsnorm(hp, ffn, src, w, B1, N, D, 1e-6, h, out)
    torch.cuda.synchronize()
    assert torch.equal(h, h_ref)
    assert torch.equal(out, out_ref)


@pytest.mark.parametrize("D,H,Hkv,bucket,branches,seed", [
    (3584, 28, 4, 256, False, 0),    # the 7B verify step
    (1536, 12, 2, 40, False, 1),     # an overflowing bucket (count > bucket)
    (3584, 28, 4, 256, True, 2),     # a batched step's per-branch positions and q scales
])
def test_qkv_rope_gated_matches_unfused(D, H, Hkv, bucket, branches, seed):
    g = torch.Generator().manual_seed(seed)
    parents = TREE_PARENTS
    B1, N, hd = len(parents), 32, 128
    BN = B1 * N
    nq = (H + 2 * Hkv) * hd
    hidden = perturbed_hidden(parents, N, D, g).reshape(BN, D).cuda()
    par = torch.tensor([0] + [int(p) for p in parents[1:]], **I32)
    ln_w = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16).cuda()
    w = (0.02 * torch.randn(nq, D, generator=g)).to(torch.bfloat16).cuda()
    wp = _lib.pack_weight(w)
    b = (0.1 * torch.randn(nq, generator=g)).to(torch.bfloat16).cuda()
    T = 4096
    ang = torch.arange(T, dtype=torch.float32)[:, None] * (1e-4 ** (torch.arange(64) / 64))
    cos = torch.cat([ang.cos(), ang.cos()], 1).to(torch.bfloat16).cuda()
    sin = torch.cat([ang.sin(), ang.sin()], 1).to(torch.bfloat16).cuda()
    if branches:
        pos = torch.randint(0, T - N, (B1,), generator=g, dtype=torch.int32).cuda()
        q_scale = (1 + 0.1 * torch.rand(BN, generator=g)).cuda()
    else:
        pos = torch.tensor([1500], **I32)
        q_scale = (1 + 0.1 * torch.rand(N, generator=g)).cuda()
    mode, delta = _lib.SF_GATE_MODEL_DTYPE, 0.1
    ws = torch.zeros(_lib.qkv_workspace_bytes(bucket, D, nq), dtype=torch.uint8, device="cuda")

    def tables():
        return (torch.full(((BN + 1) * H * hd,), 7.0, dtype=torch.bfloat16, device="cuda"),
                torch.full(((BN + 1) * 2 * Hkv * hd,), 7.0, dtype=torch.bfloat16, device="cuda"))

    u = gate_buffers(B1, N, D, bucket)
    _lib.fold_gate(hidden, par, ln_w, B1, N, bucket, delta, 1e-6, mode, u["rec"], u["f"],
                   u["src"], u["rows"], u["count"], u["seg"], u["segcnt"], u["rstd"], u["xn"],
                   slot=u["slot"])
    q_u, kv_u = tables()
    if branches:
        _lib.qkv_rope_branches(u["xn"], u["rows"], u["count"], bucket, BN, wp, b, cos, sin,
                               q_scale, N, D, H, Hkv, hd, q_u, kv_u, ws, pos)
    else:
        _lib.qkv_rope(u["xn"], u["rows"], u["count"], bucket, BN, wp, b, cos, sin, q_scale, N, D,
                      H, Hkv, hd, q_u, kv_u, ws, pos0=pos)

    fz = gate_buffers(B1, N, D, bucket)
    _lib.fold_gate(hidden, par, ln_w, B1, N, bucket, delta, 1e-6,
                   mode | _lib.SF_GATE_DEFER_COMPACT, fz["rec"], fz["f"], fz["src"], fz["rows"],
                   fz["count"], fz["seg"], fz["segcnt"], fz["rstd"], fz["xn"], slot=fz["slot"])
    torch.cuda.synchronize()
    # the deferred gate leaves the compaction's outputs alone
    assert int(fz["count"][0]) == 0 and int(fz["rows"][0]) == -7
    q_f, kv_f = tables()
    _lib.qkv_rope_gated(fz["xn"], fz["rec"], par, B1, N, bucket, fz["f"], fz["src"], fz["rows"],
                        fz["count"], fz["seg"], fz["segcnt"], fz["slot"], wp, b, cos, sin,
                        q_scale, D, H, Hkv, hd, q_f, kv_f, ws,
                        pos0=None if branches else pos, pos0_branch=pos if branches else None)
    torch.cuda.synchronize()
    for k in ("rec", "f", "src", "rows", "count", "segcnt", "slot", "rstd"):
        assert torch.equal(fz[k], u[k]), k
    for bb in range(B1):
        c = int(u["segcnt"][bb])
        assert torch.equal(fz["seg"][bb * N:bb * N + c], u["seg"][bb * N:bb * N + c])
    count = int(u["count"][0])
    assert N < count < BN
    if bucket < count:
        assert int(fz["count"][0]) == count   # the count of an overflow, rows cut at bucket
    assert torch.equal(q_f, q_u) and torch.equal(kv_f, kv_u)
    rows = u["rows"][:min(count, bucket)].long()
    assert torch.equal(fz["xn"][rows], u["xn"][rows])
    # the projection was written (not the fill) for the recomputed rows
    assert not torch.equal(q_f.view(BN + 1, H * hd)[rows], torch.full_like(
        q_f.view(BN + 1, H * hd)[rows], 7.0))
