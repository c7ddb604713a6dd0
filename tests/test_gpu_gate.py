"""sf_fold_gate: recompute mask, compaction, src, segments, rstd and the
normalized rows, against CPU restatements of the reference gate
(specfold/generate/fastdllm_v2_folded.py:136-152) on the same inputs."""

import pytest
import torch

from specfold_amd import _lib
from specfold_amd.engine import build_parent_map
from specfold_amd.synthetic import TREE_PARENTS, perturbed_hidden
from tests.helpers import src_from_mask

pytestmark = pytest.mark.gpu


def run_gate(hidden, parent, ln_w, delta, mode, bucket=None, eps=1e-6):
    B1, N, D = hidden.shape
    BN = B1 * N
    bucket = BN if bucket is None else bucket
    dev = "cuda"
    i32 = dict(dtype=torch.int32, device=dev)
    par = torch.tensor([0] + [int(p) for p in parent[1:]], **i32)
    out = dict(rec=torch.zeros(BN, dtype=torch.int8, device=dev), f=torch.zeros(BN, **i32),
               src=torch.zeros(BN, **i32), rows=torch.full((bucket,), -7, **i32),
               count=torch.zeros(1, **i32), seg=torch.full((BN,), -1, **i32),
               segcnt=torch.zeros(B1, **i32), rstd=torch.zeros(BN, dtype=torch.float32, device=dev),
               xn=torch.zeros(BN, D, dtype=torch.bfloat16, device=dev))
    _lib.fold_gate(hidden.reshape(BN, D).cuda().contiguous(), par, ln_w.cuda(), B1, N, bucket,
                   delta, eps, mode, out["rec"], out["f"], out["src"], out["rows"], out["count"],
                   out["seg"], out["segcnt"], out["rstd"], out["xn"])
    torch.cuda.synchronize()
    return {k: v.cpu() for k, v in out.items()}


def ref_mask(hidden, parent, delta, mode):
    """The reference gate on CPU: bf16 norms (mode 0) or fp32 squared norms (mode 1)."""
    B1, N, D = hidden.shape
    rec = torch.zeros(B1, N, dtype=torch.bool)
    rec[0] = True
    for i in range(1, B1):
        x, xp = hidden[i], hidden[parent[i]]
        if mode == _lib.SF_GATE_MODEL_DTYPE:
            rec[i] = (x - xp).norm(dim=-1) > delta * xp.norm(dim=-1)
        elif mode == _lib.SF_GATE_FP32_SQUARED:
            d = x.float() - xp.float()
            rec[i] = (d * d).sum(-1) > (torch.tensor(delta, dtype=torch.float32) ** 2) * \
                (xp.float() ** 2).sum(-1)
        else:
            rec[i] = True
    return rec


def check_outputs(out, hidden, parent, rec, ln_w, eps=1e-6, bucket=None):
    B1, N, D = hidden.shape
    BN = B1 * N
    bucket = BN if bucket is None else bucket
    assert torch.equal(out["rec"].view(B1, N).bool(), rec)
    cnt = int(rec.sum())
    assert int(out["count"][0]) == cnt
    rows_ref = rec.flatten().nonzero().flatten().to(torch.int32)
    k = min(cnt, bucket)
    assert torch.equal(out["rows"][:k], rows_ref[:k])
    assert torch.all(out["rows"][k:] == BN)
    src_ref = src_from_mask(parent, rec)
    assert torch.equal(out["src"].view(B1, N).long(), src_ref)
    f_ref = torch.where(rec, torch.arange(B1)[:, None],
                        torch.tensor([0] + [int(p) for p in parent[1:]])[:, None])
    assert torch.equal(out["f"].view(B1, N).long(), f_ref)
    for b in range(B1):
        mine = rec[b].nonzero().flatten() + b * N
        assert int(out["segcnt"][b]) == mine.numel()
        assert torch.equal(out["seg"][b * N:b * N + mine.numel()].long(), mine)
    # rstd and normalized rows vs Qwen2RMSNorm in bf16
    xf = hidden.reshape(BN, D).float()
    var = xf.pow(2).mean(-1, keepdim=True)
    rstd_ref = torch.rsqrt(var + eps).flatten()
    assert torch.allclose(out["rstd"], rstd_ref, rtol=2e-6, atol=0)
    xn_ref = ln_w * (xf * torch.rsqrt(var + eps)).to(torch.bfloat16)
    r = rows_ref.long()
    diff = (out["xn"][r].float() - xn_ref[r].float()).abs()
    assert float(diff.max()) <= float((xn_ref[r].float().abs() * 2 ** -7).max()) + 1e-6
    assert float((diff > 0).float().mean()) < 0.01


@pytest.mark.parametrize("mode", [_lib.SF_GATE_MODEL_DTYPE, _lib.SF_GATE_FP32_SQUARED])
@pytest.mark.parametrize("D", [1536, 3584])
def test_gate_tree_margin(mode, D):
    gen = torch.Generator().manual_seed(D + mode)
    parents = list(TREE_PARENTS)
    hidden = perturbed_hidden(parents, 32, D, gen)
    ln_w = (1 + 0.1 * torch.randn(D, generator=gen)).to(torch.bfloat16)
    rec = ref_mask(hidden, parents, 0.1, mode)
    out = run_gate(hidden, parents, ln_w, 0.1, mode)
    check_outputs(out, hidden, parents, rec, ln_w)
    frac = 1 - rec[1:].float().mean()
    assert 0.3 < frac < 0.9   # both outcomes occur


def test_gate_all_mode_is_dense():
    gen = torch.Generator().manual_seed(3)
    parents = list(TREE_PARENTS)
    hidden = perturbed_hidden(parents, 32, 512, gen)
    ln_w = torch.ones(512, dtype=torch.bfloat16)
    out = run_gate(hidden, parents, ln_w, 0.1, _lib.SF_GATE_ALL)
    check_outputs(out, hidden, parents, torch.ones(8, 32, dtype=torch.bool), ln_w)


@pytest.mark.parametrize("seed", range(6))
def test_gate_random_parent_maps(seed):
    """Random draft blocks -> arbitrary parent forests, random thresholds."""
    gen = torch.Generator().manual_seed(100 + seed)
    B1 = int(torch.randint(2, 17, (1,), generator=gen))
    N = int(torch.randint(4, 64, (1,), generator=gen))
    main = torch.randint(0, 5, (N,), generator=gen)
    toks = main.repeat(B1, 1)
    for i in range(1, B1):
        m = torch.rand(N, generator=gen) < 0.15
        toks[i][m] = torch.randint(5, 9, (int(m.sum()),), generator=gen)
    parents = build_parent_map(toks)[0]
    D = 256
    hidden = torch.zeros(B1, N, D)
    hidden[0] = torch.randn(N, D, generator=gen)
    for i in range(1, B1):
        hidden[i] = hidden[parents[i]] + 0.2 * torch.rand(N, 1, generator=gen) * \
            torch.randn(N, D, generator=gen)
    hidden = hidden.to(torch.bfloat16)
    ln_w = torch.ones(D, dtype=torch.bfloat16)
    delta = float(torch.rand(1, generator=gen)) * 0.2
    rec = ref_mask(hidden, parents, delta, _lib.SF_GATE_MODEL_DTYPE)
    out = run_gate(hidden, parents, ln_w, delta, _lib.SF_GATE_MODEL_DTYPE)
    check_outputs(out, hidden, parents, rec, ln_w)


def test_gate_bucket_overflow_truncates():
    gen = torch.Generator().manual_seed(7)
    parents = list(TREE_PARENTS)
    hidden = perturbed_hidden(parents, 32, 512, gen)
    ln_w = torch.ones(512, dtype=torch.bfloat16)
    rec = ref_mask(hidden, parents, 0.1, 0)
    out = run_gate(hidden, parents, ln_w, 0.1, 0, bucket=40)
    check_outputs(out, hidden, parents, rec, ln_w, bucket=40)
    assert int(out["count"][0]) > 40


def test_gate_rejects_bad_shapes():
    dev = "cuda"
    x = torch.zeros(2 * 600, 64, dtype=torch.bfloat16, device=dev)
    z32 = torch.zeros(1200, dtype=torch.int32, device=dev)
    with pytest.raises(_lib.SpecFoldKernelError):
        _lib.fold_gate(x, torch.zeros(2, dtype=torch.int32, device=dev),
                       torch.ones(64, dtype=torch.bfloat16, device=dev), 2, 600, 1200, 0.1, 1e-6,
                       0, torch.zeros(1200, dtype=torch.int8, device=dev), z32, z32.clone(),
                       z32.clone(), z32.clone(), z32.clone(), z32.clone(),
                       torch.zeros(1200, device=dev), x.clone())
