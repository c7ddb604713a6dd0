"""sf_chain_correct (the reference's incremental chain correction) on the GPU at
the 7B attention shape (cfg3: H 28, Hkv 4, hd 128, B1 8, N 32, a 2048-key prefix
in shuffled 16-token pages), against the oracle's own telescoped correction on
identical q/k/v.

One cfg3-shaped layer runs the verify step on Mode B inputs (branch = parent +
sigma z with sigma 0.2 on a seeded 38% of positions, 0.05 elsewhere; fold ratio
~0.62), so that folded rows sit one to three hops below their recomputing
ancestor.  The step's own gate outputs and roped q/k/v then feed:

* HIP: sf_attn_prefix_block for the recomputed rows, then sf_chain_correct for
  the folded rows (specfold/generate/triton_kernels.py:364-429);
* oracle: ``folded_layer`` with the same q/k/v forced in (``qkv_rows``) on the
  same GPU, i.e. fastdllm_v2_folded.py:164-204 in fp32: exact attention of the
  recomputed rows, then one hop per branch in topological order.

Bounds (measured values are printed beside them): folded and recomputed rows'
O within 1e-3 of max(1, max|O|) and m + log Z within 1e-3 of the oracle's; the
same against exact float64 attention of the same q/k/v; and HIP's chain form
within 1e-3 of the direct form the verify step uses (sf_attn_rows).  m itself
may differ where a replaced key held a row's maximum (the chain keeps the
bound max(m_parent, new scores)), so (m, Z) is compared through m + log Z.
"""

from __future__ import annotations

from dataclasses import replace

import pytest
import torch

from oracle.folded_reference import parent_map
from specfold_amd import _lib
from specfold_amd.configs import workload
from specfold_amd.engine import FoldedVerifyEngine
from specfold_amd.generate.synthetic_model import build_qwen2
from specfold_amd.kv_cache import PagedKVCache
from specfold_amd.synthetic import TREE_DIFFS, draft_tree_block, perturbed_hidden
from tests.helpers import err_stats
from tests.parity import attention_forced, oracle_layer

pytestmark = pytest.mark.gpu

N = 32
BOUND = 1e-3


def test_chain_correct_cfg3_shape_matches_oracle():
    w = workload("cfg3_7b")
    sh = replace(w.shape, layers=1)
    H, Hkv, hd, D = sh.heads, sh.kv_heads, sh.head_dim, sh.hidden
    P = 2048
    print(f"[chain] cfg3 shape H={H} Hkv={Hkv} D={D} P={P}", flush=True)
    model = build_qwen2(sh, w.seed, device="cuda", dtype=torch.bfloat16)
    eng = FoldedVerifyEngine(model)
    cache = PagedKVCache(1, Hkv, hd, P + 2 * N, page_size=16, device="cuda",
                         page_order="shuffled", seed=7)
    g = torch.Generator(device="cuda").manual_seed(7)
    cache.k_pages.normal_(generator=g)
    cache.v_pages.normal_(generator=g)
    cache.advance(P)
    tokens = draft_tree_block(N, sh.vocab - 1, torch.Generator().manual_seed(8),
                              diffs=TREE_DIFFS[:8])
    B1 = tokens.shape[0]
    BN = B1 * N
    parent, counts = parent_map(tokens)
    hid = perturbed_hidden(parent, N, D, torch.Generator().manual_seed(9))
    trace = []
    eng.forward(tokens.cuda(), cache, 0.1, trace=trace, teacher={0: hid.cuda()},
                compute_logits=False)
    torch.cuda.synchronize()
    ht = trace[0]
    rec = ht["rec"].view(B1, N).bool().cpu()
    cnt = int(ht["count"].item())
    folded = int((~rec).sum())
    print(f"[chain] recomputed {cnt} of {BN}, folded {folded}", flush=True)
    assert folded > 0 and cnt > N

    # HIP: recomputed rows (prefix + block), then the chain correction of the rest
    pv = cache.view(0)
    o32 = torch.full((BN, H * hd), float("nan"), device="cuda")
    obf = torch.zeros(BN, H * hd, dtype=torch.bfloat16, device="cuda")
    mt = torch.full((BN, H), float("nan"), device="cuda")
    zt = torch.full((BN, H), float("nan"), device="cuda")
    ws = torch.empty(_lib.attn_workspace_bytes(BN, H, pv.capacity), dtype=torch.uint8,
                     device="cuda")
    _lib.attn_prefix_block(ht["q"], ht["kv"], pv.k, pv.v, pv.page_table, pv.capacity,
                           pv.page_size, pv.page_stride, pv.head_stride, ht["src"], ht["rows"],
                           ht["count"], BN, B1, N, H, Hkv, hd, eng.scaling, o32, obf, mt, zt, ws,
                           prefix_len=pv.length_dev)
    par = torch.tensor([0] + [int(p) for p in parent[1:]], dtype=torch.int32, device="cuda")
    _lib.chain_correct(ht["q"], ht["kv"], ht["src"], par, ht["rec"], ht["seg"], ht["segcnt"], B1,
                       N, H, Hkv, hd, eng.scaling, o32, obf, mt, zt)
    torch.cuda.synchronize()
    assert not torch.isnan(o32).any() and not torch.isnan(mt).any()
    assert torch.equal(obf, o32.to(torch.bfloat16))

    # oracle on the same GPU with the step's own q/k/v forced in
    q_rows = ht["q"][:BN].view(BN, H, hd)
    kv_rows = ht["kv"][:BN].view(BN, 2, Hkv, hd)

    def qkv_rows(i, rsel):
        r = i * N + rsel.to("cuda")
        return (q_rows[r].transpose(0, 1), kv_rows[r, 0].transpose(0, 1),
                kv_rows[r, 1].transpose(0, 1))

    cos, sin = eng.rope_tables(P + N)
    lt = oracle_layer(eng.layers[0], hid, parent, counts, cache[0], cos[P:P + N], sin[P:P + N],
                      0.1, H, Hkv, device="cuda", qkv_rows=qkv_rows)
    assert torch.equal(lt.rec, rec), "the oracle's gate disagrees with the step's"
    o_ref = lt.O.permute(0, 2, 1, 3).reshape(B1, N, H, hd)        # [B1, N, H, hd]
    lse_ref = (lt.m.double() + torch.log(lt.Z.double())).permute(0, 2, 1)
    o_hip = o32.view(B1, N, H, hd).cpu()
    lse_hip = (mt.double() + torch.log(zt.double())).view(B1, N, H).cpu()
    ex_o, ex_m, ex_z = attention_forced(ht, cache[0], B1, N, H, Hkv, hd, eng.scaling)
    ex_lse = ex_m + torch.log(ex_z)
    o_rows = ht["o32"].view(B1, N, H, hd).cpu()                    # the step's direct form
    fails = []
    for part, sel in (("folded", ~rec), ("recomputed", rec)):
        for nm, a, b, ref_kind in (
                ("O", o_hip[sel], o_ref[sel], "oracle chain"),
                ("lse", lse_hip[sel], lse_ref[sel], "oracle chain"),
                ("O", o_hip[sel], ex_o[sel], "exact fp64"),
                ("lse", lse_hip[sel], ex_lse[sel], "exact fp64"),
                ("O", o_hip[sel], o_rows[sel], "sf_attn_rows"),
                ("O oracle", o_ref[sel], ex_o[sel], "exact fp64")):
            st = err_stats(a.float(), b.float())
            ok = st["max_abs"] <= BOUND * max(1.0, st["ref_absmax"])
            print(f"[chain] {part:10s} {nm:8s} vs {ref_kind:12s}: max {st['max_abs']:.3g} "
                  f"mean_rel {st['mean_rel']:.2e} |ref| {st['ref_absmax']:.3g}", flush=True)
            if not ok:
                fails.append((part, nm, ref_kind, st))
    # the chain's m is the running bound max(m_parent, new scores): never below
    # the row's own maximum
    assert bool((mt.view(B1, N, H).cpu().double() >= ex_m - 1e-4).all())
    assert not fails, fails
