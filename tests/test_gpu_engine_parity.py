"""HIP verify step vs the oracle, stage by stage and end to end.

Each layer is teacher-forced with the oracle's layer input, so the integer
outputs (recompute mask, compacted rows, src, counts) must match bit-exactly
and the float outputs are compared against the oracle's at that stage:
q/k/v and hidden states within bf16 rounding, attention state within fp32
attention rounding.  Tolerances (written here, per quantity):
  q/k/v, hidden      |hip - ref| <= 2^-7 * |ref| + 2^-7   (<= ~2 bf16 ulps)
  O (fp32), m, Z     max |hip - ref| / max|ref| <= 2e-3
  logits             max abs <= 2e-2 * max(1, max|ref|); mean rel <= max(1e-3,
                     2 x the spread of the oracle itself run on the GPU vs the CPU)
"""

import pytest
import torch

from oracle.folded_reference import StepTrace, folded_verify_step
from specfold_amd.engine import FoldedVerifyEngine, build_parent_map
from specfold_amd.kv_cache import PagedKVCache
from tests.helpers import (SHAPE_G2, SHAPE_G6, SHAPE_G7, err_stats, make_case, src_from_mask,
                           to_gpu_model)

pytestmark = pytest.mark.gpu


def bf16_close(a, b, rel=2 ** -7, abs_=2 ** -7):
    a = a.detach().float().cpu()
    b = b.detach().float().cpu()
    bad = (a - b).abs() > rel * b.abs() + abs_
    return int(bad.sum()), err_stats(a, b)


def run_pair(case, teacher=True, cache_kind="paged", q_scale=None):
    tr = StepTrace()
    ref_logits = folded_verify_step(case.model_cpu, case.tokens, case.kv, case.delta, trace=tr,
                                    shift=False, q_scale=q_scale)
    model = to_gpu_model(case.model_cpu)
    eng = FoldedVerifyEngine(model)
    cache = None
    if case.kv is not None:
        if cache_kind == "paged":
            cache = PagedKVCache(len(case.kv), case.kv[0][0].shape[1], 128, 4096, page_size=16,
                                 device="cuda", page_order="shuffled", seed=5)
            cache.load_dense(case.kv)
        else:
            cache = [(k.cuda(), v.cuda()) for k, v in case.kv]
    trace = []
    tf = {li: lt.h_in.cuda() for li, lt in enumerate(tr.layers)} if teacher else None
    logits = eng.forward(case.tokens.cuda(), cache, case.delta, trace=trace, teacher=tf,
                         q_scale=None if q_scale is None else q_scale.cuda())
    torch.cuda.synchronize()
    return tr, ref_logits, trace, logits


CASES = [
    ("g2_p100", SHAPE_G2, 1, 100, 0.1),
    ("g2_p0", SHAPE_G2, 2, 0, 0.1),
    ("g7_p300", SHAPE_G7, 3, 300, 0.05),
    ("g6_p517", SHAPE_G6, 4, 517, 0.02),
]


@pytest.mark.parametrize("name,shape,seed,P,delta", CASES)
def test_layers_teacher_forced(name, shape, seed, P, delta):
    case = make_case(shape, seed, P=P, delta=delta)
    tr, _, trace, _ = run_pair(case)
    check_layers(case, shape, tr, trace)


def check_layers(case, shape, tr, trace):
    """Stage-by-stage comparison of a teacher-forced step (tolerances above)."""
    B1, N = case.tokens.shape
    H, Hkv, hd, D = shape.heads, shape.kv_heads, shape.head_dim, shape.hidden
    parent = tr.parent
    assert parent == build_parent_map(case.tokens)[0]
    for li, (lt, ht) in enumerate(zip(tr.layers, trace)):
        rec_ref = lt.rec
        rec_hip = ht["rec"].cpu().view(B1, N).bool()
        assert torch.equal(rec_hip, rec_ref), f"layer {li}: recompute mask differs"
        cnt = int(ht["count"].item())
        assert cnt == int(rec_ref.sum())
        rows_ref = rec_ref.flatten().nonzero().flatten().to(torch.int32)
        assert torch.equal(ht["rows"].cpu()[:cnt], rows_ref)
        assert torch.all(ht["rows"].cpu()[cnt:] == B1 * N)
        src_ref = src_from_mask(parent, rec_ref)
        assert torch.equal(ht["src"].cpu().view(B1, N).long(), src_ref)

        r = rows_ref.long()
        bb, nn = r // N, r % N
        q_hip = ht["q"].cpu().view(-1, H, hd)[r]
        q_ref = lt.q[bb, :, nn, :]
        kv = ht["kv"].cpu().view(-1, 2, Hkv, hd)[r]
        k_ref = lt.k[bb, :, nn, :]
        v_ref = lt.v[bb, :, nn, :]
        for nm, a, b in (("q", q_hip, q_ref), ("k", kv[:, 0], k_ref), ("v", kv[:, 1], v_ref)):
            nbad, st = bf16_close(a, b)
            print(f"layer {li} {nm}: {st}")
            assert nbad == 0, f"layer {li} {nm}: {nbad} elements off ({st})"

        o_hip = ht["o32"].cpu().view(B1, N, H, hd)
        o_ref = lt.O.permute(0, 2, 1, 3)
        st = err_stats(o_hip, o_ref)
        print(f"layer {li} O: {st}")
        assert st["max_abs"] <= 2e-3 * max(st["ref_absmax"], 1e-6)
        m_hip = ht["m"].cpu().view(B1, N, H)
        z_hip = ht["z"].cpu().view(B1, N, H)
        for nm, a, b in (("m", m_hip, lt.m.permute(0, 2, 1)), ("Z", z_hip, lt.Z.permute(0, 2, 1))):
            st = err_stats(a, b)
            print(f"layer {li} {nm}: {st}")
            assert st["max_abs"] <= 2e-3 * max(st["ref_absmax"], 1.0)

        nbad, st = bf16_close(ht["h_out"].cpu().view(B1, N, D), lt.h_out)
        print(f"layer {li} h_out: {st}")
        assert nbad == 0, f"layer {li} h_out: {nbad} elements off ({st})"


@pytest.mark.parametrize("name,shape,seed,P,delta", CASES[:3])
def test_end_to_end_logits(name, shape, seed, P, delta):
    check_end_to_end(name, make_case(shape, seed, P=P, delta=delta))


def check_end_to_end(name, case, q_scale=None):
    """No teacher forcing.  bf16 turns fp32-level differences in attention into
    1-ulp flips that every following GEMM spreads, so the reference itself,
    evaluated on the GPU instead of the CPU, lands a measurable distance from
    its CPU result.  The HIP path must be no further from the CPU oracle than
    that spread (x2), and within the absolute bound max|d| <= 2e-2*max(1, |ref|)."""
    tr, ref_logits, trace, logits = run_pair(case, teacher=False, q_scale=q_scale)
    B1, N = case.tokens.shape
    flips = sum(int((ht["rec"].cpu().view(B1, N).bool() != lt.rec).sum())
                for lt, ht in zip(tr.layers, trace))
    model_gpu = to_gpu_model(case.model_cpu)
    kv_gpu = [(k.cuda(), v.cuda()) for k, v in case.kv] if case.kv else None
    ref_gpu = folded_verify_step(model_gpu, case.tokens.cuda(), kv_gpu, case.delta, shift=False,
                                 q_scale=q_scale)
    spread = err_stats(ref_gpu.float(), ref_logits.float())
    st = err_stats(logits.float(), ref_logits.float())
    print(f"{name}: mask flips {flips}\n  hip vs oracle(cpu) {st}\n  oracle(gpu) vs oracle(cpu) {spread}")
    assert flips == 0
    assert st["max_abs"] <= 2e-2 * max(1.0, st["ref_absmax"])
    assert st["mean_rel"] <= max(1e-3, 2.0 * spread["mean_rel"])


def test_contiguous_and_paged_prefix_identical():
    case = make_case(SHAPE_G2, 9, P=200, delta=0.1)
    _, _, _, a = run_pair(case, teacher=False, cache_kind="paged")
    _, _, _, b = run_pair(case, teacher=False, cache_kind="list")
    assert torch.equal(a, b)


def test_run_twice_bitwise():
    case = make_case(SHAPE_G7, 10, P=150, delta=0.05)
    model = to_gpu_model(case.model_cpu)
    eng = FoldedVerifyEngine(model)
    cache = [(k.cuda(), v.cuda()) for k, v in case.kv]
    t = case.tokens.cuda()
    a = eng.forward(t, cache, case.delta)
    b = eng.forward(t, cache, case.delta)
    assert torch.equal(a, b)


def test_bucket_overflow_recomputes_full():
    case = make_case(SHAPE_G2, 11, P=64, delta=0.1)
    model = to_gpu_model(case.model_cpu)
    eng = FoldedVerifyEngine(model)
    cache = [(k.cuda(), v.cuda()) for k, v in case.kv]
    t = case.tokens.cuda()
    full = eng.forward(t, cache, case.delta)
    small = eng.forward(t, cache, case.delta, bucket=8)   # main alone needs 32 rows
    assert torch.equal(full, small)


def test_graph_replays_match_eager():
    """The layer loop replayed from a captured HIP graph equals the eager launch
    sequence bit for bit, on every replay, with eager work and host syncs in
    between, and when the prefix grows (a new capture)."""
    case = make_case(SHAPE_G7, 12, P=130, delta=0.05)
    model = to_gpu_model(case.model_cpu)
    eng = FoldedVerifyEngine(model)
    cache = PagedKVCache(len(case.kv), case.kv[0][0].shape[1], 128, 1024, page_size=16,
                         device="cuda", page_order="shuffled", seed=1)
    cache.load_dense(case.kv)
    t = case.tokens.cuda()
    gen = torch.Generator().manual_seed(3)
    others = [t.clone() for _ in range(3)]
    for o in others:
        o[1:, 0] = torch.randint(0, SHAPE_G7.vocab, (t.shape[0] - 1,), generator=gen).cuda()
    eng.use_graphs = False
    eager = [eng.forward(x, cache, case.delta) for x in [t] + others]
    eng.use_graphs = True
    for rep in range(3):
        for x, ref in zip([t] + others, eager):
            out = eng.forward(x, cache, case.delta)
            torch.cuda.synchronize()
            assert torch.equal(out, ref), f"replay {rep} differs from eager"
            _ = (out.float() * 2).sum().item()          # unrelated eager work + sync
    # grow the prefix by one block commit: a new graph for the new length
    blk = torch.randint(0, SHAPE_G7.vocab, (1, 32), generator=gen).cuda()
    eng.use_graphs = False
    from specfold_amd import _lib
    eng.gate_mode = _lib.SF_GATE_ALL
    eng.forward(blk, cache, 0.0, append=True)
    eng.gate_mode = _lib.SF_GATE_MODEL_DTYPE
    ref2 = eng.forward(t, cache, case.delta)
    eng.use_graphs = True
    for _ in range(2):
        assert torch.equal(eng.forward(t, cache, case.delta), ref2)
