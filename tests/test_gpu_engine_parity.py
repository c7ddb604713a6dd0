"""HIP verify step vs the oracle, stage by stage and end to end.

Each layer is teacher-forced with the oracle's layer input, so the integer
outputs (recompute mask, compacted rows, src, counts) must match bit-exactly
and the float outputs are compared against the oracle's at that stage, with
the FFN also forced with the oracle's attention residual; the tolerances are
tests/parity.py's.  End to end (no forcing) the logits are compared against
the oracle on the CPU and on the same GPU (check_end_to_end).
"""

import pytest
import torch

from oracle.folded_reference import StepTrace, folded_verify_step
from specfold_amd.engine import FoldedVerifyEngine, build_parent_map
from specfold_amd.kv_cache import PagedKVCache
from tests.helpers import SHAPE_G2, SHAPE_G6, SHAPE_G7, err_stats, make_case, to_gpu_model
from tests.parity import (LOGITS_SPREAD_FACTOR, NS_MAX_ABS, NS_MEAN_REL, compare_layer,
                          oracle_layer)

pytestmark = pytest.mark.gpu


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
    return tr, ref_logits, trace, logits, eng


CASES = [
    ("g2_p100", SHAPE_G2, 1, 100, 0.1),
    ("g2_p0", SHAPE_G2, 2, 0, 0.1),
    ("g7_p300", SHAPE_G7, 3, 300, 0.05),
    ("g6_p517", SHAPE_G6, 4, 517, 0.02),
]


@pytest.mark.parametrize("name,shape,seed,P,delta", CASES)
def test_layers_teacher_forced(name, shape, seed, P, delta):
    case = make_case(shape, seed, P=P, delta=delta)
    tr, _, trace, _, eng = run_pair(case)
    check_layers(case, shape, tr, trace, eng)


def check_layers(case, shape, tr, trace, eng, q_scale=None):
    """Stage-by-stage comparison of a teacher-forced step (tests/parity.py),
    with the oracle also run on the GPU on the same layer inputs."""
    B1, N = case.tokens.shape
    H, Hkv, hd, D = shape.heads, shape.kv_heads, shape.head_dim, shape.hidden
    parent = tr.parent
    assert parent == build_parent_map(case.tokens)[0]
    P = case.kv[0][0].shape[-2] if case.kv else 0
    cos, sin = eng.rope_tables(P + N)
    for li, (lt, ht) in enumerate(zip(tr.layers, trace)):
        kv = case.kv[li] if case.kv else None
        lt_gpu = None
        if eng.device.type == "cuda":
            lt_gpu = oracle_layer(eng.layers[li], lt.h_in, parent, tr.counts, kv, cos[P:P + N],
                                  sin[P:P + N], case.delta, H, Hkv, q_scale=q_scale,
                                  device="cuda")
        compare_layer(li, lt, ht, parent, B1, N, H, Hkv, hd, D, eng=eng, lt_gpu=lt_gpu, prefix_kv=kv)


@pytest.mark.parametrize("name,shape,seed,P,delta", CASES[:3])
def test_end_to_end_logits(name, shape, seed, P, delta):
    check_end_to_end(name, make_case(shape, seed, P=P, delta=delta))


# End to end against the CPU oracle (2-layer cases): measured at most 5.55e-3 mean rel
# (g7_p300; the oracle's own GPU-vs-CPU spread there is 3.99e-3), bound with a 25% margin.
LOGITS_MEAN_REL_MAX = 7e-3


def check_end_to_end(name, case, q_scale=None):
    """No teacher forcing.  bf16 turns fp32-level differences (summation order in
    attention and the GEMMs) into 1-ulp flips that every following GEMM spreads,
    so the reference itself, evaluated in torch on the GPU instead of the CPU,
    lands a measurable distance from its CPU result.  Bounds:
      * zero mask flips against the CPU oracle at every layer;
      * max |d| <= 2e-2 * max(1, |ref|) against the CPU oracle and against the
        oracle on the same GPU;
      * mean rel against the oracle on the same GPU <= max(1e-3,
        LOGITS_SPREAD_FACTOR x the oracle's own GPU-vs-CPU spread), and against
        the CPU oracle <= LOGITS_MEAN_REL_MAX;
      * the head alone (HIP final hidden state -> the oracle's norm + head on the
        same GPU) within max abs 2e-2 and mean rel 1e-3."""
    tr, ref_logits, trace, logits, eng = run_pair(case, teacher=False, q_scale=q_scale)
    B1, N = case.tokens.shape
    flips = sum(int((ht["rec"].cpu().view(B1, N).bool() != lt.rec).sum())
                for lt, ht in zip(tr.layers, trace))
    model_gpu = eng.model
    kv_gpu = [(k.cuda(), v.cuda()) for k, v in case.kv] if case.kv else None
    ref_gpu = folded_verify_step(model_gpu, case.tokens.cuda(), kv_gpu, case.delta, shift=False,
                                 q_scale=q_scale)
    spread = err_stats(ref_gpu.float(), ref_logits.float())
    st_cpu = err_stats(logits.float(), ref_logits.float())
    st_gpu = err_stats(logits.float(), ref_gpu.float())
    head_ref = eng.head(eng.base.norm(eng.last_hidden.view(B1, N, -1)))
    st_head = err_stats(logits.float(), head_ref.float())
    print(f"{name}: mask flips {flips}\n  hip vs oracle(cpu)         {st_cpu}"
          f"\n  hip vs oracle(gpu)         {st_gpu}\n  oracle(gpu) vs oracle(cpu) {spread}"
          f"\n  head alone                 {st_head}", flush=True)
    assert flips == 0
    for st in (st_cpu, st_gpu):
        assert st["max_abs"] <= NS_MAX_ABS * max(1.0, st["ref_absmax"]), st
    assert st_gpu["mean_rel"] <= max(NS_MEAN_REL, LOGITS_SPREAD_FACTOR * spread["mean_rel"]), \
        (st_gpu, spread)
    assert st_cpu["mean_rel"] <= LOGITS_MEAN_REL_MAX, st_cpu
    assert st_head["max_abs"] <= NS_MAX_ABS * max(1.0, st_head["ref_absmax"]) and \
        st_head["mean_rel"] <= NS_MEAN_REL, st_head


def test_contiguous_and_paged_prefix_identical():
    case = make_case(SHAPE_G2, 9, P=200, delta=0.1)
    a = run_pair(case, teacher=False, cache_kind="paged")[3]
    b = run_pair(case, teacher=False, cache_kind="list")[3]
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


def test_reference_cache_graph_survives_commits():
    """A transformers DynamicCache (the reference's cache, fastdllm_v2_folded.py:122)
    grown by torch.cat over three block commits: the engine reads it through its
    mirror, so the verify step is captured once for the branch count and every
    replay equals the eager step bit for bit, before and after each commit."""
    from transformers.cache_utils import DynamicCache
    case = make_case(SHAPE_G7, 13, P=130, delta=0.05)
    model = to_gpu_model(case.model_cpu)
    eng = FoldedVerifyEngine(model)
    cache = DynamicCache()
    for li, (k, v) in enumerate(case.kv):
        cache.update(k.cuda(), v.cuda(), li)
    Hkv, hd = case.kv[0][0].shape[1], case.kv[0][0].shape[3]
    t = case.tokens.cuda()
    gen = torch.Generator().manual_seed(4)
    captures = 0
    for commit in range(4):
        eng.use_graphs = False
        ref = eng.forward(t, cache, case.delta)
        eng.use_graphs = True
        n0 = len(eng._graphs)
        for _ in range(2):
            out = eng.forward(t, cache, case.delta)
            torch.cuda.synchronize()
            assert torch.equal(out, ref), f"commit {commit}: replay differs from eager"
        captures += len(eng._graphs) - n0
        for li in range(len(case.kv)):   # commit 32 tokens: every layer grows by torch.cat
            kn = torch.randn(1, Hkv, 32, hd, generator=gen).to(torch.bfloat16).cuda()
            vn = torch.randn(1, Hkv, 32, hd, generator=gen).to(torch.bfloat16).cuda()
            cache.update(kn, vn, li)
    assert cache.get_seq_length() == 130 + 4 * 32
    assert captures == 1, f"{captures} captures over four prefix lengths"
