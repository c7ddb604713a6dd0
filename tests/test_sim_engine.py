"""The whole HIP verify step on the CPU: FoldedVerifyEngine.forward (both model
families) with every kernel it launches compiled from its own source for the
SIMT simulator of tests/sim (tests/simlib.py), stage by stage against the oracle
with the same checks and tolerances as the GPU parity tests
(tests/test_gpu_engine_parity.py: integer outputs bit-exact, q/k/v and hidden
states within bf16 rounding, attention state within fp32 attention rounding).

Test infrastructure: the engine refuses a model outside the GPU
(FoldedVerifyEngine._check_device); the subclass below lifts that check for the
simulated library only, and runs without HIP graphs."""

import pytest
import torch

from oracle.folded_reference import StepTrace, folded_verify_step, llama4_q_scale
from specfold_amd.engine import FoldedVerifyEngine
from specfold_amd.kv_cache import PagedKVCache
from tests.helpers import (SHAPE_G2, SHAPE_G7, SHAPE_N4, err_stats, make_case, make_nld_case,
                           plain_events)
from tests.simlib import build_sim_library, compiler, use_sim_library
from tests.test_gpu_engine_parity import check_layers


class SimEngine(FoldedVerifyEngine):
    """The engine over CPU tensors, for the simulated kernels only."""

    @staticmethod
    def _check_device(device):
        if device.type != "cpu":
            raise ValueError("SimEngine runs the simulated kernels on CPU tensors")


@pytest.fixture(scope="module")
def sim(tmp_path_factory):
    if compiler() is None:
        pytest.skip("no clang++ (the simulator needs clang's vector extensions)")
    path = build_sim_library(tmp_path_factory.mktemp("simlib"))
    with use_sim_library(path) as lib:
        yield lib


def run(case, q_scale=None):
    tr = StepTrace()
    ref_logits = folded_verify_step(case.model_cpu, case.tokens, case.kv, case.delta, trace=tr,
                                    shift=False, q_scale=q_scale)
    eng = SimEngine(case.model_cpu)
    eng.use_graphs = False
    cache = None
    if case.kv is not None:
        cache = PagedKVCache(len(case.kv), case.kv[0][0].shape[1], 128, 512, page_size=16,
                             device="cpu", page_order="shuffled", seed=5)
        cache.load_dense(case.kv)
    trace = []
    tf = {li: lt.h_in for li, lt in enumerate(tr.layers)}
    logits = eng.forward(case.tokens, cache, case.delta, trace=trace, teacher=tf, q_scale=q_scale)
    return tr, ref_logits, trace, logits, eng


@pytest.mark.parametrize("name,shape,seed,P,delta", [
    ("g2_p100", SHAPE_G2, 1, 100, 0.1),
    ("g7_p300", SHAPE_G7, 3, 300, 0.05),
])
def test_fastdllm_layers_teacher_forced(sim, name, shape, seed, P, delta):
    case = make_case(shape, seed, P=P, delta=delta)
    tr, ref_logits, trace, logits, eng = run(case)
    check_layers(case, shape, tr, trace, eng)
    st = err_stats(logits.float(), ref_logits.float())
    print(f"{name} logits (teacher-forced last layer): {st}")
    assert st["max_abs"] <= 2e-2 * max(1.0, st["ref_absmax"])


@pytest.mark.parametrize("name,shape,seed,P,delta,omax", [
    ("n4_p100", SHAPE_N4, 1, 100, 0.1, 64),    # llama-4 q scale active
    ("n4_p0", SHAPE_N4, 3, 0, 0.1, 16),
])
def test_nld_layers_teacher_forced(sim, name, shape, seed, P, delta, omax):
    case = make_nld_case(shape, seed, P=P, delta=delta, omax=omax)
    qs = llama4_q_scale(case.model_cpu.config, P, case.tokens.shape[1])
    assert (qs is not None) == (P + case.tokens.shape[1] > omax)
    tr, ref_logits, trace, logits, eng = run(case, q_scale=qs)
    check_layers(case, shape, tr, trace, eng, q_scale=qs)


def _paged(kv):
    if kv is None:
        return None
    cache = PagedKVCache(len(kv), kv[0][0].shape[1], 128, 512, page_size=16, device="cpu",
                         page_order="shuffled", seed=5)
    cache.load_dense(kv)
    return cache


def _batched_vs_single(model, seqs, delta, q_scales=None):
    """forward_batched over `seqs` [(tokens, kv)] against forward on each alone:
    every sequence's logits and per-layer recomputed-row counts identical."""
    from specfold_amd.engine import StepStats
    q_scales = q_scales or [None] * len(seqs)
    eng = SimEngine(model)
    eng.use_graphs = False
    single, counts = [], []
    for (tok, kv), qs in zip(seqs, q_scales):
        st = StepStats()
        single.append(eng.forward(tok, _paged(kv), delta, q_scale=qs, stats=st))
        counts.append(st.counts)
    # unpadded, and every sequence padded with copies of its main branch (they fold
    # at every layer, so the recomputed-row counts are unchanged too)
    for pad_to in (None, max(t.shape[0] for t, _ in seqs) + 2):
        stb = StepStats()
        batched = eng.forward_batched([t for t, _ in seqs], [_paged(kv) for _, kv in seqs],
                                      delta, q_scales=q_scales, stats=stb, pad_to=pad_to)
        assert len(batched) == len(seqs)
        for s, (a, b) in enumerate(zip(batched, single)):
            assert a.shape == b.shape
            assert torch.equal(a, b), (pad_to, s, err_stats(a.float(), b.float()))
        assert stb.counts == [sum(c) for c in zip(*counts)], (pad_to, stb.counts, counts)
    return counts


def test_batched_step_equals_single_steps(sim):
    """Three Fast-dLLM sequences (prefix 100 / none / 37; 8, 1 and 5 branches) in one
    verify step give each sequence's own verify step, bit for bit."""
    from tests.helpers import draft_tree_block, random_prefix_kv
    shape = SHAPE_G2
    model = make_case(shape, 1, P=0).model_cpu
    seqs = []
    for P, k, seed in ((100, 8, 11), (0, 1, 12), (37, 5, 13)):
        gen = torch.Generator().manual_seed(seed)
        tok = draft_tree_block(32, shape.vocab, gen)[:k].contiguous()
        kv = random_prefix_kv(shape.layers, shape.kv_heads, P, shape.head_dim, gen) if P else None
        seqs.append((tok, kv))
    counts = _batched_vs_single(model, seqs, 0.1)
    assert counts[1] == [32] * shape.layers        # a lone main branch: every row recomputed
    assert any(c < 8 * 32 for c in counts[0])      # some rows of the 8-branch tree folded


def test_batched_nld_step_with_q_scales(sim):
    """NLD sequences, the llama-4 q scale active for one (prefix 70 + block > 64) and
    not for the other (no prefix)."""
    from tests.helpers import draft_tree_block, random_prefix_kv
    shape = SHAPE_N4
    model = make_nld_case(shape, 1, P=0, omax=64).model_cpu
    seqs, qss = [], []
    for P, k, seed in ((70, 6, 21), (0, 4, 22)):
        gen = torch.Generator().manual_seed(seed)
        tok = draft_tree_block(32, shape.vocab - 1, gen)[:k].contiguous()
        kv = random_prefix_kv(shape.layers, shape.kv_heads, P, shape.head_dim, gen) if P else None
        seqs.append((tok, kv))
        qss.append(llama4_q_scale(model.config, P, 32))
    assert qss[0] is not None and qss[1] is None
    _batched_vs_single(model, seqs, 0.1, q_scales=qss)


def test_nld_lockstep_decode_matches_separate_decodes(sim, monkeypatch):
    """Two NLD sequences decoded in lockstep (LockstepDecoder: one forward_batched
    per round) produce the tokens and events of the same generators decoding each
    sequence alone (engine forward per verify step), prefill and block commits
    included, all on the simulated kernels."""
    from specfold_amd.configs import SYNTHETIC_DRAFT_GRAPH
    from specfold_amd.generate import nld_model_executor as nme
    from specfold_amd.generate.lockstep import LockstepDecoder
    from specfold_amd.generate.nld_folded import SpecFoldHIPNLDGeneration

    monkeypatch.setattr(nme, "FoldedVerifyEngine", SimEngine)
    shape = SHAPE_N4
    ex = nme.NLDModelExecutor(make_nld_case(shape, 1, P=0, omax=64).model_cpu, device="cpu",
                              block_length=8, max_length=128, page_order="shuffled", page_seed=3)
    ex.engine.use_graphs = False
    g = torch.Generator().manual_seed(9)
    prompts = [torch.randint(0, shape.vocab - 2, (1, n), generator=g) for n in (12, 21)]
    budgets = (16, 8)       # two blocks (a commit mid-run) / one: the loops end apart

    def make():
        return [SpecFoldHIPNLDGeneration(block_length=8, model_executor=ex,
                                         calibration_graph=SYNTHETIC_DRAFT_GRAPH,
                                         threshold=0.9, max_new_tokens=b, max_length=128,
                                         delta=0.1, device="cpu") for b in budgets]

    alone = []
    for gen, p in zip(make(), prompts):
        alone.append((list(gen.decode_steps(p)), gen._state["x_accum"].clone()))
    gens = make()
    dec = LockstepDecoder(gens)
    per_seq = [[] for _ in prompts]
    for rnd in dec.rounds(prompts):
        for i, ev in rnd["events"]:
            per_seq[i].append(ev)
    for i, (ev, x) in enumerate(alone):
        assert plain_events(per_seq[i]) == plain_events(ev), i
        assert torch.equal(gens[i]._state["x_accum"], x), i
    assert dec.batched_steps > 0 and dec.draft_positions > 0
    print(f"rounds {dec.rounds_run}, batched steps {dec.batched_steps}, "
          f"fold ratio {dec.fold_ratio:.3f}")


def test_batched_step_rejects_bad_arguments(sim):
    """forward_batched's host checks, before any launch."""
    shape = SHAPE_G2
    eng = SimEngine(make_case(shape, 1, P=0).model_cpu)
    eng.use_graphs = False
    a = torch.zeros(3, 32, dtype=torch.int64)
    with pytest.raises(ValueError, match="one cache"):
        eng.forward_batched([a, a], [None])
    with pytest.raises(ValueError, match="one q scale"):
        eng.forward_batched([a], [None], q_scales=[None, None])
    with pytest.raises(ValueError, match="same N"):
        eng.forward_batched([a, torch.zeros(2, 16, dtype=torch.int64)], [None, None])
    with pytest.raises(TypeError, match="PagedKVCache"):
        eng.forward_batched([a], [[(torch.zeros(1), torch.zeros(1))]])
    with pytest.raises(ValueError, match="pad_to"):
        eng.forward_batched([a], [None], pad_to=2)
    with pytest.raises(ValueError, match="one cache"):
        eng.forward_batched([], [])
    with pytest.raises(ValueError, match="at most 64 branches and 1024 rows"):
        eng.forward_batched([a] * 4, [None] * 4, pad_to=9)      # 4 x 9 x 32 = 1152 rows


def test_batched_step_bucket_overflow_retry(sim):
    """A bucket below the recomputed count overflows; forward_batched then redoes
    the step with every row (padding kept), and its logits equal the unbucketed
    step's."""
    from specfold_amd.engine import StepStats
    from tests.helpers import draft_tree_block, random_prefix_kv
    shape = SHAPE_G2
    model = make_case(shape, 1, P=0).model_cpu
    eng = SimEngine(model)
    eng.use_graphs = False
    blocks, kvs = [], []
    for P, k, seed in ((50, 4, 41), (0, 2, 42)):
        gen = torch.Generator().manual_seed(seed)
        blocks.append(draft_tree_block(32, shape.vocab, gen)[:k].contiguous())
        kvs.append(random_prefix_kv(shape.layers, shape.kv_heads, P, shape.head_dim, gen)
                   if P else None)
    ref = eng.forward_batched(blocks, [_paged(kv) for kv in kvs], 0.1, pad_to=5)
    st = StepStats()
    got = eng.forward_batched(blocks, [_paged(kv) for kv in kvs], 0.1, bucket=40, pad_to=5,
                              stats=st)
    assert st.overflow is False and st.bucket == 10 * 32     # the retry's stats
    assert [g.shape[0] for g in got] == [4, 2]
    for a, b in zip(got, ref):
        assert torch.equal(a, b)


def test_batched_padding_at_delta_zero(sim):
    """At delta = 0 a padding copy of a main branch can be recomputed at a later
    layer (its chain-corrected attention output rounds one bf16 step off its main
    branch's); every real sequence's logits stay those of its own step.  The
    case an engine-level random sweep found: NLD, four sequences padded to 7."""
    from specfold_amd.engine import StepStats
    from tests.helpers import draft_tree_block, random_prefix_kv
    shape = SHAPE_N4
    model = make_nld_case(shape, 1, P=0, omax=64).model_cpu
    eng = SimEngine(model)
    eng.use_graphs = False
    seqs, qss = [], []
    for k, P, seed in ((2, 6, 470481935), (7, 60, 166478675), (1, 129, 143982545),
                       (2, 97, 416689676)):
        g = torch.Generator().manual_seed(seed)
        tok = draft_tree_block(32, shape.vocab - 1, g)[:k].contiguous()
        kv = random_prefix_kv(shape.layers, shape.kv_heads, P, shape.head_dim, g) if P else None
        seqs.append((tok, kv))
        qss.append(llama4_q_scale(model.config, P, 32))
    single, counts = [], []
    for (t, kv), q in zip(seqs, qss):
        st = StepStats()
        single.append(eng.forward(t, _paged(kv), 0.0, q_scale=q, stats=st))
        counts.append(st.counts)
    st = StepStats()
    got = eng.forward_batched([t for t, _ in seqs], [_paged(kv) for _, kv in seqs], 0.0,
                              q_scales=qss, stats=st, pad_to=7)
    for a, b in zip(got, single):
        assert torch.equal(a, b)
    real = [sum(c) for c in zip(*counts)]
    assert all(b >= r for b, r in zip(st.counts, real)) and st.counts[0] == real[0]
