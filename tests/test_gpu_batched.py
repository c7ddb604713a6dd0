"""GPU check of FoldedVerifyEngine.forward_batched (sf_qkv_rope_branches and the
SF_GATE_ROOTS_BY_PARENT gate): several sequences in one verify step against each
sequence's own forward.  Integer outputs (per-layer recomputed-row counts) must
be identical, and so must the final hidden state, bit for bit (every kernel's
per-row summation order is independent of the other sequences' rows); the
logits too when the head runs on the library's own kernel, else within the
north star's bound (hipBLASLt's tile choice follows M = total rows)."""

import pytest
import torch

from oracle.folded_reference import llama4_q_scale
from specfold_amd.engine import FoldedVerifyEngine, StepStats
from specfold_amd.generate.nld_model_executor import llama4_q_scale as q_scale_dev
from specfold_amd.kv_cache import PagedKVCache
from tests.helpers import (SHAPE_G2, SHAPE_N4, draft_tree_block, err_stats, make_case,
                           make_nld_case, random_prefix_kv, to_gpu_model)

pytestmark = pytest.mark.gpu


def _paged(kv):
    if kv is None:
        return None
    cache = PagedKVCache(len(kv), kv[0][0].shape[1], 128, 512, page_size=16, device="cuda",
                         page_order="shuffled", seed=5)
    cache.load_dense([(k.cuda(), v.cuda()) for k, v in kv])
    return cache


@pytest.mark.parametrize("family", ["fastdllm", "nld"])
def test_batched_step_gpu(family):
    if family == "fastdllm":
        shape, specs = SHAPE_G2, ((100, 8, 11), (0, 1, 12), (37, 5, 13))
        model = to_gpu_model(make_case(shape, 1, P=0).model_cpu)
        vocab = shape.vocab
    else:
        shape, specs = SHAPE_N4, ((70, 6, 21), (0, 4, 22))
        model = to_gpu_model(make_nld_case(shape, 1, P=0, omax=64).model_cpu)
        vocab = shape.vocab - 1
    seqs, qss = [], []
    for P, k, seed in specs:
        gen = torch.Generator().manual_seed(seed)
        tok = draft_tree_block(32, vocab, gen)[:k].contiguous()
        kv = random_prefix_kv(shape.layers, shape.kv_heads, P, shape.head_dim, gen) if P else None
        seqs.append((tok.cuda(), kv))
        qs = llama4_q_scale(model.config, P, 32) if family == "nld" else None
        qss.append(qs.cuda() if qs is not None else None)
    print(f"[batched_gpu] {family} specs={specs}", flush=True)
    eng = FoldedVerifyEngine(model)
    single, counts, hidden = [], [], []
    for (tok, kv), qs in zip(seqs, qss):
        st = StepStats()
        single.append(eng.forward(tok, _paged(kv), 0.1, q_scale=qs, stats=st))
        hidden.append(eng.last_hidden.clone())
        counts.append(st.counts)
    stb = StepStats()
    batched = eng.forward_batched([t for t, _ in seqs], [_paged(kv) for _, kv in seqs], 0.1,
                                  q_scales=qss, stats=stb)
    torch.cuda.synchronize()
    assert stb.counts == [sum(c) for c in zip(*counts)]
    o = 0
    for a, b, h, (tok, _) in zip(batched, single, hidden, seqs):
        n = tok.shape[0] * 32
        assert torch.equal(eng.last_hidden[o:o + n], h), "final hidden differs from alone"
        o += n
        st = err_stats(a.float(), b.float())
        print(f"[batched_gpu] logits vs alone {st}", flush=True)
        if getattr(eng, "head_kernel", "hipblaslt") == "hip":
            assert torch.equal(a, b), st
        assert st["max_abs"] <= 2e-2 * max(1.0, st["ref_absmax"]), st


def test_batched_graph_replays_gpu():
    """forward_batched through its captured HIP graph (padded shape) against the
    eager run, three times, each sequence's cache grown by a committed block
    between replays (the graph must re-read every prefix length and take the new
    q scales), with eager work in between."""
    shape = SHAPE_N4
    model = to_gpu_model(make_nld_case(shape, 1, P=0, omax=64).model_cpu)
    blocks, caches = [], []
    for P, k, seed in ((40, 5, 31), (0, 3, 32), (17, 1, 33)):
        gen = torch.Generator().manual_seed(seed)
        blocks.append(draft_tree_block(32, shape.vocab - 1, gen)[:k].contiguous().cuda())
        kv = random_prefix_kv(shape.layers, shape.kv_heads, P, shape.head_dim, gen) if P else None
        c = _paged(kv)
        if c is None:
            c = PagedKVCache(shape.layers, shape.kv_heads, 128, 512, page_size=16,
                             device="cuda", page_order="shuffled", seed=5)
        caches.append(c)
    eng = FoldedVerifyEngine(model)
    for rep in range(3):
        qss = [q_scale_dev(model.config, c.length, 32, "cuda") for c in caches]
        print(f"[batched_gpu] graph replay {rep} lengths={[c.length for c in caches]}",
              flush=True)
        eng.use_graphs = False
        ref = eng.forward_batched(blocks, caches, 0.1, q_scales=qss, pad_to=6)
        eng.use_graphs = True
        got = eng.forward_batched(blocks, caches, 0.1, q_scales=qss, pad_to=6)
        torch.cuda.synchronize()
        for a, b in zip(got, ref):
            assert torch.equal(a, b), err_stats(a.float(), b.float())
        for c, b in zip(caches, blocks):      # commit each main branch: the prefixes grow
            eng.use_graphs = False
            eng.forward(b[0:1], c, 0.0, append=True,
                        q_scale=q_scale_dev(model.config, c.length, 32, "cuda"))
        torch.cuda.synchronize()
