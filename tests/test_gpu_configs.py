"""The verify step at the benchmark's five configurations, at their real shapes.

Every config builds its model on the GPU at the full shape (random init with
the config's seed; bf16), a prefix of the config's length in a paged KV cache
(K/V ~ N(0, 1) drawn on the GPU from the config's seed; cfg5: 16-token pages in
shuffled order) and the draft-tree token block (B+1 branches, row 0 = main).
Then, on one verify step at full depth:

* per-layer parity: at the first, a middle and the last layer, the oracle's
  folded layer runs on the CPU on the HIP path's own layer input (teacher
  forcing with the HIP input, so deep layers are compared without the
  oracle having to run every layer before them): recompute mask, compacted
  rows, src and count bit-exact; q/k/v, hp and h_out within ~2 bf16 ulps per
  element and within the north star's max abs 2e-2 / mean rel 1e-3; O, m, Z
  within 2e-3 of max|ref| (tests/parity.py);
* zero mask flips at every layer: the gate restated on the CPU on the HIP
  layer input gives the HIP recompute mask at all L layers;
* the head: HIP logits against torch's ``head(norm(h_L))`` on the same GPU from
  the HIP final hidden state, max abs <= 2e-2 and mean rel <= 1e-3;
* graph replay == eager bit for bit, twice; delta < 0 (every row recomputed
  by the gate) == the dense gate mode (SF_GATE_ALL) bit for bit.

cfg1 (the reference's CPU case, fp32) runs here in bf16, the dtype of the HIP
path; its oracle comparison is in bf16, and a Mode-B case (per-branch hidden
states perturbed so that ~38% of draft positions recompute, fold ratio ~0.62)
is also checked against the oracle in fp32 (masks identical, h_out within
max abs 2e-2).  cfg4 also runs its 4 sequences in one batched step against
each sequence's own step.
"""

from __future__ import annotations

import copy
import gc
from dataclasses import replace

import pytest
import torch

from oracle.folded_reference import llama4_q_scale, parent_map
from specfold_amd import _lib
from specfold_amd.configs import workload
from specfold_amd.engine import FoldedVerifyEngine, StepStats
from specfold_amd.generate.synthetic_model import build_nld, build_qwen2
from specfold_amd.kv_cache import PagedKVCache
from specfold_amd.synthetic import TREE_DIFFS, draft_tree_block, perturbed_hidden
from tests.helpers import err_stats
from tests.parity import NS_MAX_ABS, NS_MEAN_REL, compare_layer, gate_flips, oracle_layer

pytestmark = pytest.mark.gpu

N = 32


def _model(w, layers=None):
    sh = w.shape if layers is None else replace(w.shape, layers=layers)
    build = build_nld if w.family == "nld" else build_qwen2
    return build(sh, w.seed, device="cuda", dtype=torch.bfloat16)


def _cache(w, model, P, seed):
    """A paged cache holding a P-token prefix with N(0, 1) K/V in every layer."""
    sh = w.shape
    cache = PagedKVCache(sh.layers if model is None else model.config.num_hidden_layers,
                         sh.kv_heads, sh.head_dim, P + 4 * N, page_size=w.page_size, device="cuda",
                         page_order="shuffled" if w.shuffled_pages else "sequential", seed=seed)
    g = torch.Generator(device="cuda").manual_seed(seed)
    cache.k_pages.normal_(generator=g)
    cache.v_pages.normal_(generator=g)
    if P:
        cache.advance(P)
    return cache


def _tokens(w, seed, branches=None):
    gen = torch.Generator().manual_seed(seed)
    diffs = TREE_DIFFS[:branches or w.branches]
    return draft_tree_block(N, w.shape.vocab - 1, gen, diffs=diffs)


def _rope(eng, P):
    cos, sin = eng.rope_tables(P + N)
    return cos[P:P + N], sin[P:P + N]


def _gc():
    gc.collect()
    torch.cuda.empty_cache()


def check_step(w, model, eng, tokens, cache, q_scale, layers_checked, teacher=None):
    """Traced HIP step + the per-layer oracle comparisons + the head; returns
    (logits, per-layer counts)."""
    cfg = model.config
    H, Hkv, hd, D = cfg.num_attention_heads, cfg.num_key_value_heads, 128, w.shape.hidden
    B1 = tokens.shape[0]
    P = cache.length if cache is not None else 0
    parent, counts = parent_map(tokens)
    trace = []
    st = StepStats()
    logits = eng.forward(tokens.cuda(), cache, w.delta, trace=trace, stats=st,
                         teacher=teacher, q_scale=None if q_scale is None else q_scale.cuda())
    torch.cuda.synchronize()
    L = len(trace)
    print(f"[{w.name}] P={P} B1={B1} counts per layer {st.counts}", flush=True)
    # zero mask flips at every layer (HIP layer input -> the oracle's gate)
    flips = []
    for li, ht in enumerate(trace):
        flips += [(li,) + f for f in gate_flips(ht["h_in"].view(B1, N, D), ht["rec"].view(B1, N),
                                                parent, w.delta)]
    assert not flips, f"mask flips (layer, branch, pos, margin): {flips[:20]}"
    cos_n, sin_n = _rope(eng, P)
    for li in layers_checked:
        li = li % L
        kv = cache[li] if cache is not None and P else None
        h_in = trace[li]["h_in"].view(B1, N, D)
        lt = oracle_layer(eng.layers[li], h_in, parent, counts, kv, cos_n, sin_n, w.delta, H, Hkv,
                          q_scale=q_scale)
        lt_gpu = oracle_layer(eng.layers[li], h_in, parent, counts, kv, cos_n, sin_n, w.delta, H,
                              Hkv, q_scale=q_scale, device="cuda")
        compare_layer(li, lt, trace[li], parent, B1, N, H, Hkv, hd, D, eng=eng, lt_gpu=lt_gpu,
                      prefix_kv=kv)
        del lt, lt_gpu
    # the head on the same GPU from the HIP final hidden state
    base, head = eng.base, eng.head
    ref = head(base.norm(eng.last_hidden.view(B1, N, D)))
    hs = err_stats(logits.float(), ref.float())
    print(f"[{w.name}] head: {hs}", flush=True)
    assert hs["max_abs"] <= NS_MAX_ABS * max(1.0, hs["ref_absmax"]) and \
        hs["mean_rel"] <= NS_MEAN_REL, hs
    del trace, ref
    return logits, st.counts


def check_properties(w, eng, tokens, cache, q_scale, traced_logits):
    """Graph replay == eager (twice), run twice bitwise, delta < 0 == dense gate."""
    t = tokens.cuda()
    qs = None if q_scale is None else q_scale.cuda()
    eng.use_graphs = False
    eager = eng.forward(t, cache, w.delta, q_scale=qs)
    assert torch.equal(eager, traced_logits)
    eng.use_graphs = True
    for rep in range(2):
        g = eng.forward(t, cache, w.delta, q_scale=qs)
        torch.cuda.synchronize()
        assert torch.equal(g, eager), f"[{w.name}] graph replay {rep} differs from eager"
    del g
    eng.use_graphs = False
    neg = eng.forward(t, cache, -1.0, q_scale=qs)
    mode = eng.gate_mode
    eng.gate_mode = _lib.SF_GATE_ALL
    try:
        dense = eng.forward(t, cache, w.delta, q_scale=qs)
    finally:
        eng.gate_mode = mode
        eng.use_graphs = True
    assert torch.equal(neg, dense), f"[{w.name}] delta<0 folded step != dense gate mode"
    print(f"[{w.name}] graph == eager (x2), delta<0 == dense: ok", flush=True)


@pytest.mark.parametrize("name,P", [("cfg2_1p5b", 1024), ("cfg3_7b", 2048), ("cfg5_14b_16k", 16384)])
def test_config_full_depth(name, P):
    w = workload(name)
    model = _model(w)
    eng = FoldedVerifyEngine(model)
    cache = _cache(w, model, P, seed=w.seed + 100)
    tokens = _tokens(w, seed=w.seed + 200)
    q_scale = llama4_q_scale(model.config, P, N) if w.family == "nld" else None
    if name == "cfg5_14b_16k":
        assert q_scale is not None       # the llama-4 q scale is active at a 16k prefix
    L = w.shape.layers
    logits, _ = check_step(w, model, eng, tokens, cache, q_scale, (0, L // 2, L - 1))
    check_properties(w, eng, tokens, cache, q_scale, logits)
    del eng, model, cache, logits
    _gc()


def test_config_cfg1_layer():
    """cfg1: one 1.5B-shaped layer (I = 8960), P = 512, delta 0.1 — token input
    (Mode A) and perturbed hidden states (Mode B, fold ratio ~0.62)."""
    w = workload("cfg1_1p5b_layer")
    model = _model(w)
    eng = FoldedVerifyEngine(model)
    cache = _cache(w, model, 512, seed=100)
    tokens = _tokens(w, seed=200)
    logits, _ = check_step(w, model, eng, tokens, cache, None, (0,))
    check_properties(w, eng, tokens, cache, None, logits)
    # Mode B: x_child = x_parent + sigma * z, sigma 0.2 on 38% of positions, else 0.05
    parent, counts = parent_map(tokens)
    gen = torch.Generator().manual_seed(300)
    hid = perturbed_hidden(parent, N, w.shape.hidden, gen)
    _, cnt = check_step(w, model, eng, tokens, cache, None, (0,), teacher={0: hid.cuda()})
    B1 = tokens.shape[0]
    fold = 1 - (cnt[0] - N) / ((B1 - 1) * N)
    print(f"[cfg1 mode B] recomputed {cnt[0]} of {B1 * N}, fold ratio {fold:.3f}", flush=True)
    assert 0.4 <= fold <= 0.8
    # the same layer input against the oracle in fp32 (cfg1's reference dtype)
    trace = []
    eng.forward(tokens.cuda(), cache, w.delta, trace=trace, teacher={0: hid.cuda()})
    ht = trace[0]
    lyr32 = copy.deepcopy(eng.layers[0]).to("cpu").float()
    cos_n, sin_n = _rope(eng, 512)
    kv = cache[0]
    lt = oracle_layer(lyr32, hid.float(), parent, counts, (kv[0].float(), kv[1].float()),
                      cos_n.float(), sin_n.float(), w.delta, w.shape.heads, w.shape.kv_heads)
    assert torch.equal(ht["rec"].cpu().view(B1, N).bool(), lt.rec)
    st = err_stats(ht["h_out"].float().view(B1, N, -1), lt.h_out)
    print(f"[cfg1 mode B] HIP bf16 vs oracle fp32 h_out: {st}", flush=True)
    assert st["max_abs"] <= NS_MAX_ABS * max(1.0, st["ref_absmax"])
    del eng, model, cache, trace, ht, lt
    _gc()


def test_config_cfg4_batched():
    """cfg4: the 8B NLD shape, B = 4 (5 branches), delta 0.2, P = 4096 — one
    sequence against the oracle, then 4 sequences in one batched step against
    each sequence's own step (per-layer counts identical, logits within the
    north star's bound)."""
    w = workload("cfg4_8b_x4")
    P = w.prefix
    model = _model(w)
    eng = FoldedVerifyEngine(model)
    caches = [_cache(w, model, P, seed=w.seed + 100 + s) for s in range(w.batch)]
    blocks = [_tokens(w, seed=w.seed + 200 + s) for s in range(w.batch)]
    assert blocks[0].shape[0] == 5
    q_scale = llama4_q_scale(model.config, P, N)
    L = w.shape.layers
    logits0, _ = check_step(w, model, eng, blocks[0], caches[0], q_scale, (0, L - 1))
    check_properties(w, eng, blocks[0], caches[0], q_scale, logits0)
    single, counts = [], []
    for b, c in zip(blocks, caches):
        st = StepStats()
        single.append(eng.forward(b.cuda(), c, w.delta, stats=st))
        counts.append(st.counts)
    for pad in (None, 5):
        stb = StepStats()
        got = eng.forward_batched([b.cuda() for b in blocks], caches, w.delta, stats=stb,
                                  pad_to=pad)
        torch.cuda.synchronize()
        assert stb.counts == [sum(c) for c in zip(*counts)]
        for s, (a, b) in enumerate(zip(got, single)):
            st = err_stats(a.float(), b.float())
            print(f"[cfg4 batched pad={pad}] seq {s}: {st}", flush=True)
            assert st["max_abs"] <= NS_MAX_ABS * max(1.0, st["ref_absmax"]) and \
                st["mean_rel"] <= NS_MEAN_REL, st
    del eng, model, caches, got, single, logits0
    _gc()
