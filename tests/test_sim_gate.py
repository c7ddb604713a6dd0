"""The integer core of the folded verify step and the attention of folded rows,
on the CPU: the kernels' own sources for the delta gate and fold compaction
(sf_fold_gate, with the previous layer's residual fused in:
sf_fold_gate_residual), the branch parent map (sf_parent_map) and the chain
correction (sf_chain_correct, after sf_attn_prefix_block), built for the SIMT
simulator of tests/sim and driven through the library's own Python wrappers
(tests/simlib.py).  Against the same CPU restatements of the reference the GPU
tests use (recompute mask, compacted rows, src, one-hop parents, segments:
bit-exact; rstd and normalized rows: rounding) and, for attention, float64
attention of every row of the folded step."""

import pytest
import torch

from oracle.folded_reference import parent_map
from specfold_amd import _lib
from specfold_amd.engine import build_parent_map
from specfold_amd.synthetic import TREE_PARENTS, draft_tree_block, perturbed_hidden
from tests.simlib import build_sim_library, compiler, use_sim_library
from tests.test_gpu_gate import check_outputs, ref_mask


@pytest.fixture(scope="module")
def sim(tmp_path_factory):
    if compiler() is None:
        pytest.skip("no clang++ (the simulator needs clang's vector extensions)")
    path = build_sim_library(tmp_path_factory.mktemp("simlib"))
    with use_sim_library(path) as lib:
        yield lib


def gate_outputs(B1, N, D, bucket):
    BN = B1 * N
    i32 = dict(dtype=torch.int32)
    return dict(rec=torch.zeros(BN, dtype=torch.int8), f=torch.zeros(BN, **i32),
                src=torch.zeros(BN, **i32), rows=torch.full((bucket,), -7, **i32),
                count=torch.zeros(1, **i32), seg=torch.full((BN,), -1, **i32),
                segcnt=torch.zeros(B1, **i32), rstd=torch.zeros(BN, dtype=torch.float32),
                xn=torch.zeros(BN, D, dtype=torch.bfloat16))


def run_gate(lib, hidden, parent, ln_w, delta, mode, bucket=None, eps=1e-6):
    B1, N, D = hidden.shape
    bucket = B1 * N if bucket is None else bucket
    par = torch.tensor([0] + [int(p) for p in parent[1:]], dtype=torch.int32)
    out = gate_outputs(B1, N, D, bucket)
    lib.fold_gate(hidden.reshape(B1 * N, D).contiguous(), par, ln_w, B1, N, bucket, delta, eps,
                  mode, out["rec"], out["f"], out["src"], out["rows"], out["count"], out["seg"],
                  out["segcnt"], out["rstd"], out["xn"])
    return out


@pytest.mark.parametrize("mode", [_lib.SF_GATE_MODEL_DTYPE, _lib.SF_GATE_FP32_SQUARED])
def test_gate_tree(sim, mode):
    gen = torch.Generator().manual_seed(11 + mode)
    parents = list(TREE_PARENTS)
    hidden = perturbed_hidden(parents, 32, 1536, gen)
    ln_w = (1 + 0.1 * torch.randn(1536, generator=gen)).to(torch.bfloat16)
    rec = ref_mask(hidden, parents, 0.1, mode)
    out = run_gate(sim, hidden, parents, ln_w, 0.1, mode)
    check_outputs(out, hidden, parents, rec, ln_w)
    assert 0.3 < 1 - rec[1:].float().mean() < 0.9   # both outcomes occur


@pytest.mark.parametrize("seed", range(3))
def test_gate_random_forests_and_bucket(sim, seed):
    gen = torch.Generator().manual_seed(200 + seed)
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
    bucket = max(1, int(rec.sum()) - 3) if seed == 2 else None   # last: an overflowing bucket
    out = run_gate(sim, hidden, parents, ln_w, delta, _lib.SF_GATE_MODEL_DTYPE, bucket=bucket)
    check_outputs(out, hidden, parents, rec, ln_w, bucket=bucket)


def test_gate_residual_fused(sim):
    """Layer > 0: the input x = bf16(hp + ffn[src_prev*N + n]) is formed inside the
    gate (written to hidden_out) and then gated exactly like sf_fold_gate's input."""
    gen = torch.Generator().manual_seed(5)
    parents = list(TREE_PARENTS)
    B1, N, D = len(parents), 32, 512
    x = perturbed_hidden(parents, N, D, gen)
    hp = (x.float() * 0.5).to(torch.bfloat16)
    src_prev = torch.randint(0, B1, (B1 * N,), generator=gen, dtype=torch.int32)
    src_prev[:N] = 0
    ffn = torch.randn(B1 * N, D, generator=gen).to(torch.bfloat16) * 0.01
    # the residual rows the kernel forms, and the gate they must then produce
    r = torch.arange(B1 * N)
    xin = (hp.reshape(B1 * N, D).float() + ffn[(src_prev.long() * N + r % N)].float())
    xin = xin.to(torch.bfloat16).view(B1, N, D)
    ln_w = torch.ones(D, dtype=torch.bfloat16)
    rec = ref_mask(xin, parents, 0.1, _lib.SF_GATE_MODEL_DTYPE)
    out = gate_outputs(B1, N, D, B1 * N)
    par = torch.tensor([0] + [int(p) for p in parents[1:]], dtype=torch.int32)
    hidden_out = torch.zeros(B1 * N, D, dtype=torch.bfloat16)
    sim.fold_gate_residual(hp.reshape(B1 * N, D), ffn, src_prev, par, ln_w, B1, N, D, B1 * N, 0.1,
                           1e-6, _lib.SF_GATE_MODEL_DTYPE, hidden_out, out["rec"], out["f"],
                           out["src"], out["rows"], out["count"], out["seg"], out["segcnt"],
                           None, out["rstd"], out["xn"])
    assert torch.equal(hidden_out.view(B1, N, D), xin)
    check_outputs(out, xin, parents, rec, ln_w)


def device_map(lib, tokens):
    B1 = tokens.shape[0]
    par = torch.full((B1,), -1, dtype=torch.int32)
    cnt = torch.full((B1,), -1, dtype=torch.int32)
    lib.parent_map(tokens.contiguous(), par, cnt)
    return par.tolist(), cnt.tolist()


def oracle_map(tokens):
    parent, counts = parent_map(tokens)
    return [0] + [int(p) for p in parent[1:]], [int(c) for c in counts]


def test_parent_map(sim):
    g = torch.Generator().manual_seed(9)
    for _ in range(3):
        tokens = draft_tree_block(32, 151936, g)
        assert device_map(sim, tokens) == oracle_map(tokens)
    for B1, N, vocab in [(8, 32, 3), (64, 64, 2), (17, 7, 3), (1, 32, 10)]:
        for _ in range(4):
            main = torch.randint(0, vocab, (1, N), generator=g)
            flips = torch.rand(B1, N, generator=g) < 0.15
            tokens = torch.where(flips, torch.randint(0, vocab, (B1, N), generator=g), main)
            tokens[0] = main[0]
            assert device_map(sim, tokens) == oracle_map(tokens)


@pytest.mark.parametrize("P,seed", [(0, 1), (70, 2), (300, 3)])
def test_gate_attention_chain(sim, P, seed):
    """Gate -> attention of the recomputed rows -> chain correction of the folded
    rows, every row then checked against float64 attention of the folded step:
    row (b, n) attends with the query of its source row src[b*N+n]*N + n over the
    prefix and the block keys src[b*N+j]*N + j (the nearest recomputing ancestor's
    K/V at every block position).  A folded row may keep an upper bound of its
    row maximum (the ancestor's, when a changed key held it), so (m, Z) is checked
    through the log-sum-exp m + log Z."""
    gen = torch.Generator().manual_seed(seed)
    parents = list(TREE_PARENTS)
    B1, N, D, H, Hkv, hd = len(parents), 16, 256, 4, 2, 128
    BN = B1 * N
    hidden = perturbed_hidden(parents, N, D, gen)
    ln_w = torch.ones(D, dtype=torch.bfloat16)
    g = run_gate(sim, hidden, parents, ln_w, 0.1, _lib.SF_GATE_MODEL_DTYPE)
    rec = g["rec"].view(B1, N).bool()
    assert 0 < int((~rec).sum()) and int(rec[1:].sum()) > 0
    q = torch.randn((BN + 1) * H * hd, generator=gen).to(torch.bfloat16)
    kv = torch.randn((BN + 1) * 2 * Hkv * hd, generator=gen).to(torch.bfloat16)
    ps = 16
    npages = max(1, (P + ps - 1) // ps)
    pk = torch.randn(npages * Hkv * ps * hd, generator=gen).to(torch.bfloat16)
    pv = torch.randn(npages * Hkv * ps * hd, generator=gen).to(torch.bfloat16)
    table = torch.randperm(npages, generator=gen).to(torch.int32)
    o32 = torch.full((BN * H * hd,), float("nan"))
    obf = torch.zeros(BN * H * hd, dtype=torch.bfloat16)
    mt = torch.full((BN * H,), float("nan"))
    zt = torch.full((BN * H,), float("nan"))
    nws = max(sim.attn_workspace_bytes(BN, H, P), 256)
    raw = torch.zeros(nws + 256, dtype=torch.uint8)          # a 256-byte aligned view
    off = (-raw.data_ptr()) % 256
    ws = raw[off:off + nws]
    scaling = hd ** -0.5
    par = torch.tensor([0] + [int(p) for p in parents[1:]], dtype=torch.int32)
    sim.attn_prefix_block(q, kv, pk, pv, table, P, ps, Hkv * ps * hd, ps * hd, g["src"], g["rows"],
                          g["count"], BN, B1, N, H, Hkv, hd, scaling, o32, obf, mt, zt, ws)
    sim.chain_correct(q, kv, g["src"], par, g["rec"], g["seg"], g["segcnt"], B1, N, H, Hkv, hd,
                      scaling, o32, obf, mt, zt)
    G = H // Hkv
    qv = q.double().view(BN + 1, H, hd)
    kvv = kv.double().view(BN + 1, 2, Hkv, hd)
    src = g["src"].long()

    def prefix(t, h):
        rows = [t.view(npages, Hkv, ps, hd)[int(table[p // ps]), h, p % ps] for p in range(P)]
        return torch.stack(rows).double() if rows else torch.zeros(0, hd, dtype=torch.float64)
    pref = [(prefix(pk, h), prefix(pv, h)) for h in range(Hkv)]
    worst_o = worst_lse = 0.0
    for b in range(B1):
        blk = src[b * N:(b + 1) * N] * N + torch.arange(N)
        for n in range(N):
            r = b * N + n
            qrow = int(src[r]) * N + n
            for hq in range(H):
                h = hq // G
                keys = torch.cat([pref[h][0], kvv[blk, 0, h]])
                vals = torch.cat([pref[h][1], kvv[blk, 1, h]])
                s = keys @ qv[qrow, hq] * scaling
                m = float(s.max())
                p = torch.exp(s - m)
                z = float(p.sum())
                o = (p @ vals) / z
                got_o = o32.view(BN, H, hd)[r, hq].double()
                worst_o = max(worst_o, float((got_o - o).abs().max()) / max(1.0, float(o.abs().max())))
                lse_got = float(mt.view(BN, H)[r, hq]) + float(torch.log(zt.view(BN, H)[r, hq].double()))
                worst_lse = max(worst_lse, abs(lse_got - (m + float(torch.log(torch.tensor(z, dtype=torch.float64))))))
                assert float(mt.view(BN, H)[r, hq]) >= m - 1e-4
    print(f"P={P}: O max err {worst_o:.3g}, lse max err {worst_lse:.3g}, "
          f"folded rows {int((~rec).sum())}")
    assert worst_o <= 2e-5 and worst_lse <= 2e-5


# -- greedy decode statistics (sf_logit_stats) and the paged KV append ------------------

def sim_logit_stats(lib, logits, top_p, ws=None):
    """sf_logit_stats on CPU rows, with the wrapper's argument layout (the wrapper
    itself accepts GPU tensors only)."""
    M, V = logits.shape
    x = logits.contiguous()
    need = int(lib._LIB.sf_logit_stats_workspace_bytes(M))
    ws = torch.zeros(need, dtype=torch.uint8) if ws is None else ws
    out = lib.LogitStats(M, "cpu")
    st = lib._LIB.sf_logit_stats(lib._ptr(x), M, V, V, float(top_p), lib._ptr(out.top_idx),
                                 lib._ptr(out.top_val), lib._ptr(out.zfull), lib._ptr(out.znuc),
                                 lib._ptr(out.greedy_tok), lib._ptr(out.conf),
                                 lib._ptr(out.conf_full), lib._ptr(ws), ws.numel(), None)
    assert st == 0
    return out, ws


@pytest.mark.parametrize("M,V,scale,top_p", [(4, 152064, 1.0, 0.95), (3, 20000, 3.0, 0.5),
                                             (2, 131072, 0.3, 1.0)])
def test_logit_stats(sim, M, V, scale, top_p):
    """Against the reference sampler's torch sequence on the CPU and the softmax /
    topk statistics (the checks of the GPU test, tests/test_gpu_logit_stats.py)."""
    from tests.test_gpu_logit_stats import nucleus_mass64, reference_greedy, ulp_bf16
    g = torch.Generator().manual_seed(M * 31 + V)
    logits = (torch.randn(M, V, generator=g) * scale).to(torch.bfloat16)
    logits[0, 17] = logits[0].max() + 2.0           # a clear winner in one row
    st, ws = sim_logit_stats(sim, logits, top_p)
    assert torch.equal(st.top_idx[:, 0].long(), torch.argmax(logits, dim=-1))
    assert torch.equal(st.top_val, torch.topk(logits.float(), 8, dim=-1).values)
    zn64, z64 = nucleus_mass64(logits, top_p)
    assert torch.allclose(st.zfull.double(), z64, rtol=1e-5)
    assert bool(((st.znuc.double() - zn64).abs() <= 1e-5 * z64 + 2.0).all())
    tok, conf = reference_greedy(logits, top_p)
    same = st.conf == conf.float()
    assert bool(((st.conf - conf.float()).abs() <= ulp_bf16(conf)).all())
    assert torch.equal(st.greedy_tok[same].long(), tok[same])
    cfull = torch.softmax(logits, dim=-1).max(dim=-1).values
    assert bool(((st.conf_full - cfull.float()).abs() <= ulp_bf16(cfull)).all())
    # the histograms (the workspace's first M x 65536 counters) are left zero; the
    # per-slice candidates after them are overwritten by every call; a second call
    # on the same workspace gives the same statistics
    assert int(ws[:M * 65536 * 4].count_nonzero()) == 0
    st2, _ = sim_logit_stats(sim, logits, top_p, ws)
    for f in ("top_idx", "top_val", "zfull", "znuc", "greedy_tok", "conf", "conf_full"):
        assert torch.equal(getattr(st, f), getattr(st2, f)), f


def test_logit_stats_top8_ties(sim):
    """The packed order keys of the top-8: +0 and -0 tie (lower index first), -inf
    entries follow the finite values in index order, ties across slices go to the
    lower index (tests/test_gpu_logit_stats.py has the same rows at V = 152064)."""
    from tests.test_gpu_logit_stats import top8_order
    V = 24576
    a = torch.full((V,), -30.0)
    a[[500, 9000, 300, 20000]] = torch.tensor([3.0, 2.0, 2.0, 1.0])
    a[[77, 12, 16000, 5]] = torch.tensor([0.0, -0.0, 0.0, -0.0])
    b = torch.full((V,), float("-inf"))
    b[[1000, 20, 17000]] = torch.tensor([1.0, 0.5, 0.5])
    c = torch.full((V,), 2.0)   # every token tied: the first 8 indices
    logits = torch.stack([a, b, c]).to(torch.bfloat16)
    st, _ = sim_logit_stats(sim, logits, 0.95)
    for r in range(3):
        idx, val = top8_order(logits[r])
        assert st.top_idx[r].tolist() == idx, r
        assert st.top_val[r].tolist() == val, r
    assert st.top_idx[0].tolist() == [500, 300, 9000, 20000, 5, 12, 77, 16000]
    assert st.top_idx[1].tolist() == [1000, 20, 17000, 0, 1, 2, 3, 4]
    assert st.top_idx[2].tolist() == list(range(8))


def test_logit_stats_noalloc_sequence(sim):
    """sf_logit_stats_noalloc over calls of changing row count (more, fewer, more
    again) gives exactly the workspace entry point's statistics every time: its
    fixed scratch keeps the histograms at the same place whatever M is, and a call
    with fewer rows writes nothing where a later, larger call counts."""
    g = torch.Generator().manual_seed(12)
    for i, M in enumerate([9, 2, 9, 1]):
        logits = (torch.randn(M, 4096, generator=g) * 2.0).to(torch.bfloat16)
        ref, _ = sim_logit_stats(sim, logits, 0.9)
        out = sim.LogitStats(M, "cpu")
        st = sim._LIB.sf_logit_stats_noalloc(
            sim._ptr(logits), M, 4096, 4096, 0.9, sim._ptr(out.top_idx), sim._ptr(out.top_val),
            sim._ptr(out.zfull), sim._ptr(out.znuc), sim._ptr(out.greedy_tok), sim._ptr(out.conf),
            sim._ptr(out.conf_full), None)
        assert st == 0
        for f in sim.LogitStats.__slots__:
            assert torch.equal(getattr(out, f), getattr(ref, f)), (i, M, f)
    big = sim._LIB.sf_logit_stats_noalloc_max_rows() + 1
    x = torch.zeros(big, 64, dtype=torch.bfloat16)
    out = sim.LogitStats(big, "cpu")
    p = [sim._ptr(getattr(out, f)) for f in sim.LogitStats.__slots__]
    assert sim._LIB.sf_logit_stats_noalloc(sim._ptr(x), big, 64, 64, 0.9, *p, None) == 5


def test_kv_append_paged(sim):
    """The block's K/V rows land at positions start .. start+n_tok of a paged cache
    (shuffled pages), every other cache element untouched."""
    g = torch.Generator().manual_seed(4)
    Hkv, hd, ps, npages, n_tok, start, row0 = 2, 128, 16, 9, 32, 37, 5
    kv = torch.randn((row0 + n_tok + 2) * 2 * Hkv * hd, generator=g).to(torch.bfloat16)
    kc = torch.full((npages * Hkv * ps * hd,), 7.0).to(torch.bfloat16)
    vc = kc.clone()
    table = torch.randperm(npages, generator=g).to(torch.int32)
    sim.kv_append(kv, row0, n_tok, Hkv, hd, kc, vc, table, ps, Hkv * ps * hd, ps * hd, start)
    kvv = kv.view(-1, 2, Hkv, hd)
    expect_k, expect_v = torch.full_like(kc, 7.0).view(npages, Hkv, ps, hd), \
        torch.full_like(vc, 7.0).view(npages, Hkv, ps, hd)
    for t in range(n_tok):
        p = start + t
        expect_k[int(table[p // ps]), :, p % ps] = kvv[row0 + t, 0]
        expect_v[int(table[p // ps]), :, p % ps] = kvv[row0 + t, 1]
    assert torch.equal(kc.view_as(expect_k), expect_k)
    assert torch.equal(vc.view_as(expect_v), expect_v)


@pytest.mark.parametrize("mode", [_lib.SF_GATE_MODEL_DTYPE, _lib.SF_GATE_FP32_SQUARED])
def test_gate_stacked_sequences(sim, mode):
    """SF_GATE_ROOTS_BY_PARENT: three sequences' branch trees stacked in one call
    (each root its own parent) give each tree's gate and compaction alone, indices
    shifted by the tree's offset: recompute mask, count, compacted rows, src and
    per-branch segment counts exactly, the normalized rows bit for bit."""
    gen = torch.Generator().manual_seed(40 + mode)
    N, D = 32, 512
    ln_w = (1 + 0.1 * torch.randn(D, generator=gen)).to(torch.bfloat16)
    trees = [list(TREE_PARENTS), [None], list(TREE_PARENTS[:5])]
    hid = [perturbed_hidden(p, N, D, gen) for p in trees]
    alone = [run_gate(sim, h, p, ln_w, 0.1, mode) for h, p in zip(hid, trees)]
    sizes = [len(p) for p in trees]
    offs = [sum(sizes[:i]) for i in range(len(sizes))]
    B1 = sum(sizes)
    par = torch.tensor([o + (0 if q is None else int(q)) for p, o in zip(trees, offs) for q in p],
                       dtype=torch.int32)
    out = gate_outputs(B1, N, D, B1 * N)
    sim.fold_gate(torch.cat(hid).reshape(B1 * N, D).contiguous(), par, ln_w, B1, N, B1 * N, 0.1,
                  1e-6, mode | _lib.SF_GATE_ROOTS_BY_PARENT, out["rec"], out["f"], out["src"],
                  out["rows"], out["count"], out["seg"], out["segcnt"], out["rstd"], out["xn"])
    assert torch.equal(out["rec"], torch.cat([a["rec"] for a in alone]))
    counts = [int(a["count"]) for a in alone]
    assert int(out["count"]) == sum(counts)
    assert torch.equal(out["rows"][:sum(counts)],
                       torch.cat([a["rows"][:c] + o * N for a, c, o in zip(alone, counts, offs)]))
    assert torch.equal(out["src"], torch.cat([a["src"] + o for a, o in zip(alone, offs)]))
    assert torch.equal(out["segcnt"], torch.cat([a["segcnt"] for a in alone]))
    rows = out["rows"][:sum(counts)].long()
    xn_alone = torch.cat([a["xn"] for a in alone])
    rstd_alone = torch.cat([a["rstd"] for a in alone])
    assert torch.equal(out["xn"][rows], xn_alone[rows])
    assert torch.equal(out["rstd"][rows], rstd_alone[rows])
    assert 0 < sum(counts) < B1 * N
