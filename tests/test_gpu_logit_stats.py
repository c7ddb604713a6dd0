"""sf_logit_stats against the reference's own torch ops on the same logits.

The reference's greedy top-p sampler (fastdllm_model_executor.py:129-155 at
temperature 0) and softmax/topk draft statistics run here as the literal torch
sequences; the sampler on the CPU, because torch's GPU scan kernel rounds every
partial sum of the bf16 cumsum to bf16 (so on a GPU the sum of a flat
distribution stalls below top_p and nothing is cut), while its CPU kernel
accumulates in fp32, which is the rule the statistics implement.  Integer outputs (argmax token, top-8 order) must match exactly.  The
bf16 probabilities are bf16(1/Z) for an fp32 sum Z whose summation order differs
from torch's, and the nucleus cut may differ by one token where torch's bf16
cumulative sum rounds across top_p, so: within one bf16 ulp everywhere, exact on
at least 99% of rows, and the greedy token exact wherever the probability is.
"""

import pytest
import torch

from specfold_amd import _lib

pytestmark = pytest.mark.gpu


def reference_greedy(logits, top_p):
    """fastdllm_model_executor.py:129-155, temperature 0."""
    sorted_logits, sorted_indices = torch.sort(logits, descending=True, dim=-1)
    cumulative_probs = torch.cumsum(torch.softmax(sorted_logits, dim=-1), dim=-1)
    remove = cumulative_probs > top_p
    remove[..., 1:] = remove[..., :-1].clone()
    remove[..., 0] = False
    to_remove = remove.scatter(-1, sorted_indices, remove)
    probs = torch.softmax(logits.masked_fill(to_remove, float("-inf")), dim=-1)
    tok = torch.argmax(probs, dim=-1)
    return tok, torch.gather(probs, -1, tok.unsqueeze(-1)).squeeze(-1)


def nucleus_mass64(logits, top_p):
    """Kept softmax mass, float64 restatement of the reference rule: with the bf16
    probabilities in descending order, keep tokens up to and including the first
    whose cumulative probability, rounded to bf16, exceeds top_p."""
    l = logits.double()
    e = torch.exp(l - l.max(dim=-1, keepdim=True).values)
    z = e.sum(-1, keepdim=True)
    se = torch.sort(e, descending=True, dim=-1).values
    p = (se / z).to(torch.bfloat16).double()
    crossed = torch.cumsum(p, -1).to(torch.bfloat16).double() > top_p
    k = torch.where(crossed.any(-1), crossed.double().argmax(-1), torch.full_like(
        crossed[..., 0], e.shape[-1] - 1, dtype=torch.long))
    return torch.gather(torch.cumsum(se, -1), -1, k.unsqueeze(-1)).squeeze(-1), z.squeeze(-1)


def ulp_bf16(x):
    return torch.abs(x.float()) * 2.0 ** -7


def check(logits, top_p, min_exact=0.99):
    st = _lib.logit_stats(logits, top_p=top_p)
    torch.cuda.synchronize()
    M = logits.shape[0]
    # argmax and top-8 (values exact; indices where the value is unique)
    assert torch.equal(st.top_idx[:, 0].long(), torch.argmax(logits, dim=-1))
    tv = torch.topk(logits.float(), 8, dim=-1).values
    assert torch.equal(st.top_val, tv)
    # normalisers
    zn64, z64 = nucleus_mass64(logits, top_p)
    assert torch.allclose(st.zfull.double(), z64, rtol=1e-5)
    # within two tokens' mass (each e <= 1) of the float64 restatement
    assert bool(((st.znuc.double() - zn64).abs() <= 1e-5 * z64 + 2.0).all())
    # the reference's greedy token and probability (its sampler run on the CPU,
    # where torch accumulates the bf16 cumulative sum in fp32)
    tok, conf = reference_greedy(logits.cpu(), top_p)
    tok, conf = tok.cuda(), conf.cuda()
    same = st.conf == conf.float()
    assert bool(((st.conf - conf.float()).abs() <= ulp_bf16(conf)).all())
    assert float(same.float().mean()) >= min_exact, float(same.float().mean())
    assert torch.equal(st.greedy_tok[same].long(), tok[same])
    # the draft confidence: max of the bf16 softmax
    cfull = torch.softmax(logits, dim=-1).max(dim=-1).values
    assert bool(((st.conf_full - cfull.float()).abs() <= ulp_bf16(cfull)).all())
    assert float((st.conf_full == cfull.float()).float().mean()) >= min_exact
    return st


# A near-uniform row (scale 0.3) puts ~1e5 probabilities of ~1e-5 under the cut:
# the reference's own fp32 running sum over them drifts by up to ~1e-3 relative,
# which moves its cut by many tokens, so only the one-ulp bound is tight there.
@pytest.mark.parametrize("M,V,scale,min_exact", [(8, 152064, 1.0, 0.99),
                                                 (32, 131072, 0.3, 0.9),
                                                 (1, 151936, 3.0, 0.99)])
@pytest.mark.parametrize("top_p", [0.95, 0.5, 1.0])
def test_random_rows(M, V, scale, min_exact, top_p):
    g = torch.Generator(device="cuda").manual_seed(M * 7 + int(top_p * 100))
    logits = (torch.randn(M, V, device="cuda", generator=g) * scale).to(torch.bfloat16)
    check(logits, top_p, min_exact=min_exact)


def test_peaked_rows():
    """A trained-model-like row: a few dominant tokens, the cut inside the top-8."""
    g = torch.Generator(device="cuda").manual_seed(3)
    logits = torch.randn(16, 152064, device="cuda", generator=g)
    logits[:, 5] += 14.0
    logits[:, 77] += 12.5
    logits[8:, 1234] += 14.0
    check(logits.to(torch.bfloat16), 0.95)


def test_ties_lowest_index():
    """Equal maxima, more than 8 of them (the row scan), and two near-equal logits
    whose bf16 probabilities tie (the lower index wins although its logit is
    smaller, as in the reference's argmax over bf16 probabilities)."""
    V = 152064
    logits = torch.full((3, V), -20.0, device="cuda")
    logits[0, [900, 40, 7000]] = 5.0                          # 3 exact ties
    logits[1, torch.arange(100, 2100, 100)] = 6.0             # 20 exact ties
    logits[2, 50] = 0.25
    logits[2, 20] = 0.248046875                               # bf16 neighbour of 0.25
    logits = logits.to(torch.bfloat16)
    st = check(logits, 0.95, min_exact=1.0)
    assert st.top_idx[0, 0] == 40 and st.top_idx[1, 0] == 100 and st.top_idx[2, 0] == 50
    assert st.greedy_tok.tolist() == [40, 100, 20]


def top8_order(row):
    """The 8 (index, value) pairs of a row by value descending, then index ascending
    (both zeros equal, as in a float comparison)."""
    v = row.float().tolist()
    idx = sorted(range(len(v)), key=lambda i: (-v[i], i))[:8]
    return idx, [v[i] for i in idx]


def test_top8_signed_zeros_and_infinities():
    """Top-8 order on ties the packed order keys must get right: +0 and -0 tie (lower
    index first), and -inf entries fill the list behind the finite values in index
    order."""
    V = 152064
    a = torch.full((V,), -30.0)
    a[[500, 9000, 300, 150000]] = torch.tensor([3.0, 2.0, 2.0, 1.0])
    a[[77, 12, 40000, 5]] = torch.tensor([0.0, -0.0, 0.0, -0.0])
    b = torch.full((V,), float("-inf"))
    b[[1000, 20, 70000]] = torch.tensor([1.0, 0.5, 0.5])
    logits = torch.stack([a, b]).to(torch.bfloat16)
    st = _lib.logit_stats(logits.cuda(), top_p=0.95)
    torch.cuda.synchronize()
    for r in range(2):
        idx, val = top8_order(logits[r])
        assert st.top_idx[r].tolist() == idx, r
        assert st.top_val[r].tolist() == val, r
    assert st.top_idx[0].tolist() == [500, 300, 9000, 150000, 5, 12, 77, 40000]
    assert st.top_idx[1].tolist() == [1000, 20, 70000, 0, 1, 2, 3, 4]
    assert st.greedy_tok.tolist() == [500, 1000]


def test_flat_row():
    """Every logit equal: the greedy token is index 0 (the nucleus size of such a
    row depends on how the running sum of equal probabilities rounds, so only the
    tokens are compared)."""
    logits = torch.full((2, 131072), -1.0, device="cuda").to(torch.bfloat16)
    st = _lib.logit_stats(logits, top_p=0.95)
    torch.cuda.synchronize()
    assert st.top_idx[:, 0].tolist() == [0, 0] and st.greedy_tok.tolist() == [0, 0]
    assert st.top_idx[0].tolist() == list(range(8))


def test_strided_rows_and_repeat_calls():
    """Rows that are a strided slice of a bigger tensor (the decode loop passes
    logits[0, s0:s1]); a second call on the reused workspace is bit-identical."""
    g = torch.Generator(device="cuda").manual_seed(11)
    full = torch.randn(3, 32, 152064, device="cuda", generator=g).to(torch.bfloat16)
    rows = full[0, 8:16]
    a = _lib.logit_stats(rows, top_p=0.95)
    b = _lib.logit_stats(rows.contiguous(), top_p=0.95)
    torch.cuda.synchronize()
    for f in ("top_idx", "top_val", "zfull", "znuc", "greedy_tok", "conf", "conf_full"):
        assert torch.equal(getattr(a, f), getattr(b, f)), f
    check(rows.contiguous(), 0.95)


# -- the decode-loop decisions built on the statistics ----------------------------------

def test_greedy_sampler_matches_cpu_reference():
    """The reference sampler run on the CPU (fp32-accumulated bf16 cumsum) and the
    statistics path on the GPU pick the same tokens with the same probabilities."""
    from specfold_amd.generate import greedy
    g = torch.Generator(device="cuda").manual_seed(21)
    logits = (torch.randn(64, 152064, device="cuda", generator=g) * 0.7).to(torch.bfloat16)
    x_1, conf = greedy.top_p_greedy(greedy.stats(logits, 0.95))
    tok, ref = reference_greedy(logits.cpu(), 0.95)
    same = conf[0].cpu() == ref
    assert float(same.float().mean()) >= 0.98
    assert torch.equal(x_1[0].cpu()[same], tok[same])
    assert bool(((conf[0].cpu().float() - ref.float()).abs() <= ulp_bf16(ref)).all())


def test_draft_states_match_reference_ops():
    """Draft construction from the statistics equals the softmax/topk sequence."""
    from specfold_amd.configs import SYNTHETIC_DRAFT_GRAPH
    from specfold_amd.generate import greedy
    from specfold_amd.generate.fastdllm_v2_generation import FastDLLMV2SpeculativeGeneration
    g = torch.Generator(device="cuda").manual_seed(5)
    logits = (torch.randn(8, 152064, device="cuda", generator=g) * 2.0).to(torch.bfloat16)
    x = torch.randint(0, 1000, (32,), device="cuda")
    mask = torch.ones(8, dtype=torch.bool, device="cuda")
    mask[3] = False
    active = [(n, tuple(n["ij_set"]), max(p for p, _ in n["ij_set"]))
              for n in SYNTHETIC_DRAFT_GRAPH["selected_nodes"]]
    st = greedy.stats(logits)
    a = FastDLLMV2SpeculativeGeneration._draft_states(x, logits, mask, 8, active, st)
    b = FastDLLMV2SpeculativeGeneration._draft_states(x, logits, mask, 8, active)
    assert torch.equal(a, b)


def test_nld_transfer_matches_reference_ops():
    from specfold_amd.generate import greedy
    from specfold_amd.generate.nld_generation import get_transfer_index, greedy_transfer_index
    g = torch.Generator(device="cuda").manual_seed(9)
    for scale in (0.5, 4.0):
        logits = (torch.randn(1, 32, 131072, device="cuda", generator=g) * scale).to(
            torch.bfloat16)
        mask = torch.rand(1, 32, device="cuda", generator=g) < 0.7
        x = torch.randint(0, 1000, (1, 32), device="cuda")
        ntt = torch.tensor([3], device="cuda")
        for thr in (None, 0.9, 1e-6):
            a = greedy_transfer_index(greedy.stats(logits[0]), mask, x, ntt, threshold=thr)
            b = get_transfer_index(logits, 0.0, mask, x, ntt, threshold=thr)
            assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1]), (scale, thr)
