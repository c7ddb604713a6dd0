"""HIP verify step on the NLD (Nemotron-Labs-Diffusion) layout vs the oracle.

The NLD step differs from the Fast-dLLM v2 one in the model tree (``encoder``,
``diffusion_head``), no QKV bias, RMSNorm eps 1e-5, YaRN RoPE, the llama-4 q
scale after RoPE and unshifted logits; block commits run causally within the
block.  The models here take a small original context (``omax``) so the q scale
is active at the test's prefix lengths.  Tolerances are the ones of
test_gpu_engine_parity.py: integer outputs bit-exact, bf16 quantities within
~2 bf16 ulps, logits within max abs 2e-2*max(1, |ref|) and the mean relative
spread of the oracle itself on GPU vs CPU (x2, floor 1e-3).
"""

import pytest
import torch

from oracle.folded_reference import dense_verify_step, llama4_q_scale
from specfold_amd.generate.nld_folded import SpecFoldHIPNLDGeneration
from specfold_amd.generate.nld_generation import NLDDiffusionGeneration
from specfold_amd.generate.nld_model_executor import NLDModelExecutor
from tests.helpers import SHAPE_N4, SHAPE_N8, err_stats, make_nld_case, to_gpu_model
from tests.parity import bf16_close
from tests.test_gpu_engine_parity import check_end_to_end, check_layers, run_pair

pytestmark = pytest.mark.gpu

CASES = [
    ("n4_p100", SHAPE_N4, 1, 100, 0.1, 64),
    ("n8_p300", SHAPE_N8, 2, 300, 0.05, 128),
    ("n8_p0", SHAPE_N8, 3, 0, 0.1, 16),
]


def _q_scale(case, P, N):
    return llama4_q_scale(case.model_cpu.config, P, N)


@pytest.mark.parametrize("name,shape,seed,P,delta,omax", CASES)
def test_nld_layers_teacher_forced(name, shape, seed, P, delta, omax):
    case = make_nld_case(shape, seed, P=P, delta=delta, omax=omax)
    qs = _q_scale(case, P, case.tokens.shape[1])
    assert (qs is not None) == (P + case.tokens.shape[1] > omax)
    tr, _, trace, _, eng = run_pair(case, q_scale=qs)
    check_layers(case, shape, tr, trace, eng, q_scale=qs)


@pytest.mark.parametrize("name,shape,seed,P,delta,omax", CASES[:2])
def test_nld_end_to_end_logits(name, shape, seed, P, delta, omax):
    case = make_nld_case(shape, seed, P=P, delta=delta, omax=omax)
    check_end_to_end(name, case, q_scale=_q_scale(case, P, case.tokens.shape[1]))


def _executor(case, **kw):
    model = to_gpu_model(case.model_cpu)
    for k in ("encoder", "diffusion_head", "mask_token_id"):
        assert hasattr(model, k)
    return NLDModelExecutor(model, device="cuda", page_order="shuffled", page_seed=3, **kw)


@pytest.mark.parametrize("P,L", [(70, 32), (0, 40)])
def test_nld_causal_commit(P, L):
    """The AR block commit (nld_generation.py:186-194, 298-310): logits of every
    position and the K/V appended to the paged cache equal one causal dense
    forward over the whole input, whether it spans one block or two."""
    case = make_nld_case(SHAPE_N4, 7, P=P, omax=16)
    ex = _executor(case, block_length=32, max_length=512)
    cache = ex.new_cache(512)
    if case.kv is not None:
        cache.load_dense(case.kv)
    g = torch.Generator().manual_seed(L)
    tokens = torch.randint(0, SHAPE_N4.vocab - 1, (1, L), generator=g)
    ex.set_diffusion_lm(False)
    out = ex.forward(tokens.cuda(), past_key_values=cache, use_cache=True, use_causal_mask=True)
    ex.set_diffusion_lm(True)
    torch.cuda.synchronize()
    assert cache.length == P + L
    ref, new_kv = dense_verify_step(case.model_cpu, tokens, case.kv, shift=False,
                                    return_new_kv=True, q_scale=_q_scale(case, P, L),
                                    causal=True)
    st = err_stats(out.logits.float().cpu(), ref.float())
    print(f"commit P={P} L={L}: {st}")
    assert st["max_abs"] <= 2e-2 * max(1.0, st["ref_absmax"])
    assert st["mean_rel"] <= 2e-2
    # layer 0's appended K/V sees teacher-identical inputs (the embeddings)
    k0, v0 = cache[0]
    for nm, a, b in (("k", k0[:, :, P:], new_kv[0][0]), ("v", v0[:, :, P:], new_kv[0][1])):
        nbad, s = bf16_close(a, b)
        print(f"layer 0 appended {nm}: {s}")
        assert nbad == 0
    if case.kv is not None:
        assert torch.equal(k0[:, :, :P].cpu(), case.kv[0][0])


def test_nld_bidirectional_forward_matches_dense():
    """The executor's diffusion forward (use_cache=False) is the dense block forward."""
    case = make_nld_case(SHAPE_N4, 8, P=90, omax=64)
    ex = _executor(case)
    cache = ex.new_cache(512)
    cache.load_dense(case.kv)
    tokens = case.tokens[:2]
    logits = ex.forward(tokens.cuda(), past_key_values=cache, use_cache=False).logits
    ref = dense_verify_step(case.model_cpu, tokens, case.kv, shift=False,
                            q_scale=_q_scale(case, 90, tokens.shape[1]))
    st = err_stats(logits.float().cpu(), ref.float())
    print(f"bidirectional: {st}")
    assert st["max_abs"] <= 2e-2 * max(1.0, st["ref_absmax"])
    assert cache.length == 90


def test_nld_generator_decode():
    """A short decode through the folded NLD generator: prefill, verify steps with
    draft branches, at least one block commit; the folded seam agrees with the
    dense seam at delta < 0 (every row recomputed)."""
    case = make_nld_case(SHAPE_N4, 9, P=0, omax=64)
    ex = _executor(case, block_length=32, max_length=256)
    graph = {"selected_nodes": [{"ij_set": [(0, 1)]}, {"ij_set": [(0, 0), (1, 1)]},
                                {"ij_set": [(2, 1)]}]}
    gen = SpecFoldHIPNLDGeneration(block_length=32, model_executor=ex, calibration_graph=graph,
                                   max_new_tokens=64, threshold=0.9, delta=0.1)
    prompt = torch.randint(0, SHAPE_N4.vocab - 1, (1, 20), generator=torch.Generator().manual_seed(4))
    kinds = []
    for ev in gen.decode_steps(prompt):
        kinds.append(ev["kind"])
        if gen._state["model_calls"] >= 40:
            break
    print("events", kinds[:12], "fold ratio", gen.fold_ratio)
    assert kinds[0] == "prefill" and "commit" in kinds and "verify" in kinds
    assert 0.0 <= gen.fold_ratio <= 1.0
    x = gen._state["x_accum"]
    assert int((x[0, 20:52] == ex.get_mask_id()).sum()) == 0     # the first block is complete

    cache = gen._state["cache"]
    P = cache.length
    blk = torch.stack([x[0, 20:52], x[0, 20:52].clone()])
    blk[1, 5:] = ex.get_mask_id()
    folded = SpecFoldHIPNLDGeneration(block_length=32, model_executor=ex, delta=-1.0)
    a = folded._batched_block_forward(blk, cache)
    b = NLDDiffusionGeneration._batched_block_forward(folded, blk, cache)
    torch.cuda.synchronize()
    assert cache.length == P
    st = err_stats(a.float().cpu(), b.float().cpu())
    print(f"folded(delta<0) vs dense seam: {st}")
    assert st["max_abs"] <= 2e-2 * max(1.0, st["ref_absmax"])
