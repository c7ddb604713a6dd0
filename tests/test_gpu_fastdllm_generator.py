"""The Fast-dLLM v2 generator on the GPU: its verify seam, fold accounting, a short
decode, and every decode decision against the reference's own torch sequence.

* ``SpecFoldHIPFastDLLMV2Generation._batched_block_forward`` (the drop-in for
  specfold/generate/fastdllm_v2_folded.py:226-370) over a paged prefix against
  the oracle's ``folded_verify_step(shift=True)``: shifted logits within the
  end-to-end bounds of tests/test_gpu_engine_parity.py, and the fold counters
  (draft positions and recomputed draft positions, summed over layers and
  steps; fastdllm_v2_folded.py:49-53, 142-143) equal to the oracle's
  ``FoldCounters`` exactly, over several steps.  (The golden fixtures' models
  have head_dim 16, which the kernels do not take; the oracle these tests use is
  the one the golden vectors pin.)
* ``generate_with_draft_speculation`` end to end (fastdllm_v2_generation.py:
  483-720): the result tuple, and two runs give the same tokens.
* Decisions: the decode loop takes its greedy tokens and confidences from
  sf_logit_stats.  At every verify / draft-hit step the same logits also go
  through the reference's sampler (fastdllm_model_executor.py:129-155, run on
  the CPU, where torch's bf16 cumsum accumulates in fp32 as the statistics do)
  and its unmask rule (fastdllm_v2_generation.py:666-676); the committed
  positions and tokens must be identical at every step.  The head is scaled so
  that confidences span the threshold (random weights alone give flat rows).
"""

import pytest
import torch

from oracle.folded_reference import FoldCounters, folded_verify_step
from specfold_amd.configs import draft_graph
from specfold_amd.generate import FastDLLMModelExecutor, SpecFoldHIPFastDLLMV2Generation
from specfold_amd.generate.synthetic_model import ModelShape, build_qwen2
from specfold_amd.synthetic import draft_tree_block, random_prefix_kv
from tests.helpers import err_stats, to_gpu_model
from tests.parity import NS_MAX_ABS
from tests.test_gpu_engine_parity import LOGITS_MEAN_REL_MAX

pytestmark = pytest.mark.gpu

SHAPE = ModelShape(hidden=512, heads=4, kv_heads=2, layers=2, intermediate=1024, vocab=4096)
MASK, STOP = SHAPE.vocab - 1, SHAPE.vocab - 2


def _generator(model, delta=0.1, threshold=0.9, max_new=96, **kw):
    ex = FastDLLMModelExecutor(model, device="cuda", block_length=32, max_length=1024,
                               page_order="shuffled", page_seed=4)
    return SpecFoldHIPFastDLLMV2Generation(
        block_length=32, model_executor=ex, calibration_graph=draft_graph(7), threshold=threshold,
        small_block_size=8, max_new_tokens=max_new, max_length=1024, mask_id=MASK,
        stop_token=STOP, delta=delta, **kw)


def test_batched_block_forward_and_fold_counters():
    model_cpu = build_qwen2(SHAPE, 21, device="cpu", dtype=torch.bfloat16)
    gen = _generator(to_gpu_model(model_cpu))
    ex = gen.model_executor
    gen_t = torch.Generator().manual_seed(5)
    kv = random_prefix_kv(SHAPE.layers, SHAPE.kv_heads, 120, SHAPE.head_dim, gen_t)
    cache = ex.new_cache()
    cache.load_dense(kv)
    cnt = FoldCounters()
    for step in range(3):
        tokens = draft_tree_block(32, SHAPE.vocab - 2, gen_t)
        got = gen._batched_block_forward(tokens.cuda(), cache)
        ref = folded_verify_step(model_cpu, tokens, kv, gen.delta, counters=cnt, shift=True)
        st = err_stats(got.float(), ref.float())
        print(f"step {step}: shifted logits {st}", flush=True)
        assert torch.equal(got[:, 0], got[:, 1]) and torch.equal(ref[:, 0], ref[:, 1])
        assert st["max_abs"] <= NS_MAX_ABS * max(1.0, st["ref_absmax"])
        assert st["mean_rel"] <= LOGITS_MEAN_REL_MAX
        assert gen._fold_draft_positions == cnt.draft_positions
        assert int(gen._fold_draft_recomputed) == cnt.draft_recomputed, \
            (int(gen._fold_draft_recomputed), cnt.draft_recomputed)
    assert gen.fold_ratio == cnt.fold_ratio
    print(f"fold ratio {gen.fold_ratio:.4f} over {cnt.draft_positions} draft positions", flush=True)


def _scaled_model(seed, scale):
    model = build_qwen2(SHAPE, seed, device="cuda")
    model.lm_head.weight.mul_(scale)
    return model


def test_generate_with_draft_speculation():
    prompt = torch.randint(0, SHAPE.vocab - 2, (1, 40), generator=torch.Generator().manual_seed(8))
    outs = []
    for _ in range(2):
        gen = _generator(_scaled_model(22, 12.0))
        text, n_tok, calls, drafts = gen.generate_with_draft_speculation(prompt_ids=prompt.cuda())
        print(f"tokens {n_tok}, model calls {calls}, drafts {drafts}, fold ratio "
              f"{gen.fold_ratio:.3f}", flush=True)
        assert isinstance(text, list) and n_tok > 0 and calls >= 1
        assert 0.0 <= gen.fold_ratio <= 1.0
        outs.append(gen.last_tokens.clone())
    assert torch.equal(outs[0], outs[1])


def reference_decision(logits_cpu, maskable, top_p, threshold):
    """fastdllm_model_executor.py:129-155 (temperature 0) + fastdllm_v2_generation.py:
    666-676 on logits [1, n, V]: (tokens [1, n], committed positions [1, n])."""
    sorted_logits, sorted_idx = torch.sort(logits_cpu, descending=True, dim=-1)
    cum = torch.cumsum(torch.softmax(sorted_logits, dim=-1), dim=-1)
    drop_sorted = cum > top_p
    drop_sorted[..., 1:] = drop_sorted[..., :-1].clone()
    drop_sorted[..., 0] = False
    drop = drop_sorted.scatter(-1, sorted_idx, drop_sorted)
    probs = torch.softmax(logits_cpu.masked_fill(drop, float("-inf")), dim=-1)
    x_1 = torch.argmax(probs, dim=-1)
    x1_p = torch.gather(probs, -1, x_1.unsqueeze(-1)).squeeze(-1)
    x1_p = torch.where(maskable, x1_p, -torch.inf)
    unmask = x1_p > threshold
    unmask[torch.arange(x_1.shape[0]), x1_p.argmax(dim=-1)] = True
    return x_1, unmask & maskable


@pytest.mark.parametrize("scale", [6.0, 20.0, 40.0])
def test_decode_decisions_match_reference_sampler(scale):
    gen = _generator(_scaled_model(23, scale), max_new=128)
    seen = []
    orig = gen._sample_rows

    def recording(logits):
        out = orig(logits)
        seen.append(logits.detach().to("cpu", copy=True))
        return out

    gen._sample_rows = recording
    prompt = torch.randint(0, SHAPE.vocab - 2, (1, 48), generator=torch.Generator().manual_seed(9))
    steps = mism = over = 0
    for ev in gen.decode_steps(prompt.cuda()):
        if ev["kind"] not in ("verify", "hit"):
            continue
        logits = seen[-1]
        maskable = ev["maskable"].cpu()
        tok_ref, unmask_ref = reference_decision(logits, maskable, gen.top_p, gen.threshold)
        unmask = ev["unmask"].cpu()
        tok = ev["tokens"].cpu()
        steps += 1
        over += int(unmask.sum()) > 1
        if not torch.equal(unmask, unmask_ref) or not torch.equal(tok[unmask], tok_ref[unmask_ref]):
            mism += 1
            print(f"step {steps}: statistics {unmask.int().tolist()} {tok.tolist()} vs reference "
                  f"{unmask_ref.int().tolist()} {tok_ref.tolist()}", flush=True)
    print(f"scale {scale}: {steps} decision steps, {over} committed more than one token, "
          f"{mism} mismatches", flush=True)
    assert steps >= 10
    assert mism == 0


def test_warm_graphs_then_decode_replays_only():
    """warm_graphs captures the verify step for every branch count the draft graph
    can produce (the main block alone included); the decode loop afterwards captures
    nothing new and commits the same tokens as a loop that captured on the way."""
    prompt = torch.randint(0, SHAPE.vocab - 2, (1, 40), generator=torch.Generator().manual_seed(8))
    outs = []
    for warm in (False, True):
        gen = _generator(_scaled_model(22, 12.0))
        loop = gen.decode_steps(prompt.cuda())
        assert next(loop)["kind"] == "prefill"
        n0 = 0
        if warm:
            assert gen.warm_graphs() == gen.draft_limit() + 1 >= 2
            n0 = len(gen._engine._graphs)
        for _ in loop:
            pass
        if warm:
            assert len(gen._engine._graphs) == n0, "the decode loop captured a new graph"
        outs.append(gen._state["x_t"].clone())
    assert torch.equal(outs[0], outs[1])
