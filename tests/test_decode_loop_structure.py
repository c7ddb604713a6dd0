"""The Fast-dLLM v2 and NLD decode loops, restructured around one host read per iteration
(``_loop_facts``) against the reference's control flow with a host read at every
decision point (tests/reference_loops.py), on the CPU with the deterministic
bank model of tests/test_decode_loops_stats.py: the event streams (kinds,
committed counts, sampled tokens, unmasked positions), the final tokens, the
model-call and draft counts must be identical — stop tokens, commits, draft hits
and multi-token commits included."""

import pytest
import torch

from specfold_amd.configs import SYNTHETIC_DRAFT_GRAPH
from specfold_amd.generate.fastdllm_v2_generation import FastDLLMV2SpeculativeGeneration
from specfold_amd.generate.nld_generation import NLDDiffusionGeneration
from tests.helpers import plain_events
from tests.reference_loops import fastdllm_events, nld_events
from tests.test_decode_loops_stats import FakeFastDLLM, FakeNLD, _bank


def _gen(seed, stop):
    return FastDLLMV2SpeculativeGeneration(
        block_length=32, model_executor=FakeFastDLLM(_bank(seed)),
        calibration_graph=SYNTHETIC_DRAFT_GRAPH, max_new_tokens=160, stop_token=stop,
        device="cpu")


@pytest.mark.parametrize("seed", range(6))
@pytest.mark.parametrize("stop", [7, 300])
def test_loop_control_flow_matches_reference(seed, stop):
    prompt = torch.randint(0, 256, (1, 40 + 3 * seed), generator=torch.Generator().manual_seed(seed))
    a, b = _gen(seed, stop), _gen(seed, stop)
    a.last_commits = []
    ev_a = list(a.decode_steps(prompt))
    ev_b = list(fastdllm_events(b, prompt))
    assert plain_events(ev_a) == plain_events(ev_b)
    for x, y in zip(ev_a, ev_b):
        for k in ("tokens", "unmask", "maskable"):
            if k in x:
                assert torch.equal(x[k], y[k]), k
    assert torch.equal(a._state["x_t"], b._state["x_t"])
    assert a._state["model_calls"] == b._state["model_calls"]
    assert a._state["drafts_computed"] == b._state["drafts_computed"]
    assert a.last_commits == [e["committed"] for e in ev_a if e["kind"] in ("verify", "hit")]


def test_loop_exercises_every_branch():
    kinds = set()
    stopped = 0
    for seed in range(6):
        for stop in (7, 300):
            g = _gen(seed, stop)
            g.last_commits = []
            prompt = torch.randint(0, 256, (1, 40 + 3 * seed),
                                   generator=torch.Generator().manual_seed(seed))
            ev = list(g.decode_steps(prompt))
            kinds |= {e["kind"] for e in ev}
            stopped += bool((g._state["x_t"][0, g._state["orig_len"]:] == stop).any())
    assert {"prefill", "verify", "hit", "commit"} <= kinds
    assert stopped > 0


@pytest.mark.parametrize("seed", range(6))
@pytest.mark.parametrize("threshold", [0.9, None])
def test_nld_loop_control_flow_matches_reference(seed, threshold):
    bank = _bank(100 + seed, eos=FakeNLD.EOS)
    prompt = torch.randint(0, 256, (1, 20 + 5 * seed), generator=torch.Generator().manual_seed(seed))
    gens = [NLDDiffusionGeneration(block_length=32, model_executor=FakeNLD(bank),
                                   calibration_graph=SYNTHETIC_DRAFT_GRAPH, max_new_tokens=160,
                                   threshold=threshold, device="cpu") for _ in range(2)]
    gens[0].last_commits = []
    ev_a = list(gens[0].decode_steps(prompt))
    ev_b = list(nld_events(gens[1], prompt))
    assert plain_events(ev_a) == plain_events(ev_b)
    assert torch.equal(gens[0]._state["x_accum"], gens[1]._state["x_accum"])
    assert gens[0]._state["model_calls"] == gens[1]._state["model_calls"]
    assert gens[0]._state["drafts_computed"] == gens[1]._state["drafts_computed"]
    assert {"prefill", "verify", "commit"} <= {e["kind"] for e in ev_a}
