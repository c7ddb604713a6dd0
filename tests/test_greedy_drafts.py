"""The vectorised draft construction from logit statistics (one gather and one
scatter for all nodes) against the per-node, per-pair loop it replaces, on CPU
with statistics computed by the reference's own ops (topk / softmax)."""

import types

import pytest
import torch

from specfold_amd.configs import SYNTHETIC_DRAFT_GRAPH
from specfold_amd.generate import greedy
from specfold_amd.generate.fastdllm_v2_generation import FastDLLMV2SpeculativeGeneration
from specfold_amd.generate.nld_generation import NLDDiffusionGeneration


def fake_stats(logits):
    """What sf_logit_stats returns for the fields the drafts read (lowest index
    first among equal logits: stable sort)."""
    order = torch.sort(logits.float(), dim=-1, descending=True, stable=True).indices
    z = torch.exp(logits.float() - logits.float().max(-1, keepdim=True).values).sum(-1)
    return types.SimpleNamespace(top_idx=order[:, :8].to(torch.int32), zfull=z,
                                 conf_full=(1.0 / z).to(torch.bfloat16).float())


def loop_states(x, conf, st, ij_sets, offset):
    blocks = []
    for ij in ij_sets:
        positions = torch.topk(conf, k=max(p for p, _ in ij) + 1).indices
        b = x.clone()
        for p, r in ij:
            pos = positions[p:p + 1]
            b.index_put_((pos + offset,), st.top_idx.index_select(0, pos)[:, r].long())
        blocks.append(b)
    return torch.stack(blocks)


@pytest.mark.parametrize("seed", range(6))
def test_vectorised_equals_loop(seed):
    g = torch.Generator().manual_seed(seed)
    logits = (torch.randn(8, 999, generator=g) * 3).to(torch.bfloat16)
    st = fake_stats(logits)
    conf = torch.randn(8, generator=g)
    conf[seed % 8] = float("-inf")
    x = torch.randint(0, 999, (32,), generator=g)
    ij_sets = [n["ij_set"] for n in SYNTHETIC_DRAFT_GRAPH["selected_nodes"]]
    ij_sets = ij_sets + [[(0, 1), (2, 3)], [(1, 7)]]
    a = greedy.draft_states(x, conf, st, ij_sets, offset=16)
    b = loop_states(x, conf, st, ij_sets, 16)
    assert torch.equal(a, b)
    assert greedy.draft_states(x, conf, st, [[(0, 8)]]) is None     # rank beyond the top 8


def test_fastdllm_draft_states_with_stats_equal_reference_ops():
    g = torch.Generator().manual_seed(3)
    logits = (torch.randn(8, 777, generator=g) * 2).to(torch.bfloat16)
    st = fake_stats(logits)
    mask = torch.ones(8, dtype=torch.bool)
    mask[2] = False
    x = torch.randint(0, 777, (32,), generator=g)
    active = [(n, tuple(n["ij_set"]), max(p for p, _ in n["ij_set"]))
              for n in SYNTHETIC_DRAFT_GRAPH["selected_nodes"]]
    a = FastDLLMV2SpeculativeGeneration._draft_states(x, logits, mask, 8, active, st)
    b = FastDLLMV2SpeculativeGeneration._draft_states(x, logits, mask, 8, active)
    assert torch.equal(a, b)


def test_nld_draft_blocks_with_stats_equal_reference_ops():
    g = torch.Generator().manual_seed(4)
    logits = (torch.randn(32, 555, generator=g) * 2).to(torch.bfloat16)
    st = fake_stats(logits)
    gen = NLDDiffusionGeneration.__new__(NLDDiffusionGeneration)
    gen.calibration_graph = SYNTHETIC_DRAFT_GRAPH
    mask = torch.rand(32, generator=g) < 0.5
    mask[:4] = True
    x = torch.randint(0, 555, (32,), generator=g)
    a = gen.get_draft_blocks(x, logits, mask, stats=st)
    b = gen.get_draft_blocks(x, logits, mask)
    assert len(a) == len(b) > 0
    for da, db in zip(a, b):
        assert da["node"] is db["node"] and torch.equal(da["state"], db["state"])


def test_json_style_graph_nodes():
    """Calibration graphs loaded from JSON carry [pos_rank, vocab_rank] lists."""
    g = torch.Generator().manual_seed(8)
    logits = torch.randn(8, 321, generator=g).to(torch.bfloat16)
    st = fake_stats(logits)
    conf = torch.randn(8, generator=g)
    x = torch.zeros(32, dtype=torch.long)
    ij_sets = [[[0, 0], [1, 2]], [[3, 1]]]
    a = greedy.draft_states(x, conf, st, ij_sets, offset=0)
    assert torch.equal(a, loop_states(x, conf, st, ij_sets, 0))
