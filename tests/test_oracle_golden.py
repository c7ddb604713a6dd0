"""The oracle reproduces the reference's PyTorch folded verify step bit for bit.

Golden vectors come from the reference class itself
(tests/golden/make_golden.py -> specfold/generate/fastdllm_v2_folded.py:89-223)
on tiny bf16 and fp32 models; the oracle must match its logits exactly and its
fold counters exactly.
"""

import pytest
import torch

from oracle.folded_reference import FoldCounters, folded_verify_step
from tests.golden_io import golden_cases, load_case


@pytest.mark.parametrize("name", golden_cases())
def test_oracle_matches_reference_golden(name):
    case = load_case(name)
    cnt = FoldCounters()
    logits = folded_verify_step(case["model"], case["tokens"], case["kv"], case["meta"]["delta"],
                                counters=cnt)
    assert logits.dtype == case["logits"].dtype
    assert torch.equal(logits, case["logits"]), (logits - case["logits"]).abs().max()
    assert cnt.draft_positions == case["meta"]["draft_positions"]
    assert cnt.draft_recomputed == case["meta"]["draft_recomputed"]
