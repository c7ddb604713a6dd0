"""sf_parent_map (the branch parent map computed on the device) against the
oracle's restatement of _build_parent_map (fastdllm_v2_folded.py:55-75): equal
maps on draft trees, random blocks, duplicate branches and the 64 x 64 limits."""

import pytest
import torch

from oracle.folded_reference import parent_map
from specfold_amd import _lib
from specfold_amd.synthetic import draft_tree_block

pytestmark = pytest.mark.gpu


def device_map(tokens):
    B1 = tokens.shape[0]
    par = torch.full((B1,), -1, dtype=torch.int32, device="cuda")
    cnt = torch.full((B1,), -1, dtype=torch.int32, device="cuda")
    _lib.parent_map(tokens.cuda().contiguous(), par, cnt)
    torch.cuda.synchronize()
    return par.tolist(), cnt.tolist()


def oracle_map(tokens):
    parent, counts = parent_map(tokens.cpu())
    return [0] + [int(p) for p in parent[1:]], [int(c) for c in counts]


@pytest.mark.parametrize("seed", range(4))
def test_draft_trees(seed):
    g = torch.Generator().manual_seed(seed)
    tokens = draft_tree_block(32, 151936, g)
    assert device_map(tokens) == oracle_map(tokens)


@pytest.mark.parametrize("B1,N,vocab", [(8, 32, 3), (5, 32, 2), (64, 64, 2), (1, 32, 10),
                                        (17, 7, 3)])
def test_random_blocks(B1, N, vocab):
    g = torch.Generator().manual_seed(B1 * 100 + N)
    for _ in range(20):
        main = torch.randint(0, vocab, (1, N), generator=g)
        flips = torch.rand(B1, N, generator=g) < 0.15
        tokens = torch.where(flips, torch.randint(0, vocab, (B1, N), generator=g), main)
        tokens[0] = main[0]
        assert device_map(tokens) == oracle_map(tokens)


def test_duplicates_and_identical_rows():
    tokens = torch.zeros(6, 32, dtype=torch.long)
    tokens[1, 3] = tokens[2, 3] = 1          # two identical 1-diff branches
    tokens[3, [3, 5]] = 1                    # 2-diff child of both: the first (1) wins
    tokens[4, 9] = 2                         # 1-diff, unrelated
    assert device_map(tokens) == oracle_map(tokens)
    assert device_map(tokens)[0] == [0, 0, 0, 1, 0, 0]
