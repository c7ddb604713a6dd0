"""Seeded synthetic inputs for the verify step (no datasets, no checkpoints).

* ``draft_tree_block``: a main block plus B=7 draft branches whose differing
  positions form the fixed depth-4 tree d1={0}, d2={0,1}, d3={0,2}, d4={0,3},
  d5={0,1,4}, d6={0,1,5}, d7={0,1,4,6} (position indices into ``positions``),
  one replacement token per tree position, so a child repeats its parent's
  tokens where their diff sets overlap.  Parents: d1->0, d2..d4->d1,
  d5,d6->d2, d7->d5.
* ``random_prefix_kv``: per-layer prefix K/V ~ N(0, 1) in [1, Hkv, P, hd].
* ``perturbed_hidden``: per-branch hidden states x_child = x_parent + sigma*z,
  sigma = sigma_hi on a seeded fraction of positions and sigma_lo elsewhere;
  with the relative-L2 gate at delta the recompute mask is decided with a
  margin of sigma/delta (mode used for a 0.6-ish fold ratio).
"""

from __future__ import annotations

from typing import List, Optional, Sequence, Tuple

import torch

TREE_DIFFS: Tuple[Tuple[int, ...], ...] = (
    (), (0,), (0, 1), (0, 2), (0, 3), (0, 1, 4), (0, 1, 5), (0, 1, 4, 6))
TREE_PARENTS: Tuple[Optional[int], ...] = (None, 0, 1, 1, 1, 2, 2, 5)


def draft_tree_block(N: int, vocab: int, gen: torch.Generator,
                     positions: Optional[Sequence[int]] = None,
                     diffs: Sequence[Tuple[int, ...]] = TREE_DIFFS) -> torch.Tensor:
    """[len(diffs), N] int64 token block; row 0 is the main branch."""
    n_pos = 1 + max((max(d) for d in diffs if d), default=0)
    if positions is None:
        positions = list(range(n_pos))
    main = torch.randint(0, vocab, (N,), generator=gen)
    repl = torch.randint(0, vocab, (n_pos,), generator=gen)
    # a replacement must differ from the main token, or the diff set shrinks
    for k in range(n_pos):
        while int(repl[k]) == int(main[positions[k]]):
            repl[k] = int(torch.randint(0, vocab, (1,), generator=gen))
    rows = []
    for d in diffs:
        row = main.clone()
        for k in d:
            row[positions[k]] = repl[k]
        rows.append(row)
    return torch.stack(rows)


def random_prefix_kv(layers: int, kv_heads: int, P: int, head_dim: int, gen: torch.Generator,
                     dtype=torch.bfloat16) -> List[Tuple[torch.Tensor, torch.Tensor]]:
    out = []
    for _ in range(layers):
        k = torch.randn(1, kv_heads, P, head_dim, generator=gen).to(dtype)
        v = torch.randn(1, kv_heads, P, head_dim, generator=gen).to(dtype)
        out.append((k, v))
    return out


def perturbed_hidden(parents: Sequence[Optional[int]], N: int, D: int, gen: torch.Generator,
                     sigma_hi: float = 0.2, sigma_lo: float = 0.05, frac_hi: float = 0.38,
                     dtype=torch.bfloat16) -> torch.Tensor:
    """[B1, N, D] hidden states; branch i = its parent's + sigma * N(0, 1)."""
    B1 = len(parents)
    h = torch.zeros(B1, N, D)
    h[0] = torch.randn(N, D, generator=gen)
    for i in range(1, B1):
        p = parents[i] if parents[i] is not None else 0
        hi = torch.rand(N, generator=gen) < frac_hi
        sig = torch.where(hi, torch.tensor(sigma_hi), torch.tensor(sigma_lo))
        h[i] = h[p] + sig[:, None] * torch.randn(N, D, generator=gen)
    return h.to(dtype)
