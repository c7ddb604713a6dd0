"""Greedy (temperature 0) decode decisions from per-position logit statistics.

The decode loops decide from a few numbers per block position: the greedy token
and its probability (the top-p sampler, fastdllm_model_executor.py:129-155 via
fastdllm_v2_generation.py:646-676), the maximum softmax probability and the
highest-ranked vocabulary tokens (draft construction, fastdllm_v2_generation.py:
430-470, nld_generation.py:105-151) and the argmax with its probability (NLD's
transfer rule, modeling_nemotron_labs_diffusion.py:835-861).  ``sf_logit_stats``
produces them in one pass over each logits row; the functions below turn them
into the tensors the reference's torch sequences would have produced, so the
rest of each loop is unchanged.

The top-p cut follows the reference's sampler as written: each token's bf16
probability is summed in descending order and the running sum is rounded to
bf16 before the comparison with top_p.  (torch's GPU scan kernel for bf16 also
rounds every partial sum inside its scan tree, so on a GPU the reference's sum
can stall below top_p for a flat distribution and keep the whole vocabulary;
this module, like the reference run on a CPU, accumulates the sum in fp32.)
"""

from __future__ import annotations

from typing import Optional

import torch

from specfold_amd import _lib

TOP_K = 8  # vocabulary ranks the statistics carry


def usable(logits: torch.Tensor, temperature: float) -> bool:
    """Greedy decisions come from the HIP statistics for bf16 logits on the GPU
    (vocabulary a multiple of 8, the kernel's vector width)."""
    return (temperature == 0 and logits.is_cuda and logits.dtype == torch.bfloat16
            and logits.shape[-1] % 8 == 0)


def stats(rows: torch.Tensor, top_p: float = 0.95) -> _lib.LogitStats:
    """sf_logit_stats of logits rows [n, V] (any leading shape is flattened)."""
    return _lib.logit_stats(rows, top_p=top_p)


def top_p_greedy(st: _lib.LogitStats):
    """(tokens [1, n] int64, probabilities [1, n] bf16): the reference sampler's
    argmax token and its bf16 nucleus probability."""
    return st.greedy_tok.long().unsqueeze(0), st.conf.to(torch.bfloat16).unsqueeze(0)


def max_prob_bf16(st: _lib.LogitStats) -> torch.Tensor:
    """softmax(bf16 logits).max(-1) per row (bf16)."""
    return st.conf_full.to(torch.bfloat16)


def max_prob_fp32(st: _lib.LogitStats) -> torch.Tensor:
    """softmax(logits.float()).max(-1) per row (fp32): 1 / Z."""
    return 1.0 / st.zfull


def vocab_rank(st: _lib.LogitStats, pos: torch.Tensor, rank: int) -> Optional[torch.Tensor]:
    """The rank-th most likely token at row(s) ``pos`` (int64 [k]), or None when
    the statistics do not carry that rank."""
    if rank >= TOP_K:
        return None
    return st.top_idx[pos, rank].long()


class DraftIndex:
    """Device index tensors of a fixed list of draft-graph nodes (ij_sets), built
    once: for the flattened (node, pos_rank, vocab_rank) pairs, the position in
    the concatenated per-node topk results, the vocabulary rank and the node."""

    def __init__(self, ij_sets, device):
        self.ks = [max(p for p, _ in ij) + 1 for ij in ij_sets]
        starts = [sum(self.ks[:n]) for n in range(len(ij_sets))]
        g, v, node = [], [], []
        for n, ij in enumerate(ij_sets):
            for p, r in ij:
                g.append(starts[n] + p)
                v.append(r)
                node.append(n)
        self.max_rank = max(v)
        self.g_idx = torch.tensor(g, dtype=torch.long, device=device)
        self.v_idx = torch.tensor(v, dtype=torch.long, device=device)
        self.node_idx = torch.tensor(node, dtype=torch.long, device=device)
        self.n = len(ij_sets)


_DRAFT_INDEX: dict = {}


def draft_states(x: torch.Tensor, conf: torch.Tensor, st: _lib.LogitStats, ij_sets,
                 offset: int = 0) -> Optional[torch.Tensor]:
    """Draft blocks of the given nodes, stacked [n, len(x)]: node n puts, for each
    (pos_rank, vocab_rank) of its ij_set, the vocab_rank-th most likely token of
    the pos_rank-th most confident position (positions index the statistics'
    rows; block position = row + offset).  The positions of each node come from
    its own torch.topk over ``conf`` with k = its largest rank + 1, as the
    reference's per-node call; the tokens of all nodes are then gathered and
    scattered at once.  None when a vocabulary rank exceeds the statistics."""
    key = (tuple(tuple(tuple(pair) for pair in ij) for ij in ij_sets), x.device)
    ix = _DRAFT_INDEX.get(key)
    if ix is None:
        ix = _DRAFT_INDEX[key] = DraftIndex(ij_sets, x.device)
    if ix.max_rank >= TOP_K:
        return None
    positions = torch.cat([torch.topk(conf, k=k).indices for k in ix.ks])
    # advanced indexing (one gather kernel per dtype) rather than index_select,
    # whose kernel variant changes with the index count (16 or fewer, or more): a
    # step whose node set first crossed that line paid a one-off kernel load of
    # tens of milliseconds inside the decode loop
    pos = positions[ix.g_idx]
    toks = st.top_idx[pos, ix.v_idx].long()
    states = x.unsqueeze(0).repeat(ix.n, 1)
    states.index_put_((ix.node_idx, pos + offset), toks)
    return states
