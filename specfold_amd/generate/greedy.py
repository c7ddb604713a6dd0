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
    return st.top_idx.index_select(0, pos)[:, rank].long()
