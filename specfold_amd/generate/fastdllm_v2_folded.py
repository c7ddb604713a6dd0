"""SpecFold for Fast-dLLM v2 on MI355X: the B+1-branch folded verify step.

``SpecFoldHIPFastDLLMV2Generation`` is the drop-in for the reference's fused
class ``SpecFoldTritonFastDLLMV2Generation``
(specfold/generate/fastdllm_v2_folded.py:226-370): same constructor
(``delta``, ``fold_bucket``), same ``_batched_block_forward(batched_input,
past_key_values) -> shifted logits [B1, N, V]`` seam, same ``fold_ratio``
bookkeeping and the same bucket-overflow behaviour (warn, recompute with a
full bucket — here on the GPU, not through a PyTorch prototype).  The step
runs the hand-written gfx950 kernels of ``specfold_amd.engine``; there is no
CPU or PyTorch fallback.
"""

from __future__ import annotations

import logging
from typing import List, Optional, Tuple

import torch

from specfold_amd import _lib
from specfold_amd.engine import FoldedVerifyEngine, StepStats, build_parent_map
from specfold_amd.generate.fastdllm_v2_generation import FastDLLMV2SpeculativeGeneration

logger = logging.getLogger(__name__)


class SpecFoldHIPFastDLLMV2Generation(FastDLLMV2SpeculativeGeneration):
    """Folded verify step: relative-residual gate per (branch, position) against
    the subset-parent, QKV/attention/FFN only on recomputed rows, exact chain
    correction of the attention state of folded rows, residual kept per row."""

    def __init__(self, *args, delta: float = 0.1, fold_bucket: Optional[int] = None,
                 gate_mode: int = _lib.SF_GATE_MODEL_DTYPE, **kwargs):
        super().__init__(*args, **kwargs)
        self.delta = float(delta)
        self.fold_bucket = None if fold_bucket is None else int(fold_bucket)
        self.gate_mode = gate_mode
        self._engine: Optional[FoldedVerifyEngine] = None
        self._fold_draft_positions = 0
        self._fold_draft_recomputed = None  # device scalar: read only by fold_ratio
        self.last_stats: Optional[StepStats] = None

    @property
    def fold_ratio(self) -> float:
        tot = self._fold_draft_positions
        if not tot:
            return float("nan")
        return 1.0 - int(self._fold_draft_recomputed) / tot

    @staticmethod
    def _build_parent_map(batched_input: torch.Tensor) -> Tuple[List[Optional[int]], List[int]]:
        return build_parent_map(batched_input)

    def _pack_layer_weights(self, layers=None) -> None:
        """Pack per-layer QKV weights once (inside the engine)."""
        ex = self.model_executor
        eng = getattr(ex, "engine", None)
        if eng is None or eng.model is not ex.model:
            eng = FoldedVerifyEngine(ex.model, gate_mode=self.gate_mode)
        self._engine = eng

    def draft_limit(self) -> int:
        """The most draft blocks a verify step can carry: the draft graph's nodes."""
        g = self.calibration_graph or {}
        return sum(1 for n in g.get("selected_nodes", []) if n.get("ij_set"))

    @torch.no_grad()
    def warm_graphs(self, past_key_values=None) -> int:
        """Capture the verify step's HIP graph (and select the head GEMM's kernel)
        for every branch count the draft graph can produce — B1 = 1 (the main block
        alone, the dense path) and 2 .. drafts + 1 (the folded step) — at the current
        prefix cache, so the decode loop replays from its first step: the start-up
        work of a serving engine.  Runs the steps on placeholder tokens (a verify
        step reads the cache and writes nothing back); the fold counters are
        untouched.  Returns the number of branch counts prepared."""
        cache = self._state["cache"] if past_key_values is None else past_key_values
        if self._engine is None:
            self._pack_layer_weights()
        eng = self._engine
        N = self.block_length
        main = torch.full((1, N), self.mask_id, dtype=torch.long, device=eng.device)
        FastDLLMV2SpeculativeGeneration._batched_block_forward(self, main, cache)
        n = 1
        prev_mode, eng.gate_mode = eng.gate_mode, self.gate_mode
        try:
            for B1 in range(2, self.draft_limit() + 2):
                tokens = torch.full((B1, N), self.mask_id, dtype=torch.long, device=eng.device)
                tokens[1:, 0] = torch.arange(1, B1, device=eng.device)
                bucket = B1 * N if self.fold_bucket is None else min(self.fold_bucket, B1 * N)
                eng.forward(tokens, cache, delta=self.delta, bucket=bucket)
                n += 1
        finally:
            eng.gate_mode = prev_mode
        return n

    @torch.no_grad()
    def _batched_block_forward(self, batched_input: torch.Tensor, past_key_values) -> torch.Tensor:
        B1, N = batched_input.shape
        if B1 == 1:
            return FastDLLMV2SpeculativeGeneration._batched_block_forward(
                self, batched_input, past_key_values)
        if self._engine is None:
            self._pack_layer_weights()
        eng = self._engine
        bucket = B1 * N if self.fold_bucket is None else min(self.fold_bucket, B1 * N)
        stats = StepStats()
        prev_mode, eng.gate_mode = eng.gate_mode, self.gate_mode
        try:
            logits = eng.forward(batched_input, past_key_values, delta=self.delta, bucket=bucket,
                                 stats=stats, shift=True,
                                 head_rows=self.head_rows)
        finally:
            eng.gate_mode = prev_mode
        # fold counters stay on the device (no host sync per step)
        L = eng.L
        self._fold_draft_positions += (B1 - 1) * N * L
        rec = stats.count_dev.sum(dtype=torch.int64) - L * N
        self._fold_draft_recomputed = rec if self._fold_draft_recomputed is None else \
            self._fold_draft_recomputed + rec
        self.last_stats = stats
        return logits      # shifted by the head's stores (_shift_logits, :121-126)


# The reference's fused-path class name, so callers switch without code changes.
SpecFoldTritonFastDLLMV2Generation = SpecFoldHIPFastDLLMV2Generation
