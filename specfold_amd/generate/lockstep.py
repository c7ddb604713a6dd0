"""Several independent sequences decoded in lockstep, their verify steps merged.

The decode loops (NLDDiffusionGeneration.decode_steps and
FastDLLMV2SpeculativeGeneration.decode_steps) run one sequence each; a
batch of B sequences stepped one after another streams every weight matrix B
times per round of verify steps.  LockstepDecoder runs each sequence's loop with
``defer_forward=True``: in each round every live sequence advances to its next
verify forward, and the forwards of all of them run as ONE verify step over the
stacked branch trees (FoldedVerifyEngine.forward_batched), so the weights are
streamed once per round.  Prefill and block commits (cache writes) stay per
sequence.  Each sequence's tokens are those its own loop would produce with its
verify steps computed by the engine (forward_batched gives every sequence the
result of FoldedVerifyEngine.forward on it alone).

No counterpart in the reference, whose generators decode one sequence per call.
"""

from __future__ import annotations

from typing import Callable, Dict, List, Optional, Sequence

import torch

from specfold_amd.engine import StepStats
from specfold_amd.kv_cache import cache_length

# [(batched [B1_s, N], prefix cache)] -> [logits [B1_s, N, V]]
ForwardMany = Callable[[List[tuple]], List[torch.Tensor]]


class LockstepDecoder:
    """Drives the decode loops of ``gens`` (generators of one family, one per
    sequence) in lockstep.  ``forward_many`` computes a round's verify forwards;
    the default is one batched verify step on the engine of the first generator
    (a SpecFoldHIPNLDGeneration or SpecFoldHIPFastDLLMV2Generation; every
    generator shares its delta and bucket), with the executor's per-position q
    scale where it has one (NLD) and the generator's logit shift where it has
    one (Fast-dLLM)."""

    def __init__(self, gens: Sequence, forward_many: Optional[ForwardMany] = None,
                 pad: bool = True):
        if not gens:
            raise ValueError("LockstepDecoder needs at least one generator")
        self.gens = list(gens)
        # every sequence padded to the most branches a step can have (main + one per
        # draft-graph node), so a round's shape depends on the live sequences only
        # and its captured graph is reused
        graph = getattr(self.gens[0], "calibration_graph", None) or {}
        drafts = sum(1 for n in graph.get("selected_nodes", []) if n.get("ij_set"))
        self.pad_to = 1 + drafts if pad else None
        self.forward_many = forward_many or self._engine_forward_many
        self.rounds_run = 0
        self.batched_steps = 0
        self.draft_positions = 0
        self._recomputed: Optional[torch.Tensor] = None   # device scalar
        self.last_stats: Optional[StepStats] = None

    @property
    def fold_ratio(self) -> float:
        """Share of draft rows folded over every batched step (one host read).  At
        delta = 0 a padding branch recomputed at a later layer counts as a
        recomputed draft row (see FoldedVerifyEngine.forward_batched)."""
        if not self.draft_positions:
            return float("nan")
        return 1.0 - int(self._recomputed) / self.draft_positions

    def _engine_forward_many(self, requests: List[tuple]) -> List[torch.Tensor]:
        g0 = self.gens[0]
        if g0._engine is None:
            g0._pack_layer_weights()
        eng = g0._engine
        N = requests[0][0].shape[1]
        total = sum(b.shape[0] for b, _ in requests) * N      # real (unpadded) rows
        q_scale = getattr(g0.model_executor, "q_scale", None)
        q_scales = [q_scale(cache_length(c), N) if q_scale is not None else None
                    for _, c in requests]
        # a batched step holds at most 64 branches and 1024 rows: split the round
        # into as few steps as fit
        chunks, cur, cur_b = [], [], 0
        for i, (b, _) in enumerate(requests):
            nb = self.pad_to or b.shape[0]
            if cur and (cur_b + nb > 64 or (cur_b + nb) * N > 1024):
                chunks.append(cur)
                cur, cur_b = [], 0
            cur.append(i)
            cur_b += nb
        chunks.append(cur)
        logits = [None] * len(requests)
        rec = None
        # Fast-dLLM generators take shifted logits: the head's stores shift them
        shifted = hasattr(g0, "_shift_logits")
        prev_mode, eng.gate_mode = eng.gate_mode, g0.gate_mode
        try:
            for idx in chunks:
                stats = StepStats()
                # fold_bucket bounds one sequence's recomputed rows: a stacked step
                # holds the sum of its sequences' bounds (each at most its rows)
                bucket = None if g0.fold_bucket is None else sum(
                    min(int(g0.fold_bucket), (self.pad_to or requests[i][0].shape[0]) * N)
                    for i in idx)
                out = eng.forward_batched([requests[i][0] for i in idx],
                                          [requests[i][1] for i in idx], delta=g0.delta,
                                          shift=shifted,
                                          bucket=bucket, q_scales=[q_scales[i] for i in idx],
                                          stats=stats, pad_to=self.pad_to)
                for i, x in zip(idx, out):
                    logits[i] = x
                # fold counters stay on the device: every sequence's main branch is a root
                r = stats.count_dev.sum(dtype=torch.int64) - eng.L * N * len(idx)
                rec = r if rec is None else rec + r
                self.last_stats = stats
        finally:
            eng.gate_mode = prev_mode
        self.batched_steps += len(chunks) - 1      # rounds() counts one step per round
        self.draft_positions += (total - len(requests) * N) * eng.L
        self._recomputed = rec if self._recomputed is None else self._recomputed + rec
        return logits

    def rounds(self, prompts: Sequence[torch.Tensor]):
        """Generator: one event per round, {"kind": "round", "committed": tokens
        unmasked in the round (all sequences), "forwards": sequences in the round's
        batched verify step, "events": [(sequence, loop event), ...]}.  The first
        round holds the prefills.  Ends when every loop has ended; states stay on
        each generator's ``_state``."""
        if len(prompts) != len(self.gens):
            raise ValueError("one prompt per generator")
        loops = [g.decode_steps(p, defer_forward=True) for g, p in zip(self.gens, prompts)]
        reply: Dict[int, Optional[torch.Tensor]] = {i: None for i in range(len(loops))}
        started = [False] * len(loops)
        live = list(range(len(loops)))
        while live:
            events, requests, still = [], [], []
            for i in live:
                lp = loops[i]
                try:
                    ev = lp.send(reply[i]) if started[i] else next(lp)
                    started[i] = True
                    reply[i] = None
                    while ev["kind"] != "forward":
                        events.append((i, ev))
                        ev = next(lp)
                except StopIteration:
                    continue
                requests.append((i, ev))
                still.append(i)
            live = still
            if requests:
                outs = self.forward_many([(ev["batched"], ev["cache"]) for _, ev in requests])
                if len(outs) != len(requests):
                    raise RuntimeError("forward_many returned the wrong number of results")
                for (i, _), out in zip(requests, outs):
                    reply[i] = out
                self.batched_steps += 1
            self.rounds_run += 1
            yield {"kind": "round", "committed": sum(e["committed"] for _, e in events),
                   "forwards": len(requests), "events": events}

    def generate(self, prompts: Sequence) -> List[tuple]:
        """Each sequence's ``generate_with_draft_speculation`` result (texts,
        tokens_generated, model_calls, drafts_computed), the sequences decoded in
        lockstep.  prompts: strings or [1, L] token ids, one per generator."""
        def prompt_ids(g, p):
            if not isinstance(p, str):
                return p
            if hasattr(g, "_init_generation_state"):     # Fast-dLLM: its prompt template
                return g._init_generation_state(p)[1]
            return g.tokenizer(p, return_tensors="pt").input_ids

        ids = [prompt_ids(g, p) for g, p in zip(self.gens, prompts)]
        for g in self.gens:
            g.last_commits = []
        for _ in self.rounds(ids):
            pass
        return [g._result() for g in self.gens]
