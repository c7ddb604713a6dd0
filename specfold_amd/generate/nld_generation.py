"""Block-diffusion decoding for Nemotron-Labs-Diffusion with draft speculation —
the caller of the NLD verify seam ``_batched_block_forward``.

Mirrors ``NLDDiffusionGeneration`` of the reference
(specfold/generate/nld_generation.py:27-326): the same constructor knobs, the
same seam (no logit shift: the diffusion head predicts each position's own
token), the same whole-block draft construction (:105-151), the same
confidence-threshold unmasking with the transfer schedule of the checkpoint's
``generate()`` (modeling_nemotron_labs_diffusion.py:814-861), the same
draft-logit cache, and the causal refresh of the prefix cache after every block
(:298-316).  At temperature 0 the argmax tokens, probabilities and draft tokens
come from one sf_logit_stats pass over the block's logits.
"""

from __future__ import annotations

import logging
import time
from typing import Dict, List, Optional, Tuple

import torch
import torch.nn.functional as F

from specfold_amd.generate import greedy

logger = logging.getLogger(__name__)


def add_gumbel_noise(logits: torch.Tensor, temperature: float) -> torch.Tensor:
    """Scores whose argmax is a Gumbel-max sample at ``temperature``: exp(l) / E^T
    with E = -ln U, U ~ U(0, 1), all in float64; the logits themselves at
    temperature 0.  The expression and its float64 roundings are the reference's
    (modeling_nemotron_labs_diffusion.py:814-821), so that a seeded draw picks the
    same token even at a near tie."""
    if temperature == 0:
        return logits
    scores = logits.to(torch.float64)
    u = torch.rand_like(scores)
    return scores.exp() / (-torch.log(u)) ** temperature


def get_num_transfer_tokens(mask_index: torch.Tensor, steps: int) -> torch.Tensor:
    """Even split of the masked positions over ``steps``, remainder first
    (modeling_nemotron_labs_diffusion.py:824-832)."""
    mask_num = mask_index.sum(dim=1, keepdim=True)
    base = mask_num // steps
    remainder = mask_num % steps
    out = torch.zeros(mask_num.size(0), steps, device=mask_index.device, dtype=torch.int64) + base
    steps_idx = torch.arange(steps, device=mask_index.device).unsqueeze(0)
    return out + (steps_idx < remainder).to(torch.int64)


def get_transfer_index(logits: torch.Tensor, temperature: float, mask_index: torch.Tensor,
                       x: torch.Tensor, num_transfer_tokens: torch.Tensor,
                       threshold: Optional[float] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """Which masked positions to commit this denoising step
    (modeling_nemotron_labs_diffusion.py:835-861): x0 = argmax tokens (x at
    unmasked positions); the top-k masked positions by confidence, where with a
    threshold k = all masked positions and every selected position after the
    first is dropped when its confidence is below the threshold."""
    logits_with_noise = add_gumbel_noise(logits, temperature)
    x0 = torch.argmax(logits_with_noise, dim=-1)
    p = F.softmax(logits, dim=-1)
    x0_p = torch.squeeze(torch.gather(p, dim=-1, index=torch.unsqueeze(x0, -1)), -1)
    return transfer_from(x0, x0_p, mask_index, x, num_transfer_tokens, threshold)


def greedy_transfer_index(stats, mask_index: torch.Tensor, x: torch.Tensor,
                          num_transfer_tokens: torch.Tensor, threshold: Optional[float] = None,
                          ks=None):
    """get_transfer_index at temperature 0 from sf_logit_stats of the block's rows:
    x0 = the argmax token, its probability = the bf16 softmax maximum."""
    x0 = stats.top_idx[:, 0].long().unsqueeze(0)
    x0_p = greedy.max_prob_bf16(stats).unsqueeze(0)
    return transfer_from(x0, x0_p, mask_index, x, num_transfer_tokens, threshold, ks)


def transfer_from(x0, x0_p, mask_index, x, num_transfer_tokens, threshold=None, ks=None):
    """The selection part of get_transfer_index, given the argmax tokens x0 and
    their probabilities x0_p.  ``ks``: the per-row counts (masked positions with a
    threshold, else ``num_transfer_tokens``) when the caller holds them on the host."""
    x0 = torch.where(mask_index, x0, x)
    confidence = torch.where(mask_index, x0_p, float("-inf"))
    transfer_index = torch.zeros_like(x0, dtype=torch.bool)
    if ks is None:
        if threshold is not None:
            num_transfer_tokens = mask_index.sum(dim=1, keepdim=True)
        ks = num_transfer_tokens.reshape(-1).tolist()
    for j in range(confidence.shape[0]):
        k = int(ks[j])
        _, select_index = torch.topk(confidence[j], k=k)
        keep = torch.ones(k, dtype=torch.bool, device=confidence.device)
        if threshold is not None and k > 1:
            # the reference's per-position loop: drop select_index[i >= 1] if conf < thr
            keep[1:] = ~(confidence[j, select_index[1:]] < threshold)
        # transfer_index[j, select_index[keep]] = True without a host sync (the
        # topk indices are distinct and the row starts False)
        transfer_index[j].scatter_(0, select_index, keep)
    return x0, transfer_index


class NLDDiffusionGeneration:
    """Nemotron-Labs-Diffusion block-diffusion decoding (paper Sec. 3.2)."""

    def __init__(self, block_length: int, model_executor, calibration_graph=None,
                 temperature: float = 0.0, max_length: int = 4096, max_new_tokens: int = 1024,
                 threshold: Optional[float] = 0.9, causal_context: bool = True,
                 device: str = "cuda", **kwargs):
        self.block_length = block_length
        self.model_executor = model_executor
        self.calibration_graph = calibration_graph
        self.temperature = temperature
        self.max_length = max_length
        self.max_new_tokens = max_new_tokens
        self.threshold = threshold
        self.causal_context = causal_context
        self.device = getattr(model_executor, "device", torch.device(device))
        self.tokenizer = model_executor.get_tokenizer()
        self.mask_id = model_executor.get_mask_id()
        self.stop_token = model_executor.get_eos_token_id()
        self.last_commits: List[int] = []

    def _graph_nodes(self) -> List[Dict]:
        if self.calibration_graph is None:
            return []
        return [n for n in self.calibration_graph.get("selected_nodes", []) if n.get("ij_set")]

    # -- the seam ---------------------------------------------------------------------
    def _batched_block_forward(self, batched_input: torch.Tensor, past_key_values) -> torch.Tensor:
        """Dense B+1-row block forward over the prefix -> logits [B+1, N, V], no
        shift (:79-102)."""
        return self.model_executor.forward(batched_input, past_key_values=past_key_values,
                                           use_cache=False).logits

    # -- drafts -----------------------------------------------------------------------
    @torch.no_grad()
    def get_draft_blocks(self, x_block: torch.Tensor, logits_block: torch.Tensor,
                         mask_index: torch.Tensor, stats=None,
                         num_mask_positions: Optional[int] = None) -> List[Dict]:
        """One draft block per graph node over the whole block (:105-151): the
        pos_rank-th most confident masked position gets its vocab_rank-th most
        likely token.  Indices stay on the device (no host sync per node).
        ``stats``: sf_logit_stats of the block's rows (their 1/Z and top tokens
        replace the fp32 softmax and the vocabulary topk).  ``num_mask_positions``:
        the masked count when the caller holds it on the host (no device read)."""
        nodes = self._graph_nodes()
        if not nodes:
            return []
        if num_mask_positions is None:
            num_mask_positions = int(mask_index.sum().item())
        if num_mask_positions == 0:
            return []
        if stats is not None:
            confidence = greedy.max_prob_fp32(stats)
        else:
            confidence = torch.softmax(logits_block.float(), dim=-1).max(dim=-1).values
        confidence = torch.where(~mask_index, float("-inf"), confidence)
        if stats is not None:
            live = [n for n in nodes if max(pr for pr, _ in n["ij_set"]) < num_mask_positions]
            if not live:
                return []
            states = greedy.draft_states(x_block, confidence, stats, [n["ij_set"] for n in live])
            if states is not None:
                return [{"state": states[i], "node": n} for i, n in enumerate(live)]
        drafts: List[Dict] = []
        for node in nodes:
            ij_set = node["ij_set"]
            max_pos_rank = max(pr for pr, _ in ij_set)
            if max_pos_rank >= num_mask_positions:
                continue
            _, top_positions = torch.topk(confidence, k=max_pos_rank + 1)
            draft = x_block.clone()
            for pos_rank, vocab_rank in ij_set:
                pos = top_positions[pos_rank:pos_rank + 1]
                tok = greedy.vocab_rank(stats, pos, vocab_rank) if stats is not None else None
                if tok is None:
                    row = logits_block.index_select(0, pos)[0]
                    tok = torch.topk(row, k=vocab_rank + 1).indices[vocab_rank:vocab_rank + 1]
                draft.index_put_((pos,), tok)
            drafts.append({"state": draft, "node": node})
        return drafts

    def _next_ar_token(self, last_logit: torch.Tensor) -> torch.Tensor:
        """Next token [B, 1] of the autoregressive fallback: the argmax at
        temperature 0, else one draw from softmax(logits / T) (nld_generation.py:
        321-326)."""
        if self.temperature <= 0:
            return last_logit.argmax(dim=-1, keepdim=True)
        return torch.multinomial(torch.softmax(last_logit / self.temperature, dim=-1), 1)

    # -- the decode loop ----------------------------------------------------------------
    def _loop_facts(self, x_accum: torch.Tensor, block_slice: slice, called,
                    transfer=None) -> Dict:
        """What the loop's control flow reads from the token state, in one
        device-to-host copy: the block's masked count (per row and in total), the
        first cached draft state equal to the block (the draft-logit cache hit), and
        after a step its committed count and whether an EOS with no mask before it
        ends the block (:226-296).  The reference reads each with its own sync."""
        blk = x_accum[:, block_slice]
        masked = blk == self.mask_id
        parts = [masked.sum(dim=1)]
        if called:
            eq = torch.stack([st for st, _ in called]).eq(blk[0]).all(dim=1)
            parts.append(torch.where(eq.any(), eq.int().argmax(), -1).reshape(1))
        if transfer is not None:
            parts.append(transfer.sum().reshape(1))
            if self.stop_token is not None:
                eos = blk == self.stop_token
                before = masked & ~eos.cumsum(dim=1).bool()
                parts.append((eos.any() & (eos.any(dim=1) & ~before.any(dim=1)).any()).reshape(1))
        v = torch.cat([t.to(torch.long) for t in parts]).tolist()
        B = blk.shape[0]
        out = {"masked_rows": v[:B], "block_masks": sum(v[:B])}
        k = B
        out["hit"] = v[k] if called else -1
        k += 1 if called else 0
        out["n"] = v[k] if transfer is not None else None
        out["eos_break"] = bool(v[k + 1]) if (transfer is not None and
                                              self.stop_token is not None) else False
        return out

    @torch.no_grad()
    def decode_steps(self, prompt_ids: torch.Tensor, defer_forward: bool = False):
        """The decode loop of generate_with_draft_speculation (:153-316) as a
        generator: one event per iteration — {"kind": "prefill" | "verify" |
        "hit" | "commit", "committed": tokens unmasked by it}.  State on
        ``self._state``.

        The control flow is the reference's; its host reads (masked counts, cache
        hit, committed count, the EOS stop) come from one ``_loop_facts`` copy per
        iteration, taken after the iteration's decisions.

        defer_forward: instead of calling ``_batched_block_forward`` the loop yields
        {"kind": "forward", "batched": [B1, N] tokens, "cache": prefix cache,
        "committed": 0} and continues with the logits [B1, N, V] passed back by
        ``send`` (a driver that batches several sequences' verify steps into one,
        specfold_amd.generate.lockstep)."""
        executor = self.model_executor
        mask_id, eos_id = self.mask_id, self.stop_token
        prompt_ids = prompt_ids.to(self.device)
        prompt_len = prompt_ids.shape[1]
        B = prompt_ids.shape[0]
        budget = min(self.max_new_tokens, self.max_length - prompt_len)
        num_blocks = budget // self.block_length
        st = self._state = dict(model_calls=0, drafts_computed=0, x_accum=prompt_ids.clone(),
                                prompt_len=prompt_len, cache=None)
        if num_blocks <= 0:
            logger.warning("Prompt length %d leaves no room to generate (max_length=%d)",
                           prompt_len, self.max_length)
            return

        if self.causal_context:
            executor.set_diffusion_lm(False)
        output = executor.forward(prompt_ids, use_cache=True, use_causal_mask=self.causal_context)
        past_key_values = output.past_key_values
        st["cache"] = past_key_values
        st["model_calls"] += 1
        if self.causal_context:
            executor.set_diffusion_lm(True)
        next_token = None
        if self.causal_context:
            next_token = self._next_ar_token(output.logits[:, -1, :])
        yield {"kind": "prefill", "committed": 0}

        steps_per_block = self.block_length
        x_accum = st["x_accum"]
        for num_block in range(num_blocks):
            mask_block = torch.full((B, self.block_length), mask_id, dtype=prompt_ids.dtype,
                                    device=self.device)
            if self.causal_context:
                mask_block[:, 0] = next_token[:, 0]
            x_accum = torch.cat([x_accum, mask_block], dim=1)
            st["x_accum"] = x_accum
            block_start = prompt_len + num_block * self.block_length
            block_slice = slice(block_start, block_start + self.block_length)
            mask_block_idx0 = x_accum[:, block_slice] == mask_id
            num_transfer_tokens = get_num_transfer_tokens(mask_block_idx0, steps_per_block)
            draft_blocks: List[Dict] = []
            called: List[Tuple[torch.Tensor, torch.Tensor]] = []
            facts = self._loop_facts(x_accum, block_slice, called)

            for i in range(steps_per_block):
                if facts["block_masks"] == 0:
                    break
                mask_block_idx = x_accum[:, block_slice] == mask_id
                hit = facts["hit"] if called else -1
                stats = None
                if hit >= 0:
                    _, logits_block = called.pop(hit)
                    kind = "hit"
                else:
                    main_block = x_accum[:, block_slice]
                    if draft_blocks:
                        states = torch.stack([d["state"] for d in draft_blocks], dim=0)
                        batched = torch.cat([main_block, states], dim=0)
                    else:
                        batched = main_block
                    if defer_forward:
                        logits_all = yield {"kind": "forward", "batched": batched,
                                            "cache": past_key_values, "committed": 0}
                        if logits_all is None:
                            raise RuntimeError("a deferred forward needs its logits via send()")
                    else:
                        logits_all = self._batched_block_forward(batched, past_key_values)
                    st["model_calls"] += 1
                    logits_block = logits_all[0:1]
                    for k, d in enumerate(draft_blocks):
                        called.append((d["state"], logits_all[k + 1:k + 2]))
                    if B == 1 and greedy.usable(logits_block, self.temperature):
                        stats = greedy.stats(logits_block[0])
                    if self._graph_nodes():
                        draft_blocks = self.get_draft_blocks(x_accum[0, block_slice],
                                                             logits_block[0], mask_block_idx[0],
                                                             stats=stats,
                                                             num_mask_positions=facts["masked_rows"][0])
                        st["drafts_computed"] += len(draft_blocks)
                    kind = "verify"
                if stats is None and B == 1 and greedy.usable(logits_block, self.temperature):
                    stats = greedy.stats(logits_block[0])
                # with a threshold every masked position is a candidate: the counts
                # are the rows' masked counts, already on the host
                ks = facts["masked_rows"] if self.threshold is not None else None
                if stats is not None:
                    x0, transfer = greedy_transfer_index(
                        stats, mask_block_idx, x_accum[:, block_slice],
                        num_transfer_tokens[:, i], threshold=self.threshold, ks=ks)
                else:
                    x0, transfer = get_transfer_index(
                        logits_block, self.temperature, mask_block_idx, x_accum[:, block_slice],
                        num_transfer_tokens=num_transfer_tokens[:, i], threshold=self.threshold)
                cur = x_accum[:, block_slice].clone()
                cur = torch.where(transfer, x0, cur)
                x_accum[:, block_slice] = cur
                facts = self._loop_facts(x_accum, block_slice, called, transfer)
                n = facts["n"]
                self.last_commits.append(n)
                yield {"kind": kind, "committed": n}
                if facts["eos_break"]:
                    break

            if self.causal_context:
                executor.set_diffusion_lm(False)
            output = executor.forward(x_accum[:, block_slice], past_key_values=past_key_values,
                                      use_cache=True, use_causal_mask=self.causal_context)
            past_key_values = output.past_key_values
            st["cache"] = past_key_values
            st["model_calls"] += 1
            if self.causal_context:
                executor.set_diffusion_lm(True)
                next_token = self._next_ar_token(output.logits[:, -1, :])
            yield {"kind": "commit", "committed": 0}
            if eos_id is not None and bool((x_accum[:, prompt_len:] == eos_id).any(dim=1).all()):
                break

    @torch.no_grad()
    def generate_with_draft_speculation(self, prompt: str = None, prompt_ids=None,
                                        max_model_calls: Optional[int] = None, **kwargs):
        """Diffusion-mode generation with draft speculation (:153-316).

        Returns (texts, tokens_generated, model_calls, drafts_computed)."""
        t0 = time.time()
        if prompt_ids is None:
            prompt_ids = self.tokenizer(prompt, return_tensors="pt").input_ids
        self.last_commits = []
        for _ in self.decode_steps(prompt_ids):
            if max_model_calls is not None and self._state["model_calls"] >= max_model_calls:
                break
        result = self._result()
        elapsed = time.time() - t0
        logger.info("Generated %d tokens in %.2fs (%.2f tok/s)", result[1], elapsed,
                    result[1] / max(elapsed, 1e-9))
        return result

    def _result(self):
        """(texts, tokens_generated, model_calls, drafts_computed) of the decode
        state on ``self._state``: the generated ids up to the first EOS, masks
        dropped (:300-316)."""
        st = self._state
        final_ids = st["x_accum"][0, st["prompt_len"]:]
        eos_id = self.stop_token
        if eos_id is not None and bool((final_ids == eos_id).any()):
            stops = (final_ids == eos_id).nonzero()
            final_ids = final_ids[:int(stops[0]) + 1]
        kept = final_ids[final_ids != self.mask_id]
        text = self.tokenizer.batch_decode(kept.unsqueeze(0), skip_special_tokens=True)
        self.last_model_calls = st["model_calls"]
        return text, int(kept.numel()), st["model_calls"], st["drafts_computed"]
