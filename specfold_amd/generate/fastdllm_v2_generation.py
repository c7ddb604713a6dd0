"""Block-diffusion decode loop with draft speculation — the caller of the
verify-step seam ``_batched_block_forward``.

Mirrors ``FastDLLMV2SpeculativeGeneration`` of the reference
(specfold/generate/fastdllm_v2_generation.py:25-720): the same constructor
knobs, the same seam, the same draft construction from a calibration graph
(:387-474), the same unmasking rule (threshold plus the always-committed
argmax, :666-676) and the same draft-logit cache (:599-651).  The decisions
are integer logic on the logits; the forward passes go to the model executor
(dense) or, in the SpecFold subclass, to the HIP folded verify step.
"""

from __future__ import annotations

import logging
import time
from typing import Dict, List, Optional, Tuple

import torch

from specfold_amd import _lib
from specfold_amd.generate import greedy

logger = logging.getLogger(__name__)


class FastDLLMV2SpeculativeGeneration:
    MASK_ID = 151665
    STOP_TOKEN = 151645

    def __init__(self, block_length: int, model_executor, calibration_graph=None,
                 temperature: float = 0.0, top_p: float = 0.95, top_k: Optional[int] = None,
                 mask_id: int = 151665, stop_token: int = 151645, max_length: int = 4096,
                 max_new_tokens: int = 1024, small_block_size: int = 8, threshold: float = 0.9,
                 use_block_cache: bool = False, device: str = "cuda", dtype: str = "bfloat16",
                 prompt_render_mode: str = "preformatted_text", **kwargs):
        self.__dict__.update(kwargs)
        self.model_executor = model_executor
        self.device = getattr(model_executor, "device", torch.device(device))
        self.dtype = dtype
        self.target_dtype = {"bfloat16": torch.bfloat16, "float16": torch.float16}.get(
            dtype, torch.float32)
        self.block_length = block_length
        self.calibration_graph = calibration_graph
        self.temperature = temperature
        self.top_p = top_p
        self.top_k = top_k
        self.mask_id = mask_id
        self.stop_token = stop_token
        self.max_length = max_length
        self.max_new_tokens = max_new_tokens
        self.small_block_size = small_block_size
        self.threshold = threshold
        self.use_block_cache = use_block_cache
        self.prompt_render_mode = prompt_render_mode
        self.tokenizer = model_executor.get_tokenizer()
        # decode statistics of the last generate call
        self.last_model_calls = 0
        self.last_commits: List[int] = []
        # (lo, n): the positions of every branch whose logits the decode step reads,
        # set by the loop around each verify forward (None: every row); the verify
        # step's head computes only those rows
        self.head_rows = None

    # -- helpers with the reference's names ------------------------------------------
    def _shift_logits(self, logits: torch.Tensor) -> torch.Tensor:
        """Position i gets the logits of position i-1 (:121-126)."""
        return torch.cat([logits[:, :1, :], logits[:, :-1, :]], dim=1)

    @staticmethod
    def _kv_seq_length(past_key_values) -> int:
        return 0 if past_key_values is None else int(past_key_values.get_seq_length())

    def _sample_with_top_p(self, logits, top_p: float = 0.95, temperature: float = 0.0):
        return self.model_executor.sample_with_top_p(logits, top_p=top_p, temperature=temperature)

    def _sample_rows(self, logits: torch.Tensor):
        """Sampled tokens and their probabilities for logits [1, n, V] ->
        (x_1 [1, n], conf [1, n], statistics or None).  At temperature 0 on the GPU
        both come from one pass of sf_logit_stats (whose statistics the draft
        construction reuses); otherwise from the top-p sampler and a gather
        (:646-656)."""
        if greedy.usable(logits, self.temperature):
            st = greedy.stats(logits[0], self.top_p)
            x_1, conf = greedy.top_p_greedy(st)
            return x_1, conf, st
        x_1, p_1t = self._sample_with_top_p(logits, top_p=self.top_p,
                                            temperature=self.temperature)
        return x_1, torch.gather(p_1t, -1, x_1.unsqueeze(-1)).squeeze(-1), None

    def _prepare_prompt_text(self, prompt: str) -> str:
        if self.prompt_render_mode == "preformatted_text":
            if not isinstance(prompt, str):
                raise TypeError(f"Expected preformatted prompt text, got {type(prompt)}")
            return prompt
        if self.prompt_render_mode == "legacy_single_user_chat":
            return self.tokenizer.apply_chat_template([{"role": "user", "content": prompt}],
                                                      tokenize=False, add_generation_prompt=True)
        raise ValueError(f"Unsupported prompt_render_mode: {self.prompt_render_mode}")

    def _init_generation_state(self, prompt: str) -> Tuple[int, torch.Tensor]:
        ids = self.tokenizer(self._prepare_prompt_text(prompt), return_tensors="pt").input_ids
        ids = ids.to(self.device)
        return ids.shape[1], ids

    # -- the seam ---------------------------------------------------------------------
    def _batched_block_forward(self, batched_input: torch.Tensor, past_key_values) -> torch.Tensor:
        """Dense B+1-row block forward -> shifted logits [B+1, N, V] (:151-186); an
        executor with ``forward_shifted`` returns them shifted by its head's stores."""
        ex = self.model_executor
        if hasattr(ex, "forward_shifted"):
            return ex.forward_shifted(batched_input, past_key_values,
                                      head_rows=self.head_rows)
        out = ex.forward(batched_input, past_key_values=past_key_values,
                         use_cache=True, update_past_key_values=False)
        return self._shift_logits(out.logits)

    # -- drafts -----------------------------------------------------------------------
    @torch.no_grad()
    def get_draft_blocks(self, x: torch.Tensor, p: torch.Tensor,
                         mask_index: Optional[torch.Tensor] = None, start_pos=None, end_pos=None,
                         small_block_start: Optional[int] = None,
                         small_block_end: Optional[int] = None, stats=None,
                         n_masked: Optional[int] = None, **kwargs) -> List[Dict]:
        """One draft block per calibration-graph node (:387-474).

        Node ij_set = [(position rank, vocab rank), ...]: take the masked
        positions of the small block ranked by max softmax probability, and put
        the vocab_rank-th most likely token at the pos_rank-th position.
        ``stats``: sf_logit_stats of the small block's rows, when the caller has
        them (their maximum probabilities and top tokens replace the softmax and
        the vocabulary topk).  ``n_masked``: the small block's masked-position count
        when the caller already holds it on the host (no device read).
        """
        if self.calibration_graph is None:
            return []
        if small_block_start is not None and small_block_end is not None:
            small_mask = None if mask_index is None else mask_index[small_block_start:small_block_end]
            small_logits = p[small_block_start:small_block_end, :]
            offset = small_block_start
        else:
            small_mask, small_logits, offset = mask_index, p, 0
        if small_mask is None:
            return []
        if n_masked is None:
            n_masked = int(small_mask.sum().item())
        if n_masked == 0:
            return []
        active = []
        for node in self.calibration_graph.get("selected_nodes", []):
            ij_set = node.get("ij_set", [])
            if not ij_set:
                continue
            top_rank = max(pr for pr, _ in ij_set)
            if top_rank >= n_masked:
                continue
            active.append((node, tuple((int(pr), int(vr)) for pr, vr in ij_set), top_rank))
        if not active:
            return []
        # eager: torch.topk over a vocabulary row runs rocprim's radix sort, whose
        # look-back state is initialised by a memset; replayed from a captured HIP
        # graph it faulted the GPU, so the draft construction stays out of graphs
        states = self._draft_states(x, small_logits, small_mask, offset, active, stats)
        return [{"state": states[i], "start_pos": start_pos, "end_pos": end_pos, "node": node}
                for i, (node, _, _) in enumerate(active)]

    @staticmethod
    def _draft_states(x, small_logits, small_mask, offset, active, stats=None) -> torch.Tensor:
        """The draft blocks of the active nodes, stacked [n, N] (:430-470); device
        ops only (indices stay on the device), so no host sync per node."""
        if stats is not None:
            conf = greedy.max_prob_bf16(stats)
        else:
            conf = torch.softmax(small_logits, dim=-1).max(dim=-1).values
        conf = torch.where(~small_mask, float("-inf"), conf)
        if stats is not None:
            states = greedy.draft_states(x, conf, stats, [ij for _, ij, _ in active], offset)
            if states is not None:
                return states
        blocks = []
        for _, ij_set, top_rank in active:
            positions = torch.topk(conf, k=top_rank + 1).indices
            block = x.clone()
            for pos_rank, vocab_rank in ij_set:
                pos = positions[pos_rank:pos_rank + 1]
                tok = greedy.vocab_rank(stats, pos, vocab_rank) if stats is not None else None
                if tok is None:
                    row = small_logits.index_select(0, pos)[0]
                    tok = torch.topk(row, k=vocab_rank + 1).indices[vocab_rank:vocab_rank + 1]
                block.index_put_((pos + offset,), tok)
            blocks.append(block)
        return torch.stack(blocks)

    # -- the decode loop ----------------------------------------------------------------
    def _stop_reached(self, x_t: torch.Tensor, prompt_length: int) -> bool:
        tail = x_t[:, prompt_length:]
        hits = (tail == self.stop_token).nonzero()
        if hits.numel() == 0:
            return False
        first = int(hits[0][1])
        return int((tail[:, :first] == self.mask_id).sum()) == 0

    def _loop_facts(self, x_t: torch.Tensor, plen: int, called, unmask=None) -> Dict:
        """Everything the loop's control flow reads from the token state, in one
        device-to-host copy: whether the stop token ends the text (_stop_reached),
        the block's and each small block's masked positions, the first cached draft
        state equal to the current block (the draft-logit cache hit, :599-617) and
        the committed-position count of ``unmask``.  The reference reads each of
        these with its own host sync; here the decisions of a step, its draft
        construction and the next step's facts are enqueued behind the forward
        and read once."""
        bl, sbs = self.block_length, self.small_block_size
        blk = x_t[:, -bl:]
        masked = blk == self.mask_id
        tail = x_t[:, plen:]
        is_stop = tail == self.stop_token
        first = is_stop.int().argmax(dim=1, keepdim=True)      # 0 when there is none
        ahead = torch.arange(tail.shape[1], device=x_t.device).unsqueeze(0) < first
        before = ((tail == self.mask_id) & ahead).sum()
        parts = [(is_stop.any() & (before == 0)).reshape(1), masked.sum().reshape(1),
                 masked[0].view(-1, sbs).sum(dim=1)]
        if called:
            eq = torch.stack([st for st, _ in called]).eq(blk[0]).all(dim=1)
            parts.append(torch.where(eq.any(), eq.int().argmax(), -1).reshape(1))
        if unmask is not None:
            parts.append(unmask.sum().reshape(1))
        v = torch.cat([t.to(torch.long) for t in parts]).tolist()
        return self._facts_dict(v, bool(called), unmask is not None)

    def _facts_dict(self, v, has_called: bool, has_unmask: bool) -> Dict:
        n_small = self.block_length // self.small_block_size
        out = {"stop": bool(v[0]), "block_masks": v[1], "small": v[2:2 + n_small]}
        k = 2 + n_small
        out["hit"] = v[k] if has_called else -1
        k += 1 if has_called else 0
        out["n"] = v[k] if has_unmask else None
        return out

    def _decide(self, x_t: torch.Tensor, plen: int, called, s0: int, x_1: torch.Tensor,
                conf: torch.Tensor, small_mask: torch.Tensor):
        """The small block's unmask decision (:660-700: a masked position is committed
        when its probability passes the threshold or it is the most confident one),
        its write into x_t, and the loop facts after it -> (unmask [1, sbs] bool,
        facts).  On a GPU token state of one sequence with bf16 probabilities this is
        one sf_decode_facts launch; otherwise the torch sequence."""
        bl, sbs = self.block_length, self.small_block_size
        if (x_t.is_cuda and x_t.shape[0] == 1 and x_t.is_contiguous() and bl <= 64
                and conf.dtype == torch.bfloat16 and len(called) <= 16):
            buf = getattr(self, "_facts_buf", None)
            if buf is None or buf.device != x_t.device:
                buf = self._facts_buf = torch.empty(64 + 4, dtype=torch.int64, device=x_t.device)
                # torch compares a bf16 tensor with a float in bf16
                self._thr_bf16 = float(torch.tensor(self.threshold, dtype=torch.bfloat16))
            unmask8 = torch.empty(sbs, dtype=torch.int8, device=x_t.device)
            n = _lib.decode_facts(x_t, plen, bl, sbs, s0, self.mask_id, self.stop_token,
                                  conf.reshape(-1), x_1.reshape(-1).contiguous(), self._thr_bf16,
                                  [st for st, _ in called], unmask8, buf)
            facts = self._facts_dict(buf[:n].tolist(), bool(called), True)
            return unmask8.view(torch.bool).unsqueeze(0), facts
        conf = torch.where(small_mask, conf, -torch.inf)
        # the reference's unmask[arange, argmax] = True, as a compare with the argmax
        # column (an index_put_ of a host scalar syncs)
        best = conf.argmax(dim=-1, keepdim=True)
        cols = torch.arange(conf.shape[-1], device=self.device)
        unmask = ((conf > self.threshold) | (cols == best)) & small_mask
        region = x_t[:, x_t.shape[1] - bl + s0: x_t.shape[1] - bl + s0 + sbs]
        region.copy_(torch.where(unmask, x_1, region))
        return unmask, self._loop_facts(x_t, plen, called, unmask)

    @torch.no_grad()
    def decode_steps(self, prompt_ids: torch.Tensor, defer_forward: bool = False):
        """The decode loop of generate_with_draft_speculation (:483-700) as a
        generator: yields one event per loop iteration —
        {"kind": "prefill" | "commit" | "verify" | "hit", "committed": tokens
        unmasked by the iteration}.  Loop state is on ``self._state``.

        The control flow is the reference's; the host reads it needs (stop token,
        masked counts, cache hit, committed count) come from one ``_loop_facts``
        copy per iteration, taken after the iteration's decisions, so the host
        enqueues the sampling, the draft construction and the decisions while the
        forward runs.

        defer_forward: instead of calling ``_batched_block_forward`` the loop yields
        {"kind": "forward", "batched": [B1, N] tokens, "cache": prefix cache,
        "committed": 0} and continues with the shifted logits [B1, N, V] passed
        back by ``send`` (specfold_amd.generate.lockstep)."""
        input_ids = prompt_ids.to(self.device)
        orig_len = input_ids.shape[1]
        bl, sbs = self.block_length, self.small_block_size
        n_blocks = self.max_new_tokens // bl
        n_small = bl // sbs
        st = self._state = dict(cache=None, model_calls=0, drafts_computed=0, x_t=input_ids,
                                orig_len=orig_len)

        if input_ids.shape[1] > bl:
            pre = (input_ids.shape[1] // bl) * bl
            out = self.model_executor.forward(input_ids[:, :pre], past_key_values=None,
                                              use_cache=True, update_past_key_values=True)
            st["cache"] = out.past_key_values
            st["model_calls"] += 1
            if input_ids.shape[1] % bl == 0:
                input_ids = torch.cat([input_ids, out.logits[:, -1:, :].argmax(dim=-1)], dim=1)
            st["x_t"] = input_ids
            yield {"kind": "prefill", "committed": 0}

        x_t = input_ids
        draft_blocks: List[Dict] = []
        called: List[Tuple[torch.Tensor, torch.Tensor]] = []
        for _ in range(n_blocks):
            if bool((x_t[:, orig_len:] == self.stop_token).any()):
                break
            plen = x_t.shape[1]
            fill = bl - (plen % bl)
            x_t = torch.cat([x_t, torch.full((x_t.shape[0], fill), self.mask_id,
                                             device=self.device, dtype=torch.long)], dim=1)
            st["x_t"] = x_t
            facts = self._loop_facts(x_t, plen, called)
            while True:
                if facts["stop"]:
                    break
                if facts["block_masks"] == 0:
                    out = self.model_executor.forward(x_t[:, -bl:], past_key_values=st["cache"],
                                                      use_cache=True, update_past_key_values=True)
                    st["cache"] = out.past_key_values
                    st["model_calls"] += 1
                    x_t = torch.cat([x_t, out.logits[:, -1:, :].argmax(dim=-1)], dim=1)
                    st["x_t"] = x_t
                    draft_blocks, called = [], []
                    yield {"kind": "commit", "committed": 0}
                    break
                for sb in range(n_small):
                    s0, s1 = sb * sbs, sb * sbs + sbs
                    while True:
                        if facts["small"][sb] == 0 or facts["stop"]:
                            break
                        mask_idx = x_t[:, -bl:] == self.mask_id
                        small_mask = mask_idx[:, s0:s1]
                        hit = facts["hit"] if called else -1
                        if hit >= 0:
                            _, hit_logits = called.pop(hit)
                            x_1, conf, _ = self._sample_rows(hit_logits[:, s0:s1, :])
                            kind = "hit"
                        else:
                            main_block = x_t[:, -bl:]
                            if draft_blocks:
                                states = torch.stack([d["state"] for d in draft_blocks], dim=0)
                                batched = torch.cat([main_block, states], dim=0)
                            else:
                                batched = main_block
                            if defer_forward:
                                logits = yield {"kind": "forward", "batched": batched,
                                                "cache": st["cache"], "committed": 0}
                                if logits is None:
                                    raise RuntimeError(
                                        "a deferred forward needs its logits via send()")
                            else:
                                # the rows this forward's logits are read at: the small
                                # block (main branch, drafts) and the next one (a draft
                                # that fills this small block is taken at the next one's
                                # first step, :599-616); the head computes only those
                                self.head_rows = (s0, min(s1 + sbs, bl) - s0)
                                try:
                                    logits = self._batched_block_forward(batched, st["cache"])
                                finally:
                                    self.head_rows = None
                            st["model_calls"] += 1
                            main_logits = logits[0:1]
                            for i, d in enumerate(draft_blocks):
                                called.append((d["state"], logits[i + 1:i + 2]))
                            x_1, conf, stats = self._sample_rows(main_logits[:, s0:s1, :])
                            if self.calibration_graph is not None:
                                draft_blocks = self.get_draft_blocks(
                                    x_t[0, -bl:], main_logits[0], mask_idx[0],
                                    start_pos=x_t.shape[1] - bl, end_pos=x_t.shape[1],
                                    small_block_start=s0, small_block_end=s1, stats=stats,
                                    n_masked=facts["small"][sb])
                                st["drafts_computed"] += len(draft_blocks)
                            kind = "verify"
                        unmask, facts = self._decide(x_t, plen, called, s0, x_1, conf,
                                                     small_mask)
                        n = facts["n"]
                        self.last_commits.append(n)
                        # the decision itself rides along (device tensors, no sync):
                        # sampled tokens, maskable positions and the committed ones
                        yield {"kind": kind, "committed": n, "tokens": x_1,
                               "maskable": small_mask, "unmask": unmask}

    @torch.no_grad()
    def generate_with_draft_speculation(self, prompt: str = None, prompt_ids=None,
                                        max_model_calls: Optional[int] = None, **kwargs):
        """Decode with draft speculation (:483-720).

        Returns (text, tokens_generated, model_calls, drafts_computed).
        ``prompt_ids`` ([1, L] token ids) may replace the text prompt;
        ``max_model_calls`` stops early after that many forwards.
        """
        t0 = time.time()
        if prompt_ids is None:
            _, prompt_ids = self._init_generation_state(prompt)
        self.last_commits = []
        for _ in self.decode_steps(prompt_ids):
            if max_model_calls is not None and self._state["model_calls"] >= max_model_calls:
                break
        result = self._result()
        elapsed = time.time() - t0
        logger.info("Generated %d tokens in %.2fs (%.2f tok/s); model calls %d, drafts %d",
                    result[1], elapsed, result[1] / max(elapsed, 1e-9), result[2], result[3])
        return result

    def _result(self):
        """(text, tokens_generated, model_calls, drafts_computed) of the decode state
        on ``self._state``: the generated ids up to the first stop token, masks
        dropped (:700-720)."""
        st = self._state
        x_t = st["x_t"]
        final_ids = x_t[0, st["orig_len"]:]
        stops = (final_ids == self.stop_token).nonzero()
        if stops.numel() > 0:
            final_ids = final_ids[:int(stops[0]) + 1]
        kept = final_ids[final_ids != self.mask_id]
        text = self.tokenizer.batch_decode(kept.unsqueeze(0), skip_special_tokens=True)
        self.last_model_calls = st["model_calls"]
        self.last_cache = st["cache"]
        self.last_tokens = x_t
        return text, int(kept.numel()), st["model_calls"], st["drafts_computed"]
