"""Model executor with the API of the reference's FastDLLMModelExecutor
(specfold/generate/fastdllm_model_executor.py:8-167), over a Qwen2-layout
module tree that lives on the GPU.

Every forward runs through the HIP verify engine: a block forward is the
verify step with every row recomputed (gate mode SF_GATE_ALL), and
``update_past_key_values=True`` processes the input in ``block_length``
blocks, each attending to the cached prefix and bidirectionally within
itself, appending each block's K/V to the paged cache in place — the
block-diffusion prefill/commit of Fast-dLLM v2 (fastdllm_v2_generation.py:
510-524, 557-575).  The reference reaches that through HF remote code that is
not available offline; this restates its contract.
"""

from __future__ import annotations

from types import SimpleNamespace
from typing import Optional, Tuple

import torch

from specfold_amd import _lib
from specfold_amd.engine import FoldedVerifyEngine
from specfold_amd.kv_cache import PagedKVCache


class ByteTokenizer:
    """Minimal tokenizer for synthetic prompts: UTF-8 bytes <-> ids 0..255."""

    eos_token = "</s>"
    pad_token = None

    def __call__(self, text, return_tensors="pt"):
        ids = torch.tensor([list(text.encode("utf-8"))], dtype=torch.long)
        return SimpleNamespace(input_ids=ids)

    def batch_decode(self, ids, skip_special_tokens=True):
        out = []
        for row in ids:
            bs = bytes(int(t) for t in row.tolist() if 0 <= int(t) < 256)
            out.append(bs.decode("utf-8", errors="replace"))
        return out

    def apply_chat_template(self, chat, tokenize=False, add_generation_prompt=True):
        return "".join(m["content"] for m in chat)


class FastDLLMModelExecutor:
    MASK_ID = 151665
    STOP_TOKEN = 151645

    def __init__(self, model, device=None, target_dtype=torch.bfloat16, tokenizer=None,
                 block_length: int = 32, max_length: int = 4096, page_size: int = 16,
                 page_order: str = "sequential", page_seed: int = 0):
        self.model = model
        self.device = torch.device(device) if device is not None else \
            model.model.embed_tokens.weight.device
        self.target_dtype = target_dtype
        self.tokenizer = tokenizer if tokenizer is not None else ByteTokenizer()
        self.block_length = block_length
        self.max_length = max_length
        self.page_size = page_size
        self.page_order = page_order
        self.page_seed = page_seed
        self.engine = FoldedVerifyEngine(model)

    @classmethod
    def synthetic(cls, shape, seed: int, device="cuda", **kw):
        from specfold_amd.generate.synthetic_model import build_qwen2
        model = build_qwen2(shape, seed, device=device, dtype=torch.bfloat16)
        return cls(model, device=device, **kw)

    def new_cache(self, capacity: Optional[int] = None) -> PagedKVCache:
        cfg = self.model.config
        return PagedKVCache(len(self.model.model.layers), cfg.num_key_value_heads,
                            self.model.model.layers[0].self_attn.head_dim,
                            capacity or self.max_length, page_size=self.page_size,
                            device=self.device, page_order=self.page_order, seed=self.page_seed)

    def forward(self, input_seq: torch.Tensor, past_key_values=None, use_cache: bool = True,
                update_past_key_values: bool = False, use_block_cache: bool = False,
                block_past_key_values=None, replace_position: Optional[int] = None):
        """Block forward -> object with .logits [B, L, V] and .past_key_values."""
        if use_block_cache or block_past_key_values is not None or replace_position is not None:
            raise NotImplementedError("block-level KV caching is not part of the verify path")
        input_seq = input_seq.to(self.device)
        eng = self.engine
        if update_past_key_values:
            if input_seq.shape[0] != 1:
                raise ValueError("cache updates take one sequence")
            cache = past_key_values if past_key_values is not None else self.new_cache()
            if not isinstance(cache, PagedKVCache):
                raise TypeError("update_past_key_values needs a PagedKVCache")
            L = input_seq.shape[1]
            bl = self.block_length
            logits = []
            for s in range(0, L, bl):
                blk = input_seq[:, s:s + bl]
                prev_mode, eng.gate_mode = eng.gate_mode, _lib.SF_GATE_ALL
                try:
                    logits.append(eng.forward(blk, cache, delta=0.0, append=True))
                finally:
                    eng.gate_mode = prev_mode
            return SimpleNamespace(logits=torch.cat(logits, dim=1), past_key_values=cache)
        prev_mode, eng.gate_mode = eng.gate_mode, _lib.SF_GATE_ALL
        try:
            logits = eng.forward(input_seq, past_key_values, delta=0.0)
        finally:
            eng.gate_mode = prev_mode
        return SimpleNamespace(logits=logits, past_key_values=past_key_values)

    def forward_shifted(self, input_seq: torch.Tensor, past_key_values=None,
                        head_rows=None) -> torch.Tensor:
        """Dense block forward -> Fast-dLLM's shifted logits [B, L, V] (the
        generator's _shift_logits of ``forward(...).logits``, fastdllm_v2_generation.py:
        121-126, 151-186), shifted by the head kernel's stores instead of a copy.
        ``head_rows`` = (lo, n): only those positions get logits (the engine's)."""
        eng = self.engine
        prev_mode, eng.gate_mode = eng.gate_mode, _lib.SF_GATE_ALL
        try:
            return eng.forward(input_seq.to(self.device), past_key_values, delta=0.0, shift=True,
                               head_rows=head_rows)
        finally:
            eng.gate_mode = prev_mode

    @staticmethod
    def _top_p(logits: torch.Tensor, top_p: float, temperature: float):
        """Top-p filtered sampling (reference fallback, fastdllm_model_executor.py:129-155)."""
        if temperature > 0:
            logits = logits / temperature
        sorted_logits, sorted_idx = torch.sort(logits, descending=True, dim=-1)
        cum = torch.cumsum(torch.softmax(sorted_logits, dim=-1), dim=-1)
        drop_sorted = cum > top_p
        drop_sorted[..., 1:] = drop_sorted[..., :-1].clone()
        drop_sorted[..., 0] = False
        drop = drop_sorted.scatter(-1, sorted_idx, drop_sorted)
        probs = torch.softmax(logits.masked_fill(drop, float("-inf")), dim=-1)
        if temperature > 0:
            tok = torch.multinomial(probs.view(-1, probs.size(-1)), num_samples=1)
            tok = tok.view(probs.shape[:-1])
        else:
            tok = torch.argmax(probs, dim=-1)
        return tok, probs

    def sample_with_top_p(self, logits: torch.Tensor, top_p: float = 0.95,
                          temperature: float = 0.0) -> Tuple[torch.Tensor, torch.Tensor]:
        """Top-p filtered sampling, eager: replaying torch's sort / scan kernels of
        this sequence from a captured HIP graph faulted the GPU, so it stays out of
        graphs."""
        return self._top_p(logits, top_p, temperature)

    def get_tokenizer(self):
        return self.tokenizer

    def get_eos_token_id(self):
        return self.STOP_TOKEN

    def get_mask_id(self):
        return self.MASK_ID
