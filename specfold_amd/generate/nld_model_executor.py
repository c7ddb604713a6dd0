"""Model executor with the API of the reference's NLDModelExecutor
(specfold/generate/nld_model_executor.py:12-74), over a Nemotron-Labs-Diffusion
layout module tree (``encoder``, ``diffusion_head``, ``mask_token_id``) on the GPU.

Every forward runs through the HIP verify engine with every row recomputed
(gate mode SF_GATE_ALL):

* ``use_cache=True`` (the prompt prefill and the post-block refresh of
  nld_generation.py:186-194, 298-310) processes the input in ``block_length``
  blocks, each attending to the cached prefix and — with ``use_causal_mask`` —
  causally within itself (AR mode), appending its K/V to the paged cache in
  place.  A causal pass over blocks equals a causal pass over the whole input.
* ``use_cache=False`` (the diffusion forward of the dense seam, :79-102) runs the
  B rows bidirectionally within the block over the prefix, without touching
  the cache.

The llama-4 q scale (modeling_ministral.py:104-106, 148-152) is applied per
position.  The reference reaches this through its vendored modeling code,
which does not import under the installed transformers; this restates its
contract.
"""

from __future__ import annotations

from types import SimpleNamespace
from typing import Optional

import torch

from specfold_amd import _lib
from specfold_amd.engine import FoldedVerifyEngine
from specfold_amd.generate.fastdllm_model_executor import ByteTokenizer
from specfold_amd.kv_cache import PagedKVCache, cache_length


def llama4_q_scale(config, P: int, N: int, device=None) -> Optional[torch.Tensor]:
    """fp32 [N] scale 1 + beta * log(1 + floor(pos / omax)) for positions [P, P+N),
    or None when it is identically 1 (nld_folded.py:37-53)."""
    rp = getattr(config, "rope_parameters", None) or {}
    beta = rp.get("llama_4_scaling_beta")
    omax = rp.get("original_max_position_embeddings")
    if beta is None or omax is None:
        return None
    if device is None:
        return _q_scale_host(float(beta), omax, P, N)
    # a device copy per (prefix length, block): the verify steps of one block reuse
    # it instead of copying from pageable host memory (a synchronizing copy) each time
    key = (float(beta), omax, P, N, str(torch.device(device)))
    if key not in _Q_SCALE_DEV:
        scale = _q_scale_host(float(beta), omax, P, N)
        if len(_Q_SCALE_DEV) >= 64:
            _Q_SCALE_DEV.pop(next(iter(_Q_SCALE_DEV)))
        _Q_SCALE_DEV[key] = None if scale is None else scale.to(device)
    return _Q_SCALE_DEV[key]


_Q_SCALE_DEV: dict = {}


def _q_scale_host(beta: float, omax, P: int, N: int) -> Optional[torch.Tensor]:
    pos = torch.arange(P, P + N, dtype=torch.float32)
    scale = 1.0 + beta * torch.log(1.0 + torch.floor(pos / omax))
    if bool((scale == 1.0).all()):
        return None
    return scale


class NLDModelExecutor:
    """Handles a Nemotron-Labs-Diffusion-layout model's forward passes."""

    def __init__(self, model, device=None, target_dtype=torch.bfloat16, tokenizer=None,
                 block_length: int = 32, max_length: int = 4096, page_size: int = 16,
                 page_order: str = "sequential", page_seed: int = 0, eos_token_id: int = None):
        self.model = model
        self.device = torch.device(device) if device is not None else \
            model.encoder.embed_tokens.weight.device
        self.target_dtype = target_dtype
        self.tokenizer = tokenizer if tokenizer is not None else ByteTokenizer()
        self.block_length = block_length
        self.max_length = max_length
        self.page_size = page_size
        self.page_order = page_order
        self.page_seed = page_seed
        self.eos_token_id = eos_token_id
        self.diffusion_lm = True
        self.engine = FoldedVerifyEngine(model, gate_mode=_lib.SF_GATE_ALL)

    @classmethod
    def synthetic(cls, shape, seed: int, device="cuda", nld_kw: Optional[dict] = None, **kw):
        from specfold_amd.generate.synthetic_model import build_nld
        model = build_nld(shape, seed, device=device, dtype=torch.bfloat16, **(nld_kw or {}))
        return cls(model, device=device, **kw)

    def new_cache(self, capacity: Optional[int] = None) -> PagedKVCache:
        cfg = self.model.config
        return PagedKVCache(len(self.model.encoder.layers), cfg.num_key_value_heads,
                            self.model.encoder.layers[0].self_attn.head_dim,
                            capacity or self.max_length, page_size=self.page_size,
                            device=self.device, page_order=self.page_order, seed=self.page_seed)

    def set_diffusion_lm(self, enabled: bool):
        """Bidirectional (diffusion) vs causal (AR) attention (nld_model_executor.py:47-51)."""
        self.diffusion_lm = bool(enabled)

    def q_scale(self, P: int, N: int) -> Optional[torch.Tensor]:
        return llama4_q_scale(self.model.config, P, N, self.device)

    def forward(self, input_seq: torch.Tensor, past_key_values=None, use_cache: bool = False,
                use_causal_mask: bool = False):
        """One model forward -> object with .logits [B, L, V] and .past_key_values."""
        input_seq = input_seq.to(self.device)
        eng = self.engine
        causal = bool(use_causal_mask) and not self.diffusion_lm
        prev_mode, eng.gate_mode = eng.gate_mode, _lib.SF_GATE_ALL
        try:
            if use_cache:
                if input_seq.shape[0] != 1:
                    raise ValueError("cache updates take one sequence")
                cache = past_key_values if past_key_values is not None else self.new_cache()
                if not isinstance(cache, PagedKVCache):
                    raise TypeError("use_cache needs a PagedKVCache")
                L = input_seq.shape[1]
                logits = []
                for s in range(0, L, self.block_length):
                    blk = input_seq[:, s:s + self.block_length]
                    qs = self.q_scale(cache.length, blk.shape[1])
                    logits.append(eng.forward(blk, cache, delta=0.0, append=True, q_scale=qs,
                                              causal=causal))
                return SimpleNamespace(logits=torch.cat(logits, dim=1), past_key_values=cache)
            qs = self.q_scale(cache_length(past_key_values), input_seq.shape[1])
            logits = eng.forward(input_seq, past_key_values, delta=0.0, q_scale=qs, causal=causal)
            return SimpleNamespace(logits=logits, past_key_values=past_key_values)
        finally:
            eng.gate_mode = prev_mode

    def get_tokenizer(self):
        return self.tokenizer

    def get_eos_token_id(self) -> Optional[int]:
        return self.eos_token_id

    def get_mask_id(self) -> int:
        return self.model.mask_token_id
