"""Random-init Qwen2-layout and NLD-layout models (the module trees the verify
step reads).

Fast-dLLM v2 checkpoints are Qwen2.5 models loaded through HF remote code
(specfold/generate/fastdllm_model_executor.py:34-41), which is not available
offline.  This builds ``transformers.Qwen2ForCausalLM`` with the same shapes
and layout (QKV bias, RMSNorm, rotate_half RoPE with theta from the config)
directly on the target device, with seeded N(0, std) weights and unit RMSNorm
weights.  Parameters are drawn in ``named_parameters()`` order from one
generator, so a given (shape, seed, device) always yields the same model.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch


@dataclass(frozen=True)
class ModelShape:
    hidden: int
    heads: int
    kv_heads: int
    layers: int
    intermediate: int
    vocab: int
    head_dim: int = 128
    rope_theta: float = 1e6
    rms_eps: float = 1e-6
    qkv_bias: bool = True
    max_positions: int = 32768


def qwen2_config(shape: ModelShape):
    from transformers import Qwen2Config
    cfg = Qwen2Config(
        vocab_size=shape.vocab, hidden_size=shape.hidden, intermediate_size=shape.intermediate,
        num_hidden_layers=shape.layers, num_attention_heads=shape.heads,
        num_key_value_heads=shape.kv_heads, max_position_embeddings=shape.max_positions,
        rms_norm_eps=shape.rms_eps,
        rope_parameters={"rope_type": "default", "rope_theta": float(shape.rope_theta)},
        tie_word_embeddings=False)
    cfg._attn_implementation = "eager"
    if shape.hidden // shape.heads != shape.head_dim:
        cfg.head_dim = shape.head_dim
    return cfg


@torch.no_grad()
def build_qwen2(shape: ModelShape, seed: int, device="cpu", dtype=torch.bfloat16,
                std: float = 0.02):
    """Qwen2ForCausalLM with seeded weights, materialised on ``device``."""
    from transformers import Qwen2ForCausalLM
    cfg = qwen2_config(shape)
    with torch.device("meta"):
        model = Qwen2ForCausalLM(cfg)
    model = model.to_empty(device=device)
    gen = torch.Generator(device=device).manual_seed(int(seed))
    for name, p in model.named_parameters():
        if name.endswith("norm.weight") or "layernorm" in name:
            p.data.fill_(1.0)
        elif name.endswith(".bias") and not shape.qkv_bias:
            p.data.zero_()
        else:
            p.data.normal_(0.0, std, generator=gen)
    model = model.to(dtype)
    rot = model.model.rotary_emb
    inv_freq, scaling = rot.compute_default_rope_parameters(cfg, device)
    rot.inv_freq = inv_freq.to(device=device, dtype=torch.float32)
    rot.original_inv_freq = rot.inv_freq.clone()
    rot.attention_scaling = scaling
    model.eval()
    model.requires_grad_(False)
    return model


# ---------------------------------------------------------------------------
# Nemotron-Labs-Diffusion layout
# ---------------------------------------------------------------------------

def nld_config(shape: ModelShape, rope_factor: float = 16.0, original_max_positions: int = 16384,
               llama4_beta: float = 0.1):
    """Llama-layout config with the NLD (Ministral3) defaults the verify step depends
    on: no projection bias, RMSNorm eps 1e-5, YaRN RoPE (factor 16 over 16384
    positions) and the llama-4 attention-scale parameters
    (specfold/model_cache/nemotron_labs_diffusion/configuration_nemotron_labs_diffusion.py:
    54-64, modeling_ministral.py:104-106, 148-152)."""
    from transformers import LlamaConfig
    rp = {"rope_type": "yarn", "rope_theta": float(shape.rope_theta), "factor": float(rope_factor),
          "original_max_position_embeddings": int(original_max_positions),
          "llama_4_scaling_beta": float(llama4_beta)}
    cfg = LlamaConfig(
        vocab_size=shape.vocab, hidden_size=shape.hidden, intermediate_size=shape.intermediate,
        num_hidden_layers=shape.layers, num_attention_heads=shape.heads,
        num_key_value_heads=shape.kv_heads, head_dim=shape.head_dim,
        max_position_embeddings=int(rope_factor * original_max_positions),
        rms_norm_eps=shape.rms_eps, rope_parameters=rp, attention_bias=False, mlp_bias=False,
        tie_word_embeddings=False)
    cfg._attn_implementation = "eager"
    return cfg


@torch.no_grad()
def build_nld(shape: ModelShape, seed: int, device="cpu", dtype=torch.bfloat16,
              std: float = 0.02, mask_token_id: int = None, **cfg_kw):
    """A Llama-layout module tree with the NLD attribute names the folded step
    reads (``encoder``, ``diffusion_head``, ``mask_token_id``; nld_folded.py:
    105-108, 237; nld_model_executor.py:74), seeded weights as build_qwen2."""
    from transformers import LlamaForCausalLM
    from transformers.modeling_rope_utils import ROPE_INIT_FUNCTIONS
    cfg = nld_config(shape, **cfg_kw)
    with torch.device("meta"):
        model = LlamaForCausalLM(cfg)
    model = model.to_empty(device=device)
    gen = torch.Generator(device=device).manual_seed(int(seed))
    for name, p in model.named_parameters():
        if name.endswith("norm.weight") or "layernorm" in name:
            p.data.fill_(1.0)
        else:
            p.data.normal_(0.0, std, generator=gen)
    model = model.to(dtype)
    rot = model.model.rotary_emb
    inv_freq, scaling = ROPE_INIT_FUNCTIONS["yarn"](cfg, device)
    rot.inv_freq = inv_freq.to(device=device, dtype=torch.float32)
    rot.original_inv_freq = rot.inv_freq.clone()
    rot.attention_scaling = scaling
    model.encoder = model.model
    model.diffusion_head = model.lm_head
    model.mask_token_id = shape.vocab - 1 if mask_token_id is None else int(mask_token_id)
    model.eval()
    model.requires_grad_(False)
    return model
