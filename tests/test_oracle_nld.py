"""Pins of the NLD (Nemotron-Labs-Diffusion) restatement by things other than
itself (CPU only).

* the llama-4 q scale against its closed form (identity below the original
  context, 1 + beta*ln(k+1) in the k-th window above it);
* ``dense_verify_step(causal=True, q_scale=...)`` against transformers' own
  Ministral3 (the NLD backbone: Llama layout, YaRN RoPE, llama-4 attention
  scale, causal attention) run over [prefix; block] with its KV cache — an
  independent implementation of every piece of the NLD layer, with non-unit
  norm weights so a dropped norm weight fails;
* delta < 0 (every row recomputed) makes the folded NLD step equal the dense one;
* the vectorised transfer schedule and threshold unmasking of the generator
  against the per-position loops of modeling_nemotron_labs_diffusion.py:824-861.
"""

import math

import pytest
import torch
import torch.nn.functional as F

from oracle.folded_reference import dense_verify_step, folded_verify_step, llama4_q_scale
from specfold_amd.generate.nld_generation import get_num_transfer_tokens, get_transfer_index
from specfold_amd.generate.nld_model_executor import llama4_q_scale as executor_q_scale
from specfold_amd.generate.synthetic_model import ModelShape, build_nld
from specfold_amd.synthetic import draft_tree_block, random_prefix_kv

SHAPE = ModelShape(hidden=64, heads=4, kv_heads=2, layers=2, intermediate=96, vocab=80,
                   head_dim=16, rms_eps=1e-5, qkv_bias=False)
OMAX = 8


def _model(seed, omax=OMAX):
    m = build_nld(SHAPE, seed, dtype=torch.float32, original_max_positions=omax, rope_factor=4.0)
    g = torch.Generator().manual_seed(seed + 7)
    with torch.no_grad():
        for name, p in m.named_parameters():
            if "norm" in name:
                p.copy_(1.0 + 0.2 * torch.randn(p.shape, generator=g))
    return m


def test_q_scale_closed_form():
    cfg = _model(1).config
    beta = cfg.rope_parameters["llama_4_scaling_beta"]
    assert llama4_q_scale(cfg, 0, OMAX) is None              # every position < omax
    s = llama4_q_scale(cfg, OMAX - 3, 8)
    want = [1.0] * 3 + [1.0 + beta * math.log(2.0)] * 5
    assert torch.allclose(s, torch.tensor(want), rtol=0, atol=1e-7)
    s = llama4_q_scale(cfg, 3 * OMAX, 2)
    assert abs(float(s[0]) - (1.0 + beta * math.log(4.0))) < 1e-7
    # the product's host-side schedule is the same function
    for P, N in [(0, 8), (5, 8), (100, 32)]:
        a, b = llama4_q_scale(cfg, P, N), executor_q_scale(cfg, P, N)
        assert (a is None) == (b is None)
        if a is not None:
            assert torch.equal(a, b)


def _ministral3(model):
    from transformers import Ministral3Config, Ministral3ForCausalLM
    cfg = model.config
    mc = Ministral3Config(
        vocab_size=SHAPE.vocab, hidden_size=SHAPE.hidden, intermediate_size=SHAPE.intermediate,
        num_hidden_layers=SHAPE.layers, num_attention_heads=SHAPE.heads,
        num_key_value_heads=SHAPE.kv_heads, head_dim=SHAPE.head_dim,
        max_position_embeddings=cfg.max_position_embeddings, rms_norm_eps=SHAPE.rms_eps,
        rope_parameters=dict(cfg.rope_parameters), tie_word_embeddings=False,
        sliding_window=None)
    mc._attn_implementation = "eager"
    hf = Ministral3ForCausalLM(mc).float()
    sd = {k: v for k, v in model.state_dict().items()
          if not k.startswith(("encoder.", "diffusion_head."))}
    res = hf.load_state_dict(sd, strict=True)
    assert not res.missing_keys and not res.unexpected_keys
    assert hf.model.rotary_emb.rope_type == "yarn"
    return hf.eval()


@pytest.mark.parametrize("P", [4, 12, 30])
def test_causal_dense_matches_ministral3(P):
    model = _model(3)
    hf = _ministral3(model)
    N = 8
    g = torch.Generator().manual_seed(P)
    seq = torch.randint(0, SHAPE.vocab, (1, P + N), generator=g)
    with torch.no_grad():
        cache = hf(seq[:, :P], use_cache=True).past_key_values
        kv = [(cache.layers[i].keys.clone(), cache.layers[i].values.clone())
              for i in range(SHAPE.layers)]
        want = hf(seq[:, P:], past_key_values=cache, use_cache=True).logits
    qs = llama4_q_scale(model.config, P, N)
    assert qs is not None                                  # the q scale is exercised
    ours = dense_verify_step(model, seq[:, P:], kv, shift=False, causal=True, q_scale=qs)
    assert torch.allclose(ours, want, atol=1e-6, rtol=1e-5), (ours - want).abs().max()
    # dropping the q scale is visible at 100x this tolerance
    plain = dense_verify_step(model, seq[:, P:], kv, shift=False, causal=True)
    assert (plain - want).abs().max() > 1e-4


def test_bidirectional_block_differs_from_causal():
    """The diffusion forward attends to the whole block: it is not the causal one."""
    model = _model(4)
    g = torch.Generator().manual_seed(9)
    tokens = torch.randint(0, SHAPE.vocab, (1, 8), generator=g)
    kv = random_prefix_kv(SHAPE.layers, SHAPE.kv_heads, 10, SHAPE.head_dim, g,
                          dtype=torch.float32)
    qs = llama4_q_scale(model.config, 10, 8)
    a = dense_verify_step(model, tokens, kv, shift=False, q_scale=qs)
    b = dense_verify_step(model, tokens, kv, shift=False, q_scale=qs, causal=True)
    assert (a[:, 0] - b[:, 0]).abs().max() > 1e-4


@pytest.mark.parametrize("P", [0, 5, 20])
def test_nld_folded_with_gate_off_equals_dense(P):
    model = _model(5)
    g = torch.Generator().manual_seed(2 + P)
    tokens = draft_tree_block(16, SHAPE.vocab, g)
    kv = random_prefix_kv(SHAPE.layers, SHAPE.kv_heads, P, SHAPE.head_dim, g,
                          dtype=torch.float32) if P else None
    qs = llama4_q_scale(model.config, P, 16)
    folded = folded_verify_step(model, tokens, kv, delta=-1.0, shift=False, q_scale=qs)
    dense = dense_verify_step(model, tokens, kv, shift=False, q_scale=qs)
    assert torch.allclose(folded, dense, atol=1e-5, rtol=1e-5), (folded - dense).abs().max()


# -- transfer schedule -----------------------------------------------------------------

def _num_transfer_loop(mask_index, steps):
    """modeling_nemotron_labs_diffusion.py:824-832, per row."""
    mask_num = mask_index.sum(dim=1, keepdim=True)
    out = torch.zeros(mask_num.size(0), steps, dtype=torch.int64) + mask_num // steps
    rem = mask_num % steps
    for i in range(mask_num.size(0)):
        out[i, :int(rem[i])] += 1
    return out


def _transfer_loop(logits, mask_index, x, ntt, threshold):
    """modeling_nemotron_labs_diffusion.py:835-861 at temperature 0, per position."""
    x0 = torch.argmax(logits, dim=-1)
    p = F.softmax(logits, dim=-1)
    x0_p = torch.gather(p, -1, x0[..., None])[..., 0]
    x0 = torch.where(mask_index, x0, x)
    conf = torch.where(mask_index, x0_p, float("-inf"))
    out = torch.zeros_like(x0, dtype=torch.bool)
    if threshold is not None:
        ntt = mask_index.sum(dim=1, keepdim=True)
    for j in range(conf.shape[0]):
        k = int(ntt[j])
        _, sel = torch.topk(conf[j], k=k)
        out[j, sel] = True
        if threshold is not None:
            for kk in range(1, k):
                if conf[j, sel[kk]] < threshold:
                    out[j, sel[kk]] = False
    return x0, out


@pytest.mark.parametrize("steps", [1, 3, 32])
def test_num_transfer_tokens_matches_loop(steps):
    g = torch.Generator().manual_seed(steps)
    mask = torch.rand(5, 32, generator=g) < torch.linspace(0, 1, 5)[:, None]
    assert torch.equal(get_num_transfer_tokens(mask, steps), _num_transfer_loop(mask, steps))


@pytest.mark.parametrize("threshold", [None, 0.05, 0.5, 0.9])
def test_transfer_index_matches_loop(threshold):
    g = torch.Generator().manual_seed(11)
    for trial in range(6):
        logits = torch.randn(1, 32, 50, generator=g) * (0.5 + trial)
        mask = torch.rand(1, 32, generator=g) < 0.6
        mask[0, trial] = True
        x = torch.randint(0, 50, (1, 32), generator=g)
        ntt = _num_transfer_loop(mask, 4)[:, trial % 4]
        x0a, ta = get_transfer_index(logits, 0.0, mask, x, ntt, threshold=threshold)
        x0b, tb = _transfer_loop(logits, mask, x, ntt, threshold)
        assert torch.equal(x0a, x0b)
        assert torch.equal(ta, tb)
        assert bool((ta & ~mask).sum() == 0)               # only masked positions commit
        assert int(ta.sum()) >= 1                          # at least one per step
