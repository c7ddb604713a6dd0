"""Pins of the oracle by things other than itself (CPU only).

* dense_layer == transformers' Qwen2DecoderLayer (eager, no mask, prefix in a
  DynamicCache), in fp32: an independent implementation of RMSNorm, QKV+bias,
  rotate_half RoPE, GQA attention over [prefix; block], o_proj and SwiGLU.
* delta < 0 (every row recomputed) makes the folded step equal the dense one
  (the reference's docstring claim, fastdllm_v2_folded.py:5-6).
* every folded row's (m, Z, O) equals exact fp64 softmax attention of its
  inherited query over its branch's keys [prefix; branch table] — the chain
  correction is exact, whatever the fold pattern (m is compared as the
  log-sum-exp m + log Z, since a folded row's m may be an upper bound).
"""

import pytest
import torch

from oracle.folded_reference import (StepTrace, dense_layer, dense_verify_step,
                                     exact_branch_attention, expand_kv_heads, folded_verify_step,
                                     rope_tables)
from specfold_amd.generate.synthetic_model import ModelShape, build_qwen2
from specfold_amd.synthetic import draft_tree_block, random_prefix_kv

SHAPE = ModelShape(hidden=64, heads=4, kv_heads=2, layers=2, intermediate=96, vocab=80,
                   head_dim=16)


def test_dense_layer_matches_hf_qwen2_layer():
    from transformers.cache_utils import DynamicCache
    model = build_qwen2(SHAPE, 3, dtype=torch.float32)
    gen = torch.Generator().manual_seed(1)
    P, N = 10, 8
    x = torch.randn(2, N, SHAPE.hidden, generator=gen)
    kv = random_prefix_kv(1, SHAPE.kv_heads, P, SHAPE.head_dim, gen, dtype=torch.float32)[0]
    lyr = model.model.layers[0]
    cos, sin = rope_tables(model, x, P, N)
    ours = dense_layer(lyr, x, kv, cos, sin, SHAPE.heads, SHAPE.kv_heads)
    cache = DynamicCache()
    cache.update(kv[0].expand(2, -1, -1, -1).contiguous(), kv[1].expand(2, -1, -1, -1).contiguous(), 0)
    pos = torch.arange(P, P + N).unsqueeze(0).expand(2, -1)
    with torch.no_grad():
        hf = lyr(x, attention_mask=None, position_ids=pos, past_key_values=cache,
                 position_embeddings=(cos[None].expand(2, -1, -1), sin[None].expand(2, -1, -1)))
    hf = hf[0] if isinstance(hf, tuple) else hf
    assert torch.allclose(ours, hf, atol=2e-5, rtol=2e-5), (ours - hf).abs().max()


@pytest.mark.parametrize("P", [0, 12])
def test_folded_with_gate_off_equals_dense(P):
    model = build_qwen2(SHAPE, 4, dtype=torch.float32)
    gen = torch.Generator().manual_seed(2)
    tokens = draft_tree_block(16, SHAPE.vocab, gen)
    kv = random_prefix_kv(SHAPE.layers, SHAPE.kv_heads, P, SHAPE.head_dim, gen,
                          dtype=torch.float32) if P else None
    folded = folded_verify_step(model, tokens, kv, delta=-1.0)
    dense = dense_verify_step(model, tokens, kv)
    assert torch.allclose(folded, dense, atol=1e-5, rtol=1e-5), (folded - dense).abs().max()


@pytest.mark.parametrize("delta", [0.02, 0.1, 0.5])
def test_folded_state_is_exact_attention(delta):
    model = build_qwen2(SHAPE, 5, dtype=torch.float32)
    gen = torch.Generator().manual_seed(3)
    P, N = 9, 16
    tokens = draft_tree_block(N, SHAPE.vocab, gen)
    kv = random_prefix_kv(SHAPE.layers, SHAPE.kv_heads, P, SHAPE.head_dim, gen,
                          dtype=torch.float32)
    tr = StepTrace()
    folded_verify_step(model, tokens, kv, delta=delta, trace=tr)
    G = SHAPE.heads // SHAPE.kv_heads
    scaling = model.model.layers[0].self_attn.scaling
    n_folded = 0
    for li, lt in enumerate(tr.layers):
        pk = expand_kv_heads(kv[li][0], G)[0]
        pv = expand_kv_heads(kv[li][1], G)[0]
        for b in range(tokens.shape[0]):
            keys = torch.cat([pk, expand_kv_heads(lt.k[b:b + 1], G)[0]], dim=1)
            vals = torch.cat([pv, expand_kv_heads(lt.v[b:b + 1], G)[0]], dim=1)
            m, z, o = exact_branch_attention(lt.q[b], keys, vals, scaling)
            # a folded row keeps max(m_parent, new scores): an upper bound of its
            # row max when a removed key held the max, so (m, Z) is compared
            # through the log-sum-exp it encodes, m + log Z
            lse = lt.m[b].double() + torch.log(lt.Z[b].double())
            assert torch.all(lt.m[b].double() >= m - 1e-6)
            assert torch.allclose(lse, m + torch.log(z), atol=1e-5, rtol=1e-5)
            assert torch.allclose(lt.O[b].double(), o, atol=1e-5, rtol=1e-4)
            n_folded += int((~lt.rec[b]).sum())
    assert n_folded > 0
