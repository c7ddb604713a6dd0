"""Decode-loop pieces on the CPU: the draft construction (device-side indexing,
no host syncs) against a literal restatement of the reference loop
(specfold/generate/fastdllm_v2_generation.py:387-474), which indexes with
Python integers."""

import torch

from specfold_amd.configs import SYNTHETIC_DRAFT_GRAPH
from specfold_amd.generate.fastdllm_model_executor import ByteTokenizer
from specfold_amd.generate.fastdllm_v2_generation import FastDLLMV2SpeculativeGeneration


class _Exec:
    device = torch.device("cpu")

    def get_tokenizer(self):
        return ByteTokenizer()


def literal_drafts(x, p, mask_index, s0, s1, graph):
    small_mask = mask_index[s0:s1]
    small_logits = p[s0:s1, :]
    n_masked = int(small_mask.sum())
    conf = torch.softmax(small_logits, dim=-1).max(dim=-1).values
    conf = torch.where(~small_mask, float("-inf"), conf)
    out = []
    for node in graph["selected_nodes"]:
        ij = node["ij_set"]
        top = max(pr for pr, _ in ij)
        if top >= n_masked:
            continue
        positions = torch.topk(conf, k=top + 1).indices
        block = x.clone()
        for pr, vr in ij:
            pos = int(positions[pr])
            tok = torch.topk(small_logits[pos], k=vr + 1).indices[vr]
            block[s0 + pos] = tok
        out.append(block)
    return out


def test_draft_blocks_match_literal_loop():
    gen = FastDLLMV2SpeculativeGeneration(block_length=32, model_executor=_Exec(),
                                          calibration_graph=SYNTHETIC_DRAFT_GRAPH, device="cpu")
    g = torch.Generator().manual_seed(0)
    V = 500
    for trial in range(12):
        x = torch.randint(0, V, (32,), generator=g)
        p = torch.randn(32, V, generator=g).to(torch.bfloat16)
        mask = torch.rand(32, generator=g) < 0.6
        s0 = 8 * (trial % 4)
        x[s0:s0 + 8][mask[s0:s0 + 8]] = 151665
        got = gen.get_draft_blocks(x, p, mask, small_block_start=s0, small_block_end=s0 + 8)
        ref = literal_drafts(x, p, mask, s0, s0 + 8, SYNTHETIC_DRAFT_GRAPH)
        assert len(got) == len(ref)
        for d, r in zip(got, ref):
            assert torch.equal(d["state"], r)


def test_gumbel_noise_is_the_reference_expression():
    """Seeded Gumbel-max scores equal the reference's float64 expression
    exp(l) / (-log u)^T (modeling_nemotron_labs_diffusion.py:814-821) bit for
    bit, so a seeded draw transfers the same tokens, near ties included."""
    from specfold_amd.generate.nld_generation import add_gumbel_noise
    gen = torch.Generator().manual_seed(0)
    for seed, T in ((1, 1.0), (2, 0.7), (3, 0.3)):
        logits = torch.randn(4, 64, 257, generator=gen).to(torch.bfloat16)
        logits[0, 0, 3] = logits[0, 0, 5]                       # a tie
        torch.manual_seed(seed)
        got = add_gumbel_noise(logits, T)
        torch.manual_seed(seed)
        lg = logits.to(torch.float64)
        ref = lg.exp() / (-torch.log(torch.rand_like(lg, dtype=torch.float64))) ** T
        assert torch.equal(got, ref)
        assert torch.equal(got.argmax(-1), ref.argmax(-1))
    assert add_gumbel_noise(logits, 0) is logits
