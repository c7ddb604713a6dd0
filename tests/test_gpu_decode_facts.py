"""sf_decode_facts (the decode loop's small-block decision and loop facts in one
launch) against the loop's torch sequence (FastDLLMV2SpeculativeGeneration._decide
on a CPU token state runs the torch ops that restate
specfold/generate/fastdllm_v2_generation.py:660-700): the committed positions, the
written token state and every fact must be identical, over random states with
ties in the probabilities, probabilities at the threshold's bf16 neighbours, stop
tokens before and after masks, and cached draft states equal to the updated
block."""

import types

import pytest
import torch

from specfold_amd.generate.fastdllm_v2_generation import FastDLLMV2SpeculativeGeneration

pytestmark = pytest.mark.gpu

MASK, STOP = 151665, 151645


def decoder(device, bl=32, sbs=8, threshold=0.9):
    ex = types.SimpleNamespace(device=torch.device(device), get_tokenizer=lambda: None)
    return FastDLLMV2SpeculativeGeneration(bl, ex, small_block_size=sbs, threshold=threshold,
                                           mask_id=MASK, stop_token=STOP, device=device)


def case(g, bl, sbs):
    plen = 40 + int(torch.randint(0, 3 * bl, (1,), generator=g))
    fill = bl - plen % bl
    L = plen + fill
    x = torch.randint(0, 1000, (1, L), generator=g)
    blk = x[0, -bl:]
    u = torch.rand(bl, generator=g)
    blk[u < 0.55] = MASK
    blk[(u > 0.55) & (u < 0.6)] = STOP
    s0 = sbs * int(torch.randint(0, bl // sbs, (1,), generator=g))
    # probabilities with ties (a few levels) and the threshold's bf16 neighbours
    levels = torch.tensor([0.0, 0.25, 0.5, 0.8984375, 0.90234375, 0.95, 1.0])
    conf = levels[torch.randint(0, len(levels), (1, sbs), generator=g)].to(torch.bfloat16)
    x_1 = torch.randint(0, 1000, (1, sbs), generator=g)
    x_1[0, torch.rand(sbs, generator=g) < 0.2] = STOP
    return x, plen, s0, conf, x_1


@pytest.mark.parametrize("bl,sbs", [(32, 8), (64, 16), (16, 16)])
def test_decide_matches_torch_sequence(bl, sbs):
    g = torch.Generator().manual_seed(bl * 7 + sbs)
    d_cpu, d_gpu = decoder("cpu", bl, sbs), decoder("cuda", bl, sbs)
    hits = 0
    for it in range(300):
        x, plen, s0, conf, x_1 = case(g, bl, sbs)
        small_mask = (x[:, -bl:] == MASK)[:, s0:s0 + sbs]
        # the CPU reference first, so a cached state can equal its updated block
        x_ref = x.clone()
        un_ref, facts_ref = d_cpu._decide(x_ref, plen, [], s0, x_1, conf, small_mask)
        n_states = int(torch.randint(0, 8, (1,), generator=g))
        states = [torch.randint(0, 1000, (bl,), generator=g) for _ in range(n_states)]
        if n_states and it % 3 == 0:
            states[int(torch.randint(0, n_states, (1,), generator=g))] = x_ref[0, -bl:].clone()
        called = [(s, None) for s in states]
        x_ref = x.clone()
        un_ref, facts_ref = d_cpu._decide(x_ref, plen, called, s0, x_1, conf, small_mask)
        x_gpu = x.cuda()
        called_gpu = [(s.cuda(), None) for s in states]
        un, facts = d_gpu._decide(x_gpu, plen, called_gpu, s0, x_1.cuda(), conf.cuda(),
                                  small_mask.cuda())
        torch.cuda.synchronize()
        assert torch.equal(un.cpu(), un_ref), it
        assert torch.equal(x_gpu.cpu(), x_ref), it
        assert facts == facts_ref, (it, facts, facts_ref)
        hits += facts["hit"] >= 0
    assert hits > 0
