"""The decode loops with the reference's host reads, as checkers.

``fastdllm_events(gen, prompt_ids)`` walks generate_with_draft_speculation's control
flow (specfold/generate/fastdllm_v2_generation.py:483-700), and ``nld_events`` NLD's
(specfold/generate/nld_generation.py:153-296), the way the reference does: each decision point reads its own value from the device (the stop-token
check, the block's and the small block's masked counts, the draft-cache hit, the
committed count), one host sync each.  It uses the generator's own sampling,
draft construction and forward, so comparing its event stream with
``gen.decode_steps`` checks only the loop's control flow, which the product
restructures around one host read per iteration.  Test infrastructure.
"""

from typing import Dict, List, Tuple

import torch


@torch.no_grad()
def fastdllm_events(gen, prompt_ids: torch.Tensor):
    input_ids = prompt_ids.to(gen.device)
    orig_len = input_ids.shape[1]
    bl, sbs = gen.block_length, gen.small_block_size
    n_blocks = gen.max_new_tokens // bl
    n_small = bl // sbs
    st = gen._state = dict(cache=None, model_calls=0, drafts_computed=0, x_t=input_ids,
                           orig_len=orig_len)
    if input_ids.shape[1] > bl:
        pre = (input_ids.shape[1] // bl) * bl
        out = gen.model_executor.forward(input_ids[:, :pre], past_key_values=None,
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
        if bool((x_t[:, orig_len:] == gen.stop_token).any()):
            break
        plen = x_t.shape[1]
        fill = bl - (plen % bl)
        x_t = torch.cat([x_t, torch.full((x_t.shape[0], fill), gen.mask_id,
                                         device=gen.device, dtype=torch.long)], dim=1)
        st["x_t"] = x_t
        while True:
            if gen._stop_reached(x_t, plen):
                break
            mask_idx = x_t[:, -bl:] == gen.mask_id
            if int(mask_idx.sum()) == 0:
                out = gen.model_executor.forward(x_t[:, -bl:], past_key_values=st["cache"],
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
                    mask_idx = x_t[:, -bl:] == gen.mask_id
                    small_mask = mask_idx[:, s0:s1]
                    if int(small_mask.sum()) == 0:
                        break
                    if gen._stop_reached(x_t, plen):
                        break
                    hit = -1
                    if called:
                        cur = x_t[0, -bl:]
                        eq = torch.stack([s for s, _ in called]).eq(cur).all(dim=1).tolist()
                        hit = eq.index(True) if True in eq else -1
                    if hit >= 0:
                        _, hit_logits = called.pop(hit)
                        x_1, conf, _ = gen._sample_rows(hit_logits[:, s0:s1, :])
                        kind = "hit"
                    else:
                        main_block = x_t[:, -bl:]
                        if draft_blocks:
                            states = torch.stack([d["state"] for d in draft_blocks], dim=0)
                            batched = torch.cat([main_block, states], dim=0)
                        else:
                            batched = main_block
                        logits = gen._batched_block_forward(batched, st["cache"])
                        st["model_calls"] += 1
                        main_logits = logits[0:1]
                        for i, d in enumerate(draft_blocks):
                            called.append((d["state"], logits[i + 1:i + 2]))
                        x_1, conf, stats = gen._sample_rows(main_logits[:, s0:s1, :])
                        if gen.calibration_graph is not None:
                            draft_blocks = gen.get_draft_blocks(
                                x_t[0, -bl:], main_logits[0], mask_idx[0],
                                start_pos=x_t.shape[1] - bl, end_pos=x_t.shape[1],
                                small_block_start=s0, small_block_end=s1, stats=stats)
                            st["drafts_computed"] += len(draft_blocks)
                        kind = "verify"
                    conf = torch.where(small_mask, conf, -torch.inf)
                    unmask = conf > gen.threshold
                    best = conf.argmax(dim=-1)
                    unmask[torch.arange(x_1.shape[0], device=gen.device), best] = True
                    unmask = unmask & small_mask
                    region = x_t[:, x_t.shape[1] - bl + s0: x_t.shape[1] - bl + s1]
                    region.copy_(torch.where(unmask, x_1, region))
                    n = int(unmask.sum())
                    yield {"kind": kind, "committed": n, "tokens": x_1,
                           "maskable": small_mask, "unmask": unmask}


@torch.no_grad()
def nld_events(gen, prompt_ids: torch.Tensor):
    """NLD's decode loop (specfold/generate/nld_generation.py:153-296) with its
    host reads at every decision point, on the generator's own helpers."""
    from specfold_amd.generate import greedy
    from specfold_amd.generate.nld_generation import (get_num_transfer_tokens,
                                                      get_transfer_index,
                                                      greedy_transfer_index)
    executor = gen.model_executor
    mask_id, eos_id = gen.mask_id, gen.stop_token
    prompt_ids = prompt_ids.to(gen.device)
    prompt_len = prompt_ids.shape[1]
    B = prompt_ids.shape[0]
    budget = min(gen.max_new_tokens, gen.max_length - prompt_len)
    num_blocks = budget // gen.block_length
    st = gen._state = dict(model_calls=0, drafts_computed=0, x_accum=prompt_ids.clone(),
                           prompt_len=prompt_len, cache=None)
    if num_blocks <= 0:
        return
    if gen.causal_context:
        executor.set_diffusion_lm(False)
    output = executor.forward(prompt_ids, use_cache=True, use_causal_mask=gen.causal_context)
    past_key_values = output.past_key_values
    st["cache"] = past_key_values
    st["model_calls"] += 1
    if gen.causal_context:
        executor.set_diffusion_lm(True)
    next_token = None
    if gen.causal_context:
        next_token = gen._next_ar_token(output.logits[:, -1, :])
    yield {"kind": "prefill", "committed": 0}
    steps_per_block = gen.block_length
    x_accum = st["x_accum"]
    for num_block in range(num_blocks):
        mask_block = torch.full((B, gen.block_length), mask_id, dtype=prompt_ids.dtype,
                                device=gen.device)
        if gen.causal_context:
            mask_block[:, 0] = next_token[:, 0]
        x_accum = torch.cat([x_accum, mask_block], dim=1)
        st["x_accum"] = x_accum
        block_start = prompt_len + num_block * gen.block_length
        block_slice = slice(block_start, block_start + gen.block_length)
        mask_block_idx0 = x_accum[:, block_slice] == mask_id
        num_transfer_tokens = get_num_transfer_tokens(mask_block_idx0, steps_per_block)
        draft_blocks = []
        called = []
        for i in range(steps_per_block):
            mask_block_idx = x_accum[:, block_slice] == mask_id
            if int(mask_block_idx.sum()) == 0:
                break
            hit = -1
            if called:
                cur = x_accum[0, block_slice]
                eq = torch.stack([s for s, _ in called]).eq(cur).all(dim=1).tolist()
                hit = eq.index(True) if True in eq else -1
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
                logits_all = gen._batched_block_forward(batched, past_key_values)
                st["model_calls"] += 1
                logits_block = logits_all[0:1]
                for k, d in enumerate(draft_blocks):
                    called.append((d["state"], logits_all[k + 1:k + 2]))
                if B == 1 and greedy.usable(logits_block, gen.temperature):
                    stats = greedy.stats(logits_block[0])
                if gen._graph_nodes():
                    draft_blocks = gen.get_draft_blocks(x_accum[0, block_slice], logits_block[0],
                                                        mask_block_idx[0], stats=stats)
                    st["drafts_computed"] += len(draft_blocks)
                kind = "verify"
            if stats is None and B == 1 and greedy.usable(logits_block, gen.temperature):
                stats = greedy.stats(logits_block[0])
            if stats is not None:
                x0, transfer = greedy_transfer_index(
                    stats, mask_block_idx, x_accum[:, block_slice], num_transfer_tokens[:, i],
                    threshold=gen.threshold)
            else:
                x0, transfer = get_transfer_index(
                    logits_block, gen.temperature, mask_block_idx, x_accum[:, block_slice],
                    num_transfer_tokens=num_transfer_tokens[:, i], threshold=gen.threshold)
            cur = x_accum[:, block_slice].clone()
            cur = torch.where(transfer, x0, cur)
            x_accum[:, block_slice] = cur
            n = int(transfer.sum())
            yield {"kind": kind, "committed": n}
            if eos_id is not None:
                block_tokens = x_accum[:, block_slice]
                eos_mask = block_tokens == eos_id
                if bool(eos_mask.any()):
                    after_eos = eos_mask.cumsum(dim=1).bool()
                    mask_before = (block_tokens == mask_id) & ~after_eos
                    if bool((eos_mask.any(dim=1) & ~mask_before.any(dim=1)).any()):
                        break
        if gen.causal_context:
            executor.set_diffusion_lm(False)
        output = executor.forward(x_accum[:, block_slice], past_key_values=past_key_values,
                                  use_cache=True, use_causal_mask=gen.causal_context)
        past_key_values = output.past_key_values
        st["cache"] = past_key_values
        st["model_calls"] += 1
        if gen.causal_context:
            executor.set_diffusion_lm(True)
            next_token = gen._next_ar_token(output.logits[:, -1, :])
        yield {"kind": "commit", "committed": 0}
        if eos_id is not None and bool((x_accum[:, prompt_len:] == eos_id).any(dim=1).all()):
            break
