"""Both decode loops end to end on the CPU, once with the reference's torch ops
for every decision and once on the greedy-statistics path (the one the loops
take on the GPU at temperature 0), with ``sf_logit_stats`` stood in for by the
reference's own ops: the event streams, the committed tokens and the draft
counts must be identical.  This covers the plumbing around the statistics (the
top-p greedy pair, draft construction from the top-8 ranks, NLD's transfer rule)
that the GPU tests reach only through the kernel.

The model is a deterministic hash of (previous token, own token, absolute
position) into a bank of logits rows.  Every bank row holds distinct bf16
values (so no argmax / topk over the vocabulary depends on a library's tie
order) scaled by a power of two (so the rows range from flat to confident and
the loops take every branch: several commits per step, single commits, draft
hits).  The stand-in's 1/Z reproduces the fp32 softmax maximum bit for bit, so
the positions' confidences, ties included, are the same in both runs."""

import types

import pytest
import torch

from specfold_amd.configs import SYNTHETIC_DRAFT_GRAPH
from specfold_amd.generate import greedy
from specfold_amd.generate.fastdllm_model_executor import ByteTokenizer, FastDLLMModelExecutor
from specfold_amd.generate.fastdllm_v2_generation import FastDLLMV2SpeculativeGeneration
from specfold_amd.generate.nld_generation import NLDDiffusionGeneration
from tests.helpers import plain_events

V = 512
N_BANK = 97


def _bank(seed, eos=None):
    """N_BANK rows of V distinct bf16 values, each row scaled by 4, 16, 64 or 256."""
    g = torch.Generator().manual_seed(seed)
    bits = torch.arange(0x3D80, 0x4100, dtype=torch.int32)          # 1/16 .. 8
    pos = bits.to(torch.int16).view(torch.bfloat16).float()
    pool = torch.cat([pos, -pos])
    rows = []
    for r in range(N_BANK):
        vals = pool[torch.randperm(pool.numel(), generator=g)[:V]]
        row = vals * float(4 ** (1 + r % 4))
        if eos is not None and r % 47 == 5:
            top = int(row.argmax())
            row[[top, eos]] = row[[eos, top]]
        rows.append(row)
    bank = torch.stack(rows).to(torch.bfloat16)
    assert torch.equal(bank.float(), torch.stack(rows))             # exact in bf16
    assert all(bank[r].unique().numel() == V for r in range(N_BANK))
    return bank


class Cache:
    def __init__(self, n, last):
        self.n, self.last = n, last

    def get_seq_length(self):
        return self.n


def _logits(bank, toks, cache):
    start = 0 if cache is None else cache.n
    last = 0 if cache is None else cache.last
    prev = torch.cat([torch.full_like(toks[:, :1], last), toks[:, :-1]], dim=1)
    pos = start + torch.arange(toks.shape[1])
    h = (prev * 1000003 + toks * 7919 + pos * 104729) % N_BANK
    return bank[h]


class FakeFastDLLM:
    device = torch.device("cpu")

    def __init__(self, bank):
        self.bank = bank

    def get_tokenizer(self):
        return ByteTokenizer()

    def forward(self, toks, past_key_values=None, use_cache=True, update_past_key_values=False):
        out = types.SimpleNamespace(logits=_logits(self.bank, toks, past_key_values),
                                    past_key_values=past_key_values)
        if update_past_key_values:
            n = 0 if past_key_values is None else past_key_values.n
            out.past_key_values = Cache(n + toks.shape[1], int(toks[0, -1]))
        return out

    def sample_with_top_p(self, logits, top_p=0.95, temperature=0.0):
        return FastDLLMModelExecutor._top_p(logits, top_p, temperature)


class FakeNLD(FakeFastDLLM):
    MASK, EOS = 100000, 3

    def __init__(self, bank):
        super().__init__(bank)
        self.diffusion = []

    def get_mask_id(self):
        return self.MASK

    def get_eos_token_id(self):
        return self.EOS

    def set_diffusion_lm(self, flag):
        self.diffusion.append(flag)

    def forward(self, toks, past_key_values=None, use_cache=True, use_causal_mask=False):
        out = types.SimpleNamespace(logits=_logits(self.bank, toks, past_key_values),
                                    past_key_values=None)
        if use_cache:
            n = 0 if past_key_values is None else past_key_values.n
            out.past_key_values = Cache(n + toks.shape[1], int(toks[0, -1]))
        return out


def cpu_stats(rows, top_p=0.95):
    """sf_logit_stats' fields from the reference's ops: top-8 in descending order
    (lowest index first among equal values), the top-p sampler's greedy token and
    probability, the softmax normaliser (1/Z = the fp32 softmax maximum) and the
    bf16 softmax maximum."""
    f = rows.float()
    order = torch.sort(f, dim=-1, descending=True, stable=True).indices[:, :8]
    tok, probs = FastDLLMModelExecutor._top_p(rows, top_p, 0.0)
    cmax = torch.softmax(f, dim=-1).max(-1).values
    zfull = 1.0 / cmax
    assert torch.equal(1.0 / zfull, cmax)       # max_prob_fp32 reproduces it exactly
    return types.SimpleNamespace(
        top_idx=order.to(torch.int32), top_val=f.gather(1, order), zfull=zfull,
        znuc=torch.full_like(zfull, float("nan")), greedy_tok=tok.to(torch.int32),
        conf=probs.gather(-1, tok.unsqueeze(-1)).squeeze(-1).float(),
        conf_full=torch.softmax(rows, dim=-1).max(-1).values.float())


def _run(gen, prompt_ids, monkeypatch, use_stats):
    calls = []
    if use_stats:
        def stats(rows, top_p=0.95):
            calls.append(rows.shape[0])
            return cpu_stats(rows, top_p)
        monkeypatch.setattr(greedy, "usable", lambda logits, t: t == 0
                            and logits.dtype == torch.bfloat16 and logits.shape[-1] % 8 == 0)
        monkeypatch.setattr(greedy, "stats", stats)
    events = list(gen.decode_steps(prompt_ids))
    monkeypatch.undo()
    return events, gen._state, list(gen.last_commits), calls


@pytest.mark.parametrize("seed", range(4))
def test_fastdllm_loop_same_decisions_with_statistics(seed, monkeypatch):
    bank = _bank(seed)
    prompt = torch.randint(0, 256, (1, 40 + 3 * seed), generator=torch.Generator().manual_seed(seed))
    runs = []
    for use_stats in (False, True):
        gen = FastDLLMV2SpeculativeGeneration(
            block_length=32, model_executor=FakeFastDLLM(bank),
            calibration_graph=SYNTHETIC_DRAFT_GRAPH, max_new_tokens=96, stop_token=7,
            device="cpu")
        gen.last_commits = []
        runs.append(_run(gen, prompt, monkeypatch, use_stats))
    (ea, sa, ca, _), (eb, sb, cb, calls) = runs
    assert calls, "the statistics path was not taken"
    assert plain_events(ea) == plain_events(eb) and ca == cb
    assert torch.equal(sa["x_t"], sb["x_t"])
    assert sa["model_calls"] == sb["model_calls"] and sa["drafts_computed"] == sb["drafts_computed"]
    kinds = {e["kind"] for e in ea}
    assert {"verify", "commit"} <= kinds


def test_fastdllm_loop_hits_drafts():
    """The fake model exercises the draft-hit branch on at least one seed."""
    hits = 0
    for seed in range(4):
        gen = FastDLLMV2SpeculativeGeneration(
            block_length=32, model_executor=FakeFastDLLM(_bank(seed)),
            calibration_graph=SYNTHETIC_DRAFT_GRAPH, max_new_tokens=96, stop_token=7,
            device="cpu")
        gen.last_commits = []
        prompt = torch.randint(0, 256, (1, 40 + 3 * seed),
                               generator=torch.Generator().manual_seed(seed))
        hits += sum(e["kind"] == "hit" for e in gen.decode_steps(prompt))
    assert hits > 0


@pytest.mark.parametrize("seed", range(4))
def test_nld_loop_same_decisions_with_statistics(seed, monkeypatch):
    bank = _bank(100 + seed, eos=FakeNLD.EOS)
    prompt = torch.randint(0, 256, (1, 20 + 5 * seed),
                           generator=torch.Generator().manual_seed(seed))
    runs = []
    for use_stats in (False, True):
        gen = NLDDiffusionGeneration(block_length=32, model_executor=FakeNLD(bank),
                                     calibration_graph=SYNTHETIC_DRAFT_GRAPH, max_new_tokens=128,
                                     threshold=0.9, device="cpu")
        runs.append(_run(gen, prompt, monkeypatch, use_stats))
    (ea, sa, ca, _), (eb, sb, cb, calls) = runs
    assert calls, "the statistics path was not taken"
    assert plain_events(ea) == plain_events(eb) and ca == cb
    assert torch.equal(sa["x_accum"], sb["x_accum"])
    assert sa["model_calls"] == sb["model_calls"] and sa["drafts_computed"] == sb["drafts_computed"]
    assert {"prefill", "verify", "hit", "commit"} <= {e["kind"] for e in ea}


@pytest.mark.parametrize("seeds", [(0, 1, 2), (3, 5)])
def test_nld_lockstep_same_tokens_as_separate_loops(seeds):
    """LockstepDecoder over several NLD loops (deferred forwards, one merged call
    per round) gives every sequence the events, tokens and counters of its own
    loop run alone; each round's call carries one request per live sequence."""
    from specfold_amd.generate.lockstep import LockstepDecoder

    def make(seed):
        bank = _bank(100 + seed, eos=FakeNLD.EOS)
        prompt = torch.randint(0, 256, (1, 20 + 5 * seed),
                               generator=torch.Generator().manual_seed(seed))
        gen = NLDDiffusionGeneration(block_length=32, model_executor=FakeNLD(bank),
                                     calibration_graph=SYNTHETIC_DRAFT_GRAPH,
                                     max_new_tokens=64 + 32 * (seed % 2), threshold=0.9,
                                     device="cpu")
        return gen, prompt

    alone = []
    for seed in seeds:
        gen, prompt = make(seed)
        alone.append((list(gen.decode_steps(prompt)), gen._state))
    pairs = [make(seed) for seed in seeds]
    gens = [g for g, _ in pairs]
    sizes = []

    def forward_many(requests):
        sizes.append(len(requests))
        # each sequence's own forward (the fake models differ per sequence)
        return [gens[[id(g._state["cache"]) if g._state["cache"] is not None else None
                      for g in gens].index(id(c) if c is not None else None)]
                ._batched_block_forward(b, c) for b, c in requests]

    dec = LockstepDecoder(gens, forward_many=forward_many)
    per_seq = [[] for _ in seeds]
    for rnd in dec.rounds([p for _, p in pairs]):
        for i, ev in rnd["events"]:
            per_seq[i].append(ev)
    for i, (ev_alone, st_alone) in enumerate(alone):
        assert plain_events(per_seq[i]) == plain_events(ev_alone)
        assert torch.equal(gens[i]._state["x_accum"], st_alone["x_accum"])
        assert gens[i]._state["model_calls"] == st_alone["model_calls"]
    assert max(sizes) == len(seeds) and dec.batched_steps == len(sizes)


def test_nld_lockstep_generate_same_results():
    """LockstepDecoder.generate returns, per sequence, what that generator's
    generate_with_draft_speculation returns alone (texts, tokens, model calls,
    drafts)."""
    from specfold_amd.generate.lockstep import LockstepDecoder

    def make(seed):
        return NLDDiffusionGeneration(block_length=32, model_executor=FakeNLD(_bank(100 + seed,
                                                                                  eos=FakeNLD.EOS)),
                                      calibration_graph=SYNTHETIC_DRAFT_GRAPH,
                                      max_new_tokens=64 + 32 * (seed % 2), threshold=0.9,
                                      device="cpu")

    seeds = (0, 1, 3)
    prompts = ["lockstep %d" % s * (1 + s) for s in seeds]
    alone = [make(s).generate_with_draft_speculation(prompt=p) for s, p in zip(seeds, prompts)]
    gens = [make(s) for s in seeds]

    def forward_many(requests):
        # each request through its own generator's forward (the fake models differ)
        out = []
        for b, c in requests:
            g = next(g for g in gens if g._state["cache"] is c)
            out.append(g._batched_block_forward(b, c))
        return out

    got = LockstepDecoder(gens, forward_many=forward_many).generate(prompts)
    assert got == alone
    assert all(r[1] > 0 for r in got)


def test_fastdllm_lockstep_same_results():
    """Fast-dLLM loops in lockstep (deferred forwards) reproduce each sequence's
    own loop: events, final tokens, and generate_with_draft_speculation's
    results."""
    from specfold_amd.generate.lockstep import LockstepDecoder

    def make(seed):
        g = FastDLLMV2SpeculativeGeneration(
            block_length=32, model_executor=FakeFastDLLM(_bank(seed)),
            calibration_graph=SYNTHETIC_DRAFT_GRAPH, max_new_tokens=64 + 32 * (seed % 2),
            stop_token=7, device="cpu")
        g.last_commits = []
        return g

    seeds = (0, 1, 2)

    def forward_many_for(gens):
        def forward_many(requests):
            out = []
            for b, c in requests:
                g = next(g for g in gens if g._state["cache"] is c)
                out.append(g._batched_block_forward(b, c))     # shifted, as the seam
            return out
        return forward_many

    prompts = [torch.randint(0, 256, (1, 40 + 3 * s), generator=torch.Generator().manual_seed(s))
               for s in seeds]
    alone = []
    for s, p in zip(seeds, prompts):
        g = make(s)
        alone.append((list(g.decode_steps(p)), g._state["x_t"].clone()))
    gens = [make(s) for s in seeds]
    per_seq = [[] for _ in seeds]
    for rnd in LockstepDecoder(gens, forward_many=forward_many_for(gens)).rounds(prompts):
        for i, ev in rnd["events"]:
            per_seq[i].append(ev)
    for i, (ev, x) in enumerate(alone):
        assert plain_events(per_seq[i]) == plain_events(ev)
        assert torch.equal(gens[i]._state["x_t"], x)
    assert any(e["kind"] == "hit" for evs in per_seq for e in evs)

    texts = ["lockstep fast-dllm %d" % s * (1 + s) for s in seeds]
    want = [make(s).generate_with_draft_speculation(prompt=t) for s, t in zip(seeds, texts)]
    gens = [make(s) for s in seeds]
    got = LockstepDecoder(gens, forward_many=forward_many_for(gens)).generate(texts)
    assert got == want


def test_lockstep_engine_glue():
    """The default batched forward of LockstepDecoder: one forward_batched call
    with every request, the executor's q scale per sequence where it has one,
    padding to the draft graph's width, the logit shift asked of the engine's head
    exactly for generators that shift (Fast-dLLM), and the fold counters over real
    draft rows only."""
    from specfold_amd.generate.lockstep import LockstepDecoder

    class Cache:
        def __init__(self, n):
            self.length = n

        def get_seq_length(self):
            return self.length

    calls = []

    class Eng:
        L, gate_mode, device = 2, 0, torch.device("cpu")

        def forward_batched(self, blocks, caches, delta, bucket, q_scales, stats, pad_to,
                            shift=False):
            calls.append(dict(blocks=blocks, caches=caches, delta=delta, bucket=bucket,
                              q_scales=q_scales, pad_to=pad_to, shift=shift))
            stats.count_dev = torch.tensor([40, 36], dtype=torch.int32)
            out = [torch.arange(b.shape[0] * b.shape[1] * 3, dtype=torch.float32)
                   .view(b.shape[0], b.shape[1], 3) for b in blocks]
            # the engine's head shifts in its stores: the same values as the torch shift
            return [torch.cat([x[:, :1], x[:, :-1]], 1) for x in out] if shift else out

    def gen(executor, shift):
        g = types.SimpleNamespace(_engine=Eng(), gate_mode=0, delta=0.2, fold_bucket=None,
                                  model_executor=executor,
                                  calibration_graph=SYNTHETIC_DRAFT_GRAPH)
        if shift:
            g._shift_logits = FastDLLMV2SpeculativeGeneration._shift_logits.__get__(g)
        return g

    n_drafts = sum(1 for n in SYNTHETIC_DRAFT_GRAPH["selected_nodes"] if n.get("ij_set"))
    blocks = [torch.zeros(3, 8, dtype=torch.int64), torch.zeros(1, 8, dtype=torch.int64)]
    caches = [Cache(5), Cache(70)]

    # NLD-like: executor q scale, no shift
    ex = types.SimpleNamespace(q_scale=lambda P, N: torch.full((N,), float(P)))
    dec = LockstepDecoder([gen(ex, False), gen(ex, False)])
    out = dec.forward_many(list(zip(blocks, caches)))
    c = calls[-1]
    assert c["pad_to"] == 1 + n_drafts and c["delta"] == 0.2 and c["bucket"] is None
    assert c["shift"] is False
    assert [float(q[0]) for q in c["q_scales"]] == [5.0, 70.0]
    assert torch.equal(out[0], torch.arange(72, dtype=torch.float32).view(3, 8, 3))
    assert dec.draft_positions == (4 - 2) * 8 * 2
    assert int(dec._recomputed) == 76 - 2 * 8 * 2

    # Fast-dLLM-like: no q scale, logits shifted by one position per sequence
    ex2 = types.SimpleNamespace()
    dec2 = LockstepDecoder([gen(ex2, True), gen(ex2, True)])
    out2 = dec2.forward_many(list(zip(blocks, caches)))
    assert calls[-1]["q_scales"] == [None, None] and calls[-1]["shift"] is True
    raw = torch.arange(72, dtype=torch.float32).view(3, 8, 3)
    assert torch.equal(out2[0], torch.cat([raw[:, :1], raw[:, :-1]], dim=1))

    # a round beyond 1024 rows is split: 5 sequences padded to 9 branches x 32 rows
    dec3 = LockstepDecoder([gen(ex2, False)] * 5)
    dec3.pad_to = 9
    n0 = len(calls)
    big = [(torch.zeros(2, 32, dtype=torch.int64), Cache(3)) for _ in range(5)]
    out3 = dec3.forward_many(big)
    split = [len(c["blocks"]) for c in calls[n0:]]
    assert split == [3, 2] and len(out3) == 5 and dec3.batched_steps == 1
    assert int(dec3._recomputed) == 2 * 76 - 5 * 32 * 2
    assert [c["bucket"] for c in calls[n0:]] == [None, None]

    # a per-sequence fold_bucket: each stacked step gets the sum of its sequences'
    # buckets (each capped at that sequence's padded rows), so sequences that fit
    # alone fit together
    def bucketed(fb):
        g = gen(ex2, False)
        g.fold_bucket = fb
        return g
    dec4 = LockstepDecoder([bucketed(40)] * 5)
    dec4.pad_to = 9
    n0 = len(calls)
    dec4.forward_many(big)
    assert [c["bucket"] for c in calls[n0:]] == [3 * 40, 2 * 40]
    dec5 = LockstepDecoder([bucketed(1000)] * 2)
    n0 = len(calls)
    dec5.forward_many(list(zip(blocks, caches)))
    assert [c["bucket"] for c in calls[n0:]] == [2 * (1 + n_drafts) * 8]
