"""Named workloads: the five configurations the verify step is measured and
tested on (shapes of Fast-dLLM-v2-1.5B / -7B and two Llama-style diffusion
LMs), with the decoding knobs of the reference's Config
(specfold/config/config.py:13-18: block 32, depth D=8, budget B=7, per-step
limit S=3) and its default delta (specfold/generate/fastdllm_v2_folded.py:44).
"""

from __future__ import annotations

from dataclasses import dataclass, replace
from typing import Dict

from specfold_amd.generate.synthetic_model import ModelShape

QWEN2_VOCAB_15B = 151936
QWEN2_VOCAB_7B = 152064
NLD_VOCAB = 131072


@dataclass(frozen=True)
class Workload:
    name: str
    shape: ModelShape
    seed: int
    prefix: int
    budget_B: int = 7
    depth_D: int = 8
    per_step_S: int = 3
    block: int = 32
    small_block: int = 8
    delta: float = 0.1
    threshold: float = 0.9
    gen_tokens: int = 256
    batch: int = 1
    page_size: int = 16
    shuffled_pages: bool = False
    logit_shift: bool = True        # Fast-dLLM shifts logits; NLD does not
    dtype: str = "bf16"

    @property
    def branches(self) -> int:
        return self.budget_B + 1

    @property
    def family(self) -> str:
        """"fastdllm" (Qwen2 layout, shifted logits) or "nld" (Llama layout, no shift)."""
        return "fastdllm" if self.logit_shift else "nld"


WORKLOADS: Dict[str, Workload] = {
    # cfg 1: CPU reference, one Qwen2-1.5B-shaped decoder layer, fp32, 512 prefix
    "cfg1_1p5b_layer": Workload(
        "cfg1_1p5b_layer",
        ModelShape(hidden=1536, heads=12, kv_heads=2, layers=1, intermediate=8960,
                   vocab=QWEN2_VOCAB_15B),
        seed=0, prefix=512, dtype="fp32"),
    # cfg 2: full 28-layer Fast-dLLM-v2-1.5B shape
    "cfg2_1p5b": Workload(
        "cfg2_1p5b",
        ModelShape(hidden=1536, heads=12, kv_heads=2, layers=28, intermediate=8960,
                   vocab=QWEN2_VOCAB_15B),
        seed=1, prefix=1024, gen_tokens=256),
    # cfg 3: Fast-dLLM-v2-7B shape (the north-star target shape)
    "cfg3_7b": Workload(
        "cfg3_7b",
        ModelShape(hidden=3584, heads=28, kv_heads=4, layers=28, intermediate=18944,
                   vocab=QWEN2_VOCAB_7B),
        seed=2, prefix=2048, gen_tokens=512),
    # cfg 4: Llama-style 8B diffusion LM, 4 independent sequences, B=4, delta 0.2
    "cfg4_8b_x4": Workload(
        "cfg4_8b_x4",
        ModelShape(hidden=4096, heads=32, kv_heads=8, layers=32, intermediate=14336,
                   vocab=NLD_VOCAB, rms_eps=1e-5, qkv_bias=False),
        seed=3, prefix=4096, budget_B=4, delta=0.2, batch=4, logit_shift=False),
    # cfg 5: Llama-style 14B, 16k prefix in shuffled 16-token pages
    "cfg5_14b_16k": Workload(
        "cfg5_14b_16k",
        ModelShape(hidden=5120, heads=40, kv_heads=8, layers=40, intermediate=17408,
                   vocab=NLD_VOCAB, rms_eps=1e-5, qkv_bias=False),
        seed=4, prefix=16384, shuffled_pages=True, logit_shift=False),
}


def workload(name: str, **overrides) -> Workload:
    w = WORKLOADS[name]
    return replace(w, **overrides) if overrides else w


# the fixed synthetic draft graph (ij_set form: (position rank, vocab rank)),
# a depth-4 tree of B=7 nodes within D=8 levels and <= S=3 nodes per level
SYNTHETIC_DRAFT_GRAPH = {
    "selected_nodes": [
        {"ij_set": [(0, 0)]},
        {"ij_set": [(0, 0), (1, 0)]},
        {"ij_set": [(0, 0), (2, 0)]},
        {"ij_set": [(0, 0), (3, 0)]},
        {"ij_set": [(0, 0), (1, 0), (4, 0)]},
        {"ij_set": [(0, 0), (1, 0), (5, 0)]},
        {"ij_set": [(0, 0), (1, 0), (4, 0), (6, 0)]},
    ]
}


def draft_graph(budget_B: int) -> dict:
    """The first ``budget_B`` nodes of the synthetic draft graph (a valid tree:
    every node's parent precedes it, <= 3 nodes per level)."""
    nodes = SYNTHETIC_DRAFT_GRAPH["selected_nodes"]
    if not 1 <= budget_B <= len(nodes):
        raise ValueError(f"budget_B must be in [1, {len(nodes)}]")
    return {"selected_nodes": [dict(n) for n in nodes[:budget_B]]}
