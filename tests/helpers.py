"""Shared test helpers: seeded tiny models, inputs, error metrics."""

from __future__ import annotations

import copy
from dataclasses import dataclass
from typing import List, Optional

import torch

from specfold_amd.generate.synthetic_model import ModelShape, build_nld, build_qwen2
from specfold_amd.synthetic import draft_tree_block, random_prefix_kv

# hd = 128 shapes the HIP kernels take; small enough for the CPU oracle
SHAPE_G2 = ModelShape(hidden=512, heads=4, kv_heads=2, layers=2, intermediate=1024, vocab=1000)
SHAPE_G7 = ModelShape(hidden=896, heads=7, kv_heads=1, layers=2, intermediate=1536, vocab=512)
SHAPE_G6 = ModelShape(hidden=1536, heads=12, kv_heads=2, layers=1, intermediate=2048, vocab=256)


@dataclass
class Case:
    model_cpu: torch.nn.Module
    tokens: torch.Tensor
    kv: Optional[list]
    delta: float


def make_case(shape: ModelShape, seed: int, N: int = 32, P: int = 100, delta: float = 0.1,
              tokens: Optional[torch.Tensor] = None) -> Case:
    model = build_qwen2(shape, seed, device="cpu", dtype=torch.bfloat16)
    gen = torch.Generator().manual_seed(seed + 77)
    if tokens is None:
        tokens = draft_tree_block(N, shape.vocab, gen)
    kv = random_prefix_kv(shape.layers, shape.kv_heads, P, shape.head_dim, gen) if P else None
    return Case(model, tokens, kv, delta)


# NLD (Llama-layout) shapes: no QKV bias, eps 1e-5
SHAPE_N4 = ModelShape(hidden=512, heads=4, kv_heads=1, layers=2, intermediate=1024, vocab=700,
                      rms_eps=1e-5, qkv_bias=False)
SHAPE_N8 = ModelShape(hidden=1024, heads=8, kv_heads=2, layers=2, intermediate=1536, vocab=512,
                      rms_eps=1e-5, qkv_bias=False)


def make_nld_case(shape: ModelShape, seed: int, N: int = 32, P: int = 100, delta: float = 0.1,
                  omax: int = 64, dtype=torch.bfloat16) -> Case:
    """An NLD-layout model whose llama-4 q scale is active from position ``omax`` on."""
    model = build_nld(shape, seed, device="cpu", dtype=dtype, original_max_positions=omax)
    gen = torch.Generator().manual_seed(seed + 91)
    tokens = draft_tree_block(N, shape.vocab - 1, gen)
    kv = random_prefix_kv(shape.layers, shape.kv_heads, P, shape.head_dim, gen, dtype=dtype) \
        if P else None
    return Case(model, tokens, kv, delta)


def to_gpu_model(model_cpu):
    return copy.deepcopy(model_cpu).to("cuda")


def err_stats(a: torch.Tensor, b: torch.Tensor) -> dict:
    a = a.detach().double().cpu()
    b = b.detach().double().cpu()
    d = (a - b).abs()
    return dict(max_abs=float(d.max()) if d.numel() else 0.0,
                mean_rel=float(d.mean() / b.abs().mean().clamp_min(1e-30)) if d.numel() else 0.0,
                frac_diff=float((d > 0).double().mean()) if d.numel() else 0.0,
                ref_absmax=float(b.abs().max()) if b.numel() else 0.0)


def src_from_mask(parent: List[Optional[int]], rec: torch.Tensor) -> torch.Tensor:
    """Nearest recomputing ancestor branch of every (b, n), from the parent map
    and the recompute mask [B1, N] (walks the chain on the CPU)."""
    B1, N = rec.shape
    out = torch.zeros(B1, N, dtype=torch.int64)
    for b in range(B1):
        for n in range(N):
            c = b
            while not bool(rec[c, n]):
                c = parent[c] if parent[c] is not None else 0
            out[b, n] = c
    return out


def plain_events(events) -> list:
    """Decode-loop events with their tensor fields (the Fast-dLLM loop's decision
    tensors) turned into lists, so that event streams compare with ==."""
    return [{k: (v.tolist() if isinstance(v, torch.Tensor) else v) for k, v in e.items()}
            for e in events]
