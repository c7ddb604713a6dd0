"""Write golden vectors of the reference's PyTorch folded verify step.

Run in the build container only (the reference is not on the GPU box):

    python tests/golden/make_golden.py [--ref /root/reference]

It imports ``SpecFoldFastDLLMV2Generation`` from the reference checkout
(specfold/generate/fastdllm_v2_folded.py) and calls its
``_batched_block_forward`` (:89-223) on tiny seeded Qwen2-layout models
(bf16 and fp32) built with transformers, with a prefix cache and draft-tree
token blocks.  Saved per case: the model weights, the inputs, the logits and
the fold counters.  The package ``__init__`` files of the checkout are
bypassed (registered as bare packages) because ``specfold/generate/__init__.py``
also imports the NLD modules, which this path does not use.

These vectors pin the bf16 rounding trajectory of the reference, which no
closed form fixes; tests/test_oracle_golden.py checks the oracle against them.
"""

from __future__ import annotations

import argparse
import importlib
import json
import sys
import types
from pathlib import Path

import torch
from safetensors.torch import save_file

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
sys.path.insert(0, str(ROOT))

from specfold_amd.generate.synthetic_model import ModelShape, build_qwen2  # noqa: E402
from specfold_amd.synthetic import draft_tree_block, random_prefix_kv  # noqa: E402

CASES = [
    # name, dtype, delta, N, P, seed
    ("tiny_bf16_d0p1", torch.bfloat16, 0.1, 16, 24, 11),
    ("tiny_bf16_d0p02", torch.bfloat16, 0.02, 16, 24, 12),
    ("tiny_bf16_dneg", torch.bfloat16, -1.0, 16, 24, 13),
    ("tiny_fp32_d0p1", torch.float32, 0.1, 16, 24, 14),
    ("tiny_fp32_d0p01", torch.float32, 0.01, 16, 24, 15),
    ("tiny_bf16_noprefix", torch.bfloat16, 0.05, 16, 0, 16),
]

SHAPE = ModelShape(hidden=64, heads=4, kv_heads=2, layers=2, intermediate=128, vocab=96,
                   head_dim=16)


class ListCache:
    """The cache contract the reference step reads: get_seq_length, len, [li] -> (k, v)."""

    def __init__(self, kv):
        self.kv = kv

    def get_seq_length(self, layer_idx=0):
        return int(self.kv[0][0].shape[-2]) if self.kv else 0

    def __len__(self):
        return len(self.kv)

    def __getitem__(self, i):
        return self.kv[i]


def import_reference(ref: Path):
    sys.path.insert(0, str(ref))
    for name in ("specfold", "specfold.generate"):
        mod = types.ModuleType(name)
        mod.__path__ = [str(ref / Path(*name.split(".")))]
        sys.modules[name] = mod
    return importlib.import_module("specfold.generate.fastdllm_v2_folded")


def main(argv=None) -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--ref", default="/root/reference")
    args = ap.parse_args(argv)
    ref_mod = import_reference(Path(args.ref))
    Ref = ref_mod.SpecFoldFastDLLMV2Generation
    meta = {}
    for name, dtype, delta, N, P, seed in CASES:
        torch.manual_seed(seed)
        model = build_qwen2(SHAPE, seed, device="cpu", dtype=dtype)
        gen = torch.Generator().manual_seed(seed + 1000)
        tokens = draft_tree_block(N, SHAPE.vocab, gen)
        kv = random_prefix_kv(SHAPE.layers, SHAPE.kv_heads, P, SHAPE.head_dim, gen, dtype=dtype) \
            if P > 0 else None
        inst = object.__new__(Ref)
        inst.model_executor = types.SimpleNamespace(model=model)
        inst.delta = float(delta)
        with torch.no_grad():
            logits = inst._batched_block_forward(tokens, ListCache(kv) if kv else None)
        tensors = {f"w.{k}": v.contiguous() for k, v in model.state_dict().items()
                   if "rotary_emb" not in k}
        tensors["tokens"] = tokens
        tensors["logits"] = logits.contiguous()
        if kv:
            for li, (k, v) in enumerate(kv):
                tensors[f"prefix.{li}.k"] = k.contiguous()
                tensors[f"prefix.{li}.v"] = v.contiguous()
        save_file(tensors, str(HERE / f"{name}.safetensors"))
        meta[name] = dict(dtype=str(dtype).replace("torch.", ""), delta=delta, N=N, P=P, seed=seed,
                          draft_positions=int(getattr(inst, "_fold_draft_positions", 0)),
                          draft_recomputed=int(getattr(inst, "_fold_draft_recomputed", 0)),
                          shape=SHAPE.__dict__)
        print(name, "fold_ratio", inst.fold_ratio)
    (HERE / "golden_meta.json").write_text(json.dumps(meta, indent=1, sort_keys=True))
    return 0


if __name__ == "__main__":
    sys.exit(main())
