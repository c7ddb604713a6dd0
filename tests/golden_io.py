"""Loading of the committed golden fixtures (tests/golden/*.safetensors)."""

from __future__ import annotations

import json
from pathlib import Path

import torch
from safetensors.torch import load_file

from specfold_amd.generate.synthetic_model import ModelShape, build_qwen2

GOLDEN = Path(__file__).resolve().parent / "golden"


def golden_cases():
    meta = json.loads((GOLDEN / "golden_meta.json").read_text())
    return sorted(meta)


def load_case(name: str, device="cpu"):
    meta = json.loads((GOLDEN / "golden_meta.json").read_text())[name]
    t = load_file(str(GOLDEN / f"{name}.safetensors"))
    dtype = getattr(torch, meta["dtype"])
    shape = ModelShape(**meta["shape"])
    model = build_qwen2(shape, 0, device=device, dtype=dtype)
    sd = {k[2:]: v for k, v in t.items() if k.startswith("w.")}
    missing, unexpected = model.load_state_dict(sd, strict=False)
    if unexpected or any("rotary" not in m for m in missing):
        raise RuntimeError(f"state dict mismatch: {missing} {unexpected}")
    kv = None
    if meta["P"] > 0:
        kv = [(t[f"prefix.{li}.k"].to(device), t[f"prefix.{li}.v"].to(device))
              for li in range(shape.layers)]
    return dict(meta=meta, model=model, tokens=t["tokens"].to(device), kv=kv,
                logits=t["logits"], shape=shape, dtype=dtype)
