"""ORACLE — test infrastructure, not product code.

CPU restatement of chungen04/specfold's PyTorch folded verify step
(``SpecFoldFastDLLMV2Generation._batched_block_forward``,
specfold/generate/fastdllm_v2_folded.py:89-223) and of the integer decisions of
its decode loop (specfold/generate/fastdllm_v2_generation.py:387-474, 599-700).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import this package, and only as the checker / the timed CPU baseline.
The product package ``specfold_amd`` never imports it and has no CPU fallback.

How each function is pinned (checked against something other than itself):
  folded_reference.parent_map        brute force over all diff-set families
                                     (tests/test_oracle_parent_map.py)
  folded_reference.folded_layer /
  folded_reference.folded_verify_step
                                     (a) golden vectors written by importing the
                                     reference class itself on CPU
                                     (tests/golden/make_golden.py) — bit-exact;
                                     (b) delta<0 (all rows recomputed) equals an
                                     independent dense layer built on
                                     transformers' Qwen2DecoderLayer;
                                     (c) every folded row's (m, Z, O) equals
                                     exact fp64 softmax attention of its
                                     inherited query over its branch's K/V.
  decode_reference.*                 restated integer logic, checked on
                                     hand-built logits with known answers
                                     (tests/test_oracle_decode.py).
"""
