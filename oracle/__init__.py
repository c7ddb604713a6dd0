"""ORACLE — test infrastructure, not product code.

CPU restatement of chungen04/specfold's PyTorch folded verify step
(``SpecFoldFastDLLMV2Generation._batched_block_forward``,
specfold/generate/fastdllm_v2_folded.py:89-223; the NLD differences of
specfold/generate/nld_folded.py:37-53, 105-108, 237).

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
  folded_reference.delta_gate         the gate inside folded_layer (pinned with it)
  folded_reference.llama4_q_scale     its closed form at the window boundaries
                                     (tests/test_oracle_nld.py)
  folded_reference.dense_verify_step  transformers' Qwen2 / Ministral3 layers
                                     (tests/test_oracle_pins.py, test_oracle_nld.py)
The decode loops' integer decisions are restated in the tests that check them
(tests/test_decode_logic.py, tests/test_decode_loops_stats.py,
tests/test_gpu_fastdllm_generator.py), not in this package.
"""
