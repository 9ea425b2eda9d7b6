"""CPU oracle for the K-quant matmul and ragged decode attention path.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and
``bench.py``'s ``cpu_baseline`` leg may import this package, and only as the
checker or the timed CPU baseline; the product (``gmlx_amd``) never imports it.

Contents:
  kquant     numpy + C (``liboracle.so``) restatements of the GGUF Q4_K, Q6_K and
             IQ2_XXS block codecs, the quantizers, and fp64 matmul references.
  attention  fp64 ragged GQA decode attention reference
             (semantics of gmlx/qwen35_attn.py:395-493).
  moe        fp64 MoE expert-gather / fused-GLU / mix / router references
             (semantics of gmlx/modules.py:540-605, 754-763).
"""
