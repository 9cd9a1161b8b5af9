"""CPU oracle for the MoE-layer hot path: TEST INFRASTRUCTURE, never the product.

A restatement, in numpy and plain C, of the reference's CPU arithmetic for willow's Qwen3.6-35B-A3B MoE layer:
GGUF Q4_K / Q6_K dequantization (gguf/quants.py:12-25,73-116,207-227 and the per-chunk form of
gguf/metal.py:133-168), the router (engines/base.py:91-97, 448), SwiGLU experts (engines/base.py:99-107), and the
weighted combine with the sigmoid-gated shared expert (engines/base.py:445-490, 580-589).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this package, and only as the
reference that results are compared against (or, for bench.py, as the timed CPU baseline). The product path (the
gguf.hip package and libwillow_hip.so) never imports, links or calls anything here.

How each part is pinned (the reference ships no tests, fixtures or golden vectors for this path):
  quants_ref   two independent formulations (vectorized, from gguf/quants.py; per 32-value chunk, from
               gguf/metal.py, in numpy and again in C) must agree bit for bit; closed-form known answers on crafted
               blocks; fp32 exactness of every product (so evaluation order cannot matter); bf16 RNE checked
               against torch's own conversion.
  moe_ref      router logits replay the kernels' documented FMA order in C (bit-exact) and are checked against a
               float64 dot product within the fp32 error bound; route() against brute-force sorting; the layer
               against a float64 per-expert loop and against transformers' Qwen3_5MoeSparseMoeBlock on tiny
               dequantized weights (third-party pin; transformers is not needed where the GPU runs, so that test skips there).
"""
