"""CPU oracle for the block-diffusion forward hot path — TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, the reference algorithm of `kotoba-lang/dllm-qwen38`'s
block-diffusion forward (the state-fork Gated DeltaNet layer, its causal short conv with
conv-prefix carry-in, and the complementary-mask attention). It is the oracle the HIP
kernels are compared against; it is never the thing measured or shipped.

Only `tests/`, `__graft_entry__.smoke()` and the `cpu_baseline` leg of `bench.py` may import
it. The product package (`dllm_qwen38_amd`) never imports it and never falls back to it.

Modules:
  gdn_ref      chunked gated delta rule with per-chunk states (fp32, the reference's op order),
               the float64 token recurrence it must agree with, l2norm, the causal conv with
               prefix carry-in, the integer fork layout, and the whole state-fork layer.
  attn_ref     complementary / block-causal masks, allowed-pair counts, partial RoPE and the
               masked GQA attention.
  model_ref    the hybrid text model's modules (RMSNorm(1+w), gated RMSNorm, SwiGLU MLP, gated
               attention, GDN mixer), the two-stream block-diffusion forward and the per-block
               oracle forward it is checked against.

How each function is pinned (beyond restating the reference) is listed in each module header.
"""
