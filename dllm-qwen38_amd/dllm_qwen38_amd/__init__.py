"""MI355X (gfx950) block-diffusion forward hot path for Qwen3.5/3.8-family Gated DeltaNet hybrids.

Drop-in modules mirroring the reference's entry points:
  gdn          chunk_gated_delta_rule_with_states, gdn_mixer_forward, set_impl / last_impl,
               causal_conv1d_fn, and the fused two-stream state fork gdn_state_fork (one launch
               or block ranges beside the conv) with StateForkPlan for fixed-shape repeats
  attention    complementary-mask attention over cat([x_t, x_0]) (bd_attention) and block-causal
               attention against a key/value cache (block_causal_attention)
  blockdiff    block_diffusion_forward, LayerStep, BreakMode and the per-block oracles of the harness
  decode       generate (the golden decoder) and generate_cached with PrefixCache
  norms        RMSNorm with the residual add, gated RMSNorm, q/k norm + RoPE, SwiGLU, GDN gates
  equivalence  the equivalence harness (command line and run())
  model        a Qwen3.5-shaped weight container for seeded on-device initialisation
  gemm_tuning  the committed GEMM solution table for the library GEMMs around the path
  inputs       seeded synthetic workloads

All compute goes through libdllm_hip.so (hand-written HIP kernels, C ABI in include/dllm_hip.h).
"""

__all__ = ["gdn", "inputs"]
