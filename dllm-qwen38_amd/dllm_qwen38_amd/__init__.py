"""MI355X (gfx950) block-diffusion forward hot path for Qwen3.5/3.8-family Gated DeltaNet hybrids.

Drop-in modules mirroring the reference's entry points:
  gdn        chunk_gated_delta_rule_with_states, gdn_mixer_forward, set_impl / last_impl,
             causal_conv1d_fn, and the fused two-stream state fork gdn_state_fork
  inputs     seeded synthetic workloads

All compute goes through libdllm_hip.so (hand-written HIP kernels, C ABI in include/dllm_hip.h).
"""

__all__ = ["gdn", "inputs"]
