"""Shared test models and inputs: a random Qwen3.5 text model of the reference's tiny test size."""

import torch


def tiny_hf_model(seed=0, layers=8, vocab=256, norm_std=0.1, linear_heads=(2, 4), linear_head_dim=16):
    """transformers' own Qwen3_5TextModel at hidden 64 (6 GDN + 2 attention layers, attention heads
    4/2 of dim 16, GDN heads 2 key / 4 value of dim 16, conv width 4), fp32 on the CPU, plus an
    untied lm_head. Norm weights are drawn N(0, norm_std) so every weight path is exercised.
    `linear_heads` (key, value) and `linear_head_dim` change the GDN heads (128-wide heads in bf16
    run the pipelined fork kernel)."""
    from transformers.models.qwen3_5.configuration_qwen3_5 import Qwen3_5TextConfig
    from transformers.models.qwen3_5.modeling_qwen3_5 import Qwen3_5TextModel

    torch.manual_seed(seed)
    cfg = Qwen3_5TextConfig(
        vocab_size=vocab, hidden_size=64, intermediate_size=128, num_hidden_layers=layers,
        num_attention_heads=4, num_key_value_heads=2, head_dim=16, linear_num_key_heads=linear_heads[0],
        linear_num_value_heads=linear_heads[1], linear_key_head_dim=linear_head_dim,
        linear_value_head_dim=linear_head_dim, linear_conv_kernel_dim=4,
        max_position_embeddings=4096,
        rope_parameters={"rope_theta": 10000.0, "mrope_section": [2, 1, 1], "partial_rotary_factor": 0.25},
        attn_implementation="eager")
    model = Qwen3_5TextModel(cfg).eval()
    with torch.no_grad():
        for n, p in model.named_parameters():
            if n.endswith("norm.weight") and norm_std:
                p.normal_(0.0, norm_std)
    lm_head = torch.nn.Linear(64, vocab, bias=False)
    model.requires_grad_(False)
    lm_head.requires_grad_(False)
    return model, lm_head


def noised_ids(B, L, vocab=256, seed=1, p=0.5):
    """(x0, xt): uniform clean ids and a copy with each token replaced by mask id vocab-1 w.p. p."""
    g = torch.Generator().manual_seed(seed)
    x0 = torch.randint(0, vocab, (B, L), generator=g)
    xt = x0.clone()
    xt[torch.rand(B, L, generator=g) < p] = vocab - 1
    return x0, xt
