"""A Qwen3.5/3.8-shaped hybrid text model (Gated DeltaNet + gated attention) for random-init runs.

The module tree uses the attribute names of transformers' Qwen3_5TextModel (embed_tokens,
layers[i].{input_layernorm, post_attention_layernorm, mlp, linear_attn | self_attn}, norm,
rotary_emb.inv_freq, config.layer_types), so `blockdiff.block_diffusion_forward` runs unchanged on
either. It exists so that large stacks can be initialised directly on the device with seeded
weights (no checkpoint download, no CPU-side init of billions of parameters). The forward pass
lives in `blockdiff`; these modules hold weights only.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import torch
from torch import nn

FULL = "full_attention"
LINEAR = "linear_attention"


@dataclass
class HybridConfig:
    vocab_size: int = 256
    hidden_size: int = 64
    intermediate_size: int = 128
    num_hidden_layers: int = 8
    num_attention_heads: int = 4
    num_key_value_heads: int = 2
    head_dim: int = 16
    linear_num_key_heads: int = 2
    linear_num_value_heads: int = 4
    linear_key_head_dim: int = 16
    linear_value_head_dim: int = 16
    linear_conv_kernel_dim: int = 4
    rms_norm_eps: float = 1e-6
    rope_theta: float = 1e7
    partial_rotary_factor: float = 0.25
    full_attention_interval: int = 4
    layer_types: list = field(default_factory=list)

    def __post_init__(self):
        if not self.layer_types:
            # every full_attention_interval-th layer is attention (Qwen3.5 layout)
            self.layer_types = [FULL if (i + 1) % self.full_attention_interval == 0 else LINEAR
                                for i in range(self.num_hidden_layers)]


class RMSNorm(nn.Module):
    """Weight applied as (1 + w), normalised in fp32 ([hf]:720-737)."""

    def __init__(self, dim, eps):
        super().__init__()
        self.weight = nn.Parameter(torch.zeros(dim))
        self.eps = eps

    def forward(self, x):
        xf = x.float()
        y = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + self.eps)
        return (y * (1.0 + self.weight.float())).type_as(x)


class GatedRMSNorm(nn.Module):
    def __init__(self, dim, eps):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(dim))
        self.variance_epsilon = eps

    def forward(self, x, gate):
        """rmsnorm(x) * w * silu(gate): norm in fp32, weight in x's dtype ([hf]:168-184)."""
        dt = x.dtype
        xf = x.float()
        y = (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + self.variance_epsilon)).to(dt)
        return (self.weight * y * torch.nn.functional.silu(gate.float())).to(dt)


class MLP(nn.Module):
    def __init__(self, c: HybridConfig):
        super().__init__()
        self.gate_proj = nn.Linear(c.hidden_size, c.intermediate_size, bias=False)
        self.up_proj = nn.Linear(c.hidden_size, c.intermediate_size, bias=False)
        self.down_proj = nn.Linear(c.intermediate_size, c.hidden_size, bias=False)

    def forward(self, x):
        return self.down_proj(torch.nn.functional.silu(self.gate_proj(x)) * self.up_proj(x))


class GatedDeltaNet(nn.Module):
    def __init__(self, c: HybridConfig):
        super().__init__()
        self.num_k_heads = c.linear_num_key_heads
        self.num_v_heads = c.linear_num_value_heads
        self.head_k_dim = c.linear_key_head_dim
        self.head_v_dim = c.linear_value_head_dim
        self.key_dim = self.num_k_heads * self.head_k_dim
        self.value_dim = self.num_v_heads * self.head_v_dim
        self.conv_dim = 2 * self.key_dim + self.value_dim
        self.conv_kernel_size = c.linear_conv_kernel_dim
        self.activation = "silu"
        self.conv1d = nn.Conv1d(self.conv_dim, self.conv_dim, self.conv_kernel_size, groups=self.conv_dim,
                                bias=False, padding=self.conv_kernel_size - 1)
        self.dt_bias = nn.Parameter(torch.ones(self.num_v_heads))
        self.A_log = nn.Parameter(torch.zeros(self.num_v_heads))
        self.norm = GatedRMSNorm(self.head_v_dim, c.rms_norm_eps)
        self.out_proj = nn.Linear(self.value_dim, c.hidden_size, bias=False)
        self.in_proj_qkv = nn.Linear(c.hidden_size, self.conv_dim, bias=False)
        self.in_proj_z = nn.Linear(c.hidden_size, self.value_dim, bias=False)
        self.in_proj_b = nn.Linear(c.hidden_size, self.num_v_heads, bias=False)
        self.in_proj_a = nn.Linear(c.hidden_size, self.num_v_heads, bias=False)


class GatedAttention(nn.Module):
    def __init__(self, c: HybridConfig):
        super().__init__()
        self.head_dim = c.head_dim
        self.num_key_value_groups = c.num_attention_heads // c.num_key_value_heads
        self.scaling = self.head_dim ** -0.5
        self.q_proj = nn.Linear(c.hidden_size, c.num_attention_heads * c.head_dim * 2, bias=False)
        self.k_proj = nn.Linear(c.hidden_size, c.num_key_value_heads * c.head_dim, bias=False)
        self.v_proj = nn.Linear(c.hidden_size, c.num_key_value_heads * c.head_dim, bias=False)
        self.o_proj = nn.Linear(c.num_attention_heads * c.head_dim, c.hidden_size, bias=False)
        self.q_norm = RMSNorm(c.head_dim, c.rms_norm_eps)
        self.k_norm = RMSNorm(c.head_dim, c.rms_norm_eps)


class DecoderLayer(nn.Module):
    def __init__(self, c: HybridConfig, kind: str):
        super().__init__()
        self.layer_type = kind
        if kind == LINEAR:
            self.linear_attn = GatedDeltaNet(c)
        else:
            self.self_attn = GatedAttention(c)
        self.mlp = MLP(c)
        self.input_layernorm = RMSNorm(c.hidden_size, c.rms_norm_eps)
        self.post_attention_layernorm = RMSNorm(c.hidden_size, c.rms_norm_eps)


class Rotary(nn.Module):
    def __init__(self, c: HybridConfig):
        super().__init__()
        dim = int(c.head_dim * c.partial_rotary_factor)
        inv = 1.0 / (c.rope_theta ** (torch.arange(0, dim, 2, dtype=torch.float32) / dim))
        self.register_buffer("inv_freq", inv, persistent=False)


class HybridTextModel(nn.Module):
    def __init__(self, c: HybridConfig):
        super().__init__()
        self.config = c
        self.embed_tokens = nn.Embedding(c.vocab_size, c.hidden_size)
        self.layers = nn.ModuleList([DecoderLayer(c, c.layer_types[i]) for i in range(c.num_hidden_layers)])
        self.norm = RMSNorm(c.hidden_size, c.rms_norm_eps)
        self.rotary_emb = Rotary(c)


@torch.no_grad()
def init_random(model: HybridTextModel, lm_head: nn.Linear, *, std: float = 0.02, seed: int = 0):
    """Seeded init in place on the model's device: linear / embedding / conv weights ~ N(0, std),
    norm weights at their identity (0 for (1+w) norms, 1 for the gated norm), dt_bias = 1,
    A_log = log(U(1, 16)) per value head (decay rates like a trained model's)."""
    dev = next(model.parameters()).device
    gen = torch.Generator(device=dev).manual_seed(seed)
    for mod in list(model.modules()) + [lm_head]:
        if isinstance(mod, (nn.Linear, nn.Embedding, nn.Conv1d)):
            mod.weight.normal_(0.0, std, generator=gen)
        elif isinstance(mod, RMSNorm):
            mod.weight.zero_()
        elif isinstance(mod, GatedRMSNorm):
            mod.weight.fill_(1.0)
        elif isinstance(mod, GatedDeltaNet):
            mod.dt_bias.fill_(1.0)
            u = torch.rand(mod.A_log.shape, generator=gen, device=dev, dtype=torch.float32)
            mod.A_log.copy_(torch.log(1.0 + 15.0 * u))
    return model


def build(c: HybridConfig, *, device="cuda", dtype=torch.bfloat16, seed: int = 0, std: float = 0.02):
    """Model + untied lm_head, allocated and initialised directly on `device` in `dtype`."""
    with torch.device(device):
        model = HybridTextModel(c)
        lm_head = nn.Linear(c.hidden_size, c.vocab_size, bias=False)
    init_random(model, lm_head, std=std, seed=seed)
    model.to(dtype)
    lm_head.to(dtype)
    # decay parameters stay fp32, as in a checkpoint loaded with dtype bf16 they are cast but the
    # mixer upcasts them before use
    fuse_gate_up(model)
    return model.eval(), lm_head.eval()


def fuse_gate_up(model: nn.Module) -> None:
    """Store each MLP's gate and up weights as the two halves of one [2I, D] tensor (the modules'
    weights become views of it, so loading a state dict still writes into it), kept as
    `gate_up_weight`: the stack driver then runs one GEMM for both."""
    with torch.no_grad():
        for mod in model.modules():
            if hasattr(mod, "gate_proj") and hasattr(mod, "up_proj") and mod.gate_proj.bias is None \
                    and mod.up_proj.bias is None:
                w = torch.cat([mod.gate_proj.weight, mod.up_proj.weight], 0)
                n = mod.gate_proj.weight.shape[0]
                mod.gate_proj.weight = nn.Parameter(w[:n], requires_grad=mod.gate_proj.weight.requires_grad)
                mod.up_proj.weight = nn.Parameter(w[n:], requires_grad=mod.up_proj.weight.requires_grad)
                mod.gate_up_weight = w


def param_count(model: nn.Module) -> int:
    return sum(p.numel() for p in model.parameters())


def config_27b_truncated(layers: int = 16) -> HybridConfig:
    """27B-class hybrid geometry (hidden 5120, MLP 17408, GDN 16 key / 48 value heads of dim 128,
    attention 24 query / 4 key-value heads of dim 256), truncated to `layers` layers (3 GDN : 1
    attention), vocab 151936."""
    return HybridConfig(vocab_size=151936, hidden_size=5120, intermediate_size=17408, num_hidden_layers=layers,
                        num_attention_heads=24, num_key_value_heads=4, head_dim=256, linear_num_key_heads=16,
                        linear_num_value_heads=48, linear_key_head_dim=128, linear_value_head_dim=128,
                        linear_conv_kernel_dim=4, rope_theta=1e7, partial_rotary_factor=0.25)

