"""Seeded synthetic inputs of the block-diffusion forward workloads (CPU generation, fixed seeds).

All tensors are drawn on the CPU from torch.Generator().manual_seed(seed) in fp32 and cast to the
op dtype, so a CPU check and a GPU run see identical bits. Seed map: seed = 100 * workload + slot,
slots 0 raw qkv clean, 1 raw qkv noised, 2/3 beta logits clean/noised, 4/5 g logits clean/noised,
6 conv weight, 7/8/9 attention Q/K/V, 10 token ids, 11 per-block t, 12 per-token u, 13 weights.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn.functional as F


@dataclass(frozen=True)
class GdnShape:
    name: str
    B: int
    L: int
    block: int
    Hk: int
    Hv: int
    D: int
    width: int
    dtype: torch.dtype
    g_shift: float  # g = -softplus(N(0,1) + g_shift)
    seed_base: int

    @property
    def conv_dim(self) -> int:
        return 2 * self.Hk * self.D + self.Hv * self.D

    @property
    def nb(self) -> int:
        return self.L // self.block


# The three state-fork GDN layer workloads.
GDN_TINY_F32 = GdnShape("gdn-tiny-fp32: B=1 L=128 block=32 H=4 D=64 fp32", 1, 128, 32, 4, 4, 64, 4,
                        torch.float32, 0.0, 100)
GDN_08B_BF16 = GdnShape("gdn-0.8B-class: B=8 L=2048 block=32 Hk=Hv=16 D=128 bf16", 8, 2048, 32, 16, 16, 128, 4,
                        torch.bfloat16, 0.0, 200)
GDN_27B_BF16 = GdnShape("gdn-27B-class: B=4 L=4096 block=32 Hk=16 Hv=48 D=128 bf16", 4, 4096, 32, 16, 48, 128, 4,
                        torch.bfloat16, 1.0, 300)


def _randn(shape, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g, dtype=torch.float32)


def _rand(shape, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.rand(shape, generator=g, dtype=torch.float32)


def gdn_layer_inputs(s: GdnShape, *, B: int | None = None, L: int | None = None, seed_base: int | None = None,
                     g_shift: float | None = None) -> dict:
    """Pre-conv projections of both streams and the gates of a state-fork GDN layer (CPU tensors).

    raw0/rawt [B,L,conv_dim] ~ N(0,1) (op dtype); beta = sigmoid(N(0,1)) rounded to the op dtype and
    held in fp32; g = -softplus(N(0,1) + shift) fp32; conv weight ~ U(-0.5, 0.5) [conv_dim, width]
    (the nn.Conv1d default bound 1/sqrt(width), no bias). B / L / seed / shift may be overridden
    for reduced-size checks of the same shape family."""
    B = s.B if B is None else B
    L = s.L if L is None else L
    base = s.seed_base if seed_base is None else seed_base
    shift = s.g_shift if g_shift is None else g_shift
    Cd, Hv, dt = s.conv_dim, s.Hv, s.dtype
    raw0 = _randn((B, L, Cd), base + 0).to(dt)
    rawt = _randn((B, L, Cd), base + 1).to(dt)
    beta0 = torch.sigmoid(_randn((B, L, Hv), base + 2)).to(dt).float()
    betat = torch.sigmoid(_randn((B, L, Hv), base + 3)).to(dt).float()
    g0 = -F.softplus(_randn((B, L, Hv), base + 4) + shift)
    gt = -F.softplus(_randn((B, L, Hv), base + 5) + shift)
    w = (_rand((Cd, s.width), base + 6) - 0.5).to(dt)
    return {"raw0": raw0, "rawt": rawt, "beta0": beta0, "betat": betat, "g0": g0, "gt": gt, "conv_w": w}


def gdn_core_inputs(B, T, Hk, Hv, D, dtype, seed, g_shift=0.0):
    """Already-convolved q, k [B,T,Hk,D], v [B,T,Hv,D] ~ N(0,1); beta, g as above."""
    q = _randn((B, T, Hk, D), seed + 0).to(dtype)
    k = _randn((B, T, Hk, D), seed + 1).to(dtype)
    v = _randn((B, T, Hv, D), seed + 2).to(dtype)
    beta = torch.sigmoid(_randn((B, T, Hv), seed + 3)).to(dtype).float()
    g = -F.softplus(_randn((B, T, Hv), seed + 4) + g_shift)
    return q, k, v, g, beta
