"""Complementary-mask attention over a seeded spread of shapes, against the CPU oracle.

Each case draws a batch, a length of 1 to 6 blocks, a block of 8 to 64 tokens (24 included: not a
divisor of the 32-key tile), K/V heads and a GQA ratio of 1 to 6, a head size among 16, 48, 64,
80, 128, 200 and 256 (the sizes between the instantiated 32/64/128/256 are zero-padded in LDS) and
bf16 or fp32. Tolerances are those of tests/test_gpu_attn.py: fp32 1e-5 max-abs; bf16 one bf16
ulp of the probabilities the reference rounds before P.V plus the output rounding. The shapes are
drawn once from a fixed seed, the same on every run."""

import random

import pytest
import torch

from dllm_qwen38_amd import attention
from oracle import attn_ref

pytestmark = pytest.mark.gpu


def _cases(n=16, seed=20261203):
    rng = random.Random(seed)
    out = []
    for _ in range(n):
        dtype = rng.choice([torch.bfloat16, torch.bfloat16, torch.float32])
        block = rng.choice([8, 16, 24, 32, 64])
        L = block * rng.choice([1, 2, 3, 4, 6])
        Hkv = rng.choice([1, 2])
        Hq = Hkv * rng.choice([1, 2, 3, 6])
        d = rng.choice([16, 48, 64, 80, 128, 200, 256])
        B = rng.choice([1, 2, 3])
        out.append((B, L, Hq, Hkv, d, block, dtype))
    return out


CASES = _cases()


def _id(c):
    B, L, Hq, Hkv, d, block, dtype = c
    return f"B{B} L{L} Hq{Hq} Hkv{Hkv} d{d} block{block} {'bf16' if dtype == torch.bfloat16 else 'fp32'}"


@pytest.mark.parametrize("case", CASES, ids=[_id(c) for c in CASES])
def test_attention_sweep_matches_oracle(dev, case):
    B, L, Hq, Hkv, d, block, dtype = case
    g = torch.Generator().manual_seed(B * 1000003 + L * 1009 + Hq * 101 + d * 7 + block)
    q = torch.randn(B, 2 * L, Hq, d, generator=g).to(dtype)
    k = torch.randn(B, 2 * L, Hkv, d, generator=g).to(dtype)
    v = torch.randn(B, 2 * L, Hkv, d, generator=g).to(dtype)
    got = attention.bd_attention(q.to(dev), k.to(dev), v.to(dev), block=block)
    torch.cuda.synchronize()
    ref = attn_ref.bd_attention(q, k, v, block=block)
    err = (got.float().cpu() - ref.float()).abs()
    print(f"{_id(case)}: max|d|={err.max().item():.3e}", flush=True)
    if dtype == torch.float32:
        assert err.max().item() <= 1e-5
    else:
        bound = 2 ** -8 * v.float().abs().max() + 2 ** -7 * ref.float().abs()
        assert (err <= bound).all()
