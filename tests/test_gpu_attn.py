"""GPU parity of the complementary-mask attention kernel against the CPU oracle.

Bars: fp32 <= 1e-5 max-abs; bf16 within 2^-8 * max|V| + 2^-7 * |ref| of the fp32 oracle on the same
bf16 inputs: the reference's eager attention rounds the probabilities to bf16 before P.V
(transformers modeling_qwen3_5.py:621-622), which alone moves an output by up to one bf16 ulp of
P times |V|, and the output itself is rounded to bf16."""

import pytest
import torch

from dllm_qwen38_amd import attention
from oracle import attn_ref

pytestmark = pytest.mark.gpu

F32_TOL = 1e-5
BF16_RTOL = 2 ** -7


def _inputs(B, L, Hq, Hkv, d, dtype, seed, std=1.0):
    g = torch.Generator().manual_seed(seed)
    q = (torch.randn(B, 2 * L, Hq, d, generator=g) * std).to(dtype)
    k = (torch.randn(B, 2 * L, Hkv, d, generator=g) * std).to(dtype)
    v = (torch.randn(B, 2 * L, Hkv, d, generator=g) * std).to(dtype)
    return q, k, v


def _check(got, ref, dtype, name, vmax=None):
    err = (got.float().cpu() - ref.float()).abs()
    print(f"{name}: max|d|={err.max().item():.3e} max|ref|={ref.abs().max().item():.3e}")
    if dtype == torch.float32:
        assert err.max().item() <= F32_TOL, name
    else:
        atol = 2 ** -8 * vmax
        assert (err <= atol + BF16_RTOL * ref.float().abs()).all(), name


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("B,L,Hq,Hkv,d,block", [
    (1, 128, 6, 2, 256, 32),   # aligned blocks: whole tiles visible or hidden
    (2, 64, 4, 4, 128, 8),     # small blocks: element masks on partial tiles
    (1, 40, 4, 2, 64, 8),      # ragged length (L % 32 != 0)
    (2, 32, 4, 2, 16, 8),      # the tiny model's head size, padded to 32
    (1, 96, 2, 1, 32, 16),
    (1, 200, 6, 1, 256, 8),    # d = 256, six query heads on one K/V head, ragged L, element masks
    (3, 160, 4, 2, 256, 16),   # d = 256, query groups crossing blocks, B = 3
    (1, 72, 2, 1, 128, 24),    # a block that is not a divisor of the 32-key tile
    (1, 256, 4, 2, 256, 64),   # blocks longer than the 32-key tile
    (2, 192, 4, 1, 128, 64),
])
def test_bd_attention_matches_oracle(dev, dtype, B, L, Hq, Hkv, d, block):
    q, k, v = _inputs(B, L, Hq, Hkv, d, dtype, seed=L + d + block)
    got = attention.bd_attention(q.to(dev), k.to(dev), v.to(dev), block=block)
    torch.cuda.synchronize()
    ref = attn_ref.bd_attention(q, k, v, block=block)
    _check(got, ref, dtype, f"{dtype} B{B} L{L} Hq{Hq} Hkv{Hkv} d{d} block{block}", v.float().abs().max().item())


@pytest.mark.parametrize("scale", [0.2, -0.05, 0.0])
def test_custom_scales(dev, scale):
    """A positive scale runs the bf16 direct-load kernel (its softmax max is taken over the raw
    scores and scaled once, which needs scale > 0); zero or negative scales run the general kernel."""
    q, k, v = _inputs(1, 128, 4, 2, 128, torch.bfloat16, seed=77)
    got = attention.bd_attention(q.to(dev), k.to(dev), v.to(dev), block=32, scale=scale)
    torch.cuda.synchronize()
    ref = attn_ref.bd_attention(q, k, v, block=32, scale=scale)
    _check(got, ref, torch.bfloat16, f"scale {scale}", v.float().abs().max().item())


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("d", [64, 256])
def test_mask_leak_fault_matches_oracle_and_differs(dev, dtype, d):
    q, k, v = _inputs(1, 64, 4, 2, d, dtype, seed=5)
    good = attention.bd_attention(q.to(dev), k.to(dev), v.to(dev), block=16)
    bad = attention.bd_attention(q.to(dev), k.to(dev), v.to(dev), block=16, leak_xt_prefix=True)
    torch.cuda.synchronize()
    _check(bad, attn_ref.bd_attention(q, k, v, block=16, leak_xt_prefix=True), dtype, "leak",
           v.float().abs().max().item())
    assert (bad.float() - good.float()).abs().max().item() > 1e-2
    # the clean half (x_0 queries) is unaffected by the fault
    assert torch.equal(bad[:, 64:], good[:, 64:])


def test_strided_inputs_from_a_fused_projection(dev):
    """q/k/v as non-contiguous head views of one [B, 2L, (Hq+2Hkv)*d] projection buffer."""
    B, L, Hq, Hkv, d = 1, 64, 4, 2, 128
    g = torch.Generator().manual_seed(6)
    proj = torch.randn(B, 2 * L, (Hq + 2 * Hkv) * d, generator=g).to(torch.bfloat16)
    q = proj[..., : Hq * d].unflatten(-1, (Hq, d))
    k = proj[..., Hq * d: (Hq + Hkv) * d].unflatten(-1, (Hkv, d))
    v = proj[..., (Hq + Hkv) * d:].unflatten(-1, (Hkv, d))
    pd = proj.to(dev)
    got = attention.bd_attention(pd[..., : Hq * d].unflatten(-1, (Hq, d)),
                                 pd[..., Hq * d: (Hq + Hkv) * d].unflatten(-1, (Hkv, d)),
                                 pd[..., (Hq + Hkv) * d:].unflatten(-1, (Hkv, d)), block=32)
    torch.cuda.synchronize()
    _check(got, attn_ref.bd_attention(q, k, v, block=32), torch.bfloat16, "strided", v.float().abs().max().item())


def test_27b_attention_shape_sampled_rows_and_determinism(dev):
    """Full B=2, L=4096, Hq=24, Hkv=4, d=256 layer (inputs N(0,1)/16): rows of a few query blocks of
    both halves against the oracle restricted to those rows; two runs bit-identical."""
    B, L, Hq, Hkv, d, block = 2, 4096, 24, 4, 256, 32
    q, k, v = _inputs(B, L, Hq, Hkv, d, torch.bfloat16, seed=407, std=1.0 / 16)
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    o1 = attention.bd_attention(qd, kd, vd, block=block)
    o2 = attention.bd_attention(qd, kd, vd, block=block)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2)
    allowed = attn_ref.complementary_allowed(L, block)
    scale = d ** -0.5
    rows = [0, 31, 32, 2000, 4095, L + 0, L + 1500, L + 4095]
    kx = k.float().repeat_interleave(Hq // Hkv, 2)
    vx = v.float().repeat_interleave(Hq // Hkv, 2)
    for r in rows:
        sc = torch.einsum("bhd,bjhd->bhj", q[:, r].float(), kx) * scale
        sc = sc.masked_fill(~allowed[r][None, None], float("-inf"))
        ref = torch.einsum("bhj,bjhd->bhd", torch.softmax(sc, -1), vx)
        _check(o1[:, r], ref, torch.bfloat16, f"27B-class attention row {r}", v.float().abs().max().item())


def test_empty_queries_give_empty_outputs(dev):
    """No queries (empty batch or sequence): an empty output of the right shape, no launch, as the
    reference's eager attention returns for an empty score matrix."""
    for B, L in ((0, 64), (2, 0)):
        q = torch.randn(B, 2 * L, 4, 64, device=dev, dtype=torch.bfloat16)
        k = torch.randn(B, 2 * L, 2, 64, device=dev, dtype=torch.bfloat16)
        assert attention.bd_attention(q, k, k, block=32).shape == (B, 2 * L, 4, 64)
    q = torch.randn(2, 0, 4, 64, device=dev, dtype=torch.bfloat16)
    k = torch.randn(2, 96, 2, 64, device=dev, dtype=torch.bfloat16)
    assert attention.block_causal_attention(q, k, k, block=32, q_offset=64).shape == (2, 0, 4, 64)
    torch.cuda.synchronize()
