"""GPU parity of the prologue / epilogue kernels (RMSNorm(1+w) with fused residual, gated RMSNorm,
SwiGLU, q/k norm + partial RoPE) against the oracle's torch restatements of the transformers
modules. Bars: fp32 <= 1e-5 relative to max|ref|; bf16 within one bf16 ulp (2^-7 relative) of the
oracle computed from the same bf16 inputs (the reductions may sum in a different order, which can
flip one rounding of a normalised value); for RoPE outputs, which are sums of two rounded
products, one ulp of the largest operand (2^-8 max|ref|) is added to that bound."""

import pytest
import torch
import torch.nn.functional as F

from dllm_qwen38_amd import norms
from oracle import attn_ref, model_ref

pytestmark = pytest.mark.gpu


def _close(got, ref, dtype, name, floor=2 ** -12):
    got, ref = got.float().cpu(), ref.float()
    err = (got - ref).abs()
    scale = ref.abs().max().item() + 1e-30
    print(f"{name}: max|d|={err.max().item():.3e} max|ref|={scale:.3e}")
    if dtype == torch.float32:
        assert err.max().item() <= 1e-5 * scale, name
    else:
        assert (err <= 2 ** -7 * ref.abs() + floor * scale).all(), name


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("rows,dim", [(37, 64), (64, 5120), (5, 1000), (32, 2048), (8, 8192), (300, 5120)])
def test_rmsnorm_with_and_without_residual(dev, dtype, rows, dim):
    g = torch.Generator().manual_seed(rows + dim)
    x = torch.randn(rows, dim, generator=g).to(dtype)
    r = torch.randn(rows, dim, generator=g).to(dtype)
    w = (torch.randn(dim, generator=g) * 0.1).to(dtype)
    y = norms.rmsnorm(x.to(dev), w.to(dev), 1e-6)
    _close(y, model_ref.rmsnorm(x, w, 1e-6), dtype, f"rmsnorm {dtype} {rows}x{dim}")
    y2, s2 = norms.rmsnorm(x.to(dev), w.to(dev), 1e-6, residual=r.to(dev))
    s_ref = (r + x)  # the module adds in the activation dtype
    assert torch.equal(s2.cpu(), s_ref), "residual sum must be the dtype sum"
    _close(y2, model_ref.rmsnorm(s_ref, w, 1e-6), dtype, "add+rmsnorm")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("dim", [128, 64, 512, 96])
def test_gated_rmsnorm(dev, dtype, dim):
    g = torch.Generator().manual_seed(3 + dim)
    x = torch.randn(301, dim, generator=g).to(dtype)
    z = torch.randn(301, dim, generator=g).to(dtype)
    w = (1 + 0.1 * torch.randn(dim, generator=g)).to(dtype)
    y = norms.gated_rmsnorm(x.to(dev), z.to(dev), w.to(dev), 1e-6)
    _close(y, model_ref.gated_rmsnorm(x, z, w, 1e-6), dtype, f"gated rmsnorm {dtype}")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_swiglu(dev, dtype):
    g = torch.Generator().manual_seed(4)
    a = torch.randn(3, 1000, generator=g).to(dtype)
    b = torch.randn(3, 1000, generator=g).to(dtype)
    y = norms.swiglu(a.to(dev), b.to(dev))
    _close(y, F.silu(a) * b, dtype, f"swiglu {dtype}")


class _Norm:
    def __init__(self, w):
        self.weight, self.eps = w, 1e-6


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("Hq,Hkv,hd,rd", [(4, 2, 16, 4), (6, 2, 256, 64), (3, 1, 128, 32), (2, 1, 256, 256), (2, 2, 256, 8)])
def test_qk_norm_rope(dev, dtype, Hq, Hkv, hd, rd):
    B, L = 2, 24
    S = 2 * L
    g = torch.Generator().manual_seed(hd + rd)
    qg = torch.randn(B, S, Hq, 2 * hd, generator=g).to(dtype)  # q_proj output with the gate half
    q = qg[..., :hd]
    k = torch.randn(B, S, Hkv, hd, generator=g).to(dtype)
    wq = (0.1 * torch.randn(hd, generator=g)).to(dtype)
    wk = (0.1 * torch.randn(hd, generator=g)).to(dtype)
    inv = 1.0 / (1e4 ** (torch.arange(0, rd, 2, dtype=torch.float32) / rd))
    fr = torch.arange(L, dtype=torch.float32)[:, None] * inv[None, :]
    emb = torch.cat([fr, fr], -1)
    cos, sin = emb.cos().to(dtype), emb.sin().to(dtype)
    # the strided view is built on the device, as the layer passes it (row stride 2*hd inside a
    # token of Hq*2*hd): a .to(dev) of the CPU view would make a dense copy
    qd = qg.to(dev)[..., :hd]
    assert qd.stride(-2) == 2 * hd and qd.stride(1) == Hq * 2 * hd
    qo, ko = norms.qk_norm_rope(qd, k.to(dev), _Norm(wq.to(dev)), _Norm(wk.to(dev)), cos.to(dev), sin.to(dev), L)
    c2, s2 = torch.cat([cos, cos]), torch.cat([sin, sin])
    q_ref = attn_ref.apply_rope(model_ref.rmsnorm(q, wq, 1e-6), c2, s2)
    k_ref = attn_ref.apply_rope(model_ref.rmsnorm(k, wk, 1e-6), c2, s2)
    _close(qo, q_ref, dtype, f"q {dtype} hd{hd} rd{rd}", floor=2 ** -8)
    _close(ko, k_ref, dtype, f"k {dtype} hd{hd} rd{rd}", floor=2 ** -8)


@pytest.mark.parametrize("dtype,pdtype", [(torch.bfloat16, torch.float32), (torch.bfloat16, torch.bfloat16),
                                          (torch.float32, torch.float32)])
def test_gdn_gates_match_torch(dev, dtype, pdtype):
    """beta = sigmoid(b) rounded to b's dtype: within one ulp of bf16, or within 4 fp32 ulps (two
    exp implementations and the reciprocal, each within a couple of ulps); g = -exp(A_log) *
    softplus(a + dt_bias) in fp32 (relative 1e-6), including the linear branch of softplus above 20."""
    g = torch.Generator().manual_seed(3)
    H = 48
    b = (torch.randn(7, 33, H, generator=g) * 4).to(dtype)
    a = (torch.randn(7, 33, H, generator=g) * 12).to(dtype)
    a_log = torch.log(torch.rand(H, generator=g) * 15 + 1).to(pdtype)
    dt_bias = torch.randn(H, generator=g).to(pdtype)
    beta, gg = norms.gdn_gates(b.to(dev), a.to(dev), a_log.to(dev), dt_bias.to(dev))
    torch.cuda.synchronize()
    rb = b.float().sigmoid().to(dtype).float()
    ulp = (1 if dtype == torch.bfloat16 else 4) * torch.finfo(dtype).eps * rb.abs().clamp_min(torch.finfo(dtype).tiny)
    assert ((beta.cpu() - rb).abs() <= ulp).all()
    rg = -a_log.float().exp() * torch.nn.functional.softplus(a.float() + dt_bias.float())
    assert ((gg.cpu() - rg).abs() <= 1e-6 * rg.abs() + 1e-30).all()
    assert (a.float() + dt_bias.float() > 20).any()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_swiglu_on_the_halves_of_a_fused_projection(dev, dtype):
    """The row-strided form (gate and up the column halves of one gate | up output) equals the
    contiguous form bit for bit."""
    g = torch.Generator().manual_seed(34816)
    y = torch.randn(3, 40, 2 * 272, generator=g).to(dtype).to(dev)
    gate, up = y[..., :272], y[..., 272:]
    assert not gate.is_contiguous()
    got = norms.swiglu(gate, up)
    ref = norms.swiglu(gate.contiguous(), up.contiguous())
    assert got.is_contiguous() and torch.equal(got, ref)
