"""GPU parity of the gated attention layer's core in one launch (bd_attention_gated): the q
RMSNorm(1 + w) and partial RoPE applied as the kernel loads q, and the sigmoid output gate applied
as it stores the output ([hf]:672-698 around the complementary-mask attention).

  * against the fp32 CPU oracle of the same chain (model_ref.rmsnorm, attn_ref.apply_rope,
    attn_ref.bd_attention, sigmoid gate), within the bf16 attention bar of tests/test_gpu_attn.py
    (2^-8 max|V| + 2^-7 |ref|) scaled by the gate (|sigmoid| < 1) plus one bf16 ulp of the product;
  * against the separate launches (qk_norm_rope, bd_attention, torch's sigmoid product) on the
    same inputs: within two bf16 ulps per element where the separate prologue is the 256-wide bf16
    kernel. The two kernels sum a q row's squares in different orders, so 1/rms may differ in its
    last bit; that flips the rounding of an occasional normalised q element, and through the
    scores every output of that row moves by about an ulp. Against the generic prologue kernel
    (other head sizes, fp32 norm weights), whose order differs for most rows, within the oracle bar;
  * the k-only prologue equals the k output of the two-tensor prologue bit for bit.
"""

import pytest
import torch

from dllm_qwen38_amd import attention, norms
from oracle import attn_ref, model_ref

pytestmark = pytest.mark.gpu


class _Norm:
    def __init__(self, w):
        self.weight, self.eps = w, 1e-6


def _tables(L, rd, dtype):
    inv = 1.0 / (1e7 ** (torch.arange(0, rd, 2, dtype=torch.float32) / rd))
    fr = torch.arange(L, dtype=torch.float32)[:, None] * inv[None, :]
    emb = torch.cat([fr, fr], -1)
    return emb.cos().to(dtype), emb.sin().to(dtype)


def _inputs(B, L, Hq, Hkv, d, rd, seed, wdtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    S = 2 * L
    qg = torch.randn(B, S, Hq, 2 * d, generator=g).to(torch.bfloat16)  # q_proj output: query | gate per head
    k = torch.randn(B, S, Hkv, d, generator=g).to(torch.bfloat16)
    v = torch.randn(B, S, Hkv, d, generator=g).to(torch.bfloat16)
    wq = (0.1 * torch.randn(d, generator=g)).to(wdtype)
    wk = (0.1 * torch.randn(d, generator=g)).to(wdtype)
    cos, sin = _tables(L, rd, torch.bfloat16)
    return qg, k, v, wq, wk, cos, sin


CASES = [  # B, L, Hq, Hkv, d, rd, block, leak, norm weight dtype
    (1, 128, 6, 2, 256, 64, 32, False, torch.bfloat16),   # the 27B-class attention layer's head geometry
    (2, 96, 4, 1, 256, 128, 32, False, torch.bfloat16),
    (1, 64, 4, 2, 128, 64, 16, False, torch.bfloat16),
    (1, 64, 2, 2, 64, 64, 8, False, torch.bfloat16),
    (1, 128, 6, 2, 256, 64, 32, True, torch.bfloat16),    # the mask-leak fault
    (1, 64, 4, 2, 256, 192, 32, False, torch.float32),    # three rotated slice pairs, fp32 norm weights
    (1, 96, 2, 1, 256, 256, 32, False, torch.bfloat16),   # the whole head rotated
    (2, 64, 4, 2, 128, 128, 32, False, torch.float32),
]


@pytest.mark.parametrize("B,L,Hq,Hkv,d,rd,block,leak,wdtype", CASES)
def test_gated_attention_one_launch(dev, B, L, Hq, Hkv, d, rd, block, leak, wdtype):
    qg, k, v, wq, wk, cos, sin = _inputs(B, L, Hq, Hkv, d, rd, seed=91 + d + rd + L, wdtype=wdtype)
    S = 2 * L
    qgd = qg.to(dev)
    q, gate = qgd[..., :d], qgd[..., d:]  # strided views, as the layer passes them
    kd = norms.k_norm_rope(k.to(dev), _Norm(wk.to(dev)), cos.to(dev), sin.to(dev), L)
    assert attention.gated_supported(q, d, rd)
    got = attention.bd_attention_gated(q, kd, v.to(dev), gate, block=block, q_norm_weight=wq.to(dev), q_norm_eps=1e-6,
                                       cos=cos.to(dev), sin=sin.to(dev), leak_xt_prefix=leak)
    # the separate launches on the same inputs
    qn, kn = norms.qk_norm_rope(q, k.to(dev), _Norm(wq.to(dev)), _Norm(wk.to(dev)), cos.to(dev), sin.to(dev), L)
    assert torch.equal(kn, kd), "the k-only prologue must equal the k output of the two-tensor prologue"
    sep = attention.bd_attention(qn, kn, v.to(dev), block=block, leak_xt_prefix=leak)
    sep = sep * torch.sigmoid(gate)
    torch.cuda.synchronize()
    # the fp32 oracle of the chain on the same bf16 inputs
    c2, s2 = torch.cat([cos, cos]), torch.cat([sin, sin])
    qr = attn_ref.apply_rope(model_ref.rmsnorm(qg[..., :d].float(), wq.float(), 1e-6), c2.float(), s2.float())
    kr = attn_ref.apply_rope(model_ref.rmsnorm(k.float(), wk.float(), 1e-6), c2.float(), s2.float())
    ref = attn_ref.bd_attention(qr, kr, v.float(), block=block, leak_xt_prefix=leak)
    ref = ref * torch.sigmoid(qg[..., d:].float())
    bar = 2 ** -8 * v.float().abs().max() + 2 ** -7 * ref.abs() + 2 ** -8 * ref.abs()
    for name, t in (("one launch", got), ("separate launches", sep)):
        err = (t.float().cpu() - ref).abs()
        print(f"{name} vs fp32 oracle: max|d|={err.max().item():.3e} max|ref|={ref.abs().max().item():.3e} "
              f"max |d|/bar={(err / bar).max().item():.3f}", flush=True)
        assert (err <= bar).all(), name
    diff = (got.float() - sep.float()).abs().cpu()
    frac = (diff > 0).float().mean().item()
    if d == 256 and wdtype == torch.bfloat16:
        # the separate prologue is the 256-wide bf16 kernel, whose row sums the fused load matches
        # but for an occasional last bit: within two bf16 ulps per element
        cross = 2 ** -6 * sep.float().abs().cpu() + 2 ** -9 * sep.float().abs().max().item()
    else:
        # the generic prologue kernel sums a row's squares in another order, so 1/rms differs in its
        # last bit for most rows and normalised q elements round differently throughout the tile:
        # the two launches then agree only as well as each agrees with the oracle (the same bar)
        cross = bar
    print(f"one launch vs separate launches: {frac:.2%} of elements differ, max|d|={diff.max().item():.3e}, "
          f"max |d|/bound={(diff / cross).max().item():.3f}")
    assert (diff <= cross).all()
    assert got.shape == (B, S, Hq, d) and got.is_contiguous()


def test_gated_attention_refusals(dev):
    """Shapes outside the fused form raise (callers then run the separate launches)."""
    qg, k, v, wq, wk, cos, sin = _inputs(1, 64, 2, 1, 256, 32, seed=5)
    q = qg.to(dev)[..., :256]
    assert not attention.gated_supported(q, 256, 32)
    assert not attention.gated_supported(q.float(), 256, 64)
    with pytest.raises(RuntimeError, match="multiple of 64"):
        attention.bd_attention_gated(q, k.to(dev), v.to(dev), None, block=32, q_norm_weight=wq.to(dev),
                                     cos=cos.to(dev), sin=sin.to(dev))
