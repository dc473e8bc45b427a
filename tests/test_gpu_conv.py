"""GPU parity of the causal depthwise conv kernels (conv + SiLU, conv-prefix carry-in).

Compared with the oracle's conv (transformers' cast points: the input converted to the weight
dtype, fp32 accumulation rounded to the weight dtype, SiLU in fp32 rounded to the weight dtype,
result in the input dtype) and, for fp32, with a float64 FIR loop.

Bounds. The kernels evaluate SiLU from the hardware base-2 exponential and reciprocal, each within
1 ulp, so silu(x) is within a few fp32 ulps of x / (1 + e^-x); the 4-tap sum can differ from the
oracle's accumulation order by an ulp of the partial sums.
  * bf16 weights or a bf16 result: the rounded conv and the rounded SiLU agree with the oracle unless an fp32
    value falls within those few ulps of a bf16 rounding midpoint, where they differ by one bf16
    ulp (<= 2^-7 |ref|). Asserted: every element within one ulp, at most 1% of them not equal.
  * fp32 weights: |d| <= 2^-19 (1 + |ref|) against the oracle (a few fp32 ulps of values of
    magnitude up to ~4), and <= 2^-18 (1 + |ref|) against the float64 loop.
"""

import pytest
import torch

from dllm_qwen38_amd import _lib, gdn
from oracle import gdn_ref

pytestmark = pytest.mark.gpu


def _data(B, L, Cd, K, dtx, dtw, seed, bias):
    g = torch.Generator().manual_seed(seed)
    raw0 = torch.randn(B, L, Cd, generator=g).to(dtx)
    rawt = torch.randn(B, L, Cd, generator=g).to(dtx)
    w = (torch.rand(Cd, K, generator=g) - 0.5).to(dtw)
    b = (0.1 * torch.randn(Cd, generator=g)).to(dtw) if bias else None
    return raw0, rawt, w, b


def _close(name, got, ref, lowp, f64=None):
    """lowp: a bf16 rounding anywhere in the chain (bf16 weights, or a bf16 result)."""
    got, ref = got.float(), ref.float()
    d = (got - ref).abs()
    if lowp:
        ulp = 2.0 ** -7 * ref.abs()
        frac = (d > 0).float().mean().item()
        print(f"{name}: max|d|={d.max().item():.3e} not-equal={frac:.2e}", flush=True)
        assert (d <= ulp).all(), f"{name}: more than one bf16 ulp"
        assert frac <= 0.01, f"{name}: {frac:.2%} of the elements differ"
    else:
        print(f"{name}: max|d|={d.max().item():.3e}", flush=True)
        assert (d <= 2.0 ** -19 * (1 + ref.abs())).all(), f"{name}: beyond a few fp32 ulps"
        if f64 is not None:
            d64 = (got.double() - f64).abs()
            assert (d64 <= 2.0 ** -18 * (1 + f64.abs())).all(), f"{name}: far from the float64 FIR"


def _fork_conv(raw0, rawt, w, b, block, cold, dev):
    B, L, Cd = raw0.shape
    K = w.shape[1]
    nb = L // block
    d = [t.to(dev) for t in (raw0, rawt, w)]
    bd = b.to(dev) if b is not None else None
    y0, yt = torch.empty_like(d[0]), torch.empty_like(d[0])
    tails = torch.empty(B * nb, Cd, K - 1, dtype=raw0.dtype, device=dev)
    _lib.check(_lib.lib().dllm_conv_fork_fwd(
        d[0].data_ptr(), d[1].data_ptr(), d[2].data_ptr(), _lib.ptr(bd), y0.data_ptr(), yt.data_ptr(), tails.data_ptr(),
        B, L, Cd, K, block, _lib.dtype_code(raw0.dtype), _lib.dtype_code(w.dtype), int(cold),
        _lib.stream_handle(dev)), "dllm_conv_fork_fwd")
    torch.cuda.synchronize()
    return y0.cpu(), yt.cpu(), tails.cpu()


def _fork_conv_ref(raw0, rawt, w, b, block, cold):
    B, L, Cd = raw0.shape
    K = w.shape[1]
    nb = L // block
    y0 = gdn_ref.causal_conv1d(raw0.transpose(1, 2), w, b).transpose(1, 2)
    padded = torch.cat([torch.zeros(B, Cd, K - 1, dtype=raw0.dtype), raw0.transpose(1, 2)], 2)
    tails = padded.unfold(2, K - 1, block)[:, :, :nb].permute(0, 2, 1, 3).reshape(B * nb, Cd, K - 1)
    xt = rawt.reshape(B * nb, block, Cd).transpose(1, 2)
    yt = gdn_ref.causal_conv1d(xt, w, b, prefix=None if cold else tails).transpose(1, 2).reshape(B, L, Cd)
    return y0, yt, tails.contiguous()


# (dtype_x, dtype_w, width, block, Cd, bias, cold): the bf16 block-32 8-byte-group kernel, the
# 16-byte-group kernel (other blocks), the one-channel kernel (Cd not a multiple of 8, widths 2/3),
# fp32 and mixed dtypes, bias, and the no-conv-prefix fault
CASES = [
    (torch.bfloat16, torch.bfloat16, 4, 32, 1024, False, False),
    (torch.bfloat16, torch.bfloat16, 4, 32, 1024, False, True),
    (torch.bfloat16, torch.bfloat16, 4, 16, 1024, True, False),
    (torch.bfloat16, torch.bfloat16, 4, 8, 200, False, False),
    (torch.bfloat16, torch.bfloat16, 2, 32, 96, False, False),
    (torch.bfloat16, torch.bfloat16, 3, 4, 96, True, False),
    (torch.float32, torch.float32, 4, 32, 1024, False, False),
    (torch.float32, torch.float32, 4, 16, 1024, True, True),
    (torch.float32, torch.float32, 3, 8, 100, False, False),
    (torch.float32, torch.float32, 2, 2, 100, True, False),
    (torch.bfloat16, torch.float32, 4, 32, 512, False, False),
    (torch.float32, torch.bfloat16, 4, 32, 512, True, False),
]


@pytest.mark.parametrize("dtx,dtw,K,block,Cd,bias,cold", CASES)
def test_conv_fork_matches_oracle(dev, dtx, dtw, K, block, Cd, bias, cold):
    B, L = 2, 128
    raw0, rawt, w, b = _data(B, L, Cd, K, dtx, dtw, seed=K * 1000 + block + Cd, bias=bias)
    y0, yt, tails = _fork_conv(raw0, rawt, w, b, block, cold, dev)
    r0, rt, rtails = _fork_conv_ref(raw0, rawt, w, b, block, cold)
    assert torch.equal(tails, rtails), "conv tails are copies of the clean inputs"
    tag = f"{dtx}/{dtw} K{K} block{block} Cd{Cd} bias{int(bias)} cold{int(cold)}"
    f64 = None
    if dtw == torch.float32 and dtx == torch.float32:
        f64 = torch.from_numpy(gdn_ref.causal_conv1d_bruteforce_f64(raw0.transpose(1, 2), w, b)).transpose(1, 2)
    lowp = torch.bfloat16 in (dtx, dtw)
    _close(f"y0 {tag}", y0, r0, lowp, f64)
    _close(f"yt {tag}", yt, rt, lowp)
    if cold:  # the fault: every noised block starts from zeros, so block 0 is unchanged and the rest move
        warm = _fork_conv(raw0, rawt, w, b, block, False, dev)[1]
        assert torch.equal(warm[:, :block], yt[:, :block])
        assert not torch.equal(warm, yt)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("K,P,bias,silu", [(4, 3, False, True), (4, 5, True, True), (2, 1, False, True),
                                           (6, 5, True, False), (3, 0, False, True)])
def test_causal_conv1d_fn_matches_oracle(dev, dtype, K, P, bias, silu):
    """The generic conv on a strided [B, C, T] view of token-major storage (as the mixer passes
    it) and on a dense [B, C, T] tensor, with a prefix of P positions."""
    B, T, C = 2, 48, 160
    g = torch.Generator().manual_seed(K * 100 + P)
    x_tm = torch.randn(B, T, C, generator=g).to(dtype)
    w = (torch.rand(C, K, generator=g) - 0.5).to(dtype)
    b = (0.1 * torch.randn(C, generator=g)).to(dtype) if bias else None
    pre = torch.randn(B, C, P, generator=g).to(dtype) if P else None
    act = "silu" if silu else None
    ref = gdn_ref.causal_conv1d(x_tm.transpose(1, 2), w, b, act, prefix=pre)
    f64 = None
    if dtype == torch.float32 and silu:
        f64 = torch.from_numpy(gdn_ref.causal_conv1d_bruteforce_f64(x_tm.transpose(1, 2), w, b, prefix=pre))
    for name, xd in (("strided", x_tm.to(dev).transpose(1, 2)), ("dense", x_tm.transpose(1, 2).contiguous().to(dev))):
        y = gdn.causal_conv1d_fn(xd, w.to(dev), None if b is None else b.to(dev), activation=act,
                                 conv_prefix=None if pre is None else pre.to(dev))
        torch.cuda.synchronize()
        assert y.shape == (B, C, T)
        _close(f"{name} {dtype} K{K} P{P}", y.cpu(), ref, dtype == torch.bfloat16, f64)


def test_causal_conv1d_fn_package_keywords(dev):
    """initial_states is the prefix under the causal-conv1d package's name; return_final_states
    gives the last K-1 inputs of the extended sequence; seq_idx and a doubled prefix raise."""
    g = torch.Generator().manual_seed(5)
    x = torch.randn(1, 64, 20, generator=g).to(dev)
    w = (torch.rand(64, 4, generator=g) - 0.5).to(dev)
    pre = torch.randn(1, 64, 3, generator=g).to(dev)
    a = gdn.causal_conv1d_fn(x, w, activation="silu", conv_prefix=pre)
    b, fin = gdn.causal_conv1d_fn(x, w, activation="silu", initial_states=pre, return_final_states=True)
    torch.cuda.synchronize()
    assert torch.equal(a, b)
    assert torch.equal(fin, x[:, :, -3:])
    out = torch.empty(1, 64, 3, device=dev)
    _, fin2 = gdn.causal_conv1d_fn(x[:, :, :2], w, activation="silu", initial_states=pre, return_final_states=True,
                                   final_states_out=out)
    assert fin2 is out and torch.equal(out, torch.cat([pre[:, :, -1:], x[:, :, :2]], 2))
    with pytest.raises(NotImplementedError):
        gdn.causal_conv1d_fn(x, w, seq_idx=torch.zeros(1, 20, dtype=torch.int32, device=dev))
    with pytest.raises(ValueError):
        gdn.causal_conv1d_fn(x, w, initial_states=pre, conv_prefix=pre)
