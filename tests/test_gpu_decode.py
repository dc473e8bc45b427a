"""GPU parity of the cached decoder and its block-causal attention kernel.

Bars:
  * block-causal attention vs the CPU oracle: fp32 <= 1e-5 max-abs; bf16 within
    2^-8 * max|V| + 2^-7 * |ref| (P rounded to bf16 before P.V, output rounded to bf16), the bar
    of the complementary-mask kernel; and bit-equal to the clean half of that kernel, whose rows
    walk the same key tiles in the same order;
  * fp32 tiny model: the logits of a cached denoising step vs the per-block oracle and vs the
    two-stream forward <= 1e-4 max-abs (the fork forward's own bar);
  * token streams at temperature 0: `generate` (golden, HIP forward) and `generate_cached` equal the
    oracle decoder's on the tiny fp32 model;
  * 27B-class geometry in bf16: a cached step's logits vs the two-stream forward's within
    2^-5 * max|logits| + 2^-6 * |logit| (bf16 activations, different GEMM shapes on each side).
"""

import ctypes
import copy

import pytest
import torch

from _tiny import tiny_hf_model
from dllm_qwen38_amd import attention, blockdiff, decode
from dllm_qwen38_amd import model as hybrid
from oracle import attn_ref, decode_ref, model_ref

pytestmark = pytest.mark.gpu

F32_ATT = 1e-5
F32_LOGITS = 1e-4


def _att_inputs(B, M, N, Hq, Hkv, d, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, M, Hq, d, generator=g).to(dtype)
    k = torch.randn(B, N, Hkv, d, generator=g).to(dtype)
    v = torch.randn(B, N, Hkv, d, generator=g).to(dtype)
    return q, k, v


def _check_att(got, ref, dtype, vmax, name):
    err = (got.float().cpu() - ref.float()).abs()
    print(f"{name}: max|d|={err.max().item():.3e}")
    if dtype == torch.float32:
        assert err.max().item() <= F32_ATT, name
    else:
        assert (err <= 2 ** -8 * vmax + 2 ** -7 * ref.float().abs()).all(), name


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("B,M,N,q0,Hq,Hkv,d,block", [
    (1, 32, 1024, 992, 6, 2, 256, 32),   # a decoding step: every key visible
    (2, 160, 160, 0, 4, 2, 128, 32),     # a prompt prefill: block-causal from 0
    (1, 16, 112, 96, 4, 4, 64, 16),      # decoding step, block 16
    (2, 20, 100, 80, 4, 2, 64, 20),      # ragged: N, M not multiples of 32
    (1, 37, 70, 33, 4, 2, 16, 8),        # the tiny model's head size; q0 inside a block
    (1, 64, 96, 32, 2, 1, 80, 32),       # d outside the direct-load kernel's set
])
def test_block_causal_attention_matches_oracle(dev, dtype, B, M, N, q0, Hq, Hkv, d, block):
    q, k, v = _att_inputs(B, M, N, Hq, Hkv, d, dtype, seed=M + N + d)
    got = attention.block_causal_attention(q.to(dev), k.to(dev), v.to(dev), block=block, q_offset=q0)
    torch.cuda.synchronize()
    ref = attn_ref.block_causal_attention(q, k, v, block=block, q_offset=q0)
    _check_att(got, ref, dtype, v.float().abs().max().item(), f"{dtype} M{M} N{N} q0{q0} d{d} block{block}")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("L,d,block", [(256, 256, 32), (96, 64, 16), (40, 16, 8)])
def test_prefill_is_bit_equal_to_the_clean_half_of_the_two_stream_kernel(dev, dtype, L, d, block):
    g = torch.Generator().manual_seed(L + d)
    q, k, v = (torch.randn(2, 2 * L, h, d, generator=g).to(dtype).to(dev) for h in (4, 2, 2))
    both = attention.bd_attention(q, k, v, block=block)
    clean = attention.block_causal_attention(q[:, L:], k[:, L:], v[:, L:], block=block)
    torch.cuda.synchronize()
    assert torch.equal(clean, both[:, L:])


@pytest.mark.parametrize("ks", [2, 5, 16, 32])
def test_key_split_attention_matches_oracle(dev, ks):
    """Key tiles split over workgroups and merged (flash-decoding), including more splits than key
    tiles (empty shares): within the bf16 bar of the oracle, as the unsplit kernel."""
    q, k, v = _att_inputs(2, 32, 600, 8, 2, 256, torch.bfloat16, seed=ks)
    got = attention.block_causal_attention(q.to(dev), k.to(dev), v.to(dev), block=32, q_offset=568, key_splits=ks)
    one = attention.block_causal_attention(q.to(dev), k.to(dev), v.to(dev), block=32, q_offset=568, key_splits=1)
    torch.cuda.synchronize()
    ref = attn_ref.block_causal_attention(q, k, v, block=32, q_offset=568)
    vmax = v.float().abs().max().item()
    _check_att(got, ref, torch.bfloat16, vmax, f"key splits {ks}")
    _check_att(one, ref, torch.bfloat16, vmax, "unsplit")


@pytest.mark.parametrize("ks", [1, 4])
@pytest.mark.parametrize("B,M,N,q0,Hq,Hkv,d", [
    (1, 32, 1024, 992, 6, 2, 256),   # a decoding step of the 27B-class heads
    (2, 20, 100, 80, 4, 2, 128),     # ragged rows, two sequences
    (1, 64, 600, 536, 8, 2, 64),
])
def test_block_causal_gate_equals_the_separate_product(dev, ks, B, M, N, q0, Hq, Hkv, d):
    """The output gate fused into the block-causal attention (at the output store, or at the merge
    of the key shares) against the separate bf16 product o * sigmoid(gate) on the same attention
    output: within one bf16 rounding of sigmoid (hardware exp2 / reciprocal vs torch's), 2^-7 |ref|;
    the gate read in place as the second half of each head's 2d columns, as the decoder slices it."""
    q, k, v = (t.to(dev) for t in _att_inputs(B, M, N, Hq, Hkv, d, torch.bfloat16, seed=M + N + d + ks))
    g = torch.Generator().manual_seed(ks * 1000 + d)
    qg = (torch.randn(B, M, Hq, 2 * d, generator=g) * 2).to(torch.bfloat16).to(dev)
    gate = qg[..., d:]
    assert attention.block_causal_gate_fused(q, k, v)
    got = attention.block_causal_attention(q, k, v, block=32, q_offset=q0, key_splits=ks, gate=gate)
    o = attention.block_causal_attention(q, k, v, block=32, q_offset=q0, key_splits=ks)
    ref = (o * torch.sigmoid(gate)).float()
    torch.cuda.synchronize()
    err = (got.float() - ref).abs()
    print(f"gated ks={ks} B={B} M={M} d={d}: max|d|={err.max().item():.3e}")
    assert (err <= 2 ** -7 * ref.abs() + 1e-6).all()


def test_27b_class_decoding_step_attention(dev):
    """24 query / 4 key-value heads of dim 256, 4096 cached keys, one block of 32 queries."""
    q, k, v = _att_inputs(1, 32, 4096, 24, 4, 256, torch.bfloat16, seed=27)
    got = attention.block_causal_attention(q.to(dev), k.to(dev), v.to(dev), block=32, q_offset=4064)
    torch.cuda.synchronize()
    ref = attn_ref.block_causal_attention(q, k, v, block=32, q_offset=4064)
    _check_att(got, ref, torch.bfloat16, v.float().abs().max().item(), "27b step")


@pytest.mark.parametrize("M,N,K", [(32, 5120, 5120), (32, 17408, 5120), (32, 5120, 17408), (32, 48, 5120),
                                   (1, 100, 64), (7, 300, 320), (33, 1000, 640), (64, 96, 6144)])
def test_decode_linear_matches_fp32_reference(dev, M, N, K):
    """y = x W^T against torch fp32 on the same bf16 inputs: within the bf16 rounding of the output
    (2^-8 relative) plus 2^-16 of sum|x||w| for the accumulation order."""
    g = torch.Generator().manual_seed(M + N + K)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16)
    w = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16)
    got = decode.decode_linear(x.to(dev), w.to(dev))
    torch.cuda.synchronize()
    ref = x.float() @ w.float().T
    scale = x.float().abs() @ w.float().abs().T
    err = (got.float().cpu() - ref).abs()
    print(f"M{M} N{N} K{K} workgroups {decode._lib.lib().dllm_decode_linear_workgroups(M, N, K)}: max|d|={err.max():.3e}")
    assert (err <= 2 ** -8 * ref.abs() + 2 ** -16 * scale).all()
    again = decode.decode_linear(x.to(dev), w.to(dev))
    torch.cuda.synchronize()
    assert torch.equal(got, again), "the sums of split tiles must be deterministic"


@pytest.mark.parametrize("G", [1, 2, 3, 7, 100, 191, 512])
@pytest.mark.parametrize("swiglu", [0, 1])
def test_decode_linear_any_workgroup_count(dev, G, swiglu):
    """Every split of the (tile, k step) units over workgroups (2 row tiles x 6 feature tiles x 16
    steps = 192 units; 512 asks for more workgroups than units and gets one unit each) gives the
    projections within the bound of the single-launch test, and the same bits on a repeat."""
    from dllm_qwen38_amd import _lib

    g = torch.Generator().manual_seed(G + 10 * swiglu)
    M, K, N = 40, 1024, 300
    x = torch.randn(M, K, generator=g).to(torch.bfloat16)
    ws = [(torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16) for _ in range(2)]
    L = _lib.lib()
    xd, wd = x.to(dev), [w.to(dev) for w in ws]
    outs = [torch.empty(M, N, dtype=torch.bfloat16, device=dev) for _ in range(2)]

    def run():
        work = decode._workspace(L, M, N, G, bool(swiglu), dev)
        warr = (ctypes.c_void_p * 2)(*[w.data_ptr() for w in wd])
        oarr = (ctypes.c_void_p * 2)(*[o.data_ptr() for o in outs])
        narr = (ctypes.c_int * 2)(N, N)
        _lib.check(L.dllm_decode_linear_multi_fwd(xd.data_ptr(), M, K, 2, warr, oarr, narr, work.data_ptr(), G, swiglu,
                                                  _lib.DT_BF16, _lib.stream_handle(dev)), "multi")
        torch.cuda.synchronize()
        return [o.clone().cpu() for o in outs]

    got = run()
    refs = [x.float() @ w.float().T for w in ws]
    if swiglu:
        gr, ur = (r.to(torch.bfloat16).float() for r in refs)
        ref = torch.nn.functional.silu(gr).to(torch.bfloat16).float() * ur
        err = (got[0].float() - ref).abs()
        assert (err <= 2 ** -6 * ref.abs() + 2 ** -10 * ref.abs().max()).all()
    else:
        for o, w, ref in zip(got, ws, refs):
            err = (o.float() - ref).abs()
            assert (err <= 2 ** -8 * ref.abs() + 2 ** -16 * (x.float().abs() @ w.float().abs().T)).all()
    again = run()
    assert all(torch.equal(a, b) for a, b in zip(got[: 2 - swiglu], again[: 2 - swiglu]))


def test_decode_linear_more_split_tiles_than_one_fixup_launch(dev):
    """1199 workgroups over 600 tiles of 2 steps (1200 units): 599 tiles are split, more than the 512
    one fixup launch lists, so the fixups go out in two launches; the result stays within the
    single-launch bound and equals a repeat bit for bit."""
    from dllm_qwen38_amd import _lib

    g = torch.Generator().manual_seed(1199)
    M, K, N, G = 32, 128, 128 * 600, 1199
    x = torch.randn(M, K, generator=g).to(torch.bfloat16)
    w = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16)
    L = _lib.lib()
    xd, wd = x.to(dev), w.to(dev)

    def run():
        y = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
        work = decode._workspace(L, M, 0, G, False, dev)
        _lib.check(L.dllm_decode_linear_fwd(xd.data_ptr(), wd.data_ptr(), y.data_ptr(), work.data_ptr(), M, N, K, G,
                                            _lib.DT_BF16, _lib.stream_handle(dev)), "decode linear")
        torch.cuda.synchronize()
        return y.cpu()

    got = run()
    ref = x.float() @ w.float().T
    err = (got.float() - ref).abs()
    assert (err <= 2 ** -8 * ref.abs() + 2 ** -16 * (x.float().abs() @ w.float().abs().T)).all()
    assert torch.equal(got, run())


def test_decode_linear_multi_and_swiglu_epilogue(dev):
    """Projections sharing x in one launch equal the fp32 reference as single ones do; the SwiGLU
    epilogue equals round(round(silu(g)) * u) of the rounded projections within two bf16 ulps."""
    g = torch.Generator().manual_seed(77)
    M, K = 32, 5120
    x = torch.randn(M, K, generator=g).to(torch.bfloat16)
    ws = [(torch.randn(n, K, generator=g) * 0.02).to(torch.bfloat16) for n in (10240, 6144, 48, 48)]
    outs = decode.decode_linear_multi(x.to(dev), [w.to(dev) for w in ws])
    torch.cuda.synchronize()
    for o, w in zip(outs, ws):
        ref = x.float() @ w.float().T
        err = (o.float().cpu() - ref).abs()
        assert (err <= 2 ** -8 * ref.abs() + 2 ** -16 * (x.float().abs() @ w.float().abs().T)).all()
    gw, uw = ((torch.randn(2048, K, generator=g) * 0.02).to(torch.bfloat16) for _ in range(2))
    act = decode.decode_linear_multi(x.to(dev), [gw.to(dev), uw.to(dev)], swiglu=True)
    torch.cuda.synchronize()
    gr = (x.float() @ gw.float().T).to(torch.bfloat16).float()
    ur = (x.float() @ uw.float().T).to(torch.bfloat16).float()
    ref = (torch.nn.functional.silu(gr).to(torch.bfloat16).float() * ur)
    err = (act.float().cpu() - ref).abs()
    print(f"swiglu epilogue max|d|={err.max():.3e} max|ref|={ref.abs().max():.3e}")
    assert (err <= 2 ** -6 * ref.abs() + 2 ** -10 * ref.abs().max()).all()


@pytest.mark.parametrize("M,N,K,G,wdtype,unit", [
    (32, 5120, 6144, None, torch.bfloat16, 1),   # o_proj / out_proj of the 27B-class decoder step
    (32, 5120, 17408, None, torch.float32, 1),   # down_proj, fp32 norm weight
    (1, 512, 64, 1, torch.bfloat16, 0),          # one row, one unit, w applied as is
    (40, 1024, 1024, 7, torch.bfloat16, 1),      # two row tiles, seven workgroups
    (64, 2048, 512, 191, torch.float32, 0),
    (33, 3072, 256, 4096, torch.bfloat16, 1),    # more workgroups than units: one unit each
    (17, 4096, 2048, None, torch.bfloat16, 1),
    (32, 8192, 256, None, torch.bfloat16, 1),    # the widest row: two feature slots per thread
])
def test_decode_linear_rmsnorm_equals_projection_then_norm(dev, M, N, K, G, wdtype, unit):
    """The fused projection + residual add + RMSNorm equals the projection (main and fixup launches,
    same workgroup count) followed by the row RMSNorm with the residual, bit for bit in both the
    normed output and the sum; the sum stays within the projection's bound of x W^T + r; a repeat
    gives the same bits."""
    from dllm_qwen38_amd import _lib, norms

    g = torch.Generator().manual_seed(M * 7 + N + K)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16)
    w = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16)
    r = torch.randn(M, N, generator=g).to(torch.bfloat16)
    nw = (torch.randn(N, generator=g) * 0.1).to(wdtype)
    L = _lib.lib()
    G = G or L.dllm_decode_linear_workgroups(M, N, K)
    xd, wd, rd, nwd = x.to(dev), w.to(dev), r.to(dev), nw.to(dev)
    eps = 1e-6
    print(f"decode linear rmsnorm M={M} N={N} K={K} workgroups={G}", flush=True)

    def fused():
        s = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
        y = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
        work = decode._workspace(L, M, N, G, True, dev)
        _lib.check(L.dllm_decode_linear_rmsnorm_fwd(
            xd.data_ptr(), wd.data_ptr(), work.data_ptr(), M, N, K, G, rd.data_ptr(), s.data_ptr(), nwd.data_ptr(),
            y.data_ptr(), eps, unit, _lib.DT_BF16, _lib.dtype_code(wdtype), _lib.stream_handle(dev)), "fused")
        torch.cuda.synchronize()
        return y.cpu(), s.cpu()

    p = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
    work = decode._workspace(L, M, 0, G, False, dev)
    _lib.check(L.dllm_decode_linear_fwd(xd.data_ptr(), wd.data_ptr(), p.data_ptr(), work.data_ptr(), M, N, K, G,
                                        _lib.DT_BF16, _lib.stream_handle(dev)), "projection")
    y_ref, s_ref = norms.rmsnorm(p, nwd, eps, residual=rd, unit_offset=bool(unit))
    torch.cuda.synchronize()
    y, s = fused()
    assert torch.equal(s, s_ref.cpu()), "sum differs from projection + residual"
    assert torch.equal(y, y_ref.cpu()), "normed output differs from the row RMSNorm"
    ref = x.float() @ w.float().T
    bound = 2 ** -8 * ref.abs() + 2 ** -16 * (x.float().abs() @ w.float().abs().T) + 2 ** -8 * (ref + r.float()).abs()
    assert ((s.float() - (ref + r.float())).abs() <= bound + 2 ** -8 * r.float().abs()).all()
    y2, s2 = fused()
    assert torch.equal(y, y2) and torch.equal(s, s2)


class _Mixer(torch.nn.Module):
    """The attributes of a Gated DeltaNet mixer that the decoding-step prologue reads, seeded."""

    def __init__(self, K, C, Nz, H, width, conv_bias, wdtype, pdtype, seed, dev):
        super().__init__()
        g = torch.Generator().manual_seed(seed)

        def lin(n):
            m = torch.nn.Linear(K, n, bias=False)
            m.weight.data = (torch.randn(n, K, generator=g) * 0.03).to(torch.bfloat16)
            return m

        self.in_proj_qkv, self.in_proj_z, self.in_proj_b, self.in_proj_a = lin(C), lin(Nz), lin(H), lin(H)
        self.conv1d = torch.nn.Conv1d(C, C, width, groups=C, bias=conv_bias, padding=width - 1)
        self.conv1d.weight.data = (torch.rand(C, 1, width, generator=g) - 0.5).to(wdtype)
        if conv_bias:
            self.conv1d.bias.data = (torch.rand(C, generator=g) - 0.5).to(wdtype)
        self.A_log = torch.nn.Parameter(torch.log(torch.rand(H, generator=g) * 15 + 1).to(pdtype))
        self.dt_bias = torch.nn.Parameter(torch.randn(H, generator=g).to(pdtype))
        self.activation = "silu"
        self.to(dev)


@pytest.mark.parametrize("M,T,K,C,Nz,H,width,bias,prefix,wdtype,pdtype", [
    (32, 32, 1024, 768, 512, 16, 4, False, True, torch.bfloat16, torch.float32),   # every tile split
    (32, 32, 64, 768, 512, 16, 4, False, True, torch.bfloat16, torch.float32),     # one unit per tile: none split
    (64, 32, 512, 1024, 256, 48, 4, True, False, torch.float32, torch.bfloat16),   # two sequences, no carry-in
    (64, 16, 768, 640, 384, 130, 3, True, True, torch.bfloat16, torch.bfloat16),   # four sequences of 16; 130 heads
    (8, 8, 256, 300, 200, 7, 4, False, True, torch.bfloat16, torch.float32),       # ragged widths, tile rows past M
])
def test_decode_gdn_prologue_equals_the_separate_kernels(dev, M, T, K, C, Nz, H, width, bias, prefix, wdtype,
                                                           pdtype):
    """The GDN mixer's input projections finished with the short conv (and its carry-in) and the
    gates in one launch equal the projections, the conv kernel and the gates kernel run separately,
    bit for bit: the projections, z, the conv + SiLU output, beta and g."""
    from dllm_qwen38_amd import gdn, norms

    m = _Mixer(K, C, Nz, H, width, bias, wdtype, pdtype, seed=M + K + C, dev=dev)
    g = torch.Generator().manual_seed(M * T + C)
    B = M // T
    x = torch.randn(B, T, K, generator=g).to(torch.bfloat16).to(dev)
    pre = (torch.randn(B, C, width - 1, generator=g).to(torch.bfloat16).to(dev) if prefix else None)
    print(f"gdn prologue M={M} T={T} K={K} C={C} H={H} width={width}", flush=True)
    assert decode._prologue_fused(m, x, pre, T)
    raw, mixed, z, beta, gg = decode.decode_gdn_prologue(m, x, pre, T)
    lins = (m.in_proj_qkv, m.in_proj_z, m.in_proj_b, m.in_proj_a)
    raw_r, z_r, b_r, a_r = decode.decode_linear_multi(x, [lin.weight for lin in lins])
    beta_r, g_r = norms.gdn_gates(b_r, a_r, m.A_log, m.dt_bias)
    mixed_r = gdn.causal_conv1d_fn(raw_r.transpose(1, 2), m.conv1d.weight.squeeze(1), m.conv1d.bias,
                                   activation="silu", conv_prefix=pre).transpose(1, 2)
    torch.cuda.synchronize()
    for name, got, ref in (("raw", raw, raw_r), ("z", z, z_r), ("mixed", mixed, mixed_r), ("beta", beta, beta_r),
                           ("g", gg, g_r)):
        assert got.shape == ref.shape, name
        assert torch.equal(got, ref), f"{name} differs: max|d|={(got.float() - ref.float()).abs().max().item():.3e}"


@pytest.fixture(scope="module")
def tiny(dev):
    cpu_model, cpu_head = tiny_hf_model(seed=0)
    return cpu_model, cpu_head, copy.deepcopy(cpu_model).to(dev), copy.deepcopy(cpu_head).to(dev)


def _maxdiff(a, b):
    return (a.float().cpu() - b.float().cpu()).abs().max().item()


@pytest.mark.parametrize("block,prompt_blocks", [(8, 3), (16, 2), (4, 5)])
def test_cached_step_matches_the_per_block_oracle_and_the_forward(tiny, dev, block, prompt_blocks):
    cm, ch, gm, gh = tiny
    g = torch.Generator().manual_seed(block)
    P = prompt_blocks * block
    x0 = torch.randint(0, 255, (1, P + block), generator=g)
    xt = x0.clone()
    xt[:, P:][torch.rand(1, block, generator=g) < 0.5] = 255
    cache = decode.PrefixCache(gm, batch=1, capacity=P + 2 * block, block=block)
    decode.forward_segment(gm, gh, cache, x0[:, :P].to(dev), commit=True, logits=False)
    step = decode.forward_segment(gm, gh, cache, xt[:, P:].to(dev), commit=False)
    again = decode.forward_segment(gm, gh, cache, xt[:, P:].to(dev), commit=False)
    with torch.no_grad():
        lt, _ = blockdiff.block_diffusion_forward(gm, gh, x0.to(dev), xt.to(dev), block)
    torch.cuda.synchronize()
    assert cache.length == P
    assert torch.equal(step, again)  # an uncommitted step leaves the prefix untouched
    ref = model_ref.reference_block_logits(cm, ch, x0, xt, block)[:, P:]
    d_ref, d_fwd = _maxdiff(step, ref), _maxdiff(step, lt[:, P:])
    print(f"block {block} prefix {P}: vs per-block oracle {d_ref:.2e}, vs two-stream forward {d_fwd:.2e}")
    assert d_ref <= F32_LOGITS and d_fwd <= F32_LOGITS


def test_block_by_block_commits_equal_one_prefill(tiny, dev):
    _, _, gm, gh = tiny
    block = 8
    ids = torch.randint(0, 255, (1, 5 * block), generator=torch.Generator().manual_seed(3)).to(dev)
    a = decode.PrefixCache(gm, batch=1, capacity=6 * block, block=block)
    b = decode.PrefixCache(gm, batch=1, capacity=6 * block, block=block)
    decode.forward_segment(gm, gh, a, ids[:, : 4 * block], commit=True, logits=False)
    for j in range(4):
        decode.forward_segment(gm, gh, b, ids[:, j * block:(j + 1) * block], commit=True, logits=False)
    la = decode.forward_segment(gm, gh, a, ids[:, 4 * block:], commit=False)
    lb = decode.forward_segment(gm, gh, b, ids[:, 4 * block:], commit=False)
    torch.cuda.synchronize()
    assert a.length == b.length == 4 * block
    d = _maxdiff(la, lb)
    print(f"one prefill vs four commits: {d:.2e}")
    assert d <= 1e-5


@pytest.mark.parametrize("prompt,block,threshold,sub_block", [
    ([10, 11, 12, 13, 14], 8, 0.9, None),   # the reference's seam-test setting
    (list(range(30, 46)), 8, 0.0, None),     # prompt of whole blocks, everything at once
    ([5, 6, 7], 8, 0.0, 4),                  # sub-blocks
])
def test_token_streams_match_the_oracle_decoder(tiny, dev, prompt, block, threshold, sub_block):
    cm, ch, gm, gh = tiny
    kw = dict(n_blocks=3, block=block, mask_id=255, threshold=threshold, sub_block=sub_block)
    ref = decode_ref.generate(cm, ch, prompt, **kw)
    gold = decode.generate(gm, gh, prompt, **kw)
    fast = decode.generate_cached(gm, gh, prompt, **kw)
    print(f"oracle {ref['tokens']}\ngolden {gold.tokens}\ncached {fast.tokens}")
    assert gold.tokens == ref["tokens"] and gold.steps_per_block == ref["steps_per_block"]
    assert fast.tokens == ref["tokens"] and fast.steps_per_block == ref["steps_per_block"]
    assert gold.forwards == fast.forwards == ref["forwards"]
    assert fast.commits == (1 if len(prompt) >= block else 0) + 2


@pytest.fixture(scope="module")
def stack27(dev):
    c = hybrid.config_27b_truncated(layers=4)
    return hybrid.build(c, device=dev, dtype=torch.bfloat16, seed=21)


def test_27b_class_fused_step_equals_the_separate_launches(stack27, dev):
    """A cached denoising step and a commit on 27B-class layers (GDN and attention) with the fused
    decoding-step launches (projection end + residual norm, the GDN in_proj end with conv and gates,
    the attention layer's direct cache writes) against the same forward with each of them as the
    separate launches it replaces: logits, GDN states, conv carry-in and K/V cache bit-equal."""
    model, lm_head = stack27
    block, P = 32, 256
    g = torch.Generator().manual_seed(12)
    x0 = torch.randint(0, 151936, (1, P + 2 * block), generator=g).to(dev)
    xt = x0.clone()
    xt[:, P + 7:] = 151935
    runs = {}
    try:
        for fused in (True, False):
            decode.FUSED = fused
            cache = decode.PrefixCache(model, batch=1, capacity=P + 2 * block, block=block)
            decode.forward_segment(model, lm_head, cache, x0[:, :P], commit=True, logits=False)
            step = decode.forward_segment(model, lm_head, cache, xt[:, P:P + block], commit=False)
            decode.forward_segment(model, lm_head, cache, x0[:, P:P + block], commit=True, logits=False)
            step2 = decode.forward_segment(model, lm_head, cache, xt[:, P + block:], commit=False)
            torch.cuda.synchronize()
            runs[fused] = (step, step2, cache)
    finally:
        decode.FUSED = True
    (a1, a2, ca), (b1, b2, cb) = runs[True], runs[False]
    assert torch.equal(a1, b1) and torch.equal(a2, b2), "logits differ"
    for i in ca.state:
        if ca.state[i] is not None:
            assert torch.equal(ca.state[i], cb.state[i]) and torch.equal(ca.conv[i], cb.conv[i]), f"layer {i} GDN cache"
    for i in ca.k:
        n = P + block
        assert torch.equal(ca.k[i][:, :n], cb.k[i][:, :n]) and torch.equal(ca.v[i][:, :n], cb.v[i][:, :n]), f"layer {i} K/V"


def test_27b_class_cached_step_matches_the_forward_bf16(stack27, dev):
    model, lm_head = stack27
    block, P = 32, 512
    g = torch.Generator().manual_seed(8)
    x0 = torch.randint(0, 151936, (1, P + block), generator=g).to(dev)
    xt = x0.clone()
    xt[:, P + 5:] = 151935
    cache = decode.PrefixCache(model, batch=1, capacity=P + block, block=block)
    decode.forward_segment(model, lm_head, cache, x0[:, :P], commit=True, logits=False)
    step = decode.forward_segment(model, lm_head, cache, xt[:, P:], commit=False)
    with torch.no_grad():
        lt, _ = blockdiff.block_diffusion_forward(model, lm_head, x0, xt, block)
    torch.cuda.synchronize()
    ref = lt[:, P:].float()
    err = (step.float() - ref).abs()
    bound = 2 ** -5 * ref.abs().max() + 2 ** -6 * ref.abs()
    print(f"27b-class bf16 step vs forward: max|d|={err.max().item():.3e} max|ref|={ref.abs().max().item():.3e}")
    assert (err <= bound).all()
    print(f"cache bytes {cache.nbytes()}")
