"""The v channels' short conv inside the pipelined fork kernel (gdn_state_fork(vconv=True),
StateForkPlan(vconv=True), dllm_gdn_state_fork_vconv_range_fwd): the conv launch writes only the q
and k channels, and each state wave convolves its own columns of every v row tile in LDS before it
reads them. The conv's arithmetic (fp32 sums in tap order from the bias, the weight-dtype rounding,
the hardware-exp2 SiLU) is the conv kernel's, so every output must equal conv then fork bit for bit:
the clean and noised outputs, the fp32 snapshots, the conv tails (the fork writes the v channels'
tails) and the q and k channels of the conv outputs.

Cases: the 27B-class benchmark layer at full size; the 0.8B-class layer at full size (its heads
split over two workgroups: there the two state waves that own no columns convolve those of the
other two, which wait for a per-wave LDS count; every small case below runs this layout too);
blocks 32 down to 1, where a tile has fewer real rows than the conv history (the carry then spans
several tiles); fp32 conv weights (no rounding before the SiLU); a conv bias; slow decay; block
ranges, whose fork launches start from the raw rows before the range; without snapshots or tails.
The fork with the v conv is also compared with the fp32 CPU oracle (here at small sizes, and the
27B- and 0.8B-class layers at full size in test_gpu_fullsize)."""

import dataclasses

import pytest
import torch

from _bounds import excess, out_bound, state_bound
from dllm_qwen38_amd import gdn, inputs
from oracle import gdn_ref

pytestmark = pytest.mark.gpu

SMALL = dataclasses.replace(inputs.GDN_27B_BF16, name="27B heads, B=2", B=2, L=256, Hk=2, Hv=6, g_shift=-4.0)


def _fork(x, s, **kw):
    return gdn.gdn_state_fork(x["raw0"], x["rawt"], x["conv_w"], x["beta0"], x["betat"], x["g0"], x["gt"],
                              num_k_heads=s.Hk, num_v_heads=s.Hv, head_k_dim=s.D, head_v_dim=s.D, block=s.block, **kw)


def _inputs(dev, s, wdtype=None, bias=False, **kw):
    x = {k: v.to(dev) for k, v in inputs.gdn_layer_inputs(s, **kw).items()}
    if wdtype is not None:
        x["conv_w"] = x["conv_w"].to(wdtype)
    extra = {}
    if bias:
        g = torch.Generator().manual_seed(11)
        extra["conv_bias"] = (torch.rand(x["conv_w"].shape[0], generator=g) - 0.5).to(x["conv_w"].dtype).to(dev)
    return x, extra


def _assert_same(got, ref, s, what):
    cq = 2 * s.Hk * s.D
    for k in ("o0", "ot", "states", "tails"):
        if ref[k] is None:
            assert got[k] is None, (what, k)
            continue
        assert torch.equal(got[k], ref[k]), (what, k, (got[k].float() - ref[k].float()).abs().max().item())
    for k in ("y0", "yt"):  # the conv launch's own channels
        assert torch.equal(got[k][..., :cq], ref[k][..., :cq]), (what, k)


CASES = [
    ("27b-full", inputs.GDN_27B_BF16, {}),
    ("08b-full-split", inputs.GDN_08B_BF16, {}),
    ("block32", SMALL, {}),
    ("block16", dataclasses.replace(SMALL, block=16), {}),
    ("block8", dataclasses.replace(SMALL, block=8), {}),
    ("block4", dataclasses.replace(SMALL, block=4, L=64), {}),
    ("block2", dataclasses.replace(SMALL, block=2, L=64), {}),
    ("block1", dataclasses.replace(SMALL, block=1, L=64), {}),
    ("fp32-weights", SMALL, {"wdtype": torch.float32}),
    ("bias", SMALL, {"bias": True}),
    ("fp32-weights-bias", dataclasses.replace(SMALL, block=16), {"wdtype": torch.float32, "bias": True}),
    ("odd-grid", dataclasses.replace(SMALL, B=3, Hk=1, Hv=11, L=128), {}),
]


@pytest.mark.parametrize("name,s,opt", CASES, ids=[c[0] for c in CASES])
def test_vconv_equals_conv_then_fork(dev, name, s, opt):
    x, extra = _inputs(dev, s, **opt)
    print(f"{name}: B={s.B} L={s.L} block={s.block} Hk={s.Hk} Hv={s.Hv} {opt}", flush=True)
    ref = _fork(x, s, vconv=False, pieces=1, **extra)
    torch.cuda.synchronize()
    assert "v conv" not in gdn.last_impl()[1]
    ref = {k: (None if v is None else v.clone()) for k, v in ref.items()}
    got = _fork(x, s, vconv=True, pieces=1, **extra)
    torch.cuda.synchronize()
    assert "v conv" in gdn.last_impl()[1], gdn.last_impl()
    _assert_same(got, ref, s, name)


@pytest.mark.parametrize("B,L,block,small", [(1, 512, 32, False), (4, 2048, 32, False), (2, 64, 2, True),
                                              (2, 128, 8, True)])
def test_vconv_block_ranges(dev, B, L, block, small):
    """Ranges with the v conv: each fork range reads the three raw rows before it as the conv
    history (at block 2 they span two blocks) and starts from the snapshot the range before wrote;
    equal to one unfused launch."""
    s = dataclasses.replace(SMALL if small else inputs.GDN_27B_BF16, B=B, L=L, block=block, g_shift=-4.0)
    x, extra = _inputs(dev, s, bias=True)
    ref = _fork(x, s, vconv=False, pieces=1, **extra)
    torch.cuda.synchronize()
    ref = {k: v.clone() for k, v in ref.items()}
    for pieces in (2, 3, 7):
        print(f"B={B} L={L} block={block} vconv pieces={pieces}", flush=True)
        got = _fork(x, s, vconv=True, pieces=pieces, **extra)
        torch.cuda.synchronize()
        assert "v conv" in gdn.last_impl()[1] and "block ranges" in gdn.last_impl()[1], gdn.last_impl()
        _assert_same(got, ref, s, f"pieces={pieces}")


def test_vconv_without_states_or_tails(dev):
    s = dataclasses.replace(SMALL, block=16)
    x, _ = _inputs(dev, s)
    ref = _fork(x, s, vconv=False)
    torch.cuda.synchronize()
    ref = {k: v.clone() for k, v in ref.items()}
    for kw in ({"need_states": False}, {"need_tails": False}, {"need_states": False, "need_tails": False}):
        got = _fork(x, s, vconv=True, **kw)
        torch.cuda.synchronize()
        for k in ("o0", "ot"):
            assert torch.equal(got[k], ref[k]), (kw, k)
        assert (got["states"] is None) == ("need_states" in kw) and (got["tails"] is None) == ("need_tails" in kw)
        if got["states"] is not None:
            assert torch.equal(got["states"], ref["states"])
        if got["tails"] is not None:
            assert torch.equal(got["tails"], ref["tails"])


def test_vconv_plan_and_overlap(dev):
    """StateForkPlan with the v conv: run() and run_overlapped() equal the unfused plan."""
    s = dataclasses.replace(inputs.GDN_27B_BF16, B=2, L=1024, g_shift=-4.0)
    x = {k: v.to(dev) for k, v in inputs.gdn_layer_inputs(s).items()}
    plans = {vc: gdn.StateForkPlan(x["raw0"], x["rawt"], x["conv_w"], x["beta0"], x["betat"], x["g0"], x["gt"],
                                   num_k_heads=s.Hk, num_v_heads=s.Hv, head_k_dim=s.D, head_v_dim=s.D,
                                   block=s.block, vconv=vc) for vc in (False, True)}
    assert plans[True].vconv and not plans[False].vconv
    plans[False].run()
    torch.cuda.synchronize()
    ref = {k: getattr(plans[False], k).clone() for k in ("o0", "ot", "states", "tails", "y0", "yt")}
    p = plans[True]
    for how in ("run", 3):
        for k in ("o0", "ot", "states", "tails"):
            getattr(p, k).fill_(float("nan"))
        p.run() if how == "run" else p.run_overlapped(how)
        torch.cuda.synchronize()
        _assert_same({k: getattr(p, k) for k in ref}, ref, s, how)


def test_vconv_against_oracle_slow_decay(dev):
    """The fork with the v conv against the fp32 CPU oracle on the same bf16 inputs, slow decay
    (the carried state visible), blocks 32 and 8, within the bf16 bounds of tests/_bounds.py."""
    for blk in (32, 8):
        s = dataclasses.replace(SMALL, block=blk, L=256)
        x = inputs.gdn_layer_inputs(s)
        xd = {k: v.to(dev) for k, v in x.items()}
        r = _fork(xd, s, vconv=True)
        torch.cuda.synchronize()
        o0, ot, st, tails = gdn_ref.state_fork_layer(x["raw0"], x["rawt"], x["conv_w"], x["beta0"], x["betat"],
                                                     x["g0"], x["gt"], Hk=s.Hk, Hv=s.Hv, Dk=s.D, Dv=s.D, block=blk)
        for name, got, want, bound in (("o0", r["o0"], o0, out_bound), ("ot", r["ot"], ot, out_bound),
                                       ("states", r["states"], st, state_bound)):
            over, ratio = excess(got.cpu(), want, bound)
            print(f"block {blk} {name}: max |d|/bound = {ratio:.3f}", flush=True)
            assert over <= 0, (blk, name, ratio)
        assert torch.equal(r["tails"].cpu(), tails)


def test_vconv_refusals(dev):
    """Shapes the pipelined kernel does not take, or a fault, refuse vconv=True; the automatic
    choice falls back to conv then fork there."""
    t = inputs.GDN_TINY_F32
    xt = {k: v.to(dev) for k, v in inputs.gdn_layer_inputs(t).items()}
    with pytest.raises(ValueError, match="vconv"):
        _fork(xt, t, vconv=True)
    _fork(xt, t)
    assert "v conv" not in gdn.last_impl()[1]
    x, _ = _inputs(dev, SMALL)
    with pytest.raises(ValueError, match="vconv"):
        _fork(x, SMALL, vconv=True, fault="no-conv-prefix")
    _fork(x, SMALL, fault="no-conv-prefix")
    assert "v conv" not in gdn.last_impl()[1]
    torch.cuda.synchronize()
