"""The state-fork layer cut into block ranges (StateForkPlan.run_overlapped): the conv of each range
runs on a side stream beside the fork of the range before it, and each fork range starts from the
fp32 snapshot the range before it wrote. Every output must equal the one-launch schedule (run())
bit for bit: the snapshot is the exact register state, and a block's arithmetic does not depend on
where a launch starts. Slow decay (g shift -4) keeps the carried state visible in the outputs.

Also the range entry points' argument checks (a range after block 0 needs the states tensor;
ranges need the pipelined kernel; the range must lie inside the sequence)."""

import dataclasses

import pytest
import torch

from dllm_qwen38_amd import _lib, gdn, inputs

pytestmark = pytest.mark.gpu

OUTS = ("y0", "yt", "tails", "o0", "ot", "states")


def _plan(dev, s, B, L, g_shift):
    x = {k: v.to(dev) for k, v in inputs.gdn_layer_inputs(s, B=B, L=L, g_shift=g_shift).items()}
    return gdn.StateForkPlan(x["raw0"], x["rawt"], x["conv_w"], x["beta0"], x["betat"], x["g0"], x["gt"],
                             num_k_heads=s.Hk, num_v_heads=s.Hv, head_k_dim=s.D, head_v_dim=s.D, block=s.block)


@pytest.mark.parametrize("shape,B,L", [("GDN_27B_BF16", 1, 512), ("GDN_08B_BF16", 2, 1024)])
def test_overlapped_schedule_is_bit_identical(dev, shape, B, L):
    s = getattr(inputs, shape)
    p = _plan(dev, s, B, L, g_shift=-4.0)
    assert p.overlap_supported()
    p.run()
    torch.cuda.synchronize()
    # with the v conv inside the fork the conv launches write only the q and k channels of y0, yt
    cy = 2 * s.Hk * s.D if p.vconv else s.conv_dim
    view = lambda k, t: t[..., :cy] if k in ("y0", "yt") else t  # noqa: E731
    ref = {k: view(k, getattr(p, k)).clone() for k in OUTS}
    nb = L // s.block
    for kw in ({"pieces": 2}, {"pieces": 3}, {"pieces": 5}, {"bounds": [0, 1, nb // 2, nb]},
               {"bounds": [0, nb - 1, nb]}):
        for k in OUTS:
            getattr(p, k).fill_(float("nan"))
        print(f"{shape} B={B} L={L} run_overlapped({kw})", flush=True)
        p.run_overlapped(**kw)
        torch.cuda.synchronize()
        for k in OUTS:
            assert torch.equal(view(k, getattr(p, k)), ref[k]), (kw, k)
    assert gdn.kernel_status(reset=True) == 0


def test_range_entry_argument_checks(dev):
    s = inputs.GDN_27B_BF16
    B, L = 1, 256
    p = _plan(dev, s, B, L, g_shift=None)
    lib = _lib.lib()
    Cd = p.dims[2]

    def fork(states, k0, k1, Dk=s.D):
        return lib.dllm_gdn_state_fork_range_fwd(
            p.y0.data_ptr(), p.yt.data_ptr(), L * Cd, Cd, p.beta0.data_ptr(), p.betat.data_ptr(), p.g0.data_ptr(),
            p.gt.data_ptr(), p.o0.data_ptr(), p.ot.data_ptr(), states, B, L, s.Hk, s.Hv, Dk, s.D, s.block,
            p.code, s.D ** -0.5, k0, k1, _lib.stream_handle(dev))

    def conv(k0, k1):
        return lib.dllm_conv_fork_range_fwd(
            p.raw0.data_ptr(), p.rawt.data_ptr(), p.w.data_ptr(), None, p.y0.data_ptr(), p.yt.data_ptr(),
            p.tails.data_ptr(), B, L, Cd, p.K, s.block, p.code, _lib.dtype_code(p.w.dtype), 0, k0, k1,
            _lib.stream_handle(dev))

    nb = L // s.block
    assert fork(None, 2, nb) == -1  # a range after block 0 starts from states
    assert fork(p.states.data_ptr(), 0, nb + 1) == -1
    assert fork(p.states.data_ptr(), 3, 3) == -1
    assert conv(-1, 2) == -1
    assert conv(4, nb + 1) == -1
    assert conv(5, 5) == -1
    msg = _lib.last_error()
    assert "block range" in msg, msg
    torch.cuda.synchronize()
    # nothing was launched by the rejected calls; a valid pair of ranges still runs
    assert conv(0, nb) == 0 and fork(p.states.data_ptr(), 0, nb) == 0
    torch.cuda.synchronize()
    assert gdn.kernel_status(reset=True) == 0


@pytest.mark.parametrize("shape,B,L", [("GDN_27B_BF16", 1, 512), ("GDN_08B_BF16", 2, 1024)])
def test_column_split_of_the_fork_is_bit_identical(dev, shape, B, L):
    """The pipelined fork with each head's value columns over two workgroups (the default when
    the split grid fits the chip) against one workgroup per head: identical outputs and states
    (every column is computed by the same arithmetic in either layout)."""
    s = getattr(inputs, shape)
    p = _plan(dev, s, B, L, g_shift=-4.0)
    lib = _lib.lib()
    got = {}
    prev = lib.dllm_set_fork_split(1)
    try:
        for mode in (1, 2):
            lib.dllm_set_fork_split(mode)
            for k in OUTS[3:]:
                getattr(p, k).fill_(float("nan"))
            print(f"{shape} B={B} L={L} split mode {mode}", flush=True)
            p.run()
            torch.cuda.synchronize()
            got[mode] = {k: getattr(p, k).clone() for k in OUTS[3:]}
    finally:
        lib.dllm_set_fork_split(prev)
    for k in OUTS[3:]:
        assert torch.equal(got[1][k], got[2][k]), k
    assert lib.dllm_set_fork_split(3) == -1
    assert gdn.kernel_status(reset=True) == 0


def _fork(x, s, **kw):
    return gdn.gdn_state_fork(x["raw0"], x["rawt"], x["conv_w"], x["beta0"], x["betat"], x["g0"], x["gt"],
                              num_k_heads=s.Hk, num_v_heads=s.Hv, head_k_dim=s.D, head_v_dim=s.D, block=s.block, **kw)


@pytest.mark.parametrize("shape,B,L", [("GDN_27B_BF16", 1, 512), ("GDN_08B_BF16", 2, 1024),
                                       ("GDN_27B_BF16", 4, 2048)])
def test_state_fork_api_schedules_are_bit_identical(dev, shape, B, L):
    """gdn_state_fork with its default schedule, explicit range counts and one launch: identical
    outputs, conv tails and snapshots, with a conv bias and under the no-conv-prefix fault too."""
    s = getattr(inputs, shape)
    x = {k: v.to(dev) for k, v in inputs.gdn_layer_inputs(s, B=B, L=L, g_shift=-4.0).items()}
    g = torch.Generator().manual_seed(5)
    bias = (torch.rand(x["conv_w"].shape[0], generator=g) - 0.5).to(x["conv_w"].dtype).to(dev)
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    auto_ranges = gdn.default_pieces(cus, B, s.Hv, L // s.block) > 1
    for kw in ({}, {"conv_bias": bias}, {"fault": "no-conv-prefix"}):
        ref = _fork(x, s, pieces=1, **kw)
        torch.cuda.synchronize()
        assert "block ranges" not in gdn.last_impl()[1]
        # with the v conv inside the fork (the automatic choice where it pays) the conv launch
        # leaves the v channels of y0 and yt unwritten: compare its own channels there
        cy = 2 * s.Hk * s.D if "v conv" in gdn.last_impl()[1] else None
        ref = {k: (v[..., :cy] if k in ("y0", "yt") else v).clone() for k, v in ref.items() if v is not None}
        for pieces in (None, 2, 3, 7):
            print(f"{shape} B={B} L={L} {sorted(kw)} pieces={pieces}", flush=True)
            got = _fork(x, s, pieces=pieces, **kw)
            torch.cuda.synchronize()
            ranges = pieces is not None or auto_ranges
            assert ("block ranges" in gdn.last_impl()[1]) == ranges, (pieces, gdn.last_impl())
            for k in ref:
                g = got[k][..., :cy] if k in ("y0", "yt") else got[k]
                assert torch.equal(g, ref[k]), (kw, pieces, k)
    assert gdn.kernel_status(reset=True) == 0


def test_state_fork_api_schedule_arguments(dev):
    """Block ranges need the snapshots and the pipelined kernel: without them the default is one
    launch and an explicit range count is refused."""
    s = inputs.GDN_27B_BF16
    x = {k: v.to(dev) for k, v in inputs.gdn_layer_inputs(s, B=1, L=256).items()}
    with pytest.raises(ValueError, match="pieces"):
        _fork(x, s, pieces=0)
    with pytest.raises(ValueError, match="states"):
        _fork(x, s, pieces=2, need_states=False)
    r = _fork(x, s, need_states=False)
    torch.cuda.synchronize()
    assert r["states"] is None and "block ranges" not in gdn.last_impl()[1]
    t = inputs.GDN_TINY_F32
    xt = {k: v.to(dev) for k, v in inputs.gdn_layer_inputs(t).items()}
    with pytest.raises(ValueError, match="pipelined"):
        _fork(xt, t, pieces=2)
    _fork(xt, t)
    torch.cuda.synchronize()
    assert "block ranges" not in gdn.last_impl()[1]
    assert gdn.kernel_status(reset=True) == 0


@pytest.mark.parametrize("block", [16, 8])
def test_ranges_at_subtile_blocks_are_bit_identical(dev, block):
    """Blocks shorter than the kernel's 32-row tile (rows past the block are padding) in block
    ranges: the plan's overlapped schedule and the drop-in's explicit ranges equal one launch."""
    s = dataclasses.replace(inputs.GDN_27B_BF16, block=block)
    B, L = 1, 256
    nb = L // block
    p = _plan(dev, s, B, L, g_shift=-4.0)
    assert p.overlap_supported()
    p.run()
    torch.cuda.synchronize()
    # with the v conv inside the fork the conv launches write only the q and k channels of y0, yt
    cy = 2 * s.Hk * s.D if p.vconv else s.conv_dim
    view = lambda k, t: t[..., :cy] if k in ("y0", "yt") else t  # noqa: E731
    ref = {k: view(k, getattr(p, k)).clone() for k in OUTS}
    for kw in ({"pieces": 3}, {"bounds": [0, 1, nb // 2 + 1, nb]}):
        for k in OUTS:
            getattr(p, k).fill_(float("nan"))
        print(f"block={block} run_overlapped({kw})", flush=True)
        p.run_overlapped(**kw)
        torch.cuda.synchronize()
        for k in OUTS:
            assert torch.equal(view(k, getattr(p, k)), ref[k]), (kw, k)
    x = {k: v.to(dev) for k, v in inputs.gdn_layer_inputs(s, B=B, L=L, g_shift=-4.0).items()}
    one = _fork(x, s, pieces=1)
    torch.cuda.synchronize()
    one = {k: view(k, v).clone() for k, v in one.items() if v is not None}
    got = _fork(x, s, pieces=5)
    torch.cuda.synchronize()
    for k in one:
        assert torch.equal(view(k, got[k]), one[k]), k
    assert gdn.kernel_status(reset=True) == 0
