"""GPU parity of the bf16 state-fork kernels where the carried state matters.

The 27B- and 0.8B-class workloads decay 25-45 nats per 32-token block, so the state a block
inherits is ~1e-11 of its own contribution and a wrong carry would not show. These tests drive
the same kernels with slow decay, g = -softplus(N(0,1) - 4) (about 0.9 nats per block), over 32
blocks, and compare with the fp32 oracle on the same bf16 inputs within the bounds of
tests/_bounds.py (which a dropped, mis-scaled or mis-forked carry exceeds: tests/test_oracle_gdn.py).
They cover the pipelined fork kernel at both head layouts, at blocks 32, 16 and 8, without
state snapshots and at grids that are not a multiple of the 8 XCDs or exceed the chip's CUs, and
the bf16 chunked rule with an initial state on both of its kernels (the pipelined kernel on one
stream for chunks that divide the tile, the chunk kernel with one and two column windows per head
for longer chunks).
"""

import numpy as np
import pytest
import torch

from _bounds import excess, out_bound, state_bound
from dllm_qwen38_amd import gdn, inputs
from oracle import gdn_ref

pytestmark = pytest.mark.gpu

SLOW = -4.0


def _shape(name, B, L, block, Hk, Hv, seed):
    return inputs.GdnShape(name, B, L, block, Hk, Hv, 128, 4, torch.bfloat16, SLOW, seed)


def _fork(s, x, dev, **kw):
    xd = {k: v.to(dev) for k, v in x.items()}
    r = gdn.gdn_state_fork(xd["raw0"], xd["rawt"], xd["conv_w"], xd["beta0"], xd["betat"], xd["g0"], xd["gt"],
                           num_k_heads=s.Hk, num_v_heads=s.Hv, head_k_dim=s.D, head_v_dim=s.D, block=s.block, **kw)
    torch.cuda.synchronize()
    return {k: (v.cpu() if v is not None else None) for k, v in r.items()}


def _oracle(s, x):
    return gdn_ref.state_fork_layer(x["raw0"], x["rawt"], x["conv_w"], x["beta0"], x["betat"], x["g0"], x["gt"],
                                    Hk=s.Hk, Hv=s.Hv, Dk=s.D, Dv=s.D, block=s.block)


def _check(name, got, ref, bound):
    over, ratio = excess(got, ref, bound)
    d = (got.float() - ref.float()).abs()
    print(f"{name}: max|d|={d.max().item():.3e} mean|d|={d.mean().item():.3e} max|ref|={ref.float().abs().max().item():.3e} "
          f"max |d|/bound={ratio:.3f}", flush=True)
    assert over <= 0, f"{name} exceeds its bf16 bound (max |d|/bound = {ratio:.3f})"


CARRY_SHAPES = [
    _shape("27B-class heads (Hk 16, Hv 48)", 1, 1024, 32, 16, 48, 3150),
    _shape("0.8B-class heads (Hk = Hv = 16)", 2, 1024, 32, 16, 16, 2150),
]


@pytest.mark.parametrize("s", CARRY_SHAPES, ids=["27b", "08b"])
def test_pipe_fork_slow_decay_matches_oracle(dev, s):
    x = inputs.gdn_layer_inputs(s)
    r = _fork(s, x, dev)
    assert gdn.last_impl()[0] == "hip" and gdn.last_impl()[1].startswith("pipelined fork kernel")
    o0, ot, st, tails = _oracle(s, x)
    assert torch.equal(r["tails"], tails)
    assert st.abs().max().item() > 0.5, "the carried state must be non-negligible"
    _check(f"{s.name} o0", r["o0"], o0, out_bound)
    _check(f"{s.name} ot", r["ot"], ot, out_bound)
    _check(f"{s.name} states", r["states"], st, state_bound)


def test_pipe_fork_clean_stream_vs_float64_recurrence(dev):
    """The clean outputs and every block state of the pipelined kernel against the float64 token
    recurrence on the same (bf16-rounded, convolved) inputs: an independent algorithm."""
    s = CARRY_SHAPES[1]
    x = inputs.gdn_layer_inputs(s, B=1)
    r = _fork(s, x, dev)
    y = gdn_ref.causal_conv1d(x["raw0"].transpose(1, 2), x["conv_w"]).transpose(1, 2)
    q, k, v = gdn_ref._split_heads(y, 1, s.L, s.Hk, s.Hv, s.D, s.D)
    ro, rs = gdn_ref.recurrent_gated_delta_rule_f64(q, k, v, x["g0"], x["beta0"], chunk_size=32)
    _check("clean vs f64 o0", r["o0"], torch.from_numpy(ro), out_bound)
    _check("clean vs f64 states", r["states"], torch.from_numpy(rs), state_bound)


@pytest.mark.parametrize("block", [16, 8])
def test_pipe_fork_subtile_blocks(dev, block):
    """Blocks shorter than the 32-row tile (zero-padded rows) through the pipelined kernel."""
    s = _shape(f"Hk 4, Hv 8, block {block}", 2, 256, block, 4, 8, 4150 + block)
    x = inputs.gdn_layer_inputs(s)
    r = _fork(s, x, dev)
    assert gdn.last_impl()[0] == "hip" and gdn.last_impl()[1].startswith("pipelined fork kernel")
    o0, ot, st, tails = _oracle(s, x)
    assert torch.equal(r["tails"], tails)
    assert r["states"].shape == (2, 256 // block, 8, 128, 128)
    _check(f"block {block} o0", r["o0"], o0, out_bound)
    _check(f"block {block} ot", r["ot"], ot, out_bound)
    _check(f"block {block} states", r["states"], st, state_bound)


@pytest.mark.parametrize("B,Hk,Hv,L", [(3, 1, 5, 128), (5, 1, 53, 64)], ids=["30 workgroups", "265 workgroups"])
def test_pipe_fork_grids_not_a_multiple_of_eight(dev, B, Hk, Hv, L):
    """Workgroup counts that are not a multiple of the 8 XCDs (the kernel maps dispatch slots to
    (sequence, head) pairs per XCD; every pair must still be reached exactly once) and more
    workgroups than the chip has CUs (several rounds): 15 heads with their columns split over two
    workgroups (30), and 265 heads one workgroup each."""
    s = _shape(f"B {B}, Hk {Hk}, Hv {Hv}", B, L, 32, Hk, Hv, 8150 + Hv)
    x = inputs.gdn_layer_inputs(s)
    r = _fork(s, x, dev)
    assert gdn.last_impl()[0] == "hip" and gdn.last_impl()[1].startswith("pipelined fork kernel")
    o0, ot, st, tails = _oracle(s, x)
    assert torch.equal(r["tails"], tails)
    _check(f"{B}x{Hv} o0", r["o0"], o0, out_bound)
    _check(f"{B}x{Hv} ot", r["ot"], ot, out_bound)
    _check(f"{B}x{Hv} states", r["states"], st, state_bound)


def test_pipe_fork_need_states_false_is_bit_identical(dev):
    """The product forward runs the fork without snapshots (states == NULL): same outputs, bitwise."""
    s = _shape("27B-class heads, L 512", 1, 512, 32, 16, 48, 6150)
    x = inputs.gdn_layer_inputs(s)
    a = _fork(s, x, dev)
    b = _fork(s, x, dev, need_states=False, need_tails=False)
    assert b["states"] is None and b["tails"] is None
    assert gdn.last_impl()[0] == "hip" and gdn.last_impl()[1].startswith("pipelined fork kernel")
    assert torch.equal(a["o0"], b["o0"]) and torch.equal(a["ot"], b["ot"])


@pytest.mark.parametrize("B,Hk,Hv", [(1, 2, 8), (2, 16, 64), (3, 16, 48)], ids=["8 heads", "128 heads", "144 heads"])
@pytest.mark.parametrize("chunk", [32, 16, 64])
def test_chunk_kernel_bf16_matches_oracle(dev, B, Hk, Hv, chunk):
    """chunk_gated_delta_rule_with_states in bf16 at Dk = Dv = 128 with an initial state and slow
    decay. Chunks of 32 and 16 run the pipelined kernel on one stream (a head's columns over two
    workgroups up to 128 (sequence, head) pairs on this chip, one workgroup each above); chunks of
    64 run the chunk kernel (two 64-column windows per head below 128 pairs, one 128-column window
    from 128)."""
    T = 512
    q, k, v, g, beta = inputs.gdn_core_inputs(B, T, Hk, Hv, 128, torch.bfloat16, seed=7150 + Hv + chunk,
                                              g_shift=SLOW)
    init = torch.randn(B, Hv, 128, 128, generator=torch.Generator().manual_seed(7160 + Hv)) * 0.5
    out, st = gdn.chunk_gated_delta_rule_with_states(q.to(dev), k.to(dev), v.to(dev), g.to(dev), beta.to(dev), chunk,
                                                     initial_state=init.to(dev))
    torch.cuda.synchronize()
    n = Hv // Hk
    ro, rs = gdn_ref.chunk_gated_delta_rule_with_states(q.repeat_interleave(n, 2), k.repeat_interleave(n, 2), v, g,
                                                        beta, chunk, initial_state=init)
    assert st.shape == (B, T // chunk, Hv, 128, 128)
    # the initial state still weighs on the last chunk's state
    lam_total = np.exp(g.double().sum(1).max().item())
    print(f"initial-state weight at the end: {lam_total:.2e}")
    _check(f"chunk {chunk} {B}x{Hv} out", out.cpu(), ro, out_bound)
    _check(f"chunk {chunk} {B}x{Hv} states", st.cpu(), rs, state_bound)



@pytest.mark.parametrize("chunk", [8, 4, 2, 1])
def test_chunk_rule_bf16_short_chunks_on_the_pipelined_kernel(dev, chunk):
    """Chunks shorter than 8 rows per 32-row tile (every chunk that divides 32 runs the pipelined
    kernel on one stream; the tile then holds `chunk` real rows and zero padding), with an initial
    state and slow decay, against the oracle and the float64 token recurrence."""
    B, Hk, Hv, T = 1, 2, 8, 64
    q, k, v, g, beta = inputs.gdn_core_inputs(B, T, Hk, Hv, 128, torch.bfloat16, seed=7350 + chunk, g_shift=SLOW)
    init = torch.randn(B, Hv, 128, 128, generator=torch.Generator().manual_seed(7360 + chunk)) * 0.5
    out, st = gdn.chunk_gated_delta_rule_with_states(q.to(dev), k.to(dev), v.to(dev), g.to(dev), beta.to(dev), chunk,
                                                     initial_state=init.to(dev))
    torch.cuda.synchronize()
    qe, ke = q.repeat_interleave(Hv // Hk, 2), k.repeat_interleave(Hv // Hk, 2)
    ro, rs = gdn_ref.chunk_gated_delta_rule_with_states(qe, ke, v, g, beta, chunk, initial_state=init)
    assert st.shape == (B, T // chunk, Hv, 128, 128)
    _check(f"chunk {chunk} out", out.cpu(), ro, out_bound)
    _check(f"chunk {chunk} states", st.cpu(), rs, state_bound)
    fo, fs = gdn_ref.recurrent_gated_delta_rule_f64(qe, ke, v, g, beta, chunk_size=chunk, initial_state=init)
    _check(f"chunk {chunk} out vs f64", out.cpu(), torch.from_numpy(fo), out_bound)
    _check(f"chunk {chunk} states vs f64", st.cpu(), torch.from_numpy(fs), state_bound)


@pytest.mark.parametrize("chunk", [32, 16, 64])
def test_chunk_rule_bf16_without_qk_l2norm(dev, chunk):
    """use_qk_l2norm_in_kernel=False: q and k enter unnormalised (the kernels' no-norm branches: unit
    k-row scales and q scaled by Dk^-1/2 alone). Inputs are drawn with rows of norm about 1, as the
    recurrence needs bounded keys, on both kernels (chunks 32 / 16 pipelined, 64 the chunk kernel)."""
    B, Hk, Hv, T = 2, 2, 8, 256
    q, k, v, g, beta = inputs.gdn_core_inputs(B, T, Hk, Hv, 128, torch.bfloat16, seed=7450 + chunk, g_shift=SLOW)
    q = (q.float() / 128 ** 0.5).to(torch.bfloat16)
    k = (k.float() / 128 ** 0.5).to(torch.bfloat16)
    out, st = gdn.chunk_gated_delta_rule_with_states(q.to(dev), k.to(dev), v.to(dev), g.to(dev), beta.to(dev), chunk,
                                                     use_qk_l2norm_in_kernel=False)
    torch.cuda.synchronize()
    qe, ke = q.repeat_interleave(Hv // Hk, 2), k.repeat_interleave(Hv // Hk, 2)
    ro, rs = gdn_ref.chunk_gated_delta_rule_with_states(qe, ke, v, g, beta, chunk, use_qk_l2norm_in_kernel=False)
    _check(f"no l2norm chunk {chunk} out", out.cpu(), ro, out_bound)
    _check(f"no l2norm chunk {chunk} states", st.cpu(), rs, state_bound)
    fo, fs = gdn_ref.recurrent_gated_delta_rule_f64(qe, ke, v, g, beta, chunk_size=chunk, use_qk_l2norm=False)
    _check(f"no l2norm chunk {chunk} out vs f64", out.cpu(), torch.from_numpy(fo), out_bound)
