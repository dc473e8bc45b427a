"""Pins the CPU oracle of the state-fork GDN layer (CPU only).

Each check compares the oracle against something it does not restate: an independent algorithm
(float64 token recurrence, float64 FIR loop, brute-force index enumeration), a closed form, an
invariant, or the installed transformers kernel.
"""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import gdn_ref


def _inputs(B, T, H, D, seed, g_shift=0.0, Hk=None):
    g = torch.Generator().manual_seed(seed)
    Hk = H if Hk is None else Hk
    q = torch.randn(B, T, Hk, D, generator=g)
    k = torch.randn(B, T, Hk, D, generator=g)
    v = torch.randn(B, T, H, D, generator=g)
    beta = torch.sigmoid(torch.randn(B, T, H, generator=g))
    gg = -F.softplus(torch.randn(B, T, H, generator=g) + g_shift)
    return q, k, v, gg, beta


@pytest.mark.parametrize("chunk", [8, 16, 32])
def test_chunked_matches_float64_recurrence_outputs_and_states(chunk):
    q, k, v, g, beta = _inputs(2, 64, 3, 16, seed=chunk, g_shift=-2.0)
    init = torch.randn(2, 3, 16, 16, generator=torch.Generator().manual_seed(7)) * 0.3
    o, s = gdn_ref.chunk_gated_delta_rule_with_states(q, k, v, g, beta, chunk, initial_state=init)
    o64, s64 = gdn_ref.recurrent_gated_delta_rule_f64(q, k, v, g, beta, chunk_size=chunk, initial_state=init)
    assert np.abs(o.double().numpy() - o64).max() < 2e-6
    assert np.abs(s.double().numpy() - s64).max() < 2e-6
    assert s.shape == (2, 64 // chunk, 3, 16, 16)


def test_chunk_size_independence_of_outputs():
    q, k, v, g, beta = _inputs(1, 128, 2, 32, seed=11, g_shift=-3.0)
    outs = [gdn_ref.chunk_gated_delta_rule_with_states(q, k, v, g, beta, c)[0] for c in (8, 16, 32, 64, 128)]
    for o in outs[1:]:
        assert (o - outs[0]).abs().max().item() < 2e-6
    # the state after 64 tokens is the same whether the chunk is 32 or 64
    s32 = gdn_ref.chunk_gated_delta_rule_with_states(q, k, v, g, beta, 32)[1]
    s64 = gdn_ref.chunk_gated_delta_rule_with_states(q, k, v, g, beta, 64)[1]
    assert (s32[:, 1] - s64[:, 0]).abs().max().item() < 2e-6


def test_need_states_does_not_change_output_bitwise():
    q, k, v, g, beta = _inputs(2, 32, 2, 16, seed=3)
    o1, s1 = gdn_ref.chunk_gated_delta_rule_with_states(q, k, v, g, beta, 16, need_states=True)
    o2, s2 = gdn_ref.chunk_gated_delta_rule_with_states(q, k, v, g, beta, 16, need_states=False)
    assert torch.equal(o1, o2) and s2 is None and s1.shape[:2] == (2, 2)


def test_ragged_sequence_raises_reference_valueerror():
    q, k, v, g, beta = _inputs(1, 40, 1, 16, seed=4)
    with pytest.raises(ValueError, match="sequence_length 40 is not a multiple of chunk_size 32"):
        gdn_ref.chunk_gated_delta_rule_with_states(q, k, v, g, beta, 32)


def test_beta_zero_is_pure_decay_closed_form():
    """beta = 0: no writes; S_t = exp(sum g) S_0 and o_t = exp(gamma_t) S_0^T q_t (q l2-normed, scaled)."""
    B, T, H, D = 1, 32, 2, 16
    q, k, v, g, _ = _inputs(B, T, H, D, seed=5, g_shift=-3.0)
    beta = torch.zeros(B, T, H)
    S0 = torch.randn(B, H, D, D, generator=torch.Generator().manual_seed(6))
    o, s = gdn_ref.chunk_gated_delta_rule_with_states(q, k, v, g, beta, 16, initial_state=S0)
    gam = g.double().cumsum(1)  # [B,T,H]
    qn = q.double() / (q.double().pow(2).sum(-1, keepdim=True) + 1e-6).sqrt() * D ** -0.5
    want = torch.einsum("bth,bhkv,bthk->bthv", gam.exp(), S0.double(), qn)
    assert (o.double() - want).abs().max().item() < 1e-6
    want_s = S0.double() * gam[:, -1].exp()[..., None, None]
    assert (s[:, -1].double() - want_s).abs().max().item() < 1e-6


def test_delta_rule_exact_overwrite_with_orthonormal_keys():
    """g = 0, beta = 1, no l2norm: writing value v under unit key e_j stores exactly v; rewriting the
    same key replaces it (delta rule), so reading with q = e_j returns the latest value * Dk^-1/2."""
    D, T = 16, 24
    keys = torch.zeros(1, T, 1, D)
    for t in range(T):
        keys[0, t, 0, t % D] = 1.0  # keys repeat after D tokens: tokens 16..23 overwrite e_0..e_7
    v = torch.randn(1, T, 1, D, generator=torch.Generator().manual_seed(8))
    q = keys.clone()
    g = torch.zeros(1, T, 1)
    beta = torch.ones(1, T, 1)
    o, s = gdn_ref.chunk_gated_delta_rule_with_states(q, keys, v, g, beta, 8, use_qk_l2norm_in_kernel=False)
    assert (o[0, :, 0] - v[0, :, 0] * D ** -0.5).abs().max().item() < 1e-6
    final = s[0, -1, 0]  # [Dk, Dv]
    latest = {t % D: v[0, t, 0] for t in range(T)}
    for j, val in latest.items():
        assert (final[j] - val).abs().max().item() < 1e-6


def test_float64_recurrence_matches_transformers_recurrent_kernel():
    from transformers.models.qwen3_5.modeling_qwen3_5 import torch_recurrent_gated_delta_rule

    q, k, v, g, beta = _inputs(2, 20, 3, 16, seed=9, g_shift=-1.0)
    o_hf, s_hf = torch_recurrent_gated_delta_rule(q, k, v, g, beta, initial_state=None, output_final_state=True,
                                                  use_qk_l2norm_in_kernel=True)
    o64, s64 = gdn_ref.recurrent_gated_delta_rule_f64(q, k, v, g, beta, chunk_size=20)
    assert np.abs(o_hf.double().numpy() - o64).max() < 2e-6
    assert np.abs(s_hf.double().numpy() - s64[:, -1]).max() < 2e-6


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_conv_matches_float64_fir_with_and_without_prefix(dtype):
    g = torch.Generator().manual_seed(10)
    x = torch.randn(2, 24, 40, generator=g).to(dtype)
    w = (torch.rand(24, 4, generator=g) - 0.5).to(dtype)
    pre = torch.randn(2, 24, 3, generator=g).to(dtype)
    for prefix in (None, pre):
        y = gdn_ref.causal_conv1d(x, w, None, "silu", prefix=prefix)
        y64 = gdn_ref.causal_conv1d_bruteforce_f64(x, w, None, prefix=prefix)
        err = np.abs(y.double().numpy() - y64)
        if dtype == torch.float32:
            assert err.max() < 1e-5
        else:  # double rounding to bf16 (conv sum, then SiLU): within two bf16 ulps of |y|
            assert (err <= 2 * 2.0 ** -8 * np.abs(y64) + 1e-6).all()


def test_conv_prefix_equals_conv_over_concatenation():
    g = torch.Generator().manual_seed(12)
    x = torch.randn(1, 8, 32, generator=g)
    pre = torch.randn(1, 8, 3, generator=g)
    w = torch.rand(8, 4, generator=g) - 0.5
    y_pre = gdn_ref.causal_conv1d(x, w, None, "silu", prefix=pre)
    y_cat = gdn_ref.causal_conv1d(torch.cat([pre, x], 2), w, None, "silu")[:, :, -32:]
    assert torch.equal(y_pre, y_cat)


@pytest.mark.parametrize("B,L,block,width", [(1, 128, 32, 4), (3, 96, 8, 4), (2, 64, 1, 4), (2, 40, 2, 4),
                                              (2, 64, 16, 3), (4, 4096, 32, 4)])
def test_fork_layout_two_constructions_agree(B, L, block, width):
    a = gdn_ref.fork_layout(B, L, block, width)
    b = gdn_ref.fork_layout_bruteforce(B, L, block, width)
    for key in ("row", "state_src", "prefix_pos"):
        assert torch.equal(a[key], b[key]), key


def test_fork_layout_rejects_ragged_length():
    with pytest.raises(ValueError, match="not a multiple of block"):
        gdn_ref.fork_layout(1, 100, 32)


@pytest.mark.parametrize("g_shift", [0.0, -4.0])
def test_state_fork_layer_matches_visibility_contract_float64(g_shift):
    """Fork machinery (shifted states, unfolded conv prefixes, relaunched rows) vs first principles:
    noised block k = recurrence over cat(clean[:kC], noised block k) with the conv over the same
    concatenation."""
    B, L, block, Hk, Hv, D = 2, 64, 16, 1, 2, 16
    Cd = 2 * Hk * D + Hv * D
    g = torch.Generator().manual_seed(13)
    raw0 = torch.randn(B, L, Cd, generator=g)
    rawt = torch.randn(B, L, Cd, generator=g)
    w = torch.rand(Cd, 4, generator=g) - 0.5
    b0 = torch.sigmoid(torch.randn(B, L, Hv, generator=g))
    bt = torch.sigmoid(torch.randn(B, L, Hv, generator=g))
    g0 = -F.softplus(torch.randn(B, L, Hv, generator=g) + g_shift)
    gt = -F.softplus(torch.randn(B, L, Hv, generator=g) + g_shift)
    o0, ot, st, tails = gdn_ref.state_fork_layer(raw0, rawt, w, b0, bt, g0, gt, Hk=Hk, Hv=Hv, Dk=D, Dv=D, block=block)
    r0, rt, rst = gdn_ref.state_fork_layer_f64(raw0, rawt, w, b0, bt, g0, gt, Hk=Hk, Hv=Hv, Dk=D, Dv=D, block=block)
    assert np.abs(o0.double().numpy() - r0).max() < 2e-6
    assert np.abs(ot.double().numpy() - rt).max() < 2e-6
    assert np.abs(st.double().numpy() - rst).max() < 2e-6
    assert tails.shape == (B * (L // block), Cd, 3)
    # faults are visible: cold conv prefix and the naive concatenated causal pass both change ot
    _, ot_cold, _, _ = gdn_ref.state_fork_layer(raw0, rawt, w, b0, bt, g0, gt, Hk=Hk, Hv=Hv, Dk=D, Dv=D, block=block,
                                                fault="no-conv-prefix")
    ot_cat, _, _, _ = gdn_ref.state_fork_layer(raw0, rawt, w, b0, bt, g0, gt, Hk=Hk, Hv=Hv, Dk=D, Dv=D, block=block,
                                               fault="concat-causal-gdn")
    assert np.abs(ot_cold.double().numpy() - rt).max() > 1e-3
    assert np.abs(ot_cat.double().numpy() - rt).max() > 1e-3


def _carry_shape(g_shift):
    from dllm_qwen38_amd import inputs

    return inputs.GdnShape("carry-check", 1, 1024, 32, 2, 6, 128, 4, torch.bfloat16, g_shift, 5150)


def test_long_carry_oracle_matches_float64_recurrence():
    """Slow decay (about 0.9 nats per 32-token block) over 32 blocks at head size 128: the fp32
    oracle's clean outputs and every block state agree with the float64 token recurrence, so the
    bf16 bounds of the GPU tests measure the kernel, not the oracle."""
    from dllm_qwen38_amd import inputs

    s = _carry_shape(-4.0)
    x = inputs.gdn_layer_inputs(s)
    o0, _, st, _ = gdn_ref.state_fork_layer(x["raw0"], x["rawt"], x["conv_w"], x["beta0"], x["betat"], x["g0"],
                                            x["gt"], Hk=s.Hk, Hv=s.Hv, Dk=s.D, Dv=s.D, block=s.block)
    y = gdn_ref.causal_conv1d(x["raw0"].transpose(1, 2), x["conv_w"]).transpose(1, 2)
    q, k, v = gdn_ref._split_heads(y, 1, s.L, s.Hk, s.Hv, s.D, s.D)
    ro, rs = gdn_ref.recurrent_gated_delta_rule_f64(q, k, v, x["g0"], x["beta0"], chunk_size=32)
    assert np.abs(o0.float().numpy() - ro).max() <= 2 ** -8 * np.abs(ro).max()  # o0 is rounded to bf16
    assert np.abs(st.numpy() - rs).max() <= 1e-4
    assert np.abs(rs).max() > 0.5  # the carried state is not negligible


@pytest.mark.parametrize("plant", ["drop-carry", "carry-scale", "fork-off-by-one"])
def test_planted_carry_mistakes_exceed_the_bf16_bounds(plant):
    """A kernel that dropped the carried state or forked from the wrong block would fail the GPU
    tests' bf16 bounds many times over on the slow-decay inputs, and one that scaled the carry by
    1.05 at least twice over (a 2% scaling sits at the resolution of bf16 state operands). On the fast
    decay of the 27B-class workload (g = -softplus(N(0,1)+1): 25-45 nats per block) a dropped
    carry stays far inside them, which is why the carry tests use slow decay."""
    from _bounds import excess, out_bound, state_bound
    from dllm_qwen38_amd import inputs

    def run(shift, p):
        s = _carry_shape(shift)
        x = inputs.gdn_layer_inputs(s)
        return gdn_ref.state_fork_layer(x["raw0"], x["rawt"], x["conv_w"], x["beta0"], x["betat"], x["g0"], x["gt"],
                                        Hk=s.Hk, Hv=s.Hv, Dk=s.D, Dv=s.D, block=s.block, _plant=p)

    good, bad = run(-4.0, None), run(-4.0, plant)
    ratios = {"o0": excess(bad[0], good[0], out_bound)[1], "ot": excess(bad[1], good[1], out_bound)[1],
              "states": excess(bad[2], good[2], state_bound)[1]}
    print(plant, ratios)
    assert max(ratios.values()) > (2.0 if plant == "carry-scale" else 8.0)
    if plant == "drop-carry":
        fast_good, fast_bad = run(1.0, None), run(1.0, plant)
        assert excess(fast_bad[1], fast_good[1], out_bound)[1] < 0.1
