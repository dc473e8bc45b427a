"""Pins the CPU oracle of the complementary-mask attention (CPU only)."""

import numpy as np
import pytest
import torch

from oracle import attn_ref


def _enumerate(L, block, leak):
    ok = np.zeros((2 * L, 2 * L), bool)
    for i in range(2 * L):
        for j in range(2 * L):
            qi, kj = i % L, j % L
            qb, kb = qi // block, kj // block
            if i < L and j < L:
                ok[i, j] = (kb <= qb) if leak else (kb == qb)
            elif i < L:
                ok[i, j] = kb < qb
            elif j >= L:
                ok[i, j] = kb <= qb
    return ok


@pytest.mark.parametrize("L,block", [(32, 8), (24, 8), (64, 32), (12, 4), (16, 1)])
@pytest.mark.parametrize("leak", [False, True])
def test_complementary_mask_matches_enumeration_and_pair_count(L, block, leak):
    allowed = attn_ref.complementary_allowed(L, block, leak_xt_prefix=leak)
    assert np.array_equal(allowed.numpy(), _enumerate(L, block, leak))
    assert int(allowed.sum()) == attn_ref.allowed_pairs(L, block, leak_xt_prefix=leak)
    m = attn_ref.complementary_mask(L, block, torch.bfloat16, leak_xt_prefix=leak)
    assert m.shape == (1, 1, 2 * L, 2 * L)
    assert torch.equal(m[0, 0] == 0, allowed)
    assert (m[0, 0][~allowed] == torch.finfo(torch.bfloat16).min).all()
    assert allowed.any(1).all()  # every query sees at least its own block: no all-masked row


def test_allowed_pair_count_at_the_27b_attention_shape():
    # L=4096, block 32: 131,072 + 8,323,072 + 8,454,144 visible pairs (25.2% of 2L x 2L)
    assert attn_ref.allowed_pairs(4096, 32) == 16_908_288
    assert attn_ref.bd_attention_flops(2, 4096, 24, 256, 32) == 831_076_171_776


def test_block_causal_mask_matches_enumeration():
    m = attn_ref.block_causal_mask(20, 4)[0, 0]
    for i in range(20):
        for j in range(20):
            assert (m[i, j] == 0) == (j // 4 <= i // 4)


@pytest.mark.parametrize("leak", [False, True])
def test_bd_attention_matches_float64_bruteforce(leak):
    g = torch.Generator().manual_seed(21)
    B, L, Hq, Hkv, d, block = 2, 24, 4, 2, 16, 8
    q = torch.randn(B, 2 * L, Hq, d, generator=g)
    k = torch.randn(B, 2 * L, Hkv, d, generator=g)
    v = torch.randn(B, 2 * L, Hkv, d, generator=g)
    for rd in (0, 8):
        got = attn_ref.bd_attention(q, k, v, block=block, rotary_dim=rd, rope_base=1e4, leak_xt_prefix=leak,
                                    q_chunk=7)
        ref = attn_ref.bd_attention_f64_bruteforce(q, k, v, block=block, rotary_dim=rd, rope_base=1e4,
                                                   leak_xt_prefix=leak)
        assert np.abs(got.double().numpy() - ref).max() < 1e-5


@pytest.mark.parametrize("block", [8, 5])
def test_block_causal_attention_is_the_clean_half_of_the_bruteforce_at_every_offset(block):
    """The x_0 rows of the complementary mask see x_0 block-causally and nothing of x_t, so the
    clean half of the float64 brute force pins the prefill (q_offset 0); a query segment at offset
    q0 must equal rows q0.. of it, with only the first q0 + M keys present (a decode step)."""
    g = torch.Generator().manual_seed(5)
    B, L, Hq, Hkv, d = 2, 30, 4, 2, 16
    q = torch.randn(B, 2 * L, Hq, d, generator=g)
    k = torch.randn(B, 2 * L, Hkv, d, generator=g)
    v = torch.randn(B, 2 * L, Hkv, d, generator=g)
    ref = attn_ref.bd_attention_f64_bruteforce(q, k, v, block=block)[:, L:]
    qc, kc, vc = q[:, L:], k[:, L:], v[:, L:]
    got = attn_ref.block_causal_attention(qc, kc, vc, block=block)
    assert np.abs(got.double().numpy() - ref).max() < 1e-5
    for q0, M in ((10, 10), (block, block), (3, 7), (L - block, block)):
        n = min(L, (q0 + M + block - 1) // block * block)
        seg = attn_ref.block_causal_attention(qc[:, q0:q0 + M], kc[:, :n], vc[:, :n], block=block, q_offset=q0)
        assert np.abs(seg.double().numpy() - ref[:, q0:q0 + M]).max() < 1e-5
    # a planted off-by-one in the query offset is caught
    bad = attn_ref.block_causal_attention(qc[:, 9:19], kc, vc, block=block, q_offset=8)
    assert np.abs(bad.double().numpy() - ref[:, 9:19]).max() > 1e-3


def test_rope_matches_transformers_apply_rotary_and_rotary_module():
    from transformers.models.qwen3_5.configuration_qwen3_5 import Qwen3_5TextConfig
    from transformers.models.qwen3_5.modeling_qwen3_5 import Qwen3_5TextRotaryEmbedding, apply_rotary_pos_emb

    cfg = Qwen3_5TextConfig(hidden_size=64, num_attention_heads=4, num_key_value_heads=2, head_dim=32,
                            rope_parameters={"rope_theta": 1e7, "mrope_section": [2, 1, 1],
                                             "partial_rotary_factor": 0.25})
    rot = Qwen3_5TextRotaryEmbedding(cfg)
    L = 40
    x = torch.zeros(1, L, 64)
    pos = torch.arange(L).view(1, 1, -1).expand(3, 1, -1)  # text positions: all three sections equal
    cos_hf, sin_hf = rot(x, pos)
    cos, sin = attn_ref.rope_tables(torch.arange(L), 8, 1e7)
    assert torch.allclose(cos_hf[0], cos, atol=1e-6) and torch.allclose(sin_hf[0], sin, atol=1e-6)
    g = torch.Generator().manual_seed(22)
    q = torch.randn(1, L, 4, 32, generator=g)
    k = torch.randn(1, L, 2, 32, generator=g)
    qh, kh = apply_rotary_pos_emb(q.transpose(1, 2), k.transpose(1, 2), cos_hf, sin_hf)
    assert torch.allclose(attn_ref.apply_rope(q, cos, sin), qh.transpose(1, 2), atol=1e-6)
    assert torch.allclose(attn_ref.apply_rope(k, cos, sin), kh.transpose(1, 2), atol=1e-6)
