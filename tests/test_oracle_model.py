"""Pins the CPU oracle of the hybrid model forward against transformers' own Qwen3.5 modules (CPU)."""

import pytest
import torch

from _tiny import noised_ids, tiny_hf_model
from oracle import model_ref

FAULTS = ("concat-causal-gdn", "mask-leak", "no-conv-prefix")


@pytest.fixture(scope="module")
def tiny():
    return tiny_hf_model(seed=0)


def test_norms_and_mlp_match_transformers(tiny):
    model, _ = tiny
    g = torch.Generator().manual_seed(2)
    x = torch.randn(2, 7, 64, generator=g)
    layer = model.layers[0]
    assert torch.allclose(model_ref.rmsnorm(x, layer.input_layernorm.weight, layer.input_layernorm.eps),
                          layer.input_layernorm(x), atol=1e-6)
    assert torch.allclose(model_ref.mlp(layer.mlp, x), layer.mlp(x), atol=1e-6)
    m = layer.linear_attn
    a = torch.randn(14, 16, generator=g)
    z = torch.randn(14, 16, generator=g)
    assert torch.allclose(model_ref.gated_rmsnorm(a, z, m.norm.weight, m.norm.variance_epsilon), m.norm(a, z), atol=1e-6)


def test_gdn_mixer_matches_transformers_linear_attention(tiny):
    """The oracle mixer (conv + chunked delta rule at chunk 8) against HF's own layer (its torch chunked
    kernel, chunk 64) on a whole sequence: agreement pins the conv, gates, GQA and gated norm."""
    model, _ = tiny
    m = model.layers[0].linear_attn
    h = torch.randn(2, 24, 64, generator=torch.Generator().manual_seed(3))
    with torch.no_grad():
        ref = m(h)
        got, states, raw = model_ref.gdn_mixer(m, h, chunk=8)
    assert (got - ref).abs().max().item() < 1e-5
    assert states.shape == (2, 3, 4, 16, 16) and raw.shape == (2, m.conv_dim, 24)


def test_attention_layer_matches_transformers_under_block_causal_mask(tiny):
    from transformers.models.qwen3_5.modeling_qwen3_5 import Qwen3_5TextRotaryEmbedding  # noqa: F401

    model, _ = tiny
    att = model.layers[3].self_attn
    S, block = 24, 8
    h = torch.randn(2, S, 64, generator=torch.Generator().manual_seed(4))
    pos = torch.arange(S).view(1, 1, -1).expand(3, 2, -1)
    cos_hf, sin_hf = model.rotary_emb(h, pos)
    blk = torch.arange(S) // block
    allowed = blk[None, :] <= blk[:, None]
    mask = torch.zeros(S, S).masked_fill(~allowed, torch.finfo(torch.float32).min)[None, None]
    with torch.no_grad():
        ref, _ = att(hidden_states=h, position_embeddings=(cos_hf, sin_hf), attention_mask=mask)
        cos, sin = model_ref.rope_cos_sin(model, S)
        got = model_ref.attention_layer(att, h, cos, sin, block=None, causal_mask=allowed)
    assert (got - ref).abs().max().item() < 1e-5


def test_causal_block_forward_matches_transformers_model(tiny):
    model, lm_head = tiny
    ids = torch.randint(0, 256, (2, 24), generator=torch.Generator().manual_seed(5))
    blk = torch.arange(24) // 8
    mask = torch.zeros(24, 24).masked_fill(~(blk[None, :] <= blk[:, None]), torch.finfo(torch.float32).min)[None, None]
    with torch.no_grad():
        hs = model(input_ids=ids, attention_mask={"full_attention": mask, "linear_attention": None},
                   use_cache=False).last_hidden_state
        ref = lm_head(hs)
        got = model_ref.causal_block_forward(model, lm_head, ids, 8)
    assert (got - ref).abs().max().item() < 1e-4


def test_fork_forward_equals_per_block_oracle_and_faults_are_detected(tiny):
    """The visibility contract: the forked two-stream forward equals, block by block, a plain forward
    of cat(x_0 prefix, x_t block); the clean stream equals the block-causal forward of x_0; every
    deliberate fault breaks the noised stream."""
    model, lm_head = tiny
    x0, xt = noised_ids(2, 32, seed=6)
    lt, l0 = model_ref.block_diffusion_forward(model, lm_head, x0, xt, 8)
    ref_t = model_ref.reference_block_logits(model, lm_head, x0, xt, 8)
    ref_0 = model_ref.reference_clean_logits(model, lm_head, x0, 8)
    assert (lt - ref_t).abs().max().item() < 1e-4
    assert (l0 - ref_0).abs().max().item() < 1e-4
    for f in FAULTS:
        lf, _ = model_ref.block_diffusion_forward(model, lm_head, x0, xt, 8, fault=f)
        assert (lf - ref_t).abs().max().item() > 1e-3, f
