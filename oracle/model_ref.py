"""CPU oracle of the hybrid text model's block-diffusion forward — TEST INFRASTRUCTURE ONLY.

Restates, reading weights from an HF-shaped module tree (transformers' Qwen3_5TextModel or the
product's lightweight model with the same attribute names):
  * Qwen3_5RMSNorm with the (1 + w) weight, computed in fp32 then cast back
    (transformers 5.15.0 models/qwen3_5/modeling_qwen3_5.py:720-737);
  * Qwen3_5RMSNormGated: norm in fp32, weight in the input dtype, * silu(z) in fp32 ([hf]:168-184);
  * the SwiGLU MLP ([hf]:704-717);
  * the gated attention layer: q_proj -> (q, gate), q/k RMSNorm, partial RoPE with positions shared
    by both halves, complementary-mask attention, * sigmoid(gate), o_proj ([hf]:656-701 driven as in
    reference src/dllm_qwen38/blockdiff.py:178-182);
  * the GDN mixer with conv prefix and initial state (reference src/dllm_qwen38/gdn.py:193-233);
  * block_diffusion_forward with the state fork and the three faults (blockdiff.py:96-203);
  * the per-block oracle (blockdiff.py:206-243): for block k, the sequence cat(x_0[:kC], x_t block k)
    through a plain causal block model (GDN without any fork, attention under the block-causal mask).

How it is pinned (tests/test_oracle_model.py): the per-module restatements against transformers' own
modules of a random Qwen3_5TextModel; the per-block oracle against transformers' full model forward
(its own torch chunked GDN kernel, chunk 64, and eager attention); the fork forward against the
per-block oracle (the visibility contract), and every fault must move the noised logits.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

from . import attn_ref, gdn_ref

FULL = "full_attention"
LINEAR = "linear_attention"


def rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    xf = x.float()
    y = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
    return (y * (1.0 + weight.float())).type_as(x)


def gated_rmsnorm(x: torch.Tensor, z: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    dt = x.dtype
    xf = x.float()
    y = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
    y = weight * y.to(dt)
    return (y * F.silu(z.float())).to(dt)


def mlp(m, x):
    return m.down_proj(F.silu(m.gate_proj(x)) * m.up_proj(x))


def _eps(layer_norm) -> float:
    return getattr(layer_norm, "eps", getattr(layer_norm, "variance_epsilon", 1e-6))


def rope_cos_sin(text_model, L: int):
    """fp32 cos/sin [L, rotary_dim] for positions 0..L-1 (the text-only case of the interleaved mRoPE:
    all three position sections equal)."""
    inv = text_model.rotary_emb.inv_freq.float().cpu()
    pos = torch.arange(L, dtype=torch.float32)
    fr = pos[:, None] * inv[None, :]
    emb = torch.cat([fr, fr], -1)
    return emb.cos(), emb.sin()


def attention_layer(att, h: torch.Tensor, cos, sin, *, block: int | None, leak: bool = False, causal_mask=None):
    """Gated attention over h [B, S, D]. With block set, S = 2L = cat([x_t, x_0]) under the
    complementary mask (positions shared by the halves); with causal_mask (a [S, S] bool), a plain
    sequence under that mask (positions 0..S-1)."""
    B, S, _ = h.shape
    hd = att.head_dim
    qg = att.q_proj(h).view(B, S, -1, hd * 2)
    q, gate = torch.chunk(qg, 2, dim=-1)
    gate = gate.reshape(B, S, -1)
    q = rmsnorm(q, att.q_norm.weight, _eps(att.q_norm))
    k = rmsnorm(att.k_proj(h).view(B, S, -1, hd), att.k_norm.weight, _eps(att.k_norm))
    v = att.v_proj(h).view(B, S, -1, hd)
    dt = q.dtype
    c, s_ = cos.to(dt), sin.to(dt)  # the rotary tables are cast to the activation dtype
    q = attn_ref.apply_rope(q, c, s_)
    k = attn_ref.apply_rope(k, c, s_)
    if block is not None:
        o = attn_ref.bd_attention(q, k, v, block=block, leak_xt_prefix=leak, scale=hd ** -0.5).to(dt)
    else:
        rep = q.shape[2] // k.shape[2]
        kx = k.repeat_interleave(rep, 2).permute(0, 2, 1, 3).float()
        vx = v.repeat_interleave(rep, 2).permute(0, 2, 1, 3).float()
        sc = (q.permute(0, 2, 1, 3).float() @ kx.transpose(-1, -2)) * hd ** -0.5
        sc = sc.masked_fill(~causal_mask, float("-inf"))
        o = (torch.softmax(sc, -1) @ vx).permute(0, 2, 1, 3).to(dt)
    o = o.reshape(B, S, -1) * torch.sigmoid(gate)
    return att.o_proj(o)


def gdn_mixer(m, h: torch.Tensor, *, chunk: int, conv_prefix=None, initial_state=None, need_states=True):
    """Reference gdn.py:193-233 on the CPU oracle core."""
    B, T, _ = h.shape
    raw = m.in_proj_qkv(h)  # [B, T, conv_dim]
    z = m.in_proj_z(h).reshape(B, T, -1, m.head_v_dim)
    beta = m.in_proj_b(h).sigmoid()
    g = -m.A_log.float().exp() * F.softplus(m.in_proj_a(h).float() + m.dt_bias)
    mixed = gdn_ref.causal_conv1d(raw.transpose(1, 2), m.conv1d.weight.squeeze(1), m.conv1d.bias, "silu",
                                  prefix=conv_prefix).transpose(1, 2)
    q, k, v = gdn_ref._split_heads(mixed, B, T, m.num_k_heads, m.num_v_heads, m.head_k_dim, m.head_v_dim)
    core, states = gdn_ref.chunk_gated_delta_rule_with_states(q, k, v, g, beta, chunk_size=chunk,
                                                             initial_state=initial_state, need_states=need_states)
    core = gated_rmsnorm(core.reshape(-1, m.head_v_dim), z.reshape(-1, m.head_v_dim), m.norm.weight,
                         getattr(m.norm, "variance_epsilon", 1e-6)).reshape(B, T, -1)
    return m.out_proj(core), states, raw.transpose(1, 2)


@torch.no_grad()
def block_diffusion_forward(text_model, lm_head, x0_ids, xt_ids, block: int, *, fault: str | None = None,
                            layers: int | None = None, output: str = "logits"):
    """Two-stream forward with the state fork (reference blockdiff.py:96-203). Returns
    (logits_t, logits_0) or the final-normed hiddens."""
    cfg = text_model.config
    B, L = x0_ids.shape
    nb = L // block
    h0 = text_model.embed_tokens(x0_ids)
    ht = text_model.embed_tokens(xt_ids)
    cos, sin = rope_cos_sin(text_model, L)
    cos2, sin2 = torch.cat([cos, cos], 0), torch.cat([sin, sin], 0)
    n = cfg.num_hidden_layers if layers is None else layers
    for i in range(n):
        layer = text_model.layers[i]
        kind = cfg.layer_types[i]
        eps = _eps(layer.input_layernorm)
        n0 = rmsnorm(h0, layer.input_layernorm.weight, eps)
        nt = rmsnorm(ht, layer.input_layernorm.weight, eps)
        if kind == LINEAR:
            m = layer.linear_attn
            if fault == "concat-causal-gdn":
                out, _, _ = gdn_mixer(m, torch.cat([nt, n0], 1), chunk=block, need_states=False)
                ot, o0 = out[:, :L], out[:, L:]
            else:
                o0, states0, raw0 = gdn_mixer(m, n0, chunk=block, need_states=True)
                init = torch.cat([torch.zeros_like(states0[:, :1]), states0[:, :-1]], 1)
                init = init.reshape(B * nb, *init.shape[2:])
                km1 = m.conv_kernel_size - 1
                prefix = None
                if fault != "no-conv-prefix":
                    padded = torch.cat([torch.zeros_like(raw0[:, :, :km1]), raw0], 2)
                    prefix = padded.unfold(2, km1, block)[:, :, :nb].permute(0, 2, 1, 3).reshape(B * nb, -1, km1)
                ot, _, _ = gdn_mixer(m, nt.reshape(B * nb, block, -1), chunk=block, conv_prefix=prefix,
                                     initial_state=init, need_states=False)
                ot = ot.reshape(B, L, -1)
        else:
            out = attention_layer(layer.self_attn, torch.cat([nt, n0], 1), cos2, sin2, block=block,
                                  leak=(fault == "mask-leak"))
            ot, o0 = out[:, :L], out[:, L:]
        h0, ht = h0 + o0, ht + ot
        epa = _eps(layer.post_attention_layernorm)
        h0 = h0 + mlp(layer.mlp, rmsnorm(h0, layer.post_attention_layernorm.weight, epa))
        ht = ht + mlp(layer.mlp, rmsnorm(ht, layer.post_attention_layernorm.weight, epa))
    ht = rmsnorm(ht, text_model.norm.weight, _eps(text_model.norm))
    h0 = rmsnorm(h0, text_model.norm.weight, _eps(text_model.norm))
    if output == "hidden":
        return ht, h0
    return lm_head(ht), lm_head(h0)


@torch.no_grad()
def causal_block_forward(text_model, lm_head, ids, block: int, *, layers: int | None = None):
    """A plain block-causal forward of one sequence batch (no fork): GDN is an ordinary causal
    recurrence, attention uses the block-causal mask. Logits [B, S, V]."""
    cfg = text_model.config
    B, S = ids.shape
    h = text_model.embed_tokens(ids)
    cos, sin = rope_cos_sin(text_model, S)
    blk = torch.arange(S) // block
    mask = blk[None, :] <= blk[:, None]
    n = cfg.num_hidden_layers if layers is None else layers
    chunk = block if S % block == 0 else 1
    for i in range(n):
        layer = text_model.layers[i]
        x = rmsnorm(h, layer.input_layernorm.weight, _eps(layer.input_layernorm))
        if cfg.layer_types[i] == LINEAR:
            o, _, _ = gdn_mixer(layer.linear_attn, x, chunk=chunk, need_states=False)
        else:
            o = attention_layer(layer.self_attn, x, cos, sin, block=None, causal_mask=mask)
        h = h + o
        h = h + mlp(layer.mlp, rmsnorm(h, layer.post_attention_layernorm.weight, _eps(layer.post_attention_layernorm)))
    return lm_head(rmsnorm(h, text_model.norm.weight, _eps(text_model.norm)))


@torch.no_grad()
def reference_block_logits(text_model, lm_head, x0_ids, xt_ids, block: int, *, layers: int | None = None):
    """Per-block oracle (reference blockdiff.py:206-228): for each block k, a block-causal forward of
    cat(x_0[:, :kC], x_t block k); returns the last block's logits concatenated over k -> [B, L, V]."""
    L = x0_ids.shape[1]
    outs = []
    for k in range(L // block):
        seq = torch.cat([x0_ids[:, : k * block], xt_ids[:, k * block: (k + 1) * block]], 1)
        outs.append(causal_block_forward(text_model, lm_head, seq, block, layers=layers)[:, -block:])
    return torch.cat(outs, 1)


@torch.no_grad()
def reference_clean_logits(text_model, lm_head, x0_ids, block: int, *, layers: int | None = None):
    """Oracle for the clean stream (blockdiff.py:231-243)."""
    return causal_block_forward(text_model, lm_head, x0_ids, block, layers=layers)
