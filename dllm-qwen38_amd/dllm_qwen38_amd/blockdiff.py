"""Block-diffusion two-stream forward of a Qwen3.5/3.8 hybrid on the MI355X HIP kernels.

Drop-in for the reference's `src/dllm_qwen38/blockdiff.py`:
  block_diffusion_forward (blockdiff.py:96-203), BreakMode (:69-88), complementary_mask /
  block_causal_mask (:43-66), the per-block oracles reference_block_logits /
  reference_clean_logits (:206-243) and tiny_text_model (:246-278), and LayerStep, the per-layer
  unit of the FSDP trainer (fsdp_train.py:83-130), which here calls the same `layer_step` function
  as the stack driver so the fork exists in one place.

Visibility contract (x_t = noised stream, x_0 = clean stream, block(i) = i // block):
x_t token i sees x_t token j iff block(j) == block(i); x_t sees x_0 iff block(j) < block(i);
x_0 sees x_0 iff block(j) <= block(i); x_0 never sees x_t.

Per layer:
  * linear-attention (Gated DeltaNet) layers: one projection GEMM per weight over both streams,
    then ONE fused fork op (`gdn.gdn_state_fork`): the short conv of both streams with the clean
    3-token prefix carried into every noised block, and the clean recurrence whose state at every
    block boundary seeds that block's noised recurrence on the fly (no state copy, no shifted
    initial-state tensor, no prefix tensor), then the gated norm and out_proj over both streams;
  * full-attention layers: projections, q/k RMSNorm and partial RoPE (positions 0..L-1 shared by
    both halves), then the complementary-mask attention kernel, which derives visibility from
    (L, block) and skips hidden tiles (no [2L, 2L] mask exists), then the sigmoid output gate and
    o_proj.
The GEMMs (hipBLASLt through torch) and the sigmoid output gate run as torch ops on the same
stream; the mixers, the norms (each residual add fused into the norm after it), the SwiGLU product
and the q/k norm + RoPE prologue are HIP kernels of libdllm_hip.so. Forward only: the HIP ops have
no backward, so a call that would need gradients raises instead of returning a graph that
silently stops at the kernels.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn.functional as F
from torch import nn

from . import attention, gdn, norms
from .attention import block_causal_mask, complementary_mask  # noqa: F401  (re-exported, reference names)

FULL = "full_attention"
LINEAR = "linear_attention"


@dataclass
class BreakMode:
    """Deliberate faults, each of which must make the equivalence check fail (blockdiff.py:69-88)."""

    name: str = "none"

    @property
    def concat_causal_gdn(self) -> bool:
        """GDN over cat([x_t, x_0]) as one causal sequence."""
        return self.name == "concat-causal-gdn"

    @property
    def leak_xt_prefix(self) -> bool:
        """x_t block k also sees x_t blocks < k in attention."""
        return self.name == "mask-leak"

    @property
    def drop_conv_prefix(self) -> bool:
        """The state is forked but the short conv starts cold at every noised block."""
        return self.name == "no-conv-prefix"


def _eps(norm) -> float:
    return float(getattr(norm, "eps", getattr(norm, "variance_epsilon", 1e-6)))


def rmsnorm(x: torch.Tensor, norm, residual: torch.Tensor | None = None):
    """Qwen3.5 RMSNorm with (1 + w) ([hf]:720-737) on the HIP kernel; with a residual, returns
    (norm(x + residual), x + residual) from one pass."""
    return norms.rmsnorm(x, norm.weight, _eps(norm), residual=residual)


def mlp(m, x: torch.Tensor) -> torch.Tensor:
    """SwiGLU ([hf]:704-717): the two projections, one fused silu-product kernel, the down projection.
    When the gate and up weights are the halves of one tensor (`model.fuse_gate_up`), the two
    projections are one GEMM and the silu product reads its halves in place."""
    w = getattr(m, "gate_up_weight", None)
    gw, uw = m.gate_proj.weight, m.up_proj.weight
    if (w is not None and gw.data_ptr() == w.data_ptr()
            and uw.data_ptr() == w.data_ptr() + gw.numel() * w.element_size() and w.dtype == x.dtype):
        y = torch.nn.functional.linear(x, w)
        n = gw.shape[0]
        return m.down_proj(norms.swiglu(y[..., :n], y[..., n:]))
    return m.down_proj(norms.swiglu(m.gate_proj(x), m.up_proj(x)))


def rotary_tables(text_model, L: int, device, dtype):
    """cos/sin [L, rotary_dim] for positions 0..L-1 in `dtype` (text-only rotary: the three mRoPE
    position sections coincide, so the table is the plain one; [hf]:84-166, blockdiff.py:91-93)."""
    inv = text_model.rotary_emb.inv_freq.to(device=device, dtype=torch.float32)
    fr = torch.arange(L, device=device, dtype=torch.float32)[:, None] * inv[None, :]
    emb = torch.cat([fr, fr], -1)
    scale = float(getattr(text_model.rotary_emb, "attention_scaling", 1.0))
    return (emb.cos() * scale).to(dtype), (emb.sin() * scale).to(dtype)


def _gdn_fork_arm(m, n: torch.Tensor, block: int, fault: BreakMode) -> torch.Tensor:
    """LINEAR arm of the layer (blockdiff.py:153-177): both streams through one fused fork op.
    n: [2B, L, D], rows 0..B-1 the noised stream, B..2B-1 the clean one; returns the same layout."""
    B2, L, _ = n.shape
    B = B2 // 2
    if fault.concat_causal_gdn:
        out, _, _ = gdn.gdn_mixer_forward(m, torch.cat([n[:B], n[B:]], 1), chunk_size=block, need_states=False)
        return torch.cat([out[:, :L], out[:, L:]], 0)
    raw = m.in_proj_qkv(n)
    z = m.in_proj_z(n)
    beta, g = gdn._beta_g(m, m.in_proj_b(n), m.in_proj_a(n))
    Hv, Dv = m.num_v_heads, m.head_v_dim
    core = torch.empty(2 * B, L, Hv, Dv, dtype=raw.dtype, device=raw.device)
    gdn.gdn_state_fork(raw[B:], raw[:B], m.conv1d.weight.squeeze(1), beta[B:], beta[:B], g[B:], g[:B],
                       num_k_heads=m.num_k_heads, num_v_heads=Hv, head_k_dim=m.head_k_dim, head_v_dim=Dv,
                       block=block, conv_bias=m.conv1d.bias, need_states=False, need_tails=False,
                       fault="no-conv-prefix" if fault.drop_conv_prefix else None,
                       out={"ot": core[:B], "o0": core[B:]})
    o = norms.gated_rmsnorm(core.reshape(-1, Dv), z.reshape(-1, Dv), m.norm.weight, _eps(m.norm)).reshape(2 * B, L, -1)
    return m.out_proj(o)


def _attention_arm(att, n: torch.Tensor, cos, sin, block: int, fault: BreakMode) -> torch.Tensor:
    """FULL arm (blockdiff.py:178-182 through [hf]:656-701) on cat([x_t, x_0]). n: [2B, L, D] as in
    the GDN arm; cos/sin: rotary tables [L, rotary_dim] for positions 0..L-1, shared by both halves."""
    B2, L, D = n.shape
    B = B2 // 2
    # [B, 2L, D] = cat([x_t, x_0], 1) per sequence: a view at B = 1
    x = n.view(2, B, L, D).transpose(0, 1).reshape(B, 2 * L, D)
    S = 2 * L
    hd = att.head_dim
    q, gate = torch.chunk(att.q_proj(x).view(B, S, -1, 2 * hd), 2, dim=-1)
    v = att.v_proj(x).view(B, S, -1, hd)
    if attention.gated_supported(q, hd, cos.shape[-1]) and _aligned16(q, v, att.q_norm.weight, cos, sin):
        # one launch: q norm + RoPE as the kernel loads q, the sigmoid gate as it stores the output
        k = norms.k_norm_rope(att.k_proj(x).view(B, S, -1, hd), att.k_norm, cos, sin, L)
        o = attention.bd_attention_gated(q, k, v, gate, block=block, q_norm_weight=att.q_norm.weight,
                                         q_norm_eps=_eps(att.q_norm), cos=cos, sin=sin, scale=float(att.scaling),
                                         leak_xt_prefix=fault.leak_xt_prefix)
        out = att.o_proj(o.reshape(B, S, -1))
    else:
        q, k = norms.qk_norm_rope(q, att.k_proj(x).view(B, S, -1, hd), att.q_norm, att.k_norm, cos, sin, L)
        o = attention.bd_attention(q, k, v, block=block, scale=float(att.scaling), leak_xt_prefix=fault.leak_xt_prefix)
        out = att.o_proj(o.reshape(B, S, -1) * torch.sigmoid(gate.reshape(B, S, -1)))
    return out.view(B, 2, L, -1).transpose(0, 1).reshape(2 * B, L, -1)


def _aligned16(*ts) -> bool:
    return all(t.data_ptr() % 16 == 0 for t in ts)


def layer_step_stacked(layer, kind: str, h: torch.Tensor, *, block: int, cos, sin, fault: BreakMode | None = None,
                       m: torch.Tensor | None = None):
    """One decoder layer for both streams held as one tensor h [2B, L, D] (rows 0..B-1 the noised
    stream, B..2B-1 the clean one), so that every norm, projection and MLP GEMM runs once over both
    streams. m: the previous layer's MLP output not yet added to h (None: nothing pending); its
    residual add is fused into this layer's input norm. Returns (h, m) with this layer's MLP
    output pending."""
    fault = fault or BreakMode()
    if m is None:
        n = rmsnorm(h, layer.input_layernorm)
    else:
        n, h = rmsnorm(m, layer.input_layernorm, residual=h)
    if kind == LINEAR:
        o = _gdn_fork_arm(layer.linear_attn, n, block, fault)
    elif kind == FULL:
        o = _attention_arm(layer.self_attn, n, cos, sin, block, fault)
    else:
        raise ValueError(f"unknown layer type {kind}")
    n, h = rmsnorm(o, layer.post_attention_layernorm, residual=h)
    return h, mlp(layer.mlp, n)


def layer_step(layer, kind: str, h0: torch.Tensor, ht: torch.Tensor, *, block: int, cos, sin,
               fault: BreakMode | None = None, m0: torch.Tensor | None = None, mt: torch.Tensor | None = None):
    """One decoder layer for both streams (blockdiff.py:147-188) on separate stream tensors: stacks
    them and runs `layer_step_stacked`. cos/sin: rotary tables [L, rotary_dim] (positions shared by
    the halves of cat([x_t, x_0])).

    m0/mt: the previous layer's MLP outputs not yet added to h0/ht (None: nothing pending); their
    residual add is fused into this layer's input norm. Returns (h0, ht, m0, mt): the streams
    after the mixer residual and this layer's MLP outputs, again pending."""
    B = h0.shape[0]
    m = None if m0 is None else torch.cat([mt, m0], 0)
    h, m = layer_step_stacked(layer, kind, torch.cat([ht, h0], 0), block=block, cos=cos, sin=sin, fault=fault, m=m)
    return h[B:], h[:B], m[B:], m[:B]


def _forbid_grad(*modules):
    if torch.is_grad_enabled() and any(p.requires_grad for mod in modules for p in mod.parameters()):
        raise RuntimeError(
            "block_diffusion_forward runs forward-only HIP kernels (no backward is built); call it under "
            "torch.no_grad() / torch.inference_mode() or freeze the parameters")


def block_diffusion_forward(text_model, lm_head, x0_ids: torch.Tensor, xt_ids: torch.Tensor, block: int, *,
                            fault: BreakMode | None = None, layers: int | None = None, output: str = "logits",
                            checkpointing: bool = False):
    """Two-stream forward (blockdiff.py:96-203). Returns (logits_t [B, L, V], logits_0 [B, L, V]) or,
    with output="hidden", the final-normed hidden states [B, L, D] of both streams.

    x0_ids / xt_ids: [B, L] with L a multiple of `block` (ValueError otherwise). `layers` truncates
    the stack. `checkpointing` is accepted for signature compatibility; there is nothing to
    checkpoint in a forward-only pass."""
    fault = fault or BreakMode()
    if output not in ("logits", "hidden"):
        raise ValueError(f"output must be 'logits' or 'hidden', got {output!r}")
    cfg = text_model.config
    if x0_ids.shape != xt_ids.shape or x0_ids.ndim != 2:
        raise ValueError("x0_ids and xt_ids must both be [B, L]")
    B, L = x0_ids.shape
    if L % block:
        raise ValueError(f"L={L} is not a multiple of block={block}")
    _forbid_grad(text_model, lm_head)
    del checkpointing

    # both streams as one tensor [2B, L, D]: rows 0..B-1 the noised stream, B..2B-1 the clean one
    h = text_model.embed_tokens(torch.cat([xt_ids, x0_ids], 0))
    cos, sin = rotary_tables(text_model, L, h.device, h.dtype)
    n = cfg.num_hidden_layers if layers is None else layers
    m = None
    for i in range(n):
        h, m = layer_step_stacked(text_model.layers[i], cfg.layer_types[i], h, block=block, cos=cos, sin=sin,
                                  fault=fault, m=m)
    h = rmsnorm(h, text_model.norm) if m is None else rmsnorm(m, text_model.norm, residual=h)[0]
    if output == "hidden":
        return h[:B], h[B:]
    logits = lm_head(h)
    return logits[:B], logits[B:]


class LayerStep(nn.Module):
    """One decoder layer for both streams as a module (fsdp_train.py:83-130).

    forward(h0, ht, pos, mask, block): pos = (cos, sin) rotary tables for cat([x_t, x_0]), shaped
    [..., 2L, rotary_dim] (leading dims broadcast; HF's rotary output is accepted). The attention
    kernel derives visibility from `block`, so `mask` must be None: a dense mask is refused rather
    than ignored (select the leak fault with `fault=BreakMode("mask-leak")`)."""

    def __init__(self, layer, kind: str, fault: BreakMode | None = None):
        super().__init__()
        self.layer = layer
        self.kind = kind
        self.fault = fault or BreakMode()

    def forward(self, h0, ht, pos, mask, block: int):
        if mask is not None:
            raise ValueError("LayerStep takes no dense attention mask: visibility is derived from block")
        _forbid_grad(self.layer)
        cos, sin = pos
        L = h0.shape[1]
        cos1 = cos.reshape(-1, 2 * L, cos.shape[-1])[0, :L].to(h0.dtype)  # both halves share positions
        sin1 = sin.reshape(-1, 2 * L, sin.shape[-1])[0, :L].to(h0.dtype)
        h0, ht, m0, mt = layer_step(self.layer, self.kind, h0, ht, block=block, cos=cos1, sin=sin1, fault=self.fault)
        return h0 + m0, ht + mt


@torch.no_grad()
def reference_block_logits(text_model, lm_head, x0_ids: torch.Tensor, xt_ids: torch.Tensor, block: int, *,
                           layers: int | None = None) -> torch.Tensor:
    """Oracle (blockdiff.py:206-228): per block k, the UNMODIFIED transformers model on
    cat([x_0 blocks < k, x_t block k]) under the block-causal 4D mask; the last block's logits,
    concatenated over k -> [B, L, V]. Runs transformers' own modules (its torch GDN kernel and eager
    attention) wherever the model lives; none of this module's kernels are involved."""
    cfg = text_model.config
    L = x0_ids.shape[1]
    saved = cfg.num_hidden_layers
    if layers is not None:
        cfg.num_hidden_layers = layers
    try:
        outs = []
        for k in range(L // block):
            seq = torch.cat([x0_ids[:, : k * block], xt_ids[:, k * block: (k + 1) * block]], 1)
            mask = block_causal_mask(seq.shape[1], block, text_model.embed_tokens.weight.dtype, seq.device)
            hs = text_model(input_ids=seq, attention_mask={FULL: mask, LINEAR: None}, use_cache=False).last_hidden_state
            outs.append(lm_head(hs[:, -block:]))
        return torch.cat(outs, 1)
    finally:
        cfg.num_hidden_layers = saved


@torch.no_grad()
def reference_clean_logits(text_model, lm_head, x0_ids: torch.Tensor, block: int, *, layers: int | None = None):
    """Oracle for the clean stream (blockdiff.py:231-243): the unmodified model on x_0 under the
    block-causal mask."""
    cfg = text_model.config
    saved = cfg.num_hidden_layers
    if layers is not None:
        cfg.num_hidden_layers = layers
    try:
        mask = block_causal_mask(x0_ids.shape[1], block, text_model.embed_tokens.weight.dtype, x0_ids.device)
        hs = text_model(input_ids=x0_ids, attention_mask={FULL: mask, LINEAR: None}, use_cache=False).last_hidden_state
        return lm_head(hs)
    finally:
        cfg.num_hidden_layers = saved


def tiny_text_model(seed: int = 0, layers: int = 8, vocab: int = 256):
    """A random transformers Qwen3.5 text model of the reference's unit-test size (blockdiff.py:246-278):
    hidden 64, 6 GDN + 2 attention layers, attention heads 4/2 of dim 16, GDN heads 2 key / 4 value
    of dim 16, conv width 4, partial RoPE 0.25 with base 1e4; CPU fp32, untied lm_head."""
    from transformers.models.qwen3_5.configuration_qwen3_5 import Qwen3_5TextConfig
    from transformers.models.qwen3_5.modeling_qwen3_5 import Qwen3_5TextModel

    torch.manual_seed(seed)
    cfg = Qwen3_5TextConfig(
        vocab_size=vocab, hidden_size=64, intermediate_size=128, num_hidden_layers=layers,
        num_attention_heads=4, num_key_value_heads=2, head_dim=16, linear_num_key_heads=2,
        linear_num_value_heads=4, linear_key_head_dim=16, linear_value_head_dim=16, linear_conv_kernel_dim=4,
        max_position_embeddings=4096,
        rope_parameters={"rope_theta": 10000.0, "mrope_section": [2, 1, 1], "partial_rotary_factor": 0.25},
        attn_implementation="eager")
    model = Qwen3_5TextModel(cfg).eval()
    lm_head = nn.Linear(cfg.hidden_size, vocab, bias=False)
    return model, lm_head
