"""CPU oracle for the complementary-mask block-diffusion attention — TEST INFRASTRUCTURE ONLY.

Restates:
  * `complementary_mask` (reference `src/dllm_qwen38/blockdiff.py:50-66`) and
    `block_causal_mask` (`blockdiff.py:43-47`): additive masks, finfo(dtype).min where blocked;
  * the allowed-pair count of the [2L,2L] mask in closed form;
  * the rotary tables with positions shared by both halves (reference `blockdiff.py:91-93,143-144`;
    transformers 5.15.0 `models/qwen3_5/modeling_qwen3_5.py:84-166`, default rope, partial factor)
    and `apply_rotary_pos_emb` (`modeling_qwen3_5.py:554-589`, rotate_half on the first rotary_dim);
  * the masked GQA softmax attention of `eager_attention_forward` (`modeling_qwen3_5.py:604-626`).

How each function is pinned (tests/test_oracle_attn.py):
  masks            brute-force enumeration of the three visibility rules (A.6) and the exact
                   allowed-pair counts of the closed form.
  bd_attention     float64 brute force: dense softmax over the materialised mask, repeat_kv'd
                   keys; RoPE checked against transformers' own apply_rotary_pos_emb and rotary
                   module on a tiny config.
  block_causal_attention
                   the x_0 half of the float64 brute force (the clean stream is block-causal), at
                   every query offset (a segment at offset q0 equals rows q0.. of the prefill).
"""

from __future__ import annotations

import numpy as np
import torch


def _neg(dtype):
    return torch.finfo(dtype).min


def block_causal_mask(seq_len: int, block: int, dtype=torch.float32, device="cpu") -> torch.Tensor:
    """[1,1,S,S] additive: i sees j iff j // block <= i // block."""
    blk = torch.arange(seq_len, device=device) // block
    ok = blk[None, :] <= blk[:, None]
    return torch.zeros(seq_len, seq_len, dtype=dtype, device=device).masked_fill(~ok, _neg(dtype))[None, None]


def complementary_allowed(L: int, block: int, *, leak_xt_prefix: bool = False) -> torch.Tensor:
    """[2L,2L] bool over cat([x_t, x_0]) (row = query, column = key):
    x_t->x_t same block (<= under the mask-leak fault); x_t->x_0 strictly earlier blocks;
    x_0->x_t never; x_0->x_0 block-causal."""
    blk = torch.arange(L) // block
    bi, bj = blk[:, None], blk[None, :]
    tt = (bj <= bi) if leak_xt_prefix else (bj == bi)
    tc = bj < bi
    ct = torch.zeros(L, L, dtype=torch.bool)
    cc = bj <= bi
    return torch.cat([torch.cat([tt, tc], 1), torch.cat([ct, cc], 1)], 0)


def complementary_mask(seq_len: int, block: int, dtype=torch.float32, device="cpu", *, leak_xt_prefix=False):
    ok = complementary_allowed(seq_len, block, leak_xt_prefix=leak_xt_prefix).to(device)
    n = 2 * seq_len
    return torch.zeros(n, n, dtype=dtype, device=device).masked_fill(~ok, _neg(dtype))[None, None]


def allowed_pairs(L: int, block: int, *, leak_xt_prefix: bool = False) -> int:
    """Closed form of the number of allowed (query, key) pairs of the [2L,2L] mask."""
    nb = L // block
    sq = block * block
    tt = sq * (nb * (nb + 1) // 2) if leak_xt_prefix else sq * nb
    tc = sq * (nb * (nb - 1) // 2)
    cc = sq * (nb * (nb + 1) // 2)
    return tt + tc + cc


def rope_tables(positions: torch.Tensor, rotary_dim: int, base: float):
    """cos, sin [S, rotary_dim] float32: inv_freq_i = base^(-2i/rotary_dim), emb = cat(freqs, freqs)."""
    inv = 1.0 / (base ** (torch.arange(0, rotary_dim, 2, dtype=torch.float32) / rotary_dim))
    freqs = positions.to(torch.float32)[:, None] * inv[None, :]
    emb = torch.cat([freqs, freqs], -1)
    return emb.cos(), emb.sin()


def apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """x [..., S, H, d] (token-major); rotate_half on the first rotary_dim channels, rest passed."""
    rd = cos.shape[-1]
    xr, xp = x[..., :rd], x[..., rd:]
    half = rd // 2
    rot = torch.cat([-xr[..., half:], xr[..., :half]], -1)
    c, s = cos[:, None, :], sin[:, None, :]
    return torch.cat([xr * c + rot * s, xp], -1)


def bd_attention(q, k, v, *, block: int, rotary_dim: int = 0, rope_base: float = 1e7,
                 scale: float | None = None, leak_xt_prefix: bool = False, q_chunk: int = 256):
    """Complementary-mask GQA attention in float32 on the CPU.

    q [B,2L,Hq,d], k/v [B,2L,Hkv,d] token-major, halves ordered cat([x_t, x_0]); RoPE positions are
    i mod L for both halves. Returns [B,2L,Hq,d] float32. Query rows are processed in chunks and
    only allowed keys are gathered, so the dense [2L,2L] scores are never built."""
    B, S, Hq, d = q.shape
    Hkv = k.shape[2]
    L = S // 2
    rep = Hq // Hkv
    scale = d ** -0.5 if scale is None else scale
    q, k, v = q.float(), k.float(), v.float()
    if rotary_dim:
        pos = torch.arange(S) % L
        cos, sin = rope_tables(pos, rotary_dim, rope_base)
        q, k = apply_rope(q, cos, sin), apply_rope(k, cos, sin)
    allowed = complementary_allowed(L, block, leak_xt_prefix=leak_xt_prefix)
    kx = k.repeat_interleave(rep, dim=2).permute(0, 2, 1, 3)  # [B,Hq,S,d]
    vx = v.repeat_interleave(rep, dim=2).permute(0, 2, 1, 3)
    qh = q.permute(0, 2, 1, 3)
    out = torch.empty(B, Hq, S, d)
    for s0 in range(0, S, q_chunk):
        s1 = min(S, s0 + q_chunk)
        sc = (qh[:, :, s0:s1] @ kx.transpose(-1, -2)) * scale
        sc = sc.masked_fill(~allowed[s0:s1], float("-inf"))
        out[:, :, s0:s1] = torch.softmax(sc, -1) @ vx
    return out.permute(0, 2, 1, 3).contiguous()


def block_causal_attention(q, k, v, *, block: int, q_offset: int = 0, scale: float | None = None):
    """Block-causal GQA attention of a query segment against a key cache, float32 on the CPU: the
    x_0 -> x_0 rule of the complementary mask (blockdiff.py:43-47, 61-62) with the queries at
    absolute positions q_offset.. and the keys at 0..N-1. q [B,M,Hq,d], k/v [B,N,Hkv,d], rotary
    already applied. Returns [B,M,Hq,d] float32. This is what one step of a decoder that keeps the
    clean prefix's K/V computes instead of re-running the forward (decode.py:63-66)."""
    B, M, Hq, d = q.shape
    N, Hkv = k.shape[1], k.shape[2]
    scale = d ** -0.5 if scale is None else scale
    qb = (torch.arange(M) + q_offset) // block
    kb = torch.arange(N) // block
    allowed = kb[None, :] <= qb[:, None]
    kx = k.float().repeat_interleave(Hq // Hkv, dim=2).permute(0, 2, 1, 3)
    vx = v.float().repeat_interleave(Hq // Hkv, dim=2).permute(0, 2, 1, 3)
    sc = (q.float().permute(0, 2, 1, 3) @ kx.transpose(-1, -2)) * scale
    sc = sc.masked_fill(~allowed, float("-inf"))
    return (torch.softmax(sc, -1) @ vx).permute(0, 2, 1, 3).contiguous()


def bd_attention_f64_bruteforce(q, k, v, *, block: int, rotary_dim: int = 0, rope_base: float = 1e7,
                                scale: float | None = None, leak_xt_prefix: bool = False):
    """numpy float64, dense [2L,2L] mask materialised, explicit per-(b, head) softmax loops."""
    B, S, Hq, d = q.shape
    Hkv = k.shape[2]
    L = S // 2
    scale = d ** -0.5 if scale is None else scale
    q64, k64, v64 = (np.asarray(x.to(torch.float64)) for x in (q, k, v))
    if rotary_dim:
        pos = np.arange(S) % L
        inv = 1.0 / (rope_base ** (np.arange(0, rotary_dim, 2, dtype=np.float64) / rotary_dim))
        fr = pos[:, None] * inv[None, :]
        cos = np.cos(np.concatenate([fr, fr], -1))[:, None, :]
        sin = np.sin(np.concatenate([fr, fr], -1))[:, None, :]

        def rope(x):
            xr = x[..., :rotary_dim]
            h = rotary_dim // 2
            rot = np.concatenate([-xr[..., h:], xr[..., :h]], -1)
            return np.concatenate([xr * cos + rot * sin, x[..., rotary_dim:]], -1)

        q64, k64 = rope(q64), rope(k64)
    ok = np.asarray(complementary_allowed(L, block, leak_xt_prefix=leak_xt_prefix))
    out = np.zeros((B, S, Hq, d))
    for b in range(B):
        for h in range(Hq):
            kh = h // (Hq // Hkv)
            sc = q64[b, :, h] @ k64[b, :, kh].T * scale
            sc = np.where(ok, sc, -np.inf)
            sc = sc - sc.max(-1, keepdims=True)
            p = np.exp(sc)
            p /= p.sum(-1, keepdims=True)
            out[b, :, h] = p @ v64[b, :, kh]
    return out


def bd_attention_flops(B: int, L: int, Hq: int, d: int, block: int) -> int:
    """4*d flops per allowed (query, key) pair per query head (QK^T and PV)."""
    return B * Hq * allowed_pairs(L, block) * 4 * d
