"""Complementary-mask block-diffusion attention on the MI355X HIP kernel.

Replaces the FULL (attention) arm of the reference's `_layer_step` (src/dllm_qwen38/blockdiff.py:
178-182): the reference builds an additive [1,1,2L,2L] mask (blockdiff.py:50-66) and runs HF's eager
attention (transformers modeling_qwen3_5.py:604-626) over cat([x_t, x_0]). Here the visibility rule is
evaluated from (L, block) inside the kernel; fully hidden tiles are never computed and no mask tensor
exists. `complementary_mask` / `block_causal_mask` are still provided (dense, for the oracle and the
mask-leak fault), as in the reference.
"""

from __future__ import annotations

import torch

from . import _lib


def _neg(dtype: torch.dtype) -> float:
    return torch.finfo(dtype).min


def block_causal_mask(seq_len: int, block: int, dtype: torch.dtype, device) -> torch.Tensor:
    """[1, 1, S, S] additive mask: token i sees j iff block(j) <= block(i) (blockdiff.py:43-47)."""
    idx = torch.arange(seq_len, device=device) // block
    allowed = idx[None, :] <= idx[:, None]
    return torch.zeros(seq_len, seq_len, dtype=dtype, device=device).masked_fill(~allowed, _neg(dtype))[None, None]


def complementary_mask(seq_len: int, block: int, dtype: torch.dtype, device, *, leak_xt_prefix: bool = False):
    """[1, 1, 2L, 2L] additive mask over cat([x_t, x_0]) (blockdiff.py:50-66); leak_xt_prefix=True is the
    deliberately wrong mask (x_t block k also sees x_t blocks < k)."""
    L = seq_len
    idx = torch.arange(L, device=device) // block
    bi, bj = idx[:, None], idx[None, :]
    tt = (bj <= bi) if leak_xt_prefix else (bj == bi)
    top = torch.cat([tt, bj < bi], 1)
    bottom = torch.cat([torch.zeros(L, L, dtype=torch.bool, device=device), bj <= bi], 1)
    allowed = torch.cat([top, bottom], 0)
    return torch.zeros(2 * L, 2 * L, dtype=dtype, device=device).masked_fill(~allowed, _neg(dtype))[None, None]


def bd_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *, block: int, scale: float | None = None,
                 leak_xt_prefix: bool = False, out: torch.Tensor | None = None) -> torch.Tensor:
    """Attention over cat([x_t, x_0]) under the complementary mask.

    q [B, 2L, Hq, d], k/v [B, 2L, Hkv, d] (token-major, any batch/token/head strides, last dim
    contiguous; rotary already applied) -> [B, 2L, Hq, d]. scale defaults to d^-1/2 ([hf]:638)."""
    dev = _lib.require_device(q, k, v)
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        raise ValueError("q, k, v must be [B, 2L, H, d]")
    B, S, Hq, d = q.shape
    if S % 2:
        raise ValueError(f"sequence {S} is not cat([x_t, x_0]) of two equal halves")
    L = S // 2
    if L % block:
        raise ValueError(f"L={L} is not a multiple of block={block}")
    if k.shape[:2] != (B, S) or v.shape != k.shape or k.shape[-1] != d:
        raise ValueError("k and v must be [B, 2L, Hkv, d] matching q")
    Hkv = k.shape[2]
    if Hq % Hkv:
        raise ValueError(f"query heads {Hq} not a multiple of key/value heads {Hkv}")
    if k.dtype != q.dtype or v.dtype != q.dtype:
        raise TypeError("q, k, v dtypes differ")
    q, k, v = (t if t.stride(-1) == 1 else t.contiguous() for t in (q, k, v))
    if out is None:
        out = torch.empty(B, S, Hq, d, dtype=q.dtype, device=dev)
    elif tuple(out.shape) != (B, S, Hq, d) or not out.is_contiguous() or out.dtype != q.dtype:
        raise ValueError("out must be a contiguous [B, 2L, Hq, d] tensor of q's dtype")
    if B == 0 or L == 0:  # no queries: an empty output, no launch
        return out
    sc = d ** -0.5 if scale is None else float(scale)
    _lib.check(_lib.lib().dllm_bd_attention_fwd(
        q.data_ptr(), _lib.strides3(q), k.data_ptr(), _lib.strides3(k), v.data_ptr(), _lib.strides3(v),
        out.data_ptr(), B, L, Hq, Hkv, d, block, sc, _lib.dtype_code(q.dtype), 1 if leak_xt_prefix else 0,
        _lib.stream_handle(dev)), "dllm_bd_attention_fwd")
    return out


def gated_supported(q: torch.Tensor, d: int, rotary_dim: int) -> bool:
    """Whether bd_attention_gated takes this shape in one launch (bf16, d in {64, 128, 256},
    rotary_dim a multiple of 64)."""
    return bool(_lib.lib().dllm_bd_attention_gated_supported(d, rotary_dim, _lib.dtype_code(q.dtype)))


def bd_attention_gated(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, gate: torch.Tensor | None, *, block: int,
                       q_norm_weight: torch.Tensor | None = None, q_norm_eps: float = 1e-6,
                       cos: torch.Tensor | None = None, sin: torch.Tensor | None = None, scale: float | None = None,
                       leak_xt_prefix: bool = False) -> torch.Tensor:
    """The gated attention layer's core in one launch ([hf]:672-698 around bd_attention): with
    q_norm_weight, q [B, 2L, Hq, d] is the raw q_proj query half, RMSNorm(1 + w)-normalised and its
    first rotary_dim dims rotated (cos/sin [L, rotary_dim], the activation dtype, row = position
    within the half) as the kernel loads it; k must already be normed and rotated
    (norms.k_norm_rope). With gate [B, 2L, Hq, d], the output is multiplied by sigmoid(gate), each
    rounded to the dtype as the separate elementwise ops round. Returns [B, 2L, Hq, d] contiguous.
    Shapes gated_supported() refuses raise; callers run the separate launches for them."""
    dev = _lib.require_device(q, k, v, gate, q_norm_weight, cos, sin)
    B, S, Hq, d = q.shape
    if S % 2:
        raise ValueError(f"sequence {S} is not cat([x_t, x_0]) of two equal halves")
    L = S // 2
    if L % block:
        raise ValueError(f"L={L} is not a multiple of block={block}")
    if k.shape[:2] != (B, S) or v.shape != k.shape or k.shape[-1] != d:
        raise ValueError("k and v must be [B, 2L, Hkv, d] matching q")
    Hkv = k.shape[2]
    if gate is not None and (tuple(gate.shape) != (B, S, Hq, d) or gate.stride(-1) != 1 or gate.dtype != q.dtype):
        raise ValueError("gate must be [B, 2L, Hq, d] of q's dtype with its last dim contiguous")
    rd = 0
    if q_norm_weight is not None:
        if cos is None or sin is None or cos.shape != sin.shape or cos.shape[0] < L:
            raise ValueError("the q prologue needs cos/sin tables [L, rotary_dim]")
        rd = int(cos.shape[-1])
        cos, sin = cos.to(q.dtype).contiguous(), sin.to(q.dtype).contiguous()
        q_norm_weight = q_norm_weight.contiguous()
    q, k, v = (t if t.stride(-1) == 1 else t.contiguous() for t in (q, k, v))
    out = torch.empty(B, S, Hq, d, dtype=q.dtype, device=dev)
    sc = d ** -0.5 if scale is None else float(scale)
    _lib.check(_lib.lib().dllm_bd_attention_gated_fwd(
        q.data_ptr(), _lib.strides3(q), k.data_ptr(), _lib.strides3(k), v.data_ptr(), _lib.strides3(v),
        _lib.ptr(gate), None if gate is None else _lib.strides3(gate), _lib.ptr(q_norm_weight),
        _lib.dtype_code(q_norm_weight.dtype) if q_norm_weight is not None else 0, float(q_norm_eps),
        _lib.ptr(cos), _lib.ptr(sin), rd, out.data_ptr(), B, L, Hq, Hkv, d, block, sc, _lib.dtype_code(q.dtype),
        1 if leak_xt_prefix else 0, _lib.stream_handle(dev)), "dllm_bd_attention_gated_fwd")
    return out


def _key_splits(q: torch.Tensor, M: int, N: int, d: int) -> int:
    """Key splits for a decoding step (bf16, the direct-load kernel's head sizes, few query rows):
    about eight 32-key tiles per workgroup; 1 otherwise."""
    if q.dtype != torch.bfloat16 or d not in (64, 128, 256) or M > 64 or N < 512:
        return 1
    return max(1, min(32, -(-N // 256)))


def block_causal_gate_fused(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> bool:
    """Whether block_causal_attention takes a gate for these q [B, M, Hq, d] and k/v [B, N, Hkv, d]:
    the direct-load kernel's inputs (bf16, d in {64, 128, 256}, 16-byte aligned rows)."""
    d = q.shape[-1]
    return (q.dtype == torch.bfloat16 and d in (64, 128, 256)
            and all(t.dtype == q.dtype and t.stride(-1) == 1 and t.data_ptr() % 16 == 0
                    and all(t.stride(i) % 8 == 0 for i in range(3)) for t in (q, k, v)))


def block_causal_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *, block: int, q_offset: int = 0,
                           scale: float | None = None, out: torch.Tensor | None = None,
                           key_splits: int | None = None, gate: torch.Tensor | None = None) -> torch.Tensor:
    """Block-causal attention of a query segment against a key/value cache (the clean-prefix cache
    of the cached decoder; the reference re-runs the whole forward instead, decode.py:63-66).

    q [B, M, Hq, d] at absolute positions q_offset..q_offset+M-1; k/v [B, N, Hkv, d] at positions
    0..N-1 (token-major, any batch/token/head strides, last dim contiguous; rotary already applied).
    Query i sees key j iff j // block <= (q_offset + i) // block (blockdiff.py:43-47 with the query
    rows offset). Returns [B, M, Hq, d]. key_splits (default: chosen for a decoding step's few query
    rows) spreads the key tiles over several workgroups whose partial results are merged. gate
    [B, M, Hq, d] (any batch/token/head strides, last dim contiguous; bf16, the direct-load kernel's
    head sizes): the output is attention * sigmoid(gate) ([hf]:698), applied at the output store."""
    dev = _lib.require_device(q, k, v)
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        raise ValueError("q must be [B, M, Hq, d] and k, v [B, N, Hkv, d]")
    B, M, Hq, d = q.shape
    N, Hkv = k.shape[1], k.shape[2]
    if k.shape[0] != B or v.shape != k.shape or k.shape[-1] != d:
        raise ValueError("k and v must be [B, N, Hkv, d] matching q")
    if Hq % Hkv:
        raise ValueError(f"query heads {Hq} not a multiple of key/value heads {Hkv}")
    if q_offset < 0 or block <= 0:
        raise ValueError(f"q_offset {q_offset} and block {block} must be >= 0 and > 0")
    if k.dtype != q.dtype or v.dtype != q.dtype:
        raise TypeError("q, k, v dtypes differ")
    q, k, v = (t if t.stride(-1) == 1 else t.contiguous() for t in (q, k, v))
    if out is None:
        out = torch.empty(B, M, Hq, d, dtype=q.dtype, device=dev)
    elif tuple(out.shape) != (B, M, Hq, d) or not out.is_contiguous() or out.dtype != q.dtype:
        raise ValueError("out must be a contiguous [B, M, Hq, d] tensor of q's dtype")
    if B == 0 or M == 0:  # no queries: an empty output, no launch
        return out
    sc = d ** -0.5 if scale is None else float(scale)
    ks = _key_splits(q, M, N, d) if key_splits is None else int(key_splits)
    work = torch.empty(ks * B * M * Hq * (d + 2), dtype=torch.float32, device=dev) if ks > 1 else None
    if gate is not None:
        if tuple(gate.shape) != (B, M, Hq, d) or gate.dtype != q.dtype or gate.stride(-1) != 1:
            raise ValueError("gate must be [B, M, Hq, d] of q's dtype with a contiguous last dim")
        _lib.check(_lib.lib().dllm_block_causal_attention_gated_fwd(
            q.data_ptr(), _lib.strides3(q), k.data_ptr(), _lib.strides3(k), v.data_ptr(), _lib.strides3(v),
            gate.data_ptr(), _lib.strides3(gate), out.data_ptr(), B, M, N, q_offset, Hq, Hkv, d, block, sc,
            _lib.dtype_code(q.dtype), _lib.ptr(work), ks, _lib.stream_handle(dev)), "dllm_block_causal_attention_gated_fwd")
        return out
    _lib.check(_lib.lib().dllm_block_causal_attention_fwd(
        q.data_ptr(), _lib.strides3(q), k.data_ptr(), _lib.strides3(k), v.data_ptr(), _lib.strides3(v),
        out.data_ptr(), B, M, N, q_offset, Hq, Hkv, d, block, sc, _lib.dtype_code(q.dtype), _lib.ptr(work), ks,
        _lib.stream_handle(dev)), "dllm_block_causal_attention_fwd")
    return out


def attention_flops(B: int, L: int, Hq: int, d: int, block: int, leak: bool = False) -> int:
    """Algorithmic flops over the visible (query, key) pairs only: 4*d per pair and query head."""
    nb = L // block
    sq = block * block
    tt = sq * (nb * (nb + 1) // 2) if leak else sq * nb
    pairs = tt + sq * (nb * (nb - 1) // 2) + sq * (nb * (nb + 1) // 2)
    return B * Hq * pairs * 4 * d
