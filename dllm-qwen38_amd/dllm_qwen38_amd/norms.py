"""Prologue / epilogue ops around the two mixers, on the HIP kernels of libdllm_hip.so.

Each replaces a chain of torch elementwise kernels of the transformers Qwen3.5 modules with one
row-wise kernel, rounding at the module's own cast points:
  rmsnorm        Qwen3_5RMSNorm, weight applied as (1 + w), optionally fused with the residual add
                 before it ([hf]:720-737; the residual adds of the decoder layer, [hf]:785,791)
  gated_rmsnorm  Qwen3_5RMSNormGated: rmsnorm(x) * w * silu(z) ([hf]:168-184)
  swiglu         silu(gate) * up of Qwen3_5MLP ([hf]:704-717)
  qk_norm_rope   q/k RMSNorm then partial RoPE with positions shared by both halves of
                 cat([x_t, x_0]) ([hf]:554-589, 667-680; reference blockdiff.py:91-93, 143-144)
Device tensors only; a CPU tensor or a missing library raises.
"""

from __future__ import annotations

import torch

from . import _lib


def _eps(norm) -> float:
    return float(getattr(norm, "eps", getattr(norm, "variance_epsilon", 1e-6)))


def _c(t: torch.Tensor) -> torch.Tensor:
    return t if t.is_contiguous() else t.contiguous()


def rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float, *, residual: torch.Tensor | None = None,
            unit_offset: bool = True):
    """y = rmsnorm(s) * (1 + w) over the last dim, s = x (+ residual, rounded to x's dtype).
    Returns y, or (y, s) when a residual is given."""
    dev = _lib.require_device(x, weight, residual)
    x = _c(x)
    dim = x.shape[-1]
    rows = x.numel() // dim
    w = _c(weight)
    r = None if residual is None else _c(residual)
    if r is not None and (r.shape != x.shape or r.dtype != x.dtype):
        raise ValueError("residual must match x in shape and dtype")
    y = torch.empty_like(x)
    s = torch.empty_like(x) if r is not None else None
    _lib.check(_lib.lib().dllm_rmsnorm_fwd(
        x.data_ptr(), _lib.ptr(r), _lib.ptr(s), w.data_ptr(), y.data_ptr(), rows, dim, float(eps),
        _lib.dtype_code(x.dtype), _lib.dtype_code(w.dtype), int(unit_offset), _lib.stream_handle(dev)),
        "dllm_rmsnorm_fwd")
    return y if r is None else (y, s)


def gated_rmsnorm(x: torch.Tensor, z: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """rmsnorm(x) * w * silu(z) over the last dim."""
    dev = _lib.require_device(x, z, weight)
    x, z, w = _c(x), _c(z), _c(weight)
    if z.shape != x.shape:
        raise ValueError("gate must match x")
    dim = x.shape[-1]
    y = torch.empty_like(x)
    _lib.check(_lib.lib().dllm_gated_rmsnorm_fwd(
        x.data_ptr(), z.data_ptr(), w.data_ptr(), y.data_ptr(), x.numel() // dim, dim, float(eps),
        _lib.dtype_code(x.dtype), _lib.dtype_code(w.dtype), _lib.stream_handle(dev)), "dllm_gated_rmsnorm_fwd")
    return y


def swiglu(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """round(round(silu(gate)) * up) ([hf]:704-717). gate and up may be the two column halves of one
    fused gate | up output (rows ld apart, last dim contiguous): read in place."""
    dev = _lib.require_device(gate, up)
    if (gate.shape == up.shape and gate.dtype == up.dtype and gate.dim() >= 2 and gate.stride(-1) == 1
            and up.stride(-1) == 1 and gate.stride(-2) == up.stride(-2) and gate.shape[-1] % 8 == 0
            and gate.stride(-2) % 8 == 0 and not gate.is_contiguous()):
        cols, ld = gate.shape[-1], gate.stride(-2)
        rows = gate.numel() // cols
        lead_ok = all(gate.stride(i) == gate.stride(i + 1) * gate.shape[i + 1] for i in range(gate.dim() - 2))
        if lead_ok and gate.data_ptr() % 16 == 0 and up.data_ptr() % 16 == 0:
            out = torch.empty(gate.shape, dtype=gate.dtype, device=dev)
            _lib.check(_lib.lib().dllm_swiglu_rows_fwd(gate.data_ptr(), up.data_ptr(), ld, out.data_ptr(), rows, cols,
                                                       _lib.dtype_code(gate.dtype), _lib.stream_handle(dev)),
                       "dllm_swiglu_rows_fwd")
            return out
    g, u = _c(gate), _c(up)
    if g.shape != u.shape or g.dtype != u.dtype:
        raise ValueError("gate and up must match")
    out = torch.empty_like(g)
    _lib.check(_lib.lib().dllm_swiglu_fwd(g.data_ptr(), u.data_ptr(), out.data_ptr(), g.numel(),
                                          _lib.dtype_code(g.dtype), _lib.stream_handle(dev)), "dllm_swiglu_fwd")
    return out


def qk_norm_rope(q: torch.Tensor, k: torch.Tensor, q_norm, k_norm, cos: torch.Tensor, sin: torch.Tensor, L: int, *,
                 k_out: torch.Tensor | None = None):
    """q [B, S, Hq, hd], k [B, S, Hkv, hd] (any batch/token/head strides, last dim contiguous) ->
    contiguous normed-and-rotated copies. cos/sin [L, rotary_dim] in the activation dtype; token t
    uses row t mod L. k_out: a contiguous [B, S, Hkv, hd] tensor to write the k result into (a
    key cache's rows)."""
    dev = _lib.require_device(q, k, cos, sin)
    B, S, Hq, hd = q.shape
    Hkv = k.shape[2]
    if q.stride(-1) != 1 or k.stride(-1) != 1:
        raise ValueError("q/k last dim must be contiguous")
    rd = cos.shape[-1]
    cs, sn = _c(cos.to(q.dtype)), _c(sin.to(q.dtype))
    wq, wk = _c(q_norm.weight), _c(k_norm.weight)
    qo = torch.empty(B, S, Hq, hd, dtype=q.dtype, device=dev)
    if k_out is None:
        ko = torch.empty(B, S, Hkv, hd, dtype=k.dtype, device=dev)
    elif tuple(k_out.shape) != (B, S, Hkv, hd) or k_out.dtype != k.dtype or not k_out.is_contiguous():
        raise ValueError(f"k_out must be a contiguous {(B, S, Hkv, hd)} tensor of k's dtype")
    else:
        ko = k_out
    _lib.check(_lib.lib().dllm_qk_norm_rope_fwd(
        q.data_ptr(), _lib.strides3(q), k.data_ptr(), _lib.strides3(k), wq.data_ptr(), wk.data_ptr(),
        cs.data_ptr(), sn.data_ptr(), qo.data_ptr(), ko.data_ptr(), B, S, L, Hq, Hkv, hd, rd, _eps(q_norm),
        _lib.dtype_code(q.dtype), _lib.dtype_code(wq.dtype), _lib.stream_handle(dev)), "dllm_qk_norm_rope_fwd")
    return qo, ko


def k_norm_rope(k: torch.Tensor, k_norm, cos: torch.Tensor, sin: torch.Tensor, L: int) -> torch.Tensor:
    """The k half of qk_norm_rope alone (its q prologue runs inside the attention kernel):
    k [B, S, Hkv, hd] -> contiguous normed-and-rotated copy."""
    dev = _lib.require_device(k, cos, sin)
    B, S, Hkv, hd = k.shape
    if k.stride(-1) != 1:
        raise ValueError("k last dim must be contiguous")
    rd = cos.shape[-1]
    cs, sn = _c(cos.to(k.dtype)), _c(sin.to(k.dtype))
    wk = _c(k_norm.weight)
    ko = torch.empty(B, S, Hkv, hd, dtype=k.dtype, device=dev)
    _lib.check(_lib.lib().dllm_qk_norm_rope_fwd(
        None, None, k.data_ptr(), _lib.strides3(k), None, wk.data_ptr(), cs.data_ptr(), sn.data_ptr(), None,
        ko.data_ptr(), B, S, L, 0, Hkv, hd, rd, _eps(k_norm), _lib.dtype_code(k.dtype), _lib.dtype_code(wk.dtype),
        _lib.stream_handle(dev)), "dllm_qk_norm_rope_fwd")
    return ko


def gdn_gates(b: torch.Tensor, a: torch.Tensor, a_log: torch.Tensor, dt_bias: torch.Tensor):
    """Gated DeltaNet gates (reference gdn.py:225-226) in one kernel: beta = sigmoid(b) rounded to
    b's dtype and returned in fp32 (the core takes fp32 beta), g = -exp(A_log) * softplus(a + dt_bias)
    in fp32. b, a [..., H] -> (beta, g) [..., H] fp32."""
    dev = _lib.require_device(b, a, a_log, dt_bias)
    H = b.shape[-1]
    if a.shape != b.shape or a.dtype != b.dtype:
        raise ValueError("b and a must share shape and dtype")
    if a_log.numel() != H or dt_bias.numel() != H:
        raise ValueError(f"A_log and dt_bias must have {H} entries")
    p_dt = a_log.dtype
    al, db = _c(a_log.reshape(H)), _c(dt_bias.reshape(H).to(p_dt))
    bc, ac = _c(b), _c(a)
    beta = torch.empty(b.shape, dtype=torch.float32, device=dev)
    g = torch.empty(b.shape, dtype=torch.float32, device=dev)
    _lib.check(_lib.lib().dllm_gdn_gates_fwd(bc.data_ptr(), ac.data_ptr(), al.data_ptr(), db.data_ptr(), beta.data_ptr(),
                                             g.data_ptr(), b.numel() // H, H, _lib.dtype_code(b.dtype),
                                             _lib.dtype_code(p_dt), _lib.stream_handle(dev)), "dllm_gdn_gates_fwd")
    return beta, g
