"""CPU oracle for the state-fork Gated DeltaNet layer — TEST INFRASTRUCTURE ONLY.

Restates, on the CPU, the reference's algorithm for:
  * `chunk_gated_delta_rule_with_states`  (reference `src/dllm_qwen38/gdn.py:48-123`), fp32,
    in the reference's op order and cast points;
  * the float64 token recurrence it is mathematically equal to (the HF recurrent kernel,
    transformers 5.15.0 `models/qwen3_5/modeling_qwen3_5.py:330-381`);
  * `l2norm` (transformers `modeling_qwen3_5.py:242-245`);
  * the causal depthwise conv + SiLU with conv-prefix carry-in (transformers
    `modeling_qwen3_5.py:219-239`, driven as in reference `gdn.py:217-219`);
  * the integer fork layout (reference `blockdiff.py:161-173`);
  * the whole state-fork GDN layer op: conv of both streams, clean pass with per-block states,
    every noised block relaunched as its own row from the clean-prefix state
    (reference `blockdiff.py:153-177` around `gdn.py:217-231`).

How each function is pinned (tests/test_oracle_gdn.py):
  chunk_gated_delta_rule_with_states  vs recurrent_gated_delta_rule_f64 (an independent
      algorithm) on seeded tiny inputs, every per-chunk state too; chunk-size independence
      (8/16/32/64); need_states invariance (bitwise); beta=0 closed form (pure decay);
      g=0, beta=1, orthonormal keys closed form (exact overwrite).
  recurrent_gated_delta_rule_f64      vs the installed transformers recurrent kernel (fp32) and
      the hand-derived closed forms above.
  causal_conv1d                       vs a float64 brute-force FIR loop; prefix carry-in vs
      conv over the concatenated sequence.
  fork_layout                         two independent constructions (the reference's tensor ops
      on index tensors, and brute-force enumeration) must agree bit-exactly.
  state_fork_layer                    vs running the clean+noised concatenation through the
      float64 recurrence block by block (the visibility contract itself).
"""

from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F


# ----------------------------------------------------------------------------------------------
# l2norm — transformers modeling_qwen3_5.py:242-245: x * rsqrt(sum(x^2) + eps), eps inside rsqrt.
# ----------------------------------------------------------------------------------------------
def l2norm(x: torch.Tensor, dim: int = -1, eps: float = 1e-6) -> torch.Tensor:
    return x * torch.rsqrt((x * x).sum(dim=dim, keepdim=True) + eps)


# ----------------------------------------------------------------------------------------------
# Chunked gated delta rule with per-chunk states — reference gdn.py:48-123.
# ----------------------------------------------------------------------------------------------
def chunk_gated_delta_rule_with_states(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    g: torch.Tensor,
    beta: torch.Tensor,
    chunk_size: int,
    initial_state: torch.Tensor | None = None,
    use_qk_l2norm_in_kernel: bool = True,
    need_states: bool = True,
    _plant: str | None = None,
):
    """(out [B,T,Hv,Dv] in the input dtype, states [B,T/C,Hv,Dk,Dv] fp32 or None).

    `_plant` injects a deliberate mistake for tests that check a tolerance can see it:
    "drop-carry" (the update forgets e^gamma_last S) or "carry-scale" (the carried state is scaled
    by 1.05). Never used to produce expected values.

    Per chunk i and head: with gamma = cumsum(g) inside the chunk and
    Gamma[r,s] = exp(gamma_r - gamma_s) for s <= r (else 0),
      A  = strict_lower((beta*K) K^T * Gamma),  U = (I+A)^-1 (beta*V),
      W  = (I+A)^-1 (beta*K*e^gamma),           P = (Q K^T) * Gamma,
      V' = U - W S;  O = (Q e^gamma) S + P V';  S <- e^gamma_last S + (K e^(gamma_last-gamma))^T V'.
    Steps follow gdn.py:76-123 (fp32 from the input dtype, l2norm, Dk^-1/2 scale, beta scaling,
    cumulative decay, -inf strict-upper mask before exp, two unit-lower triangular solves).
    """
    out_dtype = query.dtype
    B, T, _, Dk = key.shape
    Hv, Dv = value.shape[-2:]
    if T % chunk_size != 0:
        raise ValueError(f"sequence_length {T} is not a multiple of chunk_size {chunk_size}")
    C = chunk_size
    n = T // C

    def heads_first(x):  # [B,T,H,...] -> [B,H,T,...] fp32 contiguous
        return x.transpose(1, 2).to(torch.float32).contiguous()

    q, k, v, b, gg = (heads_first(x) for x in (query, key, value, beta, g))
    if use_qk_l2norm_in_kernel:
        q = l2norm(q)
        k = l2norm(k)
    q = q * (q.shape[-1] ** -0.5)

    kb = k * b[..., None]
    vb = v * b[..., None]
    split = lambda x: x.reshape(B, Hv, n, C, x.shape[-1])  # noqa: E731
    q, k, kb, vb = split(q), split(k), split(kb), split(vb)
    gamma = gg.reshape(B, Hv, n, C).cumsum(-1)
    upper = torch.ones(C, C, dtype=torch.bool).triu(1)
    Gamma = (gamma[..., :, None] - gamma[..., None, :]).masked_fill(upper, float("-inf")).exp()

    A = (kb @ k.transpose(-1, -2)) * Gamma
    P = (q @ k.transpose(-1, -2)) * Gamma
    U = torch.linalg.solve_triangular(A, vb, upper=False, unitriangular=True)
    W = torch.linalg.solve_triangular(A, kb * gamma.exp()[..., None], upper=False, unitriangular=True)

    S = (torch.zeros(B, Hv, Dk, Dv, dtype=torch.float32) if initial_state is None
         else initial_state.to(torch.float32).clone())
    q_dec = q * gamma.exp()[..., None]
    k_dec = k * (gamma[..., -1:] - gamma).exp()[..., None]
    lam = gamma[..., -1].exp()[..., None, None]

    out = torch.empty(B, Hv, n, C, Dv, dtype=torch.float32)
    snaps = []
    for i in range(n):
        v_new = U[:, :, i] - W[:, :, i] @ S
        out[:, :, i] = q_dec[:, :, i] @ S + P[:, :, i] @ v_new
        carry = S * lam[:, :, i]
        if _plant == "drop-carry":
            carry = torch.zeros_like(carry)
        elif _plant == "carry-scale":
            carry = carry * 1.05
        S = carry + k_dec[:, :, i].transpose(-1, -2) @ v_new
        if need_states:
            snaps.append(S)
    out = out.reshape(B, Hv, T, Dv).transpose(1, 2).to(out_dtype).contiguous()
    return out, (torch.stack(snaps, 1) if need_states else None)


# ----------------------------------------------------------------------------------------------
# Float64 token recurrence — transformers modeling_qwen3_5.py:330-381 (the same math per token).
# ----------------------------------------------------------------------------------------------
def recurrent_gated_delta_rule_f64(q, k, v, g, beta, *, chunk_size=None, initial_state=None,
                                   use_qk_l2norm=True):
    """numpy float64, token by token:
        S_t = e^{g_t} S_{t-1} + k_t delta_t^T,  delta_t = beta_t (v_t - (e^{g_t} S_{t-1})^T k_t),
        o_t = S_t^T q_t   (q, k l2-normalised; q scaled by Dk^-1/2).
    Returns (o [B,T,H,Dv], states [B,T/chunk,H,Dk,Dv] snapshotted after every chunk, or None)."""
    q, k, v, g, beta = (np.asarray(x.detach().to(torch.float64) if torch.is_tensor(x) else x,
                                   dtype=np.float64) for x in (q, k, v, g, beta))
    B, T, H, Dk = k.shape
    Dv = v.shape[-1]
    if use_qk_l2norm:
        q = q / np.sqrt((q * q).sum(-1, keepdims=True) + 1e-6)
        k = k / np.sqrt((k * k).sum(-1, keepdims=True) + 1e-6)
    q = q * Dk ** -0.5
    S = (np.zeros((B, H, Dk, Dv)) if initial_state is None
         else (initial_state.detach().to(torch.float64).cpu().numpy() if torch.is_tensor(initial_state)
               else np.asarray(initial_state, dtype=np.float64)).copy())
    o = np.zeros((B, T, H, Dv))
    snaps = []
    for t in range(T):
        S = S * np.exp(g[:, t])[:, :, None, None]
        kv = np.einsum("bhkv,bhk->bhv", S, k[:, t])
        delta = (v[:, t] - kv) * beta[:, t][:, :, None]
        S = S + np.einsum("bhk,bhv->bhkv", k[:, t], delta)
        o[:, t] = np.einsum("bhkv,bhk->bhv", S, q[:, t])
        if chunk_size and (t + 1) % chunk_size == 0:
            snaps.append(S.copy())
    return o, (np.stack(snaps, 1) if chunk_size else None)


# ----------------------------------------------------------------------------------------------
# Causal depthwise conv + SiLU with prefix carry-in — transformers modeling_qwen3_5.py:219-239,
# called on cat([conv_prefix, raw]) and cut to the last T outputs as in reference gdn.py:217-219.
# ----------------------------------------------------------------------------------------------
def causal_conv1d(x, weight, bias=None, activation="silu", prefix=None):
    """x [B,C,T]; weight [C,K]; prefix [B,C,P] or None -> [B,C,T] in x's dtype.

    Computes in the weight's dtype (torch CPU bf16 conv accumulates in fp32 and rounds to bf16;
    SiLU is evaluated in fp32 and rounded to the weight dtype) and returns x's dtype."""
    T = x.shape[-1]
    xin = x if prefix is None else torch.cat([prefix.to(x.dtype), x], dim=2)
    K = weight.shape[-1]
    y = F.conv1d(xin.to(weight.dtype), weight.unsqueeze(1), bias, padding=K - 1,
                 groups=x.shape[1])[:, :, : xin.shape[-1]]
    if activation is not None:
        y = F.silu(y)
    return y[:, :, -T:].to(x.dtype)


def causal_conv1d_bruteforce_f64(x, weight, bias=None, prefix=None):
    """float64 FIR loop: y[t] = silu(bias + sum_j w[j] * xin[t - (K-1) + j]) over the prefix-extended
    sequence, zeros before its start."""
    x = np.asarray(x.to(torch.float64))
    w = np.asarray(weight.to(torch.float64))
    B, C, T = x.shape
    K = w.shape[1]
    pre = np.zeros((B, C, 0)) if prefix is None else np.asarray(prefix.to(torch.float64))
    xin = np.concatenate([np.zeros((B, C, K - 1)), pre, x], axis=2)
    off = K - 1 + pre.shape[2]
    y = np.zeros((B, C, T))
    for t in range(T):
        acc = np.zeros((B, C)) if bias is None else np.broadcast_to(np.asarray(bias.to(torch.float64)), (B, C)).copy()
        for j in range(K):
            acc = acc + w[None, :, j] * xin[:, :, off + t - (K - 1) + j]
        y[:, :, t] = acc / (1.0 + np.exp(-acc))
    return y


# ----------------------------------------------------------------------------------------------
# Fork layout (integer) — reference blockdiff.py:161-173.
# ----------------------------------------------------------------------------------------------
def fork_layout(B: int, L: int, block: int, width: int = 4):
    """Index maps of the state fork, built with the reference's own tensor operations applied to
    index tensors:
      row[b,k]          fork batch row of (sequence b, block k)                 (reshape B*nb)
      state_src[row]    flat index b*nb+k' of the clean state the row starts from, -1 = zeros
                        (cat([zeros, states0[:, :-1]]) then reshape)
      prefix_pos[row,j] clean position feeding prefix slot j, -1 = zero padding
                        (cat([zeros(K-1), raw0]).unfold(2, K-1, block)[:, :, :nb])"""
    if L % block:
        raise ValueError(f"L={L} is not a multiple of block={block}")
    nb = L // block
    km1 = width - 1
    row = torch.arange(B * nb).reshape(B, nb)
    states_idx = torch.arange(B * nb).reshape(B, nb)  # stand-in for states0[b, k]
    init = torch.cat([torch.full_like(states_idx[:, :1], -1), states_idx[:, :-1]], 1).reshape(B * nb)
    pos = torch.arange(L).expand(B, 1, L)  # [B, C=1, L] positions of raw0
    padded = torch.cat([torch.full((B, 1, km1), -1, dtype=pos.dtype), pos], 2)
    prefix = padded.unfold(2, km1, block)[:, :, :nb].permute(0, 2, 1, 3).reshape(B * nb, -1, km1)[:, 0]
    return {"row": row, "state_src": init, "prefix_pos": prefix}


def fork_layout_bruteforce(B: int, L: int, block: int, width: int = 4):
    nb = L // block
    km1 = width - 1
    row = np.zeros((B, nb), np.int64)
    src = np.zeros(B * nb, np.int64)
    pre = np.zeros((B * nb, km1), np.int64)
    for b in range(B):
        for k in range(nb):
            r = b * nb + k
            row[b, k] = r
            src[r] = -1 if k == 0 else b * nb + (k - 1)
            for j in range(km1):
                p = k * block - km1 + j
                pre[r, j] = p if p >= 0 else -1
    return {"row": torch.from_numpy(row), "state_src": torch.from_numpy(src), "prefix_pos": torch.from_numpy(pre)}


# ----------------------------------------------------------------------------------------------
# The state-fork GDN layer op (conv + core + fork) — reference blockdiff.py:153-177 with the
# mixer steps of gdn.py:217-231 (projections, gated norm and out_proj excluded).
# ----------------------------------------------------------------------------------------------
def _split_heads(mixed, B, T, Hk, Hv, Dk, Dv):
    kd = Hk * Dk
    q, k, v = torch.split(mixed, [kd, kd, Hv * Dv], dim=-1)
    q = q.reshape(B, T, Hk, Dk)
    k = k.reshape(B, T, Hk, Dk)
    v = v.reshape(B, T, Hv, Dv)
    if Hv // Hk > 1:  # GQA expansion: value head j reads key head j // (Hv/Hk) (gdn.py:227-229)
        q = q.repeat_interleave(Hv // Hk, dim=2)
        k = k.repeat_interleave(Hv // Hk, dim=2)
    return q, k, v


def gdn_conv_core(raw, conv_w, beta, g, *, Hk, Hv, Dk, Dv, chunk, conv_prefix=None,
                  initial_state=None, need_states=True, _plant=None):
    """One mixer pass without projections: raw [B,T,conv_dim] (token-major) -> conv+SiLU (with an
    optional [B,conv_dim,K-1] prefix) -> split/GQA -> chunked core. Returns (o, states)."""
    B, T, _ = raw.shape
    mixed = causal_conv1d(raw.transpose(1, 2), conv_w, None, "silu", prefix=conv_prefix).transpose(1, 2)
    q, k, v = _split_heads(mixed, B, T, Hk, Hv, Dk, Dv)
    return chunk_gated_delta_rule_with_states(q, k, v, g, beta, chunk_size=chunk,
                                              initial_state=initial_state, need_states=need_states,
                                              _plant=_plant)


def state_fork_layer(raw0, rawt, conv_w, beta0, betat, g0, gt, *, Hk, Hv, Dk, Dv, block,
                     fault: str | None = None, need_states: bool = True, _plant: str | None = None):
    """The state-fork GDN layer on pre-conv projections of both streams.

    raw0/rawt [B,L,conv_dim]; beta*, g* [B,L,Hv]; conv_w [conv_dim,K].
    Returns (o0 [B,L,Hv,Dv], ot [B,L,Hv,Dv], states0 [B,nb,Hv,Dk,Dv] fp32, tails [B*nb,conv_dim,K-1]).

    fault: None | "no-conv-prefix" (noised rows' conv starts cold) | "concat-causal-gdn"
    (one causal pass over cat([x_t, x_0])) — reference blockdiff.py:69-88,155-157,168-170.
    `_plant` (tests of tolerances only): the core's "drop-carry" / "carry-scale" on the clean pass,
    or "fork-off-by-one" (noised block k starts from the clean state after block k, not k-1)."""
    B, L, Cd = raw0.shape
    if L % block:
        raise ValueError(f"L={L} is not a multiple of block={block}")
    nb = L // block
    K = conv_w.shape[-1]
    dims = dict(Hk=Hk, Hv=Hv, Dk=Dk, Dv=Dv)
    if fault == "concat-causal-gdn":
        o, _ = gdn_conv_core(torch.cat([rawt, raw0], 1), conv_w, torch.cat([betat, beta0], 1),
                             torch.cat([gt, g0], 1), chunk=block, need_states=False, **dims)
        return o[:, L:], o[:, :L], None, None
    core_plant = _plant if _plant in ("drop-carry", "carry-scale") else None
    o0, states0 = gdn_conv_core(raw0, conv_w, beta0, g0, chunk=block, need_states=True, _plant=core_plant, **dims)
    init = torch.cat([torch.zeros_like(states0[:, :1]), states0[:, :-1]], 1).reshape(B * nb, Hv, Dk, Dv)
    if _plant == "fork-off-by-one":
        init = states0.reshape(B * nb, Hv, Dk, Dv)
    raw0_t = raw0.transpose(1, 2)  # [B, Cd, L], the reference's raw_qkv layout
    padded = torch.cat([torch.zeros_like(raw0_t[:, :, : K - 1]), raw0_t], 2)
    tails = padded.unfold(2, K - 1, block)[:, :, :nb].permute(0, 2, 1, 3).reshape(B * nb, Cd, K - 1)
    prefix = None if fault == "no-conv-prefix" else tails
    ot, _ = gdn_conv_core(rawt.reshape(B * nb, block, Cd), conv_w, betat.reshape(B * nb, block, Hv),
                          gt.reshape(B * nb, block, Hv), chunk=block, conv_prefix=prefix,
                          initial_state=init, need_states=False, **dims)
    return o0, ot.reshape(B, L, Hv, Dv), (states0 if need_states else None), tails.contiguous()


def state_fork_layer_f64(raw0, rawt, conv_w, beta0, betat, g0, gt, *, Hk, Hv, Dk, Dv, block):
    """Visibility contract in float64, from first principles: clean stream = one causal recurrence;
    noised block k of sequence b = the recurrence over cat(clean[:kC], noised block k), with the
    conv also run over that concatenation, keeping only block k's outputs. No fork machinery."""
    B, L, Cd = raw0.shape
    nb = L // block
    w = conv_w.to(torch.float64)
    n_rep = Hv // Hk

    def mix(raw):  # [B', T, Cd] -> q,k,v float64 (conv in float64, no intermediate rounding)
        y = torch.from_numpy(causal_conv1d_bruteforce_f64(raw.transpose(1, 2).to(torch.float64), w)).transpose(1, 2)
        q, k, v = torch.split(y, [Hk * Dk, Hk * Dk, Hv * Dv], dim=-1)
        q = q.reshape(*q.shape[:2], Hk, Dk).repeat_interleave(n_rep, 2)
        k = k.reshape(*k.shape[:2], Hk, Dk).repeat_interleave(n_rep, 2)
        return q, k, v.reshape(*v.shape[:2], Hv, Dv)

    q, k, v = mix(raw0)
    o0, st = recurrent_gated_delta_rule_f64(q, k, v, g0, beta0, chunk_size=block)
    ot = np.zeros_like(o0)
    for kb in range(nb):
        sl = slice(kb * block, (kb + 1) * block)
        seq = torch.cat([raw0[:, : kb * block], rawt[:, sl]], 1)
        qq, kk, vv = mix(seq)
        gg = torch.cat([g0[:, : kb * block], gt[:, sl]], 1)
        bb = torch.cat([beta0[:, : kb * block], betat[:, sl]], 1)
        o, _ = recurrent_gated_delta_rule_f64(qq, kk, vv, gg, bb)
        ot[:, sl] = o[:, -block:]
    return o0, ot, st


def gdn_layer_flops(B: int, L: int, Hv: int, Dk: int, Dv: int, chunk: int) -> int:
    """Algorithmic flops of the state-fork layer's chunk contractions (clean + noised), counting
    W.S, Q.S, K^T V' (clean) and W.S, Q.S (noised) at 2*C*Dk*Dv each, plus K K^T, Q K^T, P V'
    (2*C^2*D each) and the two triangular solves (C^2*D each) per stream."""
    C = chunk
    D = Dk
    clean = 6 * C * D * Dv + 8 * C * C * D
    noised = 4 * C * D * Dv + 8 * C * C * D
    return (B * L // C) * Hv * (clean + noised)
