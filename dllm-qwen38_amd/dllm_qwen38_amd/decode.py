"""Block-wise confidence-threshold parallel decoding on the MI355X HIP kernels.

Drop-in for the reference's `src/dllm_qwen38/decode.py`:
  * `DecodeTrace` and `generate` (decode.py:23-99): the golden decoder. Every denoising step re-runs
    the whole two-stream `block_diffusion_forward` over prompt + generated tokens, here on the HIP
    path, so its temperature-0 token stream is the one a faster decoder must reproduce.
  * `generate_cached`: the same decoder with the clean prefix kept on the device instead of
    recomputed. Under the complementary mask, x_t block k sees x_0 blocks < k and itself, and x_0
    is block-causal; so the noised logits of block k are a block-causal forward of the block's own
    tokens on top of the clean prefix, whose per-layer state is everything the block needs:
      - Gated DeltaNet layers: the recurrent state after the prefix [B, Hv, Dk, Dv] (fp32) and the
        pre-conv projections of the prefix's last (conv width - 1) tokens (the conv carry-in);
      - attention layers: the prefix's keys and values after q/k norm and RoPE.
    A denoising step is then one forward over `block` tokens instead of (k + 1) * block, and a
    finished block enters the cache with one more such forward (`commit`). The prompt's whole blocks
    are prefilled in one block-causal forward.
    `PrefixCache` holds that state in HBM and `forward_segment` runs a segment through it.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass, field

import torch

from . import _lib, attention, gdn, norms
from .blockdiff import FULL, LINEAR, _eps, block_diffusion_forward, rmsnorm, rotary_tables


@dataclass
class DecodeTrace:
    """Token stream and schedule of one decode (decode.py:23-33). `commits`: cache-extending
    forwards of `generate_cached` (one per finished block, plus the prompt prefill); not counted in
    `forwards`, which counts denoising forwards as the reference does."""

    tokens: list[int]
    forwards: int = 0
    generated: int = 0
    steps_per_block: list[int] = field(default_factory=list)
    commits: int = 0

    @property
    def tokens_per_forward(self) -> float:
        return self.generated / self.forwards if self.forwards else 0.0


def _select(logits: torch.Tensor, masked: torch.Tensor, *, threshold: float, sub_block: int | None,
            temperature: float):
    """The commit rule of one denoising step (decode.py:67-88). logits [C, V] fp32 over the current
    block, masked [C] bool. Returns (commit [C] bool, pick [C] tokens): the argmax token (a sample
    at temperature > 0) and its probability per position; candidates are the masked positions,
    restricted with sub_block to the leftmost sub-block still holding a mask; every candidate at or
    above the threshold commits, and at least the most confident one does."""
    if temperature > 0:
        probs = torch.softmax(logits / temperature, -1)
        pick = torch.multinomial(probs, 1).squeeze(1)
        conf = probs.gather(1, pick.unsqueeze(1)).squeeze(1)
    else:
        conf, pick = torch.softmax(logits, -1).max(-1)
    cand = masked.clone()
    if sub_block:
        first = int(masked.nonzero()[0])
        start = (first // sub_block) * sub_block
        cand[:start] = False
        cand[start + sub_block:] = False
    conf = conf.masked_fill(~cand, -1.0)
    commit = cand & (conf >= threshold)
    if not bool(commit.any()):
        commit[int(conf.argmax())] = True
    return commit, pick


@torch.no_grad()
def generate(text_model, lm_head, prompt_ids: list[int], *, n_blocks: int, block: int, mask_id: int,
             threshold: float = 0.9, sub_block: int | None = None, eos_id: int | None = None,
             temperature: float = 0.0, layers: int | None = None) -> DecodeTrace:
    """The golden decoder (decode.py:36-99): per block, start from all-mask, re-run the whole
    two-stream forward per step and commit by `_select` until the block is clean; stop after the
    block that produced `eos_id`."""
    device = text_model.embed_tokens.weight.device
    cur = list(prompt_ids)
    trace = DecodeTrace(tokens=cur)
    for _ in range(n_blocks):
        n = len(cur)
        kb = n // block
        L = (kb + 1) * block
        known = torch.full((L,), mask_id, dtype=torch.long, device=device)
        known[:n] = torch.tensor(cur, dtype=torch.long, device=device)
        masked = torch.arange(L, device=device) >= n
        x0 = known.clone()  # x_0 block kb is invisible to x_t block kb
        steps = 0
        while bool(masked.any()):
            xt = known.masked_fill(masked, mask_id)
            lt, _ = block_diffusion_forward(text_model, lm_head, x0[None], xt[None], block, layers=layers)
            trace.forwards += 1
            steps += 1
            commit, pick = _select(lt[0, kb * block:].float(), masked[kb * block:], threshold=threshold,
                                   sub_block=sub_block, temperature=temperature)
            known[kb * block:][commit] = pick[commit]
            masked[kb * block:][commit] = False
        trace.steps_per_block.append(steps)
        # the block's host synchronisation: a kernel whose bounded wait gave up chose these tokens
        # from invalid logits
        gdn.check_kernel_status("decode block")
        new = known[n:].tolist()
        cur.extend(new)
        trace.generated += len(new)
        if eos_id is not None and eos_id in new:
            break
    trace.tokens = cur
    return trace


# False: forward_segment runs each bit-exact fused decoding-step launch (projection end + norm, the
# GDN in_proj end, the attention layer's direct cache writes) as the separate launches it replaces,
# whose results it equals bit for bit; for comparisons and measurement. (The attention output gate
# inside the attention kernel rounds its sigmoid from the hardware exponential, within one bf16
# rounding of torch's, and is not switched.)
FUSED = True

_WORKSPACES: dict = {}
_SIZES: dict = {}


def _workgroups(L, M: int, N: int, K: int) -> int:
    key = ("g", M, N, K)
    G = _SIZES.get(key)
    if G is None:
        G = _SIZES[key] = L.dllm_decode_linear_workgroups(M, N, K)
    return G


def _workspace(L, M: int, n_gate: int, G: int, swiglu: bool, dev) -> torch.Tensor:
    """Workspace of one decoding-step projection launch: the fp32 pieces of the tiles split between
    workgroups (and with swiglu the up projection's rounded tiles; for the fused residual norm the
    projection's rounded tiles, the same size with n_gate = N). One buffer per (device, stream,
    size), reused: launches on one stream run in order, and a launch's pieces are consumed by its
    own second kernel before the next launch on that stream writes them."""
    key = ("w", M, n_gate, G, bool(swiglu))
    nbytes = _SIZES.get(key)
    if nbytes is None:
        nbytes = _SIZES[key] = L.dllm_decode_linear_workspace_bytes(M, n_gate, G, int(swiglu))
    if nbytes <= 0:
        raise ValueError(f"decode linear: no workspace size for M={M} workgroups={G}")
    wkey = (dev.index, _lib.stream_handle(dev), nbytes)
    ws = _WORKSPACES.get(wkey)
    if ws is None:
        ws = _WORKSPACES[wkey] = torch.empty(-(-nbytes // 16) * 4, dtype=torch.float32, device=dev)
    return ws


def decode_linear(x: torch.Tensor, weight: torch.Tensor, *, out: torch.Tensor | None = None) -> torch.Tensor:
    """x [..., K] @ weight[N, K]^T for the few token rows of a decoding step (bf16, at most 64 rows,
    K a multiple of 64) on the HIP kernel that streams the weight into MFMA operands, every CU an
    equal share of it; fp32 accumulation, deterministic. Returns [..., N] bf16."""
    dev = _lib.require_device(x, weight)
    K = x.shape[-1]
    N = weight.shape[0]
    if weight.dim() != 2 or weight.shape[1] != K:
        raise ValueError(f"weight must be [N, {K}], got {tuple(weight.shape)}")
    if x.dtype != torch.bfloat16 or weight.dtype != torch.bfloat16:
        raise TypeError("decode_linear takes bf16 x and weight")
    x2 = x.reshape(-1, K).contiguous()
    w = weight.contiguous()
    M = x2.shape[0]
    L = _lib.lib()
    G = _workgroups(L, M, N, K)
    if G <= 0:
        raise ValueError(f"decode_linear does not take M={M} N={N} K={K} (M <= 64, K % 64 == 0)")
    y = torch.empty(M, N, dtype=torch.bfloat16, device=dev) if out is None else out
    if tuple(y.shape) != (M, N) or not y.is_contiguous() or y.dtype != torch.bfloat16:
        raise ValueError("out must be a contiguous bf16 [M, N] tensor")
    ws = _workspace(L, M, 0, G, False, dev)
    _lib.check(L.dllm_decode_linear_fwd(x2.data_ptr(), w.data_ptr(), y.data_ptr(), ws.data_ptr(), M, N, K, G,
                                        _lib.dtype_code(x.dtype), _lib.stream_handle(dev)), "dllm_decode_linear_fwd")
    return y.reshape(*x.shape[:-1], N)


def decode_linear_multi(x: torch.Tensor, weights: list, *, swiglu: bool = False, outs: list | None = None):
    """Up to four projections of the same x [..., K] in one launch (their weights [N_i, K] bf16).
    Returns the list of [..., N_i] outputs, or with swiglu (gate, up) the MLP activation
    round(round(silu(x gate^T)) * (x up^T)) as one tensor. outs (without swiglu): per projection
    None or a contiguous bf16 tensor of M x N_i elements to write it into (a cache's rows)."""
    dev = _lib.require_device(x, *weights)
    K = x.shape[-1]
    if not 1 <= len(weights) <= 4:
        raise ValueError("decode_linear_multi takes 1 to 4 weights")
    if any(w.dim() != 2 or w.shape[1] != K or w.dtype != torch.bfloat16 for w in weights) or x.dtype != torch.bfloat16:
        raise ValueError(f"weights must be bf16 [N, {K}] and x bf16")
    x2 = x.reshape(-1, K).contiguous()
    M = x2.shape[0]
    ws = [w.contiguous() for w in weights]
    Ns = [w.shape[0] for w in ws]
    if swiglu and (len(ws) != 2 or Ns[0] != Ns[1]):
        raise ValueError("swiglu takes (gate, up) of equal N")
    L = _lib.lib()
    G = _workgroups(L, M, sum(-(-n // 128) * 128 for n in Ns), K)
    if G <= 0:
        raise ValueError(f"decode_linear_multi does not take M={M} K={K} (M <= 64, K % 64 == 0)")
    given = outs
    if given is not None and (swiglu or len(given) != len(Ns)):
        raise ValueError("outs takes one entry per projection, without swiglu")
    outs = []
    for i, n in enumerate(Ns[:1] if swiglu else Ns):
        o = given[i] if given is not None else None
        if o is None:
            o = torch.empty(M, n, dtype=torch.bfloat16, device=dev)
        elif o.numel() != M * n or o.dtype != torch.bfloat16 or not o.is_contiguous() or o.device != dev:
            raise ValueError(f"outs[{i}] must be a contiguous bf16 tensor of {M} x {n} elements on {dev}")
        outs.append(o)
    if swiglu:
        outs.append(outs[0])  # not written
    work = _workspace(L, M, Ns[0], G, swiglu, dev)
    n = len(ws)
    warr = (ctypes.c_void_p * n)(*[w.data_ptr() for w in ws])
    oarr = (ctypes.c_void_p * n)(*[o.data_ptr() for o in outs])
    narr = (ctypes.c_int * n)(*Ns)
    _lib.check(L.dllm_decode_linear_multi_fwd(x2.data_ptr(), M, K, n, warr, oarr, narr, work.data_ptr(), G,
                                              int(swiglu), _lib.dtype_code(x.dtype), _lib.stream_handle(dev)),
               "dllm_decode_linear_multi_fwd")
    lead = x.shape[:-1]
    if swiglu:
        return outs[0].reshape(*lead, Ns[0])
    return [o.reshape(*lead, nn) for o, nn in zip(outs, Ns)]


def decode_linear_rmsnorm(x: torch.Tensor, weight: torch.Tensor, residual: torch.Tensor, norm_weight: torch.Tensor,
                          eps: float, *, unit_offset: bool = True):
    """A decoding-step projection followed by the residual add and RMSNorm after it: with
    p = x @ weight^T rounded to bf16, returns (rmsnorm(s) * (1 + norm_weight), s) where s = p +
    residual rounded to bf16. Equal element for element to `decode_linear` then
    `norms.rmsnorm(.., residual=residual)`, in one streaming launch and one row-wise launch (the
    split tiles' sums, the add and the norm) instead of three. x [..., K] and weight [N, K] bf16 (at
    most 64 rows, K a multiple of 64), residual [..., N] bf16, norm_weight [N] bf16 or fp32, N a
    multiple of 512 up to 8192."""
    dev = _lib.require_device(x, weight, residual, norm_weight)
    K = x.shape[-1]
    N = weight.shape[0]
    if weight.dim() != 2 or weight.shape[1] != K:
        raise ValueError(f"weight must be [N, {K}], got {tuple(weight.shape)}")
    if x.dtype != torch.bfloat16 or weight.dtype != torch.bfloat16 or residual.dtype != torch.bfloat16:
        raise TypeError("decode_linear_rmsnorm takes bf16 x, weight and residual")
    lead = x.shape[:-1]
    if tuple(residual.shape) != (*lead, N) or tuple(norm_weight.shape) != (N,):
        raise ValueError(f"residual must be {(*lead, N)} and norm_weight ({N},)")
    x2 = x.reshape(-1, K).contiguous()
    M = x2.shape[0]
    L = _lib.lib()
    G = _workgroups(L, M, N, K)
    if G <= 0:
        raise ValueError(f"decode_linear_rmsnorm does not take M={M} N={N} K={K} (M <= 64, K % 64 == 0)")
    wt = weight.contiguous()
    r = residual.reshape(M, N).contiguous()
    w = norm_weight.contiguous()
    s = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
    y = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
    ws = _workspace(L, M, N, G, True, dev)  # the pieces, then the projection's whole tiles
    _lib.check(L.dllm_decode_linear_rmsnorm_fwd(
        x2.data_ptr(), wt.data_ptr(), ws.data_ptr(), M, N, K, G, r.data_ptr(), s.data_ptr(),
        w.data_ptr(), y.data_ptr(), float(eps), int(unit_offset), _lib.dtype_code(x.dtype), _lib.dtype_code(w.dtype),
        _lib.stream_handle(dev)), "dllm_decode_linear_rmsnorm_fwd")
    return y.reshape(*lead, N), s.reshape(*lead, N)


def _fast(lins, x: torch.Tensor) -> bool:
    """Whether the decoding-step kernels take these projections of x (bf16 rows <= 64, no bias)."""
    rows = x.numel() // x.shape[-1]
    return (x.dtype == torch.bfloat16 and rows <= 64 and x.shape[-1] % 64 == 0
            and all(lin.bias is None and lin.weight.dtype == torch.bfloat16 for lin in lins))


def _proj_many(lins, x: torch.Tensor) -> list:
    """Several projections of the same x: one launch on the decoding-step kernel, else one library
    GEMM each."""
    if _fast(lins, x):
        return decode_linear_multi(x, [lin.weight for lin in lins])
    return [lin(x) for lin in lins]


def _proj(lin, x: torch.Tensor) -> torch.Tensor:
    """nn.Linear `lin` on x: the decoding-step kernel for a block of bf16 rows (at most 64), the
    library GEMM for the many rows of a prefill and for fp32 or biased projections."""
    w = lin.weight
    rows = x.numel() // x.shape[-1]
    if (lin.bias is None and x.dtype == torch.bfloat16 and w.dtype == torch.bfloat16 and rows <= 64
            and w.shape[1] % 64 == 0):
        return decode_linear(x, w)
    return lin(x)


def decode_gdn_prologue(m, x: torch.Tensor, conv_prefix: torch.Tensor | None, T: int):
    """The Gated DeltaNet mixer `m`'s input projections of a decoding segment with the short conv
    and the gates (reference gdn.py:212-226 with conv_prefix): x [..., K] bf16, rows = sequences of T
    tokens (T dividing 32, at most 64 rows), conv_prefix [sequences, conv_dim, width - 1] (the
    prefix's last projections) or None (zeros). Returns (raw, mixed, z, beta, g): the qkv projection
    and its conv + SiLU [..., conv_dim], z [..., value_dim], beta and g [..., H] fp32, equal element
    for element to the projections, `gdn._beta_g` and `gdn.causal_conv1d_fn` run separately; one
    streaming launch and one launch for the rest."""
    lins = (m.in_proj_qkv, m.in_proj_z, m.in_proj_b, m.in_proj_a)
    dev = _lib.require_device(x, *[lin.weight for lin in lins])
    K = x.shape[-1]
    x2 = x.reshape(-1, K).contiguous()
    M = x2.shape[0]
    ws = [lin.weight.contiguous() for lin in lins]
    Ns = [w.shape[0] for w in ws]
    C, H = Ns[0], Ns[2]
    cw = m.conv1d.weight.reshape(C, -1).contiguous()
    width = cw.shape[1]
    cb = None if m.conv1d.bias is None else m.conv1d.bias.contiguous()
    if conv_prefix is not None and (tuple(conv_prefix.shape) != (M // T, C, width - 1) or
                                    conv_prefix.dtype != torch.bfloat16 or not conv_prefix.is_contiguous()):
        raise ValueError(f"conv_prefix must be a contiguous bf16 [{M // T}, {C}, {width - 1}] tensor")
    L = _lib.lib()
    G = _workgroups(L, M, sum(-(-n // 128) * 128 for n in Ns), K)
    if G <= 0:
        raise ValueError(f"decode_gdn_prologue does not take M={M} K={K} (M <= 64, K % 64 == 0)")
    outs = [torch.empty(M, n, dtype=torch.bfloat16, device=dev) for n in Ns]
    mixed = torch.empty(M, C, dtype=torch.bfloat16, device=dev)
    beta = torch.empty(M, H, dtype=torch.float32, device=dev)
    g = torch.empty(M, H, dtype=torch.float32, device=dev)
    al = m.A_log.reshape(H).contiguous()
    db = m.dt_bias.reshape(H).to(al.dtype).contiguous()
    work = _workspace(L, M, Ns[0], G, False, dev)
    warr = (ctypes.c_void_p * 4)(*[w.data_ptr() for w in ws])
    oarr = (ctypes.c_void_p * 4)(*[o.data_ptr() for o in outs])
    narr = (ctypes.c_int * 4)(*Ns)
    _lib.check(L.dllm_decode_gdn_prologue_fwd(
        x2.data_ptr(), M, K, warr, oarr, narr, work.data_ptr(), G, T, _lib.ptr(conv_prefix),
        0 if conv_prefix is None else width - 1, cw.data_ptr(), _lib.ptr(cb), width, mixed.data_ptr(),
        al.data_ptr(), db.data_ptr(), beta.data_ptr(), g.data_ptr(), _lib.DT_BF16, _lib.dtype_code(cw.dtype),
        _lib.dtype_code(al.dtype), _lib.stream_handle(dev)), "dllm_decode_gdn_prologue_fwd")
    lead = x.shape[:-1]
    return (outs[0].reshape(*lead, C), mixed.reshape(*lead, C), outs[1].reshape(*lead, Ns[1]),
            beta.reshape(*lead, H), g.reshape(*lead, H))


def _prologue_fused(m, x: torch.Tensor, conv_prefix, T: int) -> bool:
    """Whether `decode_gdn_prologue` takes this mixer and segment."""
    lins = (m.in_proj_qkv, m.in_proj_z, m.in_proj_b, m.in_proj_a)
    w = m.conv1d.weight
    return (_fast(lins, x) and 32 % T == 0 and m.activation in ("silu", "swish") and 2 <= w.shape[-1] <= 4
            and w.dtype in (torch.bfloat16, torch.float32) and m.A_log.dtype in (torch.bfloat16, torch.float32)
            and m.in_proj_b.out_features == m.in_proj_a.out_features
            and (conv_prefix is None or (conv_prefix.dtype == torch.bfloat16 and conv_prefix.is_contiguous()
                                         and conv_prefix.shape[-1] == w.shape[-1] - 1)))


def _norm_width_fused(N: int) -> bool:
    """Whether dllm_decode_linear_rmsnorm_fwd takes rows of N features: N a multiple of 512 up to
    8192 whose 512-feature vectors split over at most 8 waves with at most 8 vectors per lane (the
    row RMSNorm kernel's layout)."""
    if N <= 0 or N % 512 or N > 8192:
        return False
    nv = N // 512
    nw = max(d for d in range(1, 9) if nv % d == 0)
    return nv // nw <= 8


def _proj_norm(lin, a: torch.Tensor, norm, h: torch.Tensor):
    """nn.Linear `lin` on a, then the residual add of h and RMSNorm `norm` ([hf]:778-792): returns
    (norm(lin(a) + h), lin(a) + h). One fused launch pair on the decoding-step kernels
    (`decode_linear_rmsnorm`), else the projection and the norm kernel."""
    w = lin.weight
    rows = a.numel() // a.shape[-1]
    if (FUSED and lin.bias is None and a.dtype == torch.bfloat16 and w.dtype == torch.bfloat16 and h.dtype == torch.bfloat16
            and rows <= 64 and w.shape[1] % 64 == 0 and _norm_width_fused(w.shape[0])
            and norm.weight.dtype in (torch.bfloat16, torch.float32)):
        return decode_linear_rmsnorm(a, w, h, norm.weight, _eps(norm))
    return rmsnorm(_proj(lin, a), norm, residual=h)


def _mlp_act(m, x: torch.Tensor):
    """SwiGLU MLP ([hf]:704-717) up to its down projection: gate and up in one launch with the
    activation in its reduction. Returns (down_proj, activation): the caller applies down_proj
    together with the residual add and norm that follow it."""
    if _fast((m.gate_proj, m.up_proj), x):
        act = decode_linear_multi(x, [m.gate_proj.weight, m.up_proj.weight], swiglu=True)
    else:
        act = norms.swiglu(m.gate_proj(x), m.up_proj(x))
    return m.down_proj, act


class PrefixCache:
    """Per-layer state of a committed clean prefix, resident in HBM, for `forward_segment`.

    For each Gated DeltaNet layer: `state[i]` [B, Hv, Dk, Dv] fp32 (the recurrence after the prefix)
    and `conv[i]` [B, conv_dim, width - 1] (pre-conv projections of the prefix's last tokens), both
    None while the prefix is empty. For each attention layer: `k[i]`, `v[i]` [B, capacity, Hkv, d]
    (after q/k norm and RoPE); rows >= `length` are scratch. `length` is the committed prefix in
    tokens, a multiple of `block`."""

    def __init__(self, text_model, *, batch: int, capacity: int, block: int, layers: int | None = None):
        cfg = text_model.config
        self.n_layers = cfg.num_hidden_layers if layers is None else layers
        if not 0 < self.n_layers <= cfg.num_hidden_layers:
            raise ValueError(f"layers={layers} outside 1..{cfg.num_hidden_layers}")
        if block <= 0 or capacity <= 0 or capacity % block:
            raise ValueError(f"capacity {capacity} must be a positive multiple of block {block}")
        w = text_model.embed_tokens.weight
        self.device, self.dtype = w.device, w.dtype
        self.batch, self.capacity, self.block, self.length = batch, capacity, block, 0
        self.kinds = list(cfg.layer_types[: self.n_layers])
        self.state: dict[int, torch.Tensor | None] = {}
        self.conv: dict[int, torch.Tensor | None] = {}
        self.k: dict[int, torch.Tensor] = {}
        self.v: dict[int, torch.Tensor] = {}
        for i, kind in enumerate(self.kinds):
            if kind == LINEAR:
                self.state[i] = self.conv[i] = None
            elif kind == FULL:
                att = text_model.layers[i].self_attn
                hkv = att.k_proj.out_features // att.head_dim
                shape = (batch, capacity, hkv, att.head_dim)
                self.k[i] = torch.empty(shape, dtype=self.dtype, device=self.device)
                self.v[i] = torch.empty(shape, dtype=self.dtype, device=self.device)
            else:
                raise ValueError(f"unknown layer type {kind}")
        self.cos, self.sin = rotary_tables(text_model, capacity, self.device, self.dtype)

    def reset(self) -> None:
        """Forget the prefix (buffers are kept)."""
        self.length = 0
        for i in self.state:
            self.state[i] = self.conv[i] = None

    def nbytes(self) -> int:
        tens = [t for d in (self.state, self.conv, self.k, self.v) for t in d.values() if t is not None]
        return sum(t.numel() * t.element_size() for t in tens)


def _gdn_segment(m, x: torch.Tensor, cache: PrefixCache, i: int, commit: bool) -> torch.Tensor:
    """Gated DeltaNet mixer of a segment on top of the cached prefix (the reference's
    gdn_mixer_forward with conv_prefix / initial_state, gdn.py:193-233): the conv carries the
    prefix's last projections in, the recurrence starts from the prefix state; with commit, the
    state after the segment and its last projections replace the cached ones."""
    B, T, _ = x.shape
    if FUSED and _prologue_fused(m, x, cache.conv[i], T):
        raw, mixed, z, beta, g = decode_gdn_prologue(m, x, cache.conv[i], T)  # raw, mixed [B, T, conv_dim]
    else:
        raw, z, bp, ap = _proj_many((m.in_proj_qkv, m.in_proj_z, m.in_proj_b, m.in_proj_a), x)
        beta, g = gdn._beta_g(m, bp, ap)
        mixed = gdn.causal_conv1d_fn(raw.transpose(1, 2), m.conv1d.weight.squeeze(1), m.conv1d.bias,
                                     activation=m.activation, conv_prefix=cache.conv[i]).transpose(1, 2)
    q, k, v = gdn._split_qkv(mixed, m, B, T)
    core, states = gdn._core(q, k, v, g, beta, chunk_size=cache.block, initial_state=cache.state[i],
                             need_states=commit)
    if commit:
        km1 = m.conv1d.weight.shape[-1] - 1
        hist = raw.transpose(1, 2) if cache.conv[i] is None or T >= km1 else torch.cat([cache.conv[i], raw.transpose(1, 2)], 2)
        if hist.shape[2] < km1:  # a prefix shorter than the conv window: zero history before it
            hist = torch.nn.functional.pad(hist, (km1 - hist.shape[2], 0))
        cache.conv[i] = hist[:, :, -km1:].contiguous()
        cache.state[i] = states[:, -1].contiguous()
    Dv = m.head_v_dim
    o = norms.gated_rmsnorm(core.reshape(-1, Dv), z.reshape(-1, Dv), m.norm.weight, _eps(m.norm))
    return m.out_proj, o.reshape(B, T, -1)


def _attention_segment(att, x: torch.Tensor, cache: PrefixCache, i: int, pos0: int) -> torch.Tensor:
    """Gated attention of a segment at positions pos0.. over the cached prefix ([hf]:656-701 under
    the block-causal rule): q/k norm + RoPE, the segment's K/V written into the cache at pos0..,
    block-causal attention against cache rows 0..pos0+T-1, sigmoid gate; returns (o_proj, its input)."""
    B, T, _ = x.shape
    hd = att.head_dim
    kc, vc = cache.k[i][:, pos0:pos0 + T], cache.v[i][:, pos0:pos0 + T]
    # one sequence: the segment's cache rows are contiguous, and the projections and the k prologue
    # write into them directly
    direct = FUSED and B == 1 and kc.is_contiguous() and vc.is_contiguous()
    lins = (att.q_proj, att.k_proj, att.v_proj)
    if direct and _fast(lins, x):
        qg, kp, _ = decode_linear_multi(x, [lin.weight for lin in lins], outs=[None, None, vc])
    else:
        qg, kp, vp = _proj_many(lins, x)
        vc.copy_(vp.view(B, T, -1, hd))
    q, gate = torch.chunk(qg.view(B, T, -1, 2 * hd), 2, dim=-1)
    cos, sin = cache.cos[pos0:pos0 + T], cache.sin[pos0:pos0 + T]
    q, k = norms.qk_norm_rope(q, kp.view(B, T, -1, hd), att.q_norm, att.k_norm, cos, sin, T,
                              k_out=kc if direct else None)
    if not direct:
        kc.copy_(k)
    kv = (cache.k[i][:, :pos0 + T], cache.v[i][:, :pos0 + T])
    if attention.block_causal_gate_fused(q, *kv):
        o = attention.block_causal_attention(q, *kv, block=cache.block, q_offset=pos0, scale=float(att.scaling),
                                             gate=gate)
        return att.o_proj, o.reshape(B, T, -1)
    o = attention.block_causal_attention(q, *kv, block=cache.block, q_offset=pos0, scale=float(att.scaling))
    return att.o_proj, o.reshape(B, T, -1) * torch.sigmoid(gate.reshape(B, T, -1))


@torch.no_grad()
def forward_segment(text_model, lm_head, cache: PrefixCache, ids: torch.Tensor, *, commit: bool,
                    logits: bool = True):
    """Run ids [B, T] (T a multiple of the block) at positions cache.length.. through the stack on
    top of the cached prefix, block-causally. Returns the logits [B, T, V] (or None with
    logits=False). With commit, the segment becomes part of the prefix; without, the cache's
    committed state is untouched (attention rows past `length` are scratch). Runs without autograd:
    the HIP kernels are forward-only."""
    if ids.dim() != 2 or ids.shape[0] != cache.batch:
        raise ValueError(f"ids must be [B={cache.batch}, T]")
    B, T = ids.shape
    P = cache.length
    if T == 0 or T % cache.block:
        raise ValueError(f"segment length {T} is not a positive multiple of block={cache.block}")
    if P + T > cache.capacity:
        raise ValueError(f"segment at {P}..{P + T} exceeds the cache capacity {cache.capacity}")
    h = text_model.embed_tokens(ids)
    pending = None  # (the last MLP's down_proj, its input): applied with the norm after it
    for i, kind in enumerate(cache.kinds):
        layer = text_model.layers[i]
        if pending is None:
            x = rmsnorm(h, layer.input_layernorm)
        else:
            x, h = _proj_norm(*pending, layer.input_layernorm, h)
        if kind == LINEAR:
            lin, a = _gdn_segment(layer.linear_attn, x, cache, i, commit)
        else:
            lin, a = _attention_segment(layer.self_attn, x, cache, i, P)
        x, h = _proj_norm(lin, a, layer.post_attention_layernorm, h)
        pending = _mlp_act(layer.mlp, x)
    if commit:
        cache.length = P + T
    if not logits:
        return None  # the cache is complete; the last MLP's down projection feeds only the logits
    return _proj(lm_head, _proj_norm(*pending, text_model.norm, h)[0])


@torch.no_grad()
def generate_cached(text_model, lm_head, prompt_ids: list[int], *, n_blocks: int, block: int, mask_id: int,
                    threshold: float = 0.9, sub_block: int | None = None, eos_id: int | None = None,
                    temperature: float = 0.0, layers: int | None = None,
                    cache: PrefixCache | None = None) -> DecodeTrace:
    """`generate` with the clean prefix cached: same arguments, same commit rule and trace, one
    block per denoising forward. The prompt's whole blocks are prefilled in one forward; each
    finished block is committed with one more. A `cache` of batch 1 and enough capacity may be
    passed in to reuse its buffers (it is reset)."""
    device = text_model.embed_tokens.weight.device
    cur = list(prompt_ids)
    trace = DecodeTrace(tokens=cur)
    kb = len(cur) // block
    need = (kb + n_blocks) * block
    if cache is None:
        cache = PrefixCache(text_model, batch=1, capacity=need, block=block, layers=layers)
    elif cache.batch != 1 or cache.capacity < need or cache.block != block:
        raise ValueError("cache must have batch 1, the same block and capacity >= (prompt blocks + n_blocks) * block")
    cache.reset()
    if kb:
        forward_segment(text_model, lm_head, cache, torch.tensor([cur[:kb * block]], device=device), commit=True,
                        logits=False)
        trace.commits += 1
    for nb in range(n_blocks):
        n = len(cur)
        kb = n // block
        have = n - kb * block  # prompt tokens already in this block
        known = torch.full((block,), mask_id, dtype=torch.long, device=device)
        known[:have] = torch.tensor(cur[kb * block:], dtype=torch.long, device=device)
        masked = torch.arange(block, device=device) >= have
        steps = 0
        while bool(masked.any()):
            lt = forward_segment(text_model, lm_head, cache, known.masked_fill(masked, mask_id)[None], commit=False)
            trace.forwards += 1
            steps += 1
            commit, pick = _select(lt[0].float(), masked, threshold=threshold, sub_block=sub_block,
                                   temperature=temperature)
            known[commit] = pick[commit]
            masked[commit] = False
        trace.steps_per_block.append(steps)
        gdn.check_kernel_status("decode block")
        new = known[have:].tolist()
        cur.extend(new)
        trace.generated += len(new)
        done = eos_id is not None and eos_id in new
        if done or nb == n_blocks - 1:
            break
        forward_segment(text_model, lm_head, cache, known[None], commit=True, logits=False)
        trace.commits += 1
    trace.tokens = cur
    return trace
