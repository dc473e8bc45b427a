"""Gated DeltaNet forward with per-chunk states and the state fork, on MI355X HIP kernels.

Drop-in for the reference's `src/dllm_qwen38/gdn.py` entry points:
  chunk_gated_delta_rule_with_states (gdn.py:48-123), set_impl / last_impl (gdn.py:39-45),
  gdn_mixer_forward (gdn.py:193-233), plus the conv seam causal_conv1d_fn
  (transformers modeling_qwen3_5.py:219-239) and the fused two-stream fork op used by
  `blockdiff.block_diffusion_forward` (reference blockdiff.py:153-177).

Every core runs the hand-written gfx950 kernels of libdllm_hip.so through its C ABI. There is no
CPU or torch implementation behind these functions: a CPU tensor, a missing library or a kernel
error raises. GQA is handled by indexing the key head (value head j reads key head j // (Hv/Hk));
q/k are never expanded.
"""

from __future__ import annotations

import threading

import torch

from . import _lib, norms

# Which core the last call used and why — reports name the path they measured (gdn.py:22-24).
_IMPL = {"force": None, "last": "hip", "reason": ""}


def set_impl(name):
    """'hip' | None. The reference also accepts 'torch' / 'fla'; this package has only the HIP
    core, so forcing anything else raises (gdn.py:39-41, 158-159)."""
    if name not in (None, "hip"):
        raise RuntimeError(f"{name} forced but unavailable: this package runs the HIP core only")
    _IMPL["force"] = name


def last_impl():
    return _IMPL["last"], _IMPL["reason"]


def _fp32c(t: torch.Tensor) -> torch.Tensor:
    return t.to(torch.float32).contiguous()


def _lastdim_contig(t: torch.Tensor) -> torch.Tensor:
    return t if t.stride(-1) == 1 else t.contiguous()


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
):
    """Return (core_attn_out [B, T, Hv, Dv], states [B, n_chunks, Hv, Dk, Dv] fp32 or None).

    Same contract as the reference (gdn.py:48-123): states[:, i] is the recurrent state after
    chunk i; T must be a multiple of chunk_size (ValueError otherwise). q/k may carry Hk <= Hv
    heads (Hv % Hk == 0) in addition to the reference's already-expanded layout."""
    dev = _lib.require_device(query, key, value, g, beta, initial_state)
    if query.dim() != 4 or key.dim() != 4 or value.dim() != 4:
        raise ValueError("query/key/value must be [B, T, H, D]")
    B, T, Hk, Dk = key.shape
    Hv, Dv = value.shape[-2:]
    if query.shape != key.shape:
        raise ValueError(f"query {tuple(query.shape)} and key {tuple(key.shape)} differ")
    if value.shape[:2] != (B, T):
        raise ValueError("value must share [B, T] with key")
    if T % chunk_size != 0:
        raise ValueError(f"sequence_length {T} is not a multiple of chunk_size {chunk_size}")
    if Hv % Hk:
        raise ValueError(f"num value heads {Hv} is not a multiple of num key heads {Hk}")
    dt = query.dtype
    if key.dtype != dt or value.dtype != dt:
        raise TypeError(f"query/key/value dtypes differ ({dt}, {key.dtype}, {value.dtype})")
    code = _lib.dtype_code(dt)
    q, k, v = _lastdim_contig(query), _lastdim_contig(key), _lastdim_contig(value)
    gg, bb = _fp32c(g), _fp32c(beta)
    if gg.shape != (B, T, Hv) or bb.shape != (B, T, Hv):
        raise ValueError(f"g and beta must be [B, T, Hv] = {(B, T, Hv)}")
    init = None
    if initial_state is not None:
        if tuple(initial_state.shape) != (B, Hv, Dk, Dv):
            raise ValueError(f"initial_state must be {(B, Hv, Dk, Dv)}, got {tuple(initial_state.shape)}")
        init = _fp32c(initial_state)
    out = torch.empty(B, T, Hv, Dv, dtype=dt, device=dev)
    states = (torch.empty(B, T // chunk_size, Hv, Dk, Dv, dtype=torch.float32, device=dev)
              if need_states else None)
    if B == 0 or T == 0:
        # nothing to compute; as the reference, an empty sequence has no chunk states to stack
        # (its torch.stack of an empty list raises, gdn.py:123)
        if T == 0 and need_states:
            raise RuntimeError("chunk_gated_delta_rule_with_states: a sequence of length 0 has no chunk states")
        _IMPL["last"], _IMPL["reason"] = "hip", "empty input"
        return out, states
    L = _lib.lib()
    _lib.check(L.dllm_gdn_chunk_fwd(
        q.data_ptr(), _lib.strides3(q), k.data_ptr(), _lib.strides3(k), v.data_ptr(), _lib.strides3(v),
        gg.data_ptr(), _lib.strides3(gg), bb.data_ptr(), _lib.strides3(bb), _lib.ptr(init), out.data_ptr(),
        _lib.ptr(states), B, T, Hk, Hv, Dk, Dv, chunk_size, code, int(bool(use_qk_l2norm_in_kernel)),
        Dk ** -0.5, _lib.stream_handle(dev)), "dllm_gdn_chunk_fwd")
    _IMPL["last"], _IMPL["reason"] = "hip", ""
    return out, states


def _core(q, k, v, g, beta, *, chunk_size, initial_state, need_states):
    """Core dispatch (reference gdn.py:147-163): the HIP kernel; forcing another impl raises."""
    if _IMPL["force"] not in (None, "hip"):
        raise RuntimeError(f"{_IMPL['force']} forced but unavailable")
    return chunk_gated_delta_rule_with_states(q, k, v, g, beta, chunk_size=chunk_size, initial_state=initial_state,
                                              use_qk_l2norm_in_kernel=True, need_states=need_states)


def causal_conv1d_fn(hidden_states: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None = None,
                     activation: str | None = None, *, seq_idx=None, initial_states: torch.Tensor | None = None,
                     return_final_states: bool = False, final_states_out: torch.Tensor | None = None,
                     conv_prefix: torch.Tensor | None = None):
    """Causal depthwise conv [B, C, T] -> [B, C, T] (transformers modeling_qwen3_5.py:219-239), with
    an optional [B, C, P] prefix: equal to the conv over cat([prefix, x]) cut to the last T outputs
    (reference gdn.py:217-219). The result is a [B, C, T] view of token-major [B, T, C] storage.

    The positional parameters are those of the transformers fallback (x, weight, bias, activation).
    The causal-conv1d package's other arguments, which the seam passes by keyword, are
    keyword-only here and are honoured or refused, never dropped: `initial_states` [B, C, K-1] is the prefix under that
    package's name; `return_final_states` also returns the last K-1 inputs of the extended sequence
    ([B, C, K-1], written into `final_states_out` when given); `seq_idx` (packed sequences) is
    not supported and raises."""
    if activation not in (None, "silu", "swish"):
        raise ValueError(f"activation {activation} not supported (silu or None)")
    if seq_idx is not None:
        raise NotImplementedError("causal_conv1d_fn: seq_idx (packed sequences) is not supported")
    if initial_states is not None:
        if conv_prefix is not None:
            raise ValueError("pass the prefix once: initial_states and conv_prefix are the same argument")
        conv_prefix = initial_states
    dev = _lib.require_device(hidden_states, weight, bias, conv_prefix)
    B, C, T = hidden_states.shape
    K = weight.shape[-1]
    w = weight.reshape(C, K).contiguous()
    b = None if bias is None else bias.contiguous()
    x = hidden_states
    y = torch.empty(B, T, C, dtype=x.dtype, device=dev)
    pre = conv_prefix
    if pre is not None and (pre.shape[0] != B or pre.shape[1] != C):
        raise ValueError(f"conv_prefix must be [B, C, P] = [{B}, {C}, P], got {tuple(pre.shape)}")
    L = _lib.lib()
    if B > 0 and T > 0 and C > 0:  # an empty input has an empty output (no launch)
        _lib.check(L.dllm_causal_conv1d_fwd(
            x.data_ptr(), _lib.strides3(x), _lib.ptr(pre), None if pre is None else _lib.strides3(pre),
            0 if pre is None else pre.shape[2], w.data_ptr(), _lib.ptr(b), y.data_ptr(), B, C, T, K,
            _lib.dtype_code(x.dtype), _lib.dtype_code(w.dtype), int(activation is not None),
            _lib.stream_handle(dev)), "dllm_causal_conv1d_fwd")
    if not return_final_states:
        return y.transpose(1, 2)
    xin = x if pre is None else torch.cat([pre.to(x.dtype), x], 2)
    if xin.shape[2] < K - 1:
        xin = torch.cat([xin.new_zeros(B, C, K - 1 - xin.shape[2]), xin], 2)
    fin = xin[:, :, xin.shape[2] - (K - 1):]
    if final_states_out is not None:
        final_states_out.copy_(fin)
        fin = final_states_out
    return y.transpose(1, 2), fin


def _beta_g(m, b: torch.Tensor, a: torch.Tensor):
    """beta = sigmoid(b) rounded to the projection dtype (returned in fp32, as the core takes it);
    g = -exp(A_log) * softplus(a + dt_bias) in fp32 (reference gdn.py:225-226); one HIP kernel."""
    return norms.gdn_gates(b, a, m.A_log, m.dt_bias)


def _split_qkv(mixed: torch.Tensor, m, B: int, T: int):
    """Views (no copies) of q [B,T,Hk,Dk], k, v [B,T,Hv,Dv] inside token-major [B,T,conv_dim]."""
    kd, vd = m.key_dim, m.value_dim
    q = mixed[..., :kd].unflatten(-1, (m.num_k_heads, m.head_k_dim))
    k = mixed[..., kd: 2 * kd].unflatten(-1, (m.num_k_heads, m.head_k_dim))
    v = mixed[..., 2 * kd: 2 * kd + vd].unflatten(-1, (m.num_v_heads, m.head_v_dim))
    return q, k, v


def gdn_mixer_forward(
    m,
    hidden_states: torch.Tensor,
    *,
    chunk_size: int,
    conv_prefix: torch.Tensor | None = None,
    initial_state: torch.Tensor | None = None,
    need_states: bool = True,
):
    """Run a Qwen3.5 Gated DeltaNet module `m` on hidden_states [B, T, D] (reference gdn.py:193-233).

    conv_prefix: [B, conv_dim, K-1] pre-conv projections of the tokens before this segment, or None.
    initial_state: [B, Hv, Dk, Dv] recurrent state before the segment, or None for zeros.
    Returns (output [B, T, D], states [B, T/chunk, Hv, Dk, Dv] | None, raw_qkv [B, conv_dim, T])."""
    B, T, _ = hidden_states.shape
    raw = m.in_proj_qkv(hidden_states)  # [B, T, conv_dim]
    z = m.in_proj_z(hidden_states).reshape(B, T, -1, m.head_v_dim)
    beta, g = _beta_g(m, m.in_proj_b(hidden_states), m.in_proj_a(hidden_states))
    mixed = causal_conv1d_fn(raw.transpose(1, 2), m.conv1d.weight.squeeze(1), m.conv1d.bias,
                             activation=m.activation, conv_prefix=conv_prefix).transpose(1, 2)
    q, k, v = _split_qkv(mixed, m, B, T)
    core, states = _core(q, k, v, g, beta, chunk_size=chunk_size, initial_state=initial_state,
                         need_states=need_states)
    # the module's gated RMSNorm (Qwen3_5RMSNormGated: rmsnorm(core) * w * silu(z), [hf]:168-184) on
    # the HIP kernel, with the module's weight and epsilon
    Dv = m.head_v_dim
    eps = float(getattr(m.norm, "variance_epsilon", getattr(m.norm, "eps", 1e-6)))
    core = norms.gated_rmsnorm(core.reshape(-1, Dv), z.reshape(-1, Dv), m.norm.weight, eps).reshape(B, T, -1)
    return m.out_proj(core), states, raw.transpose(1, 2)


# ----------------------------------------------------------------------------------------------
# Fused state fork of one GDN layer (both streams)
# ----------------------------------------------------------------------------------------------
def gdn_state_fork(raw0: torch.Tensor, rawt: torch.Tensor, conv_weight: torch.Tensor,
                   beta0: torch.Tensor, betat: torch.Tensor, g0: torch.Tensor, gt: torch.Tensor, *,
                   num_k_heads: int, num_v_heads: int, head_k_dim: int, head_v_dim: int, block: int,
                   conv_bias: torch.Tensor | None = None, need_states: bool = True,
                   need_tails: bool = True, fault: str | None = None, out: dict | None = None,
                   pieces: int | None = None, vconv: bool | None = None):
    """The state-fork GDN layer core on pre-conv projections of both streams
    (reference blockdiff.py:153-177 with gdn.py:217-231, projections excluded).

    raw0/rawt [B, L, conv_dim] (token-major, the in_proj_qkv output); beta*/g* [B, L, Hv];
    conv_weight [conv_dim, K]. Returns dict(o0, ot [B, L, Hv, Dv], states [B, nb, Hv, Dk, Dv] fp32
    or None, tails [B*nb, conv_dim, K-1] or None).

    fault: None | "no-conv-prefix" (noised blocks' conv starts cold). `out` may pass preallocated
    buffers (keys o0, ot, states, tails, y0, yt) to keep the call allocation-free.

    pieces: the schedule. 1 runs the conv, then the fork, as two launches. k > 1 cuts the layer
    into k ranges of blocks: the conv of each range runs on a side stream beside the fork of the
    range before it (each fork range starts from the snapshot the one before wrote), which needs
    the pipelined fork kernel and the states. None (default) takes 4 ranges where that applies and
    the fork's grid leaves compute units free for the conv, else 1. Every schedule returns the same
    results bit for bit.

    vconv: the v channels' conv inside the fork kernel (the conv launch then convolves only the q
    and k channels, and the v channels of y0/yt are left unwritten), which saves their round trip
    through HBM. None (default) takes it where the pipelined kernel runs, there is no fault and the
    states are kept; True requires it. Results are bit-identical either way. Measured (step
    medians, interleaved): the 27B-class layer (B = 4, L = 4096) 0.740 vs 0.819 ms, the 0.8B-class
    layer (B = 8, L = 2048, a head's columns over two workgroups) 381 vs 405 us. Without the
    states the fork is bound by its tile chain rather than by its stores, so the conv's arithmetic
    costs it more than the conv launch saves (the 16-layer stack's layers, B = 1, L = 2048: fork
    258 vs 224 us, conv 19 vs 34 us)."""
    dev = _lib.require_device(raw0, rawt, conv_weight, beta0, betat, g0, gt, conv_bias)
    if raw0.shape != rawt.shape or raw0.dim() != 3:
        raise ValueError("raw0 and rawt must both be [B, L, conv_dim]")
    B, L, Cd = raw0.shape
    if L % block:
        raise ValueError(f"L={L} is not a multiple of block={block}")
    Hk, Hv, Dk, Dv = num_k_heads, num_v_heads, head_k_dim, head_v_dim
    if Cd != 2 * Hk * Dk + Hv * Dv:
        raise ValueError(f"conv_dim {Cd} != 2*Hk*Dk + Hv*Dv = {2 * Hk * Dk + Hv * Dv}")
    if fault not in (None, "no-conv-prefix"):
        raise ValueError(f"fault {fault!r} is not a fork-level fault")
    nb = L // block
    K = conv_weight.shape[-1]
    dt = raw0.dtype
    code = _lib.dtype_code(dt)
    r0, rt = raw0.contiguous(), rawt.contiguous()
    w = conv_weight.reshape(Cd, K).contiguous()
    bufs = out or {}

    def buf(name, shape, dtype):
        t = bufs.get(name)
        if t is None:
            t = torch.empty(shape, dtype=dtype, device=dev)
        elif tuple(t.shape) != tuple(shape) or t.dtype != dtype or not t.is_contiguous():
            raise ValueError(f"buffer {name} must be contiguous {shape} {dtype}")
        return t

    y0 = buf("y0", (B, L, Cd), dt)
    yt = buf("yt", (B, L, Cd), dt)
    tails = buf("tails", (B * nb, Cd, K - 1), dt) if need_tails else None
    o0 = buf("o0", (B, L, Hv, Dv), dt)
    ot = buf("ot", (B, L, Hv, Dv), dt)
    states = buf("states", (B, nb, Hv, Dk, Dv), torch.float32) if need_states else None
    b0, bt_, gg0, ggt = (_fp32c(x) for x in (beta0, betat, g0, gt))
    for name, x in (("beta0", b0), ("betat", bt_), ("g0", gg0), ("gt", ggt)):
        if tuple(x.shape) != (B, L, Hv):
            raise ValueError(f"{name} must be [B, L, Hv] = {(B, L, Hv)}")
    Lb = _lib.lib()
    sh = _lib.stream_handle(dev)
    wcode = _lib.dtype_code(w.dtype)
    cflags = 1 if fault == "no-conv-prefix" else 0
    bias = None if conv_bias is None else conv_bias.contiguous()
    # block ranges run on the pipelined kernel, which reads 16-byte rows of the conv outputs
    ranges_ok = (states is not None and nb >= 2 and Lb.dllm_gdn_state_fork_path(Dk, Dv, block, code) == 2
                 and y0.data_ptr() % 16 == 0 and yt.data_ptr() % 16 == 0)
    vc_ok = (vconv_supported(Lb, K, Dk, Dv, block, code) and fault is None
             and all(t.data_ptr() % 16 == 0 for t in (r0, rt, y0, yt)))
    if vconv is None:
        vconv = vc_ok and states is not None
    elif vconv and not vc_ok:
        raise ValueError("vconv needs the pipelined fork kernel (bf16, Dk = Dv = 128, block dividing 32), a width-4 "
                         "conv, 16-byte aligned buffers and no fault")
    vconv = bool(vconv)
    if pieces is None:
        pieces = default_pieces(_device_cus(dev), B, Hv, nb) if ranges_ok else 1
    pieces = int(pieces)
    if pieces < 1:
        raise ValueError(f"pieces={pieces} must be at least 1")
    if pieces > 1:
        if not ranges_ok:
            raise ValueError("pieces > 1 needs the pipelined fork kernel (bf16, Dk = Dv = 128), the states "
                             "and at least two blocks")
        pieces = min(pieces, nb)
        cuts = [nb * i // pieces for i in range(pieces + 1)]
        _launch_ranges(Lb, dev, cuts, (r0, rt, w, bias, y0, yt, tails, cflags),
                       (y0, yt, b0, bt_, gg0, ggt, o0, ot, states), (B, L, Cd, K, Hk, Hv, Dk, Dv, block, code),
                       vconv=vconv)
        _IMPL["last"], _IMPL["reason"] = "hip", (f"pipelined fork kernel{' with the v conv' if vconv else ''}, "
                                                 f"{pieces} block ranges beside the conv")
        return {"o0": o0, "ot": ot, "states": states, "tails": tails, "y0": y0, "yt": yt}
    if vconv:
        _launch_vconv(Lb, sh, 0, nb, (r0, rt, w, bias, y0, yt, tails),
                      (b0, bt_, gg0, ggt, o0, ot, states), (B, L, Cd, K, Hk, Hv, Dk, Dv, block, code))
        _IMPL["last"], _IMPL["reason"] = "hip", "pipelined fork kernel with the v conv"
        return {"o0": o0, "ot": ot, "states": states, "tails": tails, "y0": y0, "yt": yt}
    _lib.check(Lb.dllm_conv_fork_fwd(
        r0.data_ptr(), rt.data_ptr(), w.data_ptr(), _lib.ptr(bias), y0.data_ptr(), yt.data_ptr(),
        _lib.ptr(tails), B, L, Cd, K, block, code, wcode, cflags, sh), "dllm_conv_fork_fwd")
    if Lb.dllm_gdn_fused_fork_supported(Dk, block, code):
        _lib.check(Lb.dllm_gdn_state_fork_fwd(
            y0.data_ptr(), yt.data_ptr(), L * Cd, Cd, b0.data_ptr(), bt_.data_ptr(), gg0.data_ptr(), ggt.data_ptr(),
            o0.data_ptr(), ot.data_ptr(), _lib.ptr(states), B, L, Hk, Hv, Dk, Dv, block, code, Dk ** -0.5, sh),
            "dllm_gdn_state_fork_fwd")
        path = Lb.dllm_gdn_state_fork_path(Dk, Dv, block, code)
        _IMPL["last"], _IMPL["reason"] = "hip", _FORK_PATHS.get(path, "")
    else:
        # two-pass fork on the same HIP core: clean pass with states, then the B*nb noised rows
        # relaunched from the shifted states (reference blockdiff.py:160-176)
        class _Dims:
            key_dim, value_dim = Hk * Dk, Hv * Dv
            num_k_heads, num_v_heads, head_k_dim, head_v_dim = Hk, Hv, Dk, Dv

        q0, k0, v0 = _split_qkv(y0, _Dims, B, L)
        o0c, st0 = chunk_gated_delta_rule_with_states(q0, k0, v0, gg0, b0, block, need_states=True)
        o0.copy_(o0c)
        init = torch.cat([torch.zeros_like(st0[:, :1]), st0[:, :-1]], 1).reshape(B * nb, Hv, Dk, Dv)
        qt, kt, vt = _split_qkv(yt.view(B * nb, block, Cd), _Dims, B * nb, block)
        otc, _ = chunk_gated_delta_rule_with_states(
            qt, kt, vt, ggt.view(B * nb, block, Hv), bt_.view(B * nb, block, Hv), block, initial_state=init,
            need_states=False)
        ot.copy_(otc.view(B, L, Hv, Dv))
        if states is not None:
            states.copy_(st0)
        _IMPL["last"], _IMPL["reason"] = "hip", "two-pass fork (fused kernel does not take this shape)"
    return {"o0": o0, "ot": ot, "states": states, "tails": tails, "y0": y0, "yt": yt}


# kernel names reported through last_impl() for the fused fork (dllm_gdn_state_fork_path)
_FORK_PATHS = {2: "pipelined fork kernel", 1: "fused fork kernel"}

_CUS: dict = {}
_SIDE = threading.local()


def _device_cus(dev: torch.device) -> int:
    idx = dev.index if dev.index is not None else torch.cuda.current_device()
    if idx not in _CUS:
        _CUS[idx] = torch.cuda.get_device_properties(idx).multi_processor_count
    return _CUS[idx]


def fork_workgroups(cus: int, B: int, Hv: int) -> int:
    """Workgroups of the pipelined fork on a chip of `cus` compute units: one per (sequence, value
    head), or two (a head's columns split) when those fit in the chip, as the library's dispatch
    chooses."""
    return 2 * B * Hv if 2 * B * Hv <= cus else B * Hv


def default_pieces(cus: int, B: int, Hv: int, nb: int) -> int:
    """Block ranges of gdn_state_fork's default schedule: 1, the conv then the fork as two
    launches. Ranges (the conv of each range beside the fork of the range before) measured within
    the clock spread of it once the fork's outputs went out as 16-byte row runs: at the 27B-class
    layer (B = 4, L = 4096) four ranges 0.838-0.841 ms per step against 0.846-0.847 ms after 30
    warm-ups, and, in fresh processes after 5, 0.879-0.889 ms against 0.882-0.891 ms (interleaved,
    4 runs each), where the schedule timed first is the one the clock ramp penalises.
    At B = 1, L = 2048 (the column split) each extra range costs more than the short conv it hides
    (277 vs 241 us). `pieces` still selects ranges explicitly; every schedule is bit-identical."""
    return 1


def vconv_supported(Lb, K: int, Dk: int, Dv: int, block: int, code: int) -> bool:
    """Whether the fork kernel can take the v channels' conv: the pipelined kernel (bf16,
    Dk = Dv = 128, a block dividing 32) and a width-4 conv."""
    return K == 4 and Lb.dllm_gdn_state_fork_path(Dk, Dv, block, code) == 2


def _launch_vconv(Lb, sh, k0, k1, conv, fork, dims):
    """Blocks [k0, k1) of the layer with the v conv inside the fork: the conv launch over the q and
    k channels (their y and tails), then the fork reading the v channels' raw rows (writing their
    tails), both on stream handle `sh`."""
    r0, rt, w, bias, y0, yt, tails = conv
    b0, bt_, gg0, ggt, o0, ot, states = fork
    B, L, Cd, K, Hk, Hv, Dk, Dv, block, code = dims
    wcode = _lib.dtype_code(w.dtype)
    _lib.check(Lb.dllm_conv_fork_channels_range_fwd(
        r0.data_ptr(), rt.data_ptr(), w.data_ptr(), _lib.ptr(bias), y0.data_ptr(), yt.data_ptr(), _lib.ptr(tails),
        B, L, Cd, K, block, code, wcode, 0, k0, k1, 2 * Hk * Dk, sh), "dllm_conv_fork_channels_range_fwd")
    _lib.check(Lb.dllm_gdn_state_fork_vconv_range_fwd(
        y0.data_ptr(), yt.data_ptr(), r0.data_ptr(), rt.data_ptr(), L * Cd, Cd, w.data_ptr(), _lib.ptr(bias), wcode,
        _lib.ptr(tails), Cd, b0.data_ptr(), bt_.data_ptr(), gg0.data_ptr(), ggt.data_ptr(), o0.data_ptr(),
        ot.data_ptr(), _lib.ptr(states), B, L, Hk, Hv, Dk, Dv, block, code, Dk ** -0.5, k0, k1, sh),
        "dllm_gdn_state_fork_vconv_range_fwd")


def _side_stream(dev: torch.device) -> torch.cuda.Stream:
    """This thread's side stream on `dev` (default priority), created once."""
    streams = getattr(_SIDE, "streams", None)
    if streams is None:
        streams = _SIDE.streams = {}
    idx = dev.index if dev.index is not None else torch.cuda.current_device()
    if idx not in streams:
        streams[idx] = torch.cuda.Stream(device=idx)
    return streams[idx]


def _launch_ranges(Lb, dev, cuts, conv, fork, dims, vconv=False):
    """The layer in block ranges [cuts[i], cuts[i+1]): every conv range on this thread's side
    stream, in order, each followed by an event; each fork range on the current stream after its
    conv range's event, starting from the snapshot the range before wrote (the kernels' arithmetic
    per block does not depend on where a launch starts, so the results equal one launch's)."""
    r0, rt, w, bias, y0, yt, tails, cflags = conv
    c0, ct, b0, bt_, gg0, ggt, o0, ot, states = fork
    B, L, Cd, K, Hk, Hv, Dk, Dv, block, code = dims
    main = torch.cuda.current_stream(dev)
    side = _side_stream(dev)
    side.wait_stream(main)  # the inputs as the caller's stream leaves them
    wcode = _lib.dtype_code(w.dtype)
    events = []
    # with vconv: the conv ranges cover the q and k channels; each fork range convolves its v rows
    # (reading the three raw rows before the range) and writes their tails
    yc = 2 * Hk * Dk if vconv else Cd
    for k0, k1 in zip(cuts, cuts[1:]):
        _lib.check(Lb.dllm_conv_fork_channels_range_fwd(
            r0.data_ptr(), rt.data_ptr(), w.data_ptr(), _lib.ptr(bias), y0.data_ptr(), yt.data_ptr(), _lib.ptr(tails),
            B, L, Cd, K, block, code, wcode, cflags, k0, k1, yc, side.cuda_stream), "dllm_conv_fork_channels_range_fwd")
        ev = torch.cuda.Event()
        ev.record(side)
        events.append(ev)
    for ev, (k0, k1) in zip(events, zip(cuts, cuts[1:])):
        main.wait_event(ev)
        if vconv:
            _lib.check(Lb.dllm_gdn_state_fork_vconv_range_fwd(
                c0.data_ptr(), ct.data_ptr(), r0.data_ptr(), rt.data_ptr(), L * Cd, Cd, w.data_ptr(), _lib.ptr(bias),
                wcode, _lib.ptr(tails), Cd, b0.data_ptr(), bt_.data_ptr(), gg0.data_ptr(), ggt.data_ptr(),
                o0.data_ptr(), ot.data_ptr(), _lib.ptr(states), B, L, Hk, Hv, Dk, Dv, block, code, Dk ** -0.5, k0,
                k1, main.cuda_stream), "dllm_gdn_state_fork_vconv_range_fwd")
            continue
        _lib.check(Lb.dllm_gdn_state_fork_range_fwd(
            c0.data_ptr(), ct.data_ptr(), L * Cd, Cd, b0.data_ptr(), bt_.data_ptr(), gg0.data_ptr(), ggt.data_ptr(),
            o0.data_ptr(), ot.data_ptr(), _lib.ptr(states), B, L, Hk, Hv, Dk, Dv, block, code, Dk ** -0.5, k0, k1,
            main.cuda_stream), "dllm_gdn_state_fork_range_fwd")
    # every side-stream launch is joined into the caller's stream above; the caching allocator is
    # told of the side stream's use all the same
    for t in (r0, rt, w, bias, y0, yt, tails):
        if t is not None:
            t.record_stream(side)


def check_kernel_status(where: str) -> None:
    """Raise RuntimeError when a bounded wait inside a kernel gave up since the last check (the
    outputs of the launches since then are invalid); resets the bits. Synchronises the device, so
    callers place it where they synchronise anyway."""
    st = kernel_status(reset=True)
    if st:
        raise RuntimeError(f"{where}: a bounded wait inside a HIP kernel gave up (status bits {st:#x}); the outputs "
                           "of the launches since the last status check are invalid")


def kernel_status(reset: bool = True) -> int:
    """Bits set by bounded waits inside kernels that gave up since the last reset (0 = none), after
    a device synchronisation: 1 = the pipelined fork's LDS row-buffer wait. A set bit means the
    launch that set it produced invalid outputs."""
    st = _lib.lib().dllm_status(int(bool(reset)))
    if st < 0:
        raise RuntimeError(f"dllm_status failed: {_lib.last_error()}")
    return st


def fork_layout(B: int, L: int, block: int, width: int = 4, device="cuda"):
    """Integer fork maps computed on the device by the kernels' own index functions
    (reference blockdiff.py:161-173): row [B, nb], state_src [B*nb], prefix_pos [B*nb, width-1]."""
    if L % block:
        raise ValueError(f"L={L} is not a multiple of block={block}")
    nb = L // block
    dev = torch.device(device)
    row = torch.empty(B * nb, dtype=torch.int32, device=dev)
    src = torch.empty(B * nb, dtype=torch.int32, device=dev)
    pre = torch.empty(B * nb, max(width - 1, 1), dtype=torch.int32, device=dev)
    _lib.require_device(row)
    _lib.check(_lib.lib().dllm_fork_layout(B, L, block, width, row.data_ptr(), src.data_ptr(), pre.data_ptr(),
                                           _lib.stream_handle(dev)), "dllm_fork_layout")
    return {"row": row.view(B, nb), "state_src": src, "prefix_pos": pre[:, : width - 1]}


def layer_flops(B: int, L: int, Hv: int, Dk: int, Dv: int, chunk: int) -> int:
    """Algorithmic flops of the state-fork layer's chunk contractions (both streams): per chunk and
    value head 6*C*Dk*Dv + 8*C^2*Dk (clean) and 4*C*Dk*Dv + 8*C^2*Dk (noised)."""
    C = chunk
    per = (6 * C * Dk * Dv + 8 * C * C * Dk) + (4 * C * Dk * Dv + 8 * C * C * Dk)
    return (B * L // C) * Hv * per


def layer_bytes(B: int, L: int, Hk: int, Hv: int, Dk: int, Dv: int, chunk: int, esize: int = 2, K: int = 4) -> int:
    """Algorithmic HBM bytes of the layer op (inputs read once, outputs written once): raw qkv of both
    streams, beta (input dtype) and g (fp32) of both streams, both outputs, the per-chunk fp32
    states and the conv tails."""
    Cd = 2 * Hk * Dk + Hv * Dv
    T = B * L
    raw = 2 * T * Cd * esize
    bg = 2 * T * Hv * (esize + 4)
    o = 2 * T * Hv * Dv * esize
    states = (T // chunk) * Hv * Dk * Dv * 4
    tails = (T // chunk) * Cd * (K - 1) * esize
    return raw + bg + o + states + tails



class StateForkPlan:
    """Pre-validated, pre-allocated state-fork layer launches for repeated calls on fixed shapes
    (benchmarks, serving loops): run() enqueues the conv kernel and the fused fork kernel on the
    current stream with no allocation and no host synchronisation. Inputs are the tensors given
    at construction (their contents may be rewritten between runs)."""

    def __init__(self, raw0, rawt, conv_weight, beta0, betat, g0, gt, *, num_k_heads, num_v_heads, head_k_dim,
                 head_v_dim, block, need_states=True, need_tails=True, vconv=None):
        dev = _lib.require_device(raw0, rawt, conv_weight, beta0, betat, g0, gt)
        B, L, Cd = raw0.shape
        self.dims = (B, L, Cd, num_k_heads, num_v_heads, head_k_dim, head_v_dim, block)
        self.code = _lib.dtype_code(raw0.dtype)
        if not _lib.lib().dllm_gdn_fused_fork_supported(head_k_dim, block, self.code):
            raise ValueError("StateForkPlan needs a shape the fused fork kernel takes")
        if not (raw0.is_contiguous() and rawt.is_contiguous()):
            raise ValueError("raw0/rawt must be contiguous [B, L, conv_dim]")
        self.raw0, self.rawt = raw0, rawt
        self.w = conv_weight.reshape(Cd, -1).contiguous()
        self.beta0, self.betat, self.g0, self.gt = (_fp32c(x) for x in (beta0, betat, g0, gt))
        dt = raw0.dtype
        nb = L // block
        K = self.w.shape[1]
        self.K = K
        self.y0 = torch.empty(B, L, Cd, dtype=dt, device=dev)
        self.yt = torch.empty(B, L, Cd, dtype=dt, device=dev)
        self.tails = torch.empty(B * nb, Cd, K - 1, dtype=dt, device=dev) if need_tails else None
        self.o0 = torch.empty(B, L, num_v_heads, head_v_dim, dtype=dt, device=dev)
        self.ot = torch.empty_like(self.o0)
        self.states = (torch.empty(B, nb, num_v_heads, head_k_dim, head_v_dim, dtype=torch.float32, device=dev)
                       if need_states else None)
        self.device = dev
        self._lib = _lib.lib()
        # the v channels' conv inside the fork (gdn_state_fork's vconv): None takes it where supported
        # and the states are kept
        ok = (vconv_supported(self._lib, K, head_k_dim, head_v_dim, block, self.code)
              and raw0.data_ptr() % 16 == 0 and rawt.data_ptr() % 16 == 0)
        if vconv is None:
            vconv = ok and need_states
        elif vconv and not ok:
            raise ValueError("vconv needs the pipelined fork kernel (bf16, Dk = Dv = 128) and a width-4 conv")
        self.vconv = bool(vconv)

    def run_conv(self, stream=None):
        B, L, Cd, Hk, Hv, Dk, Dv, block = self.dims
        sh = stream if stream is not None else _lib.stream_handle(self.device)
        if self.vconv:  # the q and k channels only; the fork convolves the v channels
            _lib.check(self._lib.dllm_conv_fork_channels_range_fwd(
                self.raw0.data_ptr(), self.rawt.data_ptr(), self.w.data_ptr(), None, self.y0.data_ptr(),
                self.yt.data_ptr(), _lib.ptr(self.tails), B, L, Cd, self.K, block, self.code,
                _lib.dtype_code(self.w.dtype), 0, 0, L // block, 2 * Hk * Dk, sh), "dllm_conv_fork_channels_range_fwd")
            return
        _lib.check(self._lib.dllm_conv_fork_fwd(
            self.raw0.data_ptr(), self.rawt.data_ptr(), self.w.data_ptr(), None, self.y0.data_ptr(),
            self.yt.data_ptr(), _lib.ptr(self.tails), B, L, Cd, self.K, block, self.code,
            _lib.dtype_code(self.w.dtype), 0, sh), "dllm_conv_fork_fwd")

    def run_core(self, stream=None):
        B, L, Cd, Hk, Hv, Dk, Dv, block = self.dims
        sh = stream if stream is not None else _lib.stream_handle(self.device)
        if self.vconv:
            _lib.check(self._lib.dllm_gdn_state_fork_vconv_range_fwd(
                self.y0.data_ptr(), self.yt.data_ptr(), self.raw0.data_ptr(), self.rawt.data_ptr(), L * Cd, Cd,
                self.w.data_ptr(), None, _lib.dtype_code(self.w.dtype), _lib.ptr(self.tails), Cd,
                self.beta0.data_ptr(),
                self.betat.data_ptr(), self.g0.data_ptr(), self.gt.data_ptr(), self.o0.data_ptr(),
                self.ot.data_ptr(), _lib.ptr(self.states), B, L, Hk, Hv, Dk, Dv, block, self.code, Dk ** -0.5, 0,
                L // block, sh), "dllm_gdn_state_fork_vconv_range_fwd")
            return
        _lib.check(self._lib.dllm_gdn_state_fork_fwd(
            self.y0.data_ptr(), self.yt.data_ptr(), L * Cd, Cd, self.beta0.data_ptr(), self.betat.data_ptr(),
            self.g0.data_ptr(), self.gt.data_ptr(), self.o0.data_ptr(), self.ot.data_ptr(), _lib.ptr(self.states),
            B, L, Hk, Hv, Dk, Dv, block, self.code, Dk ** -0.5, sh), "dllm_gdn_state_fork_fwd")

    def run(self, stream=None):
        self.run_conv(stream)
        self.run_core(stream)
        _IMPL["last"], _IMPL["reason"] = "hip", ""

    def overlap_supported(self):
        """Whether run_overlapped can split this plan's layer (the pipelined fork path, states kept)."""
        B, L, Cd, Hk, Hv, Dk, Dv, block = self.dims
        return (self.states is not None and L // block >= 2
                and self._lib.dllm_gdn_state_fork_path(Dk, Dv, block, self.code) == 2)

    def run_overlapped(self, pieces=4, bounds=None):
        """The layer cut into `pieces` ranges of blocks (or at the given block boundaries, e.g.
        [0, 16, 64, 128]): the conv of each range runs on a side stream while the fork of the range
        before it runs on the caller's stream, which waits for each range's conv by an event; each
        fork range starts from the snapshot the one before it wrote. The results equal run()'s bit
        for bit. Enqueued on the current stream."""
        if not self.overlap_supported():
            raise ValueError("run_overlapped needs the pipelined fork path with states")
        B, L, Cd, Hk, Hv, Dk, Dv, block = self.dims
        nb = L // block
        if bounds is not None:
            cuts = [int(c) for c in bounds]
            if cuts[0] != 0 or cuts[-1] != nb or any(b <= a for a, b in zip(cuts, cuts[1:])):
                raise ValueError(f"bounds must rise from 0 to {nb}")
        else:
            pieces = max(1, min(int(pieces), nb))
            cuts = [nb * i // pieces for i in range(pieces + 1)]
        _launch_ranges(self._lib, self.device, cuts,
                       (self.raw0, self.rawt, self.w, None, self.y0, self.yt, self.tails, 0),
                       (self.y0, self.yt, self.beta0, self.betat, self.g0, self.gt, self.o0, self.ot, self.states),
                       (B, L, Cd, self.K, Hk, Hv, Dk, Dv, block, self.code), vconv=self.vconv)
        _IMPL["last"], _IMPL["reason"] = "hip", ""
