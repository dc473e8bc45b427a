"""ctypes binding of libdllm_hip.so (the C ABI declared in include/dllm_hip.h).

The library must have been built in-tree (`dllm_qwen38_amd._build.build()`); a missing library
raises immediately — there is no fallback implementation behind these entry points.
"""

from __future__ import annotations

import ctypes
import os

import torch

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libdllm_hip.so")

DT_F32 = 0
DT_BF16 = 1

_c_void_p = ctypes.c_void_p
_c_int = ctypes.c_int
_c_float = ctypes.c_float
_c_i64 = ctypes.c_int64
_c_i64p = ctypes.POINTER(ctypes.c_int64)
_c_voidpp = ctypes.POINTER(ctypes.c_void_p)
_c_intp = ctypes.POINTER(ctypes.c_int)
_c_fp = ctypes.c_void_p

# name -> (restype, argtypes)
_SIGNATURES = {
    "dllm_abi_version": (_c_int, []),
    "dllm_last_error": (ctypes.c_char_p, []),
    "dllm_gdn_chunk_fwd": (_c_int, [
        _c_void_p, _c_i64p, _c_void_p, _c_i64p, _c_void_p, _c_i64p, _c_fp, _c_i64p, _c_void_p, _c_i64p,
        _c_fp, _c_void_p, _c_fp, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int,
        _c_float, _c_void_p]),
    "dllm_gdn_fused_fork_supported": (_c_int, [_c_int, _c_int, _c_int]),
    "dllm_gdn_state_fork_path": (_c_int, [_c_int, _c_int, _c_int, _c_int]),
    "dllm_set_spin_limit": (_c_int, [_c_int]),
    "dllm_set_fork_split": (_c_int, [_c_int]),
    "dllm_status": (_c_int, [_c_int]),
    "dllm_set_wait_test_mode": (_c_int, [_c_int]),
    "dllm_gdn_state_fork_fwd": (_c_int, [
        _c_void_p, _c_void_p, _c_i64, _c_i64, _c_void_p, _c_void_p, _c_fp, _c_fp, _c_void_p, _c_void_p,
        _c_fp, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_float, _c_void_p]),
    "dllm_gdn_state_fork_range_fwd": (_c_int, [
        _c_void_p, _c_void_p, _c_i64, _c_i64, _c_void_p, _c_void_p, _c_fp, _c_fp, _c_void_p, _c_void_p,
        _c_fp, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_float, _c_int, _c_int,
        _c_void_p]),
    "dllm_gdn_state_fork_vconv_range_fwd": (_c_int, [
        _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_i64, _c_i64, _c_void_p, _c_void_p, _c_int, _c_void_p,
        _c_int, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_fp, _c_int, _c_int,
        _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_float, _c_int, _c_int, _c_void_p]),
    "dllm_conv_fork_channels_range_fwd": (_c_int, [
        _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_int, _c_int, _c_int,
        _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_void_p]),
    "dllm_conv_fork_fwd": (_c_int, [
        _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_int, _c_int, _c_int,
        _c_int, _c_int, _c_int, _c_int, _c_int, _c_void_p]),
    "dllm_conv_fork_range_fwd": (_c_int, [
        _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_int, _c_int, _c_int,
        _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_void_p]),
    "dllm_causal_conv1d_fwd": (_c_int, [
        _c_void_p, _c_i64p, _c_void_p, _c_i64p, _c_int, _c_void_p, _c_void_p, _c_void_p, _c_int, _c_int,
        _c_int, _c_int, _c_int, _c_int, _c_int, _c_void_p]),
    "dllm_fork_layout": (_c_int, [_c_int, _c_int, _c_int, _c_int, _c_void_p, _c_void_p, _c_void_p, _c_void_p]),
    "dllm_rmsnorm_fwd": (_c_int, [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_int, _c_int, _c_float,
                                  _c_int, _c_int, _c_int, _c_void_p]),
    "dllm_gated_rmsnorm_fwd": (_c_int, [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_int, _c_int, _c_float, _c_int,
                                        _c_int, _c_void_p]),
    "dllm_swiglu_fwd": (_c_int, [_c_void_p, _c_void_p, _c_void_p, _c_i64, _c_int, _c_void_p]),
    "dllm_swiglu_rows_fwd": (_c_int, [_c_void_p, _c_void_p, _c_i64, _c_void_p, _c_i64, _c_i64, _c_int, _c_void_p]),
    "dllm_qk_norm_rope_fwd": (_c_int, [
        _c_void_p, _c_i64p, _c_void_p, _c_i64p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
        _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_float, _c_int, _c_int, _c_void_p]),
    "dllm_bd_attention_fwd": (_c_int, [
        _c_void_p, _c_i64p, _c_void_p, _c_i64p, _c_void_p, _c_i64p, _c_void_p, _c_int, _c_int, _c_int, _c_int,
        _c_int, _c_int, _c_float, _c_int, _c_int, _c_void_p]),
    "dllm_bd_attention_gated_supported": (_c_int, [_c_int, _c_int, _c_int]),
    "dllm_bd_attention_gated_fwd": (_c_int, [
        _c_void_p, _c_i64p, _c_void_p, _c_i64p, _c_void_p, _c_i64p, _c_void_p, _c_i64p, _c_void_p, _c_int,
        _c_float, _c_void_p, _c_void_p, _c_int, _c_void_p, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_float,
        _c_int, _c_int, _c_void_p]),
    "dllm_decode_linear_workgroups": (_c_int, [_c_int, _c_int, _c_int]),
    "dllm_decode_linear_workspace_bytes": (_c_i64, [_c_int, _c_int, _c_int, _c_int]),
    "dllm_decode_linear_fwd": (_c_int, [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_int, _c_int, _c_int, _c_int,
                                        _c_int, _c_void_p]),
    "dllm_decode_linear_noalloc_max_bytes": (_c_i64, []),
    "dllm_decode_linear_fwd_noalloc": (_c_int, [_c_void_p, _c_void_p, _c_void_p, _c_int, _c_int, _c_int, _c_int, _c_int,
                                                _c_void_p]),
    "dllm_decode_linear_multi_fwd": (_c_int, [_c_void_p, _c_int, _c_int, _c_int, _c_voidpp, _c_voidpp, _c_intp,
                                              _c_void_p, _c_int, _c_int, _c_int, _c_void_p]),
    "dllm_decode_linear_rmsnorm_fwd": (_c_int, [
        _c_void_p, _c_void_p, _c_void_p, _c_int, _c_int, _c_int, _c_int, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
        _c_float, _c_int, _c_int, _c_int, _c_void_p]),
    "dllm_decode_gdn_prologue_fwd": (_c_int, [
        _c_void_p, _c_int, _c_int, _c_voidpp, _c_voidpp, _c_intp, _c_void_p, _c_int, _c_int, _c_void_p, _c_int,
        _c_void_p, _c_void_p, _c_int, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_int, _c_int, _c_int,
        _c_void_p]),
    "dllm_gdn_gates_fwd": (_c_int, [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_i64, _c_int,
                                    _c_int, _c_int, _c_void_p]),
    "dllm_block_causal_attention_fwd": (_c_int, [
        _c_void_p, _c_i64p, _c_void_p, _c_i64p, _c_void_p, _c_i64p, _c_void_p, _c_int, _c_int, _c_int, _c_int,
        _c_int, _c_int, _c_int, _c_int, _c_float, _c_int, _c_void_p, _c_int, _c_void_p]),
    "dllm_block_causal_attention_gated_fwd": (_c_int, [
        _c_void_p, _c_i64p, _c_void_p, _c_i64p, _c_void_p, _c_i64p, _c_void_p, _c_i64p, _c_void_p, _c_int, _c_int,
        _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_float, _c_int, _c_void_p, _c_int, _c_void_p]),
}

_LIB = None


class HipLibraryMissing(RuntimeError):
    pass


def lib() -> ctypes.CDLL:
    """Load (once) and return the library with argtypes bound for every known entry point."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise HipLibraryMissing(
                f"{LIB_PATH} is not built; run __graft_entry__.build() (hipcc --offload-arch=gfx950)")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(L, name, None)
            if fn is None:
                continue
            fn.restype = res
            fn.argtypes = args
        _LIB = L
    return _LIB


def last_error() -> str:
    return lib().dllm_last_error().decode(errors="replace")


def check(status: int, what: str) -> None:
    if status != 0:
        raise RuntimeError(f"{what} failed (status {status}): {last_error()}")


def dtype_code(dt: torch.dtype) -> int:
    if dt == torch.float32:
        return DT_F32
    if dt == torch.bfloat16:
        return DT_BF16
    raise TypeError(f"unsupported dtype {dt} (float32 or bfloat16)")


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def strides3(t: torch.Tensor, dims=(0, 1, 2)):
    """int64[3] host array of element strides for the given dims."""
    arr = (ctypes.c_int64 * 3)(*(int(t.stride(d)) for d in dims))
    return arr


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_handle(device: torch.device) -> int:
    """hipStream_t of the device's current stream: torch's accessor of the raw handle (the value of
    torch.cuda.current_stream(device).cuda_stream without building a Stream object, a measurable
    share of a decoding step's ~240 launches from the host)."""
    if _raw_stream is not None:
        return _raw_stream(device.index if device.index is not None else torch.cuda.current_device())
    return torch.cuda.current_stream(device).cuda_stream


def require_device(*ts: torch.Tensor | None) -> torch.device:
    """All given tensors must live on one ROCm device; returns it. CPU tensors are an error: the
    product path has no CPU implementation."""
    idx = None
    for t in ts:
        if t is None:
            continue
        if not t.is_cuda:
            raise RuntimeError(
                f"the HIP kernels need ROCm device tensors (got a tensor on {t.device}); this library "
                "has no CPU path")
        i = t.get_device()
        if idx is None:
            idx = i
        elif i != idx:
            raise RuntimeError(f"tensors on different devices: cuda:{idx} and cuda:{i}")
    if idx is None:
        raise RuntimeError("no device tensor given")
    return _device(idx)


_DEVICES: dict = {}


def _device(idx: int) -> torch.device:
    d = _DEVICES.get(idx)
    if d is None:
        d = _DEVICES[idx] = torch.device("cuda", idx)
    return d
