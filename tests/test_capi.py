"""The C-ABI library loads on the host and exports every entry point the header declares
(host-side checks only: no kernel is launched here)."""

import ctypes
import os
import re

from dllm_qwen38_amd import _lib

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "dllm_hip.h")


def _declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(dllm_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_entry_points():
    names = _declared()
    for n in ("dllm_gdn_chunk_fwd", "dllm_gdn_state_fork_fwd", "dllm_conv_fork_fwd", "dllm_causal_conv1d_fwd",
              "dllm_fork_layout", "dllm_last_error", "dllm_abi_version"):
        assert n in names


def test_library_exports_every_declared_symbol():
    lib = _lib.lib()
    missing = [n for n in _declared() if not hasattr(lib, n)]
    assert missing == []
    for n in _declared():
        assert n in _lib._SIGNATURES, f"{n} has no ctypes signature"


def test_abi_version_and_host_side_queries():
    lib = _lib.lib()
    assert lib.dllm_abi_version() == 1
    assert lib.dllm_gdn_fused_fork_supported(128, 32, _lib.DT_BF16) == 1
    assert lib.dllm_gdn_fused_fork_supported(64, 32, _lib.DT_F32) == 1
    assert lib.dllm_gdn_fused_fork_supported(128, 32, _lib.DT_F32) == 0
    assert lib.dllm_gdn_fused_fork_supported(128, 64, _lib.DT_BF16) == 0
    assert lib.dllm_gdn_fused_fork_supported(128, 24, _lib.DT_BF16) == 0


def test_argument_validation_fails_before_any_launch():
    lib = _lib.lib()
    one = (ctypes.c_int64 * 3)(1, 1, 1)
    st = lib.dllm_gdn_chunk_fwd(1, one, 1, one, 1, one, 1, one, 1, one, None, 1, None, 1, 100, 1, 1, 64, 64, 32,
                                _lib.DT_F32, 1, 0.125, None)
    assert st == -1
    assert "sequence_length 100 is not a multiple of chunk_size 32" in _lib.last_error()
    st = lib.dllm_conv_fork_fwd(None, None, None, None, None, None, None, 1, 32, 8, 4, 32, 0, 0, 0, None)
    assert st == -1 and "null pointer" in _lib.last_error()
    st = lib.dllm_fork_layout(1, 33, 32, 4, 1, 1, 1, None)
    assert st == -1 and "not a multiple of block" in _lib.last_error()


def test_swiglu_rows_and_decode_linear_validate_before_any_launch():
    lib = _lib.lib()
    st = lib.dllm_swiglu_rows_fwd(None, None, 16, None, 1, 8, _lib.DT_BF16, None)
    assert st == -1 and "null pointer" in _lib.last_error()
    st = lib.dllm_swiglu_rows_fwd(16, 32, 4, 64, 1, 8, _lib.DT_BF16, None)  # ld < cols
    assert st == -1 and "bad sizes" in _lib.last_error()
    st = lib.dllm_swiglu_rows_fwd(16, 32, 12, 64, 1, 12, _lib.DT_BF16, None)  # cols not a multiple of 8
    assert st == -1 and "16-byte vectors" in _lib.last_error()
    w = (ctypes.c_void_p * 1)(16)
    o = (ctypes.c_void_p * 1)(16)
    n = (ctypes.c_int * 1)(128)
    st = lib.dllm_decode_linear_multi_fwd(16, 32, 128, 1, w, o, n, None, 4, 0, _lib.DT_BF16, None)
    assert st == -1 and "workspace" in _lib.last_error()
    st = lib.dllm_decode_linear_multi_fwd(16, 65, 128, 1, w, o, n, 16, 4, 0, _lib.DT_BF16, None)
    assert st == -2 and "64 rows" in _lib.last_error()


def test_fork_path_query():
    lib = _lib.lib()
    assert lib.dllm_gdn_state_fork_path(128, 128, 32, _lib.DT_BF16) == 2
    assert lib.dllm_gdn_state_fork_path(128, 128, 8, _lib.DT_BF16) == 2
    assert lib.dllm_gdn_state_fork_path(64, 64, 32, _lib.DT_BF16) == 1
    assert lib.dllm_gdn_state_fork_path(64, 64, 32, _lib.DT_F32) == 1
    assert lib.dllm_gdn_state_fork_path(128, 128, 64, _lib.DT_BF16) == 0


def test_spin_limit_setter():
    lib = _lib.lib()
    assert lib.dllm_set_spin_limit(-1) == -1
    prev = lib.dllm_set_spin_limit(1000)
    assert lib.dllm_set_spin_limit(prev) == 1000
