"""Host-side contract of the cached decoder (CPU: shapes, errors, cache layout; no kernel runs)."""

import pytest
import torch

from _tiny import tiny_hf_model
from dllm_qwen38_amd import decode


@pytest.fixture(scope="module")
def tiny():
    return tiny_hf_model(seed=0)


def test_prefix_cache_layout(tiny):
    m, _ = tiny
    c = decode.PrefixCache(m, batch=2, capacity=64, block=8)
    kinds = m.config.layer_types
    assert sorted(c.k) == [i for i, k in enumerate(kinds) if k == "full_attention"]
    assert sorted(c.state) == [i for i, k in enumerate(kinds) if k == "linear_attention"]
    for i in c.k:
        assert tuple(c.k[i].shape) == (2, 64, 2, 16) and c.k[i].dtype == torch.float32
    assert all(s is None for s in c.state.values()) and c.length == 0
    assert tuple(c.cos.shape) == (64, 4)  # partial rotary 0.25 of head_dim 16
    assert c.nbytes() == 2 * 2 * 64 * 2 * 16 * 4 * len(c.k)
    c4 = decode.PrefixCache(m, batch=1, capacity=16, block=8, layers=4)
    assert c4.n_layers == 4 and len(c4.kinds) == 4


def test_prefix_cache_rejects_bad_geometry(tiny):
    m, _ = tiny
    with pytest.raises(ValueError, match="multiple of block"):
        decode.PrefixCache(m, batch=1, capacity=20, block=8)
    with pytest.raises(ValueError, match="layers"):
        decode.PrefixCache(m, batch=1, capacity=16, block=8, layers=99)


def test_forward_segment_shape_errors_come_before_any_kernel(tiny):
    m, head = tiny
    c = decode.PrefixCache(m, batch=1, capacity=16, block=8)
    with torch.no_grad():
        with pytest.raises(ValueError, match="multiple of block"):
            decode.forward_segment(m, head, c, torch.zeros(1, 5, dtype=torch.long), commit=False)
        with pytest.raises(ValueError, match="capacity"):
            decode.forward_segment(m, head, c, torch.zeros(1, 24, dtype=torch.long), commit=False)
        with pytest.raises(ValueError, match=r"\[B=1, T\]"):
            decode.forward_segment(m, head, c, torch.zeros(2, 8, dtype=torch.long), commit=False)
    with pytest.raises(ValueError, match="cache must"):
        decode.generate_cached(m, head, [1, 2, 3], n_blocks=4, block=8, mask_id=255, cache=c)


def test_the_hip_path_fails_loudly_on_host_tensors(tiny):
    m, head = tiny
    c = decode.PrefixCache(m, batch=1, capacity=16, block=8)
    with pytest.raises(RuntimeError):
        decode.forward_segment(m, head, c, torch.zeros(1, 8, dtype=torch.long), commit=False)


def test_trace_tokens_per_forward():
    t = decode.DecodeTrace(tokens=[1, 2], forwards=4, generated=10)
    assert t.tokens_per_forward == 2.5 and decode.DecodeTrace(tokens=[]).tokens_per_forward == 0.0


def test_decode_linear_workgroup_rule_and_host_errors():
    from dllm_qwen38_amd import _lib

    L = _lib.lib()
    assert L.dllm_decode_linear_workgroups(32, 100, 100) == 0  # K not a multiple of 64
    assert L.dllm_decode_linear_workgroups(65, 100, 128) == 0  # more than 64 token rows
    assert L.dllm_decode_linear_workgroups(32, 151936, 5120) == 1187  # >= 512 tiles: one per workgroup
    assert L.dllm_decode_linear_workgroups(32, 5120, 5120) == 256  # one per CU, 15 units each
    assert L.dllm_decode_linear_workgroups(1, 100, 64) == 1  # one unit: one workgroup
    assert L.dllm_decode_linear_workgroups(33, 300, 320) == 3 * 2 * 5  # fewer units than CUs
    # pieces: two fp32 [32, 128] tiles per workgroup; swiglu adds the up projection's bf16 rows
    assert L.dllm_decode_linear_workspace_bytes(32, 0, 512, 0) == 512 * 2 * 32 * 128 * 4
    assert L.dllm_decode_linear_workspace_bytes(32, 17408, 512, 1) == 512 * 2 * 32 * 128 * 4 + 32 * 17408 * 2
    assert L.dllm_decode_linear_workspace_bytes(0, 0, 512, 0) == -1
    with pytest.raises(RuntimeError):
        decode.decode_linear(torch.zeros(32, 64, dtype=torch.bfloat16), torch.zeros(8, 64, dtype=torch.bfloat16))
