"""The allocation-free decode projection entry point against the allocating one, through the C ABI.

dllm_decode_linear_fwd_noalloc keeps the split-tile pieces in the library's fixed per-device array
instead of a caller workspace. With the same workgroup count both run the same kernels in the same
order, so their outputs must be bit-identical; calls in a row (the second smaller, then one that
splits nothing with more workgroups than the array could serve) reuse the array.
"""

import pytest
import torch

from dllm_qwen38_amd import _lib

pytestmark = pytest.mark.gpu

def _bind():
    return _lib.lib()


def _pair(L, dev, M, N, K, seed):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(M, K, generator=g) * 0.5).to(torch.bfloat16).to(dev)
    w = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16).to(dev)
    G = L.dllm_decode_linear_workgroups(M, N, K)
    assert G > 0
    ws = torch.empty(max(L.dllm_decode_linear_workspace_bytes(M, N, G, 0), 16), dtype=torch.uint8, device=dev)
    y_ref = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
    y = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=dev)
    sh = _lib.stream_handle(dev)
    print(f"decode linear M={M} N={N} K={K} workgroups={G}", flush=True)
    _lib.check(L.dllm_decode_linear_fwd(x.data_ptr(), w.data_ptr(), y_ref.data_ptr(), ws.data_ptr(), M, N, K, G,
                                        _lib.DT_BF16, sh), "dllm_decode_linear_fwd")
    _lib.check(L.dllm_decode_linear_fwd_noalloc(x.data_ptr(), w.data_ptr(), y.data_ptr(), M, N, K, G, _lib.DT_BF16,
                                                sh), "dllm_decode_linear_fwd_noalloc")
    torch.cuda.synchronize()
    ref = (x.float() @ w.float().t())
    return y, y_ref, ref


def test_noalloc_matches_the_workspace_entry_point(dev):
    L = _bind()
    assert L.dllm_decode_linear_noalloc_max_bytes() == 8 << 20
    for M, N, K, seed in ((32, 5120, 6144, 1), (32, 1024, 2048, 2), (20, 65536, 512, 3)):
        y, y_ref, ref = _pair(L, dev, M, N, K, seed)
        assert torch.equal(y, y_ref), f"M={M} N={N} K={K}: outputs differ"
        err = (y_ref.float() - ref).abs().max().item()
        assert err <= 2 ** -7 * ref.abs().max().item() + 1e-3


def test_noalloc_rejects_more_splitting_workgroups_than_the_array_holds(dev):
    L = _bind()
    # 3840 units over 300 workgroups split tiles: 300 x 32 KB of pieces exceed the 8 MiB array
    # (refused on the host, before any launch)
    x = torch.zeros(32, 6144, dtype=torch.bfloat16, device=dev)
    w = torch.zeros(5120, 6144, dtype=torch.bfloat16, device=dev)
    y = torch.zeros(32, 5120, dtype=torch.bfloat16, device=dev)
    rc = L.dllm_decode_linear_fwd_noalloc(x.data_ptr(), w.data_ptr(), y.data_ptr(), 32, 5120, 6144, 300, _lib.DT_BF16,
                                          _lib.stream_handle(dev))
    assert rc == -2
    assert "scratch" in _lib.last_error()
