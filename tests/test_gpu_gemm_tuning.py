"""On MI355X the committed GEMM solution table loads (its validators match this image), and a
projection-shaped GEMM under it equals the fp32 product within the bf16 accumulation bound."""

import pytest
import torch

from dllm_qwen38_amd import gemm_tuning

pytestmark = pytest.mark.gpu


def test_table_loads_and_tuned_gemm_is_accurate():
    from torch.cuda import tunable

    try:
        assert gemm_tuning.enable() is True
        g = torch.Generator().manual_seed(4096)
        x = torch.randn(4096, 5120, generator=g).to(torch.bfloat16)
        w = (torch.randn(10240, 5120, generator=g) * 0.02).to(torch.bfloat16)
        y = torch.nn.functional.linear(x.cuda(), w.cuda()).float().cpu()  # tn_10240_4096_5120 in the table
        ref = x.float() @ w.float().T
        scale = x.float().abs() @ w.float().abs().T
        err = (y - ref).abs()
        print(f"tuned GEMM max|d|={err.max():.3e}")
        assert (err <= 2 ** -8 * ref.abs() + 2 ** -14 * scale).all()
    finally:
        tunable.enable(False)
