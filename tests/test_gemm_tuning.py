"""The committed GEMM solution table (PyTorch TunableOp results) parses, names the architecture and
library versions it was made with, and covers the stack's projection shapes; enable() declines
without a GPU."""

import torch

from dllm_qwen38_amd import gemm_tuning


def test_table_validators_and_stack_shapes():
    t = gemm_tuning.table_entries()
    v = t["validators"]
    assert v["GCN_ARCH_NAME"].startswith("gfx950")
    for k in ("PT_VERSION", "HIP_VERSION", "HIPBLASLT_VERSION", "ROCBLAS_VERSION"):
        assert k in v
    shapes = {shape for _, shape, _, _ in t["gemms"]}
    # hidden 5120, both streams stacked (4096 rows): in_proj qkv, MLP gate/up and down; lm_head and
    # the MLP at 2048 rows (the decoder's prefill)
    for s in ("tn_10240_4096_5120_ld_5120_5120_10240", "tn_17408_4096_5120_ld_5120_5120_17408",
              "tn_5120_4096_17408_ld_17408_17408_5120", "tn_17408_2048_5120_ld_5120_5120_17408",
              "tn_151936_2048_5120_ld_5120_5120_151936"):
        assert s in shapes
    assert all(op == "GemmTunableOp_BFloat16_TN" and ms > 0 for op, _, _, ms in t["gemms"])
    assert len(shapes) == len(t["gemms"])  # one solution per shape


def test_enable_declines_without_gpu():
    if not torch.cuda.is_available():
        assert gemm_tuning.enable() is False
