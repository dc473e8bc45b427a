"""Host-side contract of the block-diffusion forward (no GPU): argument checks with the reference's
wording, the fault switches, and the refusal to run anything on the CPU."""

import pytest
import torch

from _tiny import noised_ids, tiny_hf_model
from dllm_qwen38_amd import blockdiff, gdn


@pytest.fixture(scope="module")
def tiny():
    return tiny_hf_model(seed=0, layers=4)


def test_break_mode_switches():
    assert blockdiff.BreakMode().name == "none"
    assert blockdiff.BreakMode("concat-causal-gdn").concat_causal_gdn
    assert blockdiff.BreakMode("mask-leak").leak_xt_prefix
    assert blockdiff.BreakMode("no-conv-prefix").drop_conv_prefix
    m = blockdiff.BreakMode("none")
    assert not (m.concat_causal_gdn or m.leak_xt_prefix or m.drop_conv_prefix)


def test_shape_contracts_raise_value_error(tiny):
    model, lm_head = tiny
    x0, xt = noised_ids(1, 32)
    with pytest.raises(ValueError, match="must both be"):
        blockdiff.block_diffusion_forward(model, lm_head, x0, xt[:, :16], 8)
    with pytest.raises(ValueError, match="must both be"):
        blockdiff.block_diffusion_forward(model, lm_head, x0[0], xt[0], 8)
    with pytest.raises(ValueError, match="is not a multiple of block"):
        blockdiff.block_diffusion_forward(model, lm_head, x0, xt, 12)
    with pytest.raises(ValueError, match="output"):
        blockdiff.block_diffusion_forward(model, lm_head, x0, xt, 8, output="probs")


def test_cpu_tensors_fail_loudly(tiny):
    """No CPU path: the first mixer call on host tensors raises instead of computing."""
    model, lm_head = tiny
    x0, xt = noised_ids(1, 32)
    with torch.no_grad(), pytest.raises(RuntimeError, match="no CPU path"):
        blockdiff.block_diffusion_forward(model, lm_head, x0, xt, 8)


def test_grad_mode_refused(tiny):
    model, lm_head = tiny
    x0, xt = noised_ids(1, 32)
    lm_head.weight.requires_grad_(True)
    try:
        with pytest.raises(RuntimeError, match="forward-only"):
            blockdiff.block_diffusion_forward(model, lm_head, x0, xt, 8)
    finally:
        lm_head.weight.requires_grad_(False)


def test_layer_step_refuses_dense_mask(tiny):
    model, _ = tiny
    h = torch.zeros(1, 16, 64)
    step = blockdiff.LayerStep(model.layers[0], "linear_attention")
    with pytest.raises(ValueError, match="dense attention mask"):
        step(h, h, (torch.zeros(32, 4), torch.zeros(32, 4)), blockdiff.complementary_mask(16, 8, torch.float32, "cpu"), 8)


def test_set_impl_refuses_other_cores():
    with pytest.raises(RuntimeError, match="unavailable"):
        gdn.set_impl("torch")
    gdn.set_impl(None)
    gdn.set_impl("hip")
    gdn.set_impl(None)
