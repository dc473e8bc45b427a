"""Bounded waits report instead of racing: the pipelined fork's LDS row-buffer wait (its P waves
wait for the state waves to finish reading a tile's q/k rows before overwriting them) gives up
after the spin limit and sets a status bit, which dllm_status returns; the kernel still ends.

The wait is forced to give up from the host: in test mode it waits for a count the state waves
never reach, with a spin limit of 8 sleeps, so every P wave of every tile gives up. Its outputs
are then invalid (not checked); the next launch in normal mode must be exact and report nothing.
"""

import pytest
import torch

from dllm_qwen38_amd import _lib, gdn, inputs

pytestmark = pytest.mark.gpu


def test_expired_lds_wait_is_reported_and_the_kernel_ends(dev):
    s = inputs.GDN_27B_BF16
    x = {k: v.to(dev) for k, v in inputs.gdn_layer_inputs(s, B=1, L=256).items()}
    p = gdn.StateForkPlan(x["raw0"], x["rawt"], x["conv_w"], x["beta0"], x["betat"], x["g0"], x["gt"],
                          num_k_heads=s.Hk, num_v_heads=s.Hv, head_k_dim=s.D, head_v_dim=s.D, block=s.block)
    assert gdn.kernel_status(reset=True) == 0
    p.run()
    torch.cuda.synchronize()
    ref = {k: getattr(p, k).clone() for k in ("o0", "ot", "states")}
    assert gdn.kernel_status() == 0
    L = _lib.lib()
    prev_limit = L.dllm_set_spin_limit(8)
    L.dllm_set_wait_test_mode(1)
    try:
        print("fork launch with every LDS wait forced to give up", flush=True)
        p.run()
        torch.cuda.synchronize()
    finally:
        L.dllm_set_wait_test_mode(0)
        L.dllm_set_spin_limit(prev_limit)
    assert gdn.kernel_status(reset=True) == 1
    assert gdn.kernel_status() == 0
    for k in ref:
        getattr(p, k).fill_(float("nan"))
    p.run()
    torch.cuda.synchronize()
    for k, v in ref.items():
        assert torch.equal(getattr(p, k), v), k
    assert gdn.kernel_status() == 0
