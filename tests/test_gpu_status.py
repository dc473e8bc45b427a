"""Bounded waits report instead of racing: the pipelined fork's LDS row-buffer wait (its P waves
wait for the state waves to finish reading a tile's q/k rows before overwriting them) gives up
after the spin limit and sets a status bit, which dllm_status returns; the kernel still ends.

The wait is forced to give up from the host: in test mode it waits for a count the state waves
never reach, with a spin limit of 8 sleeps, so every P wave of every tile gives up. Its outputs
are then invalid (not checked); the next launch in normal mode must be exact and report nothing.
"""

import contextlib
import copy

import pytest
import torch

from _tiny import tiny_hf_model
from dllm_qwen38_amd import _lib, decode, equivalence, gdn, inputs

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


@contextlib.contextmanager
def _every_wait_gives_up():
    """Test mode: the pipelined fork's LDS wait waits for a count its state waves never reach and
    gives up after 8 sleeps, so each of its launches sets the status bit and still ends."""
    L = _lib.lib()
    prev_limit = L.dllm_set_spin_limit(8)
    L.dllm_set_wait_test_mode(1)
    try:
        yield
    finally:
        L.dllm_set_wait_test_mode(0)
        L.dllm_set_spin_limit(prev_limit)


def _wide_gdn_models(dev):
    """The tiny Qwen3.5 test model with 128-wide GDN heads (1 key, 2 value heads): its GDN layers run
    the pipelined fork kernel in bf16. Returns the fp32 CPU oracle and a bf16 device copy."""
    oracle, ohead = tiny_hf_model(seed=0, layers=4, linear_heads=(1, 2), linear_head_dim=128)
    cand, chead = copy.deepcopy(oracle).to(dev, torch.bfloat16), copy.deepcopy(ohead).to(dev, torch.bfloat16)
    oracle.to(torch.bfloat16).float()
    ohead.to(torch.bfloat16).float()
    return oracle, ohead, cand, chead


def test_equivalence_harness_raises_on_a_wait_that_gave_up(dev):
    """The harness checks the status word after every candidate forward: with the wait forced to give
    up it raises instead of comparing invalid logits; in normal mode the same call reports."""
    oracle, ohead, cand, chead = _wide_gdn_models(dev)
    kw = dict(block=32, nblocks=2, layers=None, tol=0.25, change_floor=2.5, seed=0, device=str(dev))
    assert gdn.kernel_status(reset=True) == 0
    print("harness forward with every LDS wait forced to give up", flush=True)
    with _every_wait_gives_up(), pytest.raises(RuntimeError, match="bounded wait"):
        equivalence.run(cand, chead, oracle, ohead, **kw)
    assert gdn.kernel_status() == 0  # the check reset the bit it raised on
    rep = equivalence.run(cand, chead, oracle, ohead, **kw)
    print({c["name"]: c.get("max_abs_diff", c.get("min_abs_diff")) for c in rep["checks"]})
    assert rep["checks_total"] == 5 and rep["faults_total"] == 3


def test_decoder_raises_on_a_wait_that_gave_up(dev):
    """The decoders check the status word at each block's host synchronisation. The prompt (100
    tokens: three whole blocks) makes every forward walk at least three tiles, so the pipelined
    kernel's row-buffer wait runs (a single-tile launch has none)."""
    _, _, cand, chead = _wide_gdn_models(dev)
    prompt = list(range(10, 110))
    for fn in (decode.generate, decode.generate_cached):
        print(f"{fn.__name__} with every LDS wait forced to give up", flush=True)
        with _every_wait_gives_up(), pytest.raises(RuntimeError, match="bounded wait"):
            fn(cand, chead, prompt, n_blocks=1, block=32, mask_id=255, threshold=0.0)
        assert gdn.kernel_status() == 0
        tr = fn(cand, chead, prompt, n_blocks=1, block=32, mask_id=255, threshold=0.0)
        assert tr.generated == 28
