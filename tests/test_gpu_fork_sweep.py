"""The state fork over a seeded spread of small shapes, against the fp32 oracle on the same inputs.

Each case draws a batch, a length of 1 to 5 blocks (a single-block sequence included), a block of
8, 16 or 32 tokens, key heads and a GQA ratio of 1 to 4, a head size of 32, 64 or 128 and bf16 or
fp32, with slow decay so that every carried state shows in the outputs. bf16 cases use the bounds
of tests/_bounds.py; fp32 cases the 1e-4 of the fp32 contract. The conv tails are bit-exact
copies of the clean input. Shapes are drawn once from a fixed seed (the list is the same on every
run) and are all shapes the C ABI accepts: the fused fork needs the block to divide 32, and fp32
heads of at most 64.
"""

import random

import pytest
import torch

from _bounds import excess, out_bound, state_bound
from dllm_qwen38_amd import gdn, inputs
from oracle import gdn_ref

pytestmark = pytest.mark.gpu


def _cases(n=16, seed=20261202):
    rng = random.Random(seed)
    out = []
    while len(out) < n:
        dtype = rng.choice([torch.bfloat16, torch.bfloat16, torch.float32])
        D = rng.choice([32, 64, 128] if dtype == torch.bfloat16 else [32, 64])
        block = rng.choice([8, 16, 32])
        B = rng.choice([1, 2, 3])
        Hk = rng.choice([1, 2, 4])
        Hv = Hk * rng.choice([1, 2, 3, 4])
        nb = rng.choice([1, 2, 3, 5])
        name = f"B{B} L{nb * block} block{block} Hk{Hk} Hv{Hv} D{D} {'bf16' if dtype == torch.bfloat16 else 'fp32'}"
        out.append(inputs.GdnShape(name, B, nb * block, block, Hk, Hv, D, 4, dtype, -4.0, 9000 + 37 * len(out)))
    return out


CASES = _cases()


@pytest.mark.parametrize("s", CASES, ids=[c.name for c in CASES])
def test_fork_sweep_matches_oracle(dev, s):
    x = inputs.gdn_layer_inputs(s)
    xd = {k: v.to(dev) for k, v in x.items()}
    r = gdn.gdn_state_fork(xd["raw0"], xd["rawt"], xd["conv_w"], xd["beta0"], xd["betat"], xd["g0"], xd["gt"],
                           num_k_heads=s.Hk, num_v_heads=s.Hv, head_k_dim=s.D, head_v_dim=s.D, block=s.block)
    torch.cuda.synchronize()
    assert gdn.last_impl()[0] == "hip"
    o0, ot, st, tails = gdn_ref.state_fork_layer(x["raw0"], x["rawt"], x["conv_w"], x["beta0"], x["betat"],
                                                 x["g0"], x["gt"], Hk=s.Hk, Hv=s.Hv, Dk=s.D, Dv=s.D, block=s.block)
    assert torch.equal(r["tails"].cpu(), tails), s.name
    assert r["states"].shape == (s.B, s.nb, s.Hv, s.D, s.D)
    for key, ref, bound in (("o0", o0, out_bound), ("ot", ot, out_bound), ("states", st, state_bound)):
        got = r[key].cpu()
        if s.dtype == torch.float32:
            d = (got.float() - ref.float()).abs().max().item()
            print(f"{s.name} {key}: max|d|={d:.2e}", flush=True)
            assert d <= 1e-4, f"{s.name} {key}: {d:.3e}"
        else:
            over, ratio = excess(got, ref, bound)
            print(f"{s.name} {key}: max |d|/bound={ratio:.3f} ({gdn.last_impl()[1]})", flush=True)
            assert over <= 0, f"{s.name} {key}: max |d|/bound = {ratio:.3f}"
