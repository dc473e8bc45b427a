"""The benchmarked GDN layer workloads at their own sizes, against the CPU oracle.

bench.py times the 27B-class layer (B=4, L=4096, Hk=16, Hv=48, D=128, block 32) as the conv
launch then one fork launch, and the 0.8B-class layer (B=8, L=2048, Hk=Hv=16) as one launch whose
heads' value columns are split over two workgroups; `--pieces 4` times the 27B-class layer as 4
block ranges, the conv of each range beside the fork of the one before. Here each runs exactly as
the benchmark runs it (StateForkPlan, the bench's seeded inputs), and every output,
state snapshot and conv tail is compared with oracle/gdn_ref.state_fork_layer on the same inputs:
tails bit-exact, outputs and states within the bf16 bounds of tests/_bounds.py. Each workload is
checked on its own inputs (25-45 nats of decay per block at the 27B-class shape) and again with
slow decay (g shifted by -4: about 0.9 nats per block), where the state a block inherits carries
real weight and a wrong carry or fork would show.
"""

import os
import time

import pytest
import torch

from _bounds import excess, out_bound, state_bound
from dllm_qwen38_amd import gdn, inputs
from oracle import gdn_ref

pytestmark = pytest.mark.gpu


def _check(name, got, ref, bound):
    over, ratio = excess(got, ref, bound)
    d = (got.float() - ref.float()).abs()
    print(f"{name}: max|d|={d.max().item():.3e} mean|d|={d.mean().item():.3e} max|ref|={ref.float().abs().max().item():.3e} "
          f"max |d|/bound={ratio:.3f}", flush=True)
    assert over <= 0, f"{name} exceeds its bf16 bound (max |d|/bound = {ratio:.3f})"


def _run_like_bench(s, x, dev, pieces):
    xd = {k: v.to(dev) for k, v in x.items()}
    plan = gdn.StateForkPlan(xd["raw0"], xd["rawt"], xd["conv_w"], xd["beta0"], xd["betat"], xd["g0"], xd["gt"],
                             num_k_heads=s.Hk, num_v_heads=s.Hv, head_k_dim=s.D, head_v_dim=s.D, block=s.block)
    if pieces > 1:
        assert plan.overlap_supported()
        plan.run_overlapped(pieces)
    else:
        plan.run()
    torch.cuda.synchronize()
    gdn.check_kernel_status("full-size fork")
    return {k: getattr(plan, k).cpu() for k in ("o0", "ot", "states", "tails")}


CASES = [
    # (shape, schedule of the benchmark, g shift)
    (inputs.GDN_27B_BF16, 1, None),
    (inputs.GDN_27B_BF16, 4, None),
    (inputs.GDN_27B_BF16, 4, inputs.GDN_27B_BF16.g_shift - 4.0),
    (inputs.GDN_08B_BF16, 1, None),
    (inputs.GDN_08B_BF16, 1, inputs.GDN_08B_BF16.g_shift - 4.0),
]


@pytest.mark.parametrize("s,pieces,shift", CASES, ids=["27b-one-launch", "27b-4-ranges", "27b-4-ranges-slow-decay",
                                                        "08b-split", "08b-split-slow-decay"])
def test_benchmarked_layer_matches_oracle_at_full_size(dev, s, pieces, shift):
    torch.set_num_threads(len(os.sched_getaffinity(0)))
    x = inputs.gdn_layer_inputs(s, g_shift=shift)
    print(f"{s.name} shift={s.g_shift if shift is None else shift}: GPU, {pieces} range(s)", flush=True)
    r = _run_like_bench(s, x, dev, pieces)
    t = time.time()
    o0, ot, st, tails = gdn_ref.state_fork_layer(x["raw0"], x["rawt"], x["conv_w"], x["beta0"], x["betat"], x["g0"],
                                                 x["gt"], Hk=s.Hk, Hv=s.Hv, Dk=s.D, Dv=s.D, block=s.block)
    print(f"CPU oracle {time.time() - t:.1f} s", flush=True)
    assert torch.equal(r["tails"], tails), "conv tails must be bit-exact"
    _check("o0", r["o0"], o0, out_bound)
    _check("ot", r["ot"], ot, out_bound)
    _check("states", r["states"], st, state_bound)
