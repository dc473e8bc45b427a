"""Benchmark: state-fork Gated DeltaNet layer tokens/s at the 27B-class shape on one MI355X.

Workload (one step = one layer call on one batch): B=4, L=4096, block = chunk = 32 (128 noised
rows per sequence), 16 key heads / 48 value heads, d_k = d_v = 128, conv width 4, bf16 with fp32
state and accumulation; synthetic seeded inputs already resident in HBM. A step runs the two HIP
kernels of the layer: the two-stream causal conv with conv-prefix carry-in, and the fused
chunked delta rule (intra-chunk UT transform, sequential state pass with per-block fp32 state
snapshots, every noised block relaunched from its clean-prefix state).

tokens = B*L clean positions per layer call (each carries its noised twin).

Prints ONE JSON line. `roofline` is for the dominant kernel (the fused fork kernel): its
algorithmic HBM bytes per launch over its mean duration measured with HIP events on the launch
stream. `cpu_baseline` times the CPU oracle (torch fp32, all host cores of this process) on a
bounded sample of the same workload.
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "dllm-qwen38_amd"))

HBM_PEAK_GBS = 8000.0
BF16_MFMA_PEAK_TFLOPS = 2500.0


def _traffic_from_profiles():
    """HBM bytes per launch of the fork kernel from the committed PMC summary, if present."""
    p = os.path.join(ROOT, "profiles", "gdn_fork_27b_traffic.json")
    if os.path.exists(p):
        with open(p) as f:
            return json.load(f).get("bytes_per_launch")
    return None


def cpu_baseline(sample_L: int, budget_s: float):
    """The CPU oracle (torch fp32 on all host cores of this process) on one sequence of the workload
    (B=1, L=sample_L), re-run until `budget_s` seconds of CPU time have elapsed (at least 3 runs);
    median tokens/s."""
    import torch

    sys.path.insert(0, ROOT)
    from dllm_qwen38_amd import inputs
    from oracle import gdn_ref

    n = len(os.sched_getaffinity(0))
    torch.set_num_threads(n)
    s = inputs.GDN_27B_BF16
    x = inputs.gdn_layer_inputs(s, B=1, L=sample_L)
    args = (x["raw0"], x["rawt"], x["conv_w"], x["beta0"], x["betat"], x["g0"], x["gt"])
    kw = dict(Hk=s.Hk, Hv=s.Hv, Dk=s.D, Dv=s.D, block=s.block)
    gdn_ref.state_fork_layer(*args, **kw)  # warm-up
    times = []
    start = time.perf_counter()
    while len(times) < 3 or time.perf_counter() - start < budget_s:
        t = time.perf_counter()
        gdn_ref.state_fork_layer(*args, **kw)
        times.append(time.perf_counter() - t)
    med = statistics.median(times)
    return {"value": sample_L / med, "unit": "tokens/s", "cores": n, "kind": "port",
            "sample": f"one sequence (B=1 L={sample_L}) of the 27B-class shape (Hk=16 Hv=48 D=128 block 32), "
                      f"bf16-rounded inputs, fp32 torch CPU oracle on {n} threads; median of {len(times)} runs "
                      f"after 1 warm-up ({med:.2f} s/run, {sum(times):.1f} s timed)"}


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--cpu-sample-L", type=int, default=4096)
    ap.add_argument("--cpu-budget-s", type=float, default=10.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--calibration-copy-gib", type=float, default=0.0,
                    help="after the timed steps, copy this many GiB device-to-device (the reference transfer "
                         "that scales rocprofv3 FETCH_SIZE / WRITE_SIZE readings)")
    a = ap.parse_args(argv)
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: the state-fork layer shards over (batch, value head) with no "
              "exchange, and this build runs and reports the single-GPU share; use --gpus 1", file=sys.stderr)
        return 2

    import torch

    from dllm_qwen38_amd import gdn, inputs

    dev = torch.device("cuda:0")
    s = inputs.GDN_27B_BF16
    x = inputs.gdn_layer_inputs(s)
    xd = {k: v.to(dev) for k, v in x.items()}
    plan = gdn.StateForkPlan(xd["raw0"], xd["rawt"], xd["conv_w"], xd["beta0"], xd["betat"], xd["g0"], xd["gt"],
                             num_k_heads=s.Hk, num_v_heads=s.Hv, head_k_dim=s.D, head_v_dim=s.D, block=s.block)
    stream = torch.cuda.current_stream(dev)
    for _ in range(a.warmup):
        plan.run()
    torch.cuda.synchronize(dev)

    # timed region: K steps; events around each kernel on the launch stream
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True),
           torch.cuda.Event(enable_timing=True)) for _ in range(a.steps)]
    torch.cuda.synchronize(dev)
    t0 = time.perf_counter()
    for e0, e1, e2 in ev:
        e0.record(stream)
        plan.run_conv()
        e1.record(stream)
        plan.run_core()
        e2.record(stream)
    torch.cuda.synchronize(dev)
    wall = time.perf_counter() - t0
    conv_ms = [e0.elapsed_time(e1) for e0, e1, _ in ev]
    core_ms = [e1.elapsed_time(e2) for _, e1, e2 in ev]
    step_ms = ev[0][0].elapsed_time(ev[-1][2]) / a.steps
    tokens = s.B * s.L
    core_avg = sum(core_ms) / len(core_ms)
    conv_avg = sum(conv_ms) / len(conv_ms)

    Cd = s.conv_dim
    T = s.B * s.L
    core_bytes = (2 * T * Cd * 2 + 2 * T * s.Hv * 8 + 2 * T * s.Hv * s.D * 2 + (T // s.block) * s.Hv * s.D * s.D * 4)
    core_flops = gdn.layer_flops(s.B, s.L, s.Hv, s.D, s.D, s.block)
    achieved = core_bytes / (core_avg * 1e-3) / 1e9
    traffic = _traffic_from_profiles()
    res = {
        "metric": "state-fork GDN layer tokens/s at 27B-class shape; % MFMA/HBM roofline",
        "value": tokens / (step_ms * 1e-3),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": step_ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) projections, sigmoid/softplus gates, U(-0.5,0.5) conv weight)",
        "config": {"workload": "state-fork GDN layer, 27B-class: B=4 L=4096 block=chunk=32 Hk=16 Hv=48 "
                               "Dk=Dv=128 conv width 4, bf16 in/out, fp32 state", "global_batch": s.B,
                   "seq_len": s.L, "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": traffic},
        "kernels_ms": {"conv_fork": conv_avg, "gdn_state_fork": core_avg},
        "mfma": {"kernel": "gdn_state_fork", "algorithmic_tflops": core_flops / (core_avg * 1e-3) / 1e12,
                 "peak_tflops": BF16_MFMA_PEAK_TFLOPS,
                 "frac": core_flops / (core_avg * 1e-3) / 1e12 / BF16_MFMA_PEAK_TFLOPS},
        "wall_s_timed": wall,
        "cpu_baseline": None,
    }
    if a.calibration_copy_gib > 0:
        n = int(a.calibration_copy_gib * (1 << 28))
        src = torch.ones(n, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize(dev)
        del src, dst
    if not a.no_cpu_baseline:
        res["cpu_baseline"] = cpu_baseline(a.cpu_sample_L, a.cpu_budget_s)
        res["speedup_vs_cpu"] = res["value"] / res["cpu_baseline"]["value"]
    print(json.dumps(res))
    return 0


if __name__ == "__main__":
    sys.exit(main())
