"""Benchmark: state-fork Gated DeltaNet layer tokens/s at the 27B-class shape on one MI355X.

Workload (one step = one layer call on one batch): B=4, L=4096, block = chunk = 32 (128 noised
rows per sequence), 16 key heads / 48 value heads, d_k = d_v = 128, conv width 4, bf16 with fp32
state and accumulation; synthetic seeded inputs already resident in HBM. A step runs the two HIP
kernels of the layer: the two-stream causal conv of the q and k channels with conv-prefix
carry-in, and the fused chunked delta rule, which convolves the v channels itself as their rows
arrive (intra-chunk UT transform, sequential state pass with per-block fp32 state snapshots,
every noised block relaunched from its clean-prefix state).

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


def _calibration_copy(a, dev):
    """With --calibration-copy-gib G: one device-to-device copy of G GiB after the timed steps, the
    known-size kernel that PMC traffic counts are scaled by."""
    import torch

    if a.calibration_copy_gib > 0:
        n = int(a.calibration_copy_gib * (1 << 28))
        src = torch.ones(n, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize(dev)
        del src, dst


def _traffic_from_profiles(name):
    """HBM bytes per launch of the dominant kernel from a committed PMC summary, if present."""
    p = os.path.join(ROOT, "profiles", name)
    if os.path.exists(p):
        with open(p) as f:
            return json.load(f).get("bytes_per_launch")
    return None


def cpu_baseline(s, sample_L: int, budget_s: float):
    """The CPU oracle (torch fp32 on all host cores of this process) on one sequence of the workload
    (B=1, L=sample_L), re-run until `budget_s` seconds of CPU time have elapsed (at least 3 runs);
    median tokens/s."""
    import torch

    sys.path.insert(0, ROOT)
    from dllm_qwen38_amd import inputs
    from oracle import gdn_ref

    n = len(os.sched_getaffinity(0))
    torch.set_num_threads(n)
    x = inputs.gdn_layer_inputs(s, B=1, L=sample_L)
    args = (x["raw0"], x["rawt"], x["conv_w"], x["beta0"], x["betat"], x["g0"], x["gt"])
    kw = dict(Hk=s.Hk, Hv=s.Hv, Dk=s.D, Dv=s.D, block=s.block)
    ref = gdn_ref.state_fork_layer(*args, **kw)  # warm-up
    times = []
    start = time.perf_counter()
    while len(times) < 3 or time.perf_counter() - start < budget_s:
        t = time.perf_counter()
        gdn_ref.state_fork_layer(*args, **kw)
        times.append(time.perf_counter() - t)
    med = statistics.median(times)
    return {"value": sample_L / med, "unit": "tokens/s", "cores": n, "kind": "port",
            "sample": f"one sequence (B=1 L={sample_L}) of the workload's shape (Hk={s.Hk} Hv={s.Hv} D={s.D} "
                    f"block {s.block}): the workload's own sequence 0, bf16-rounded inputs, fp32 torch CPU oracle "
                    f"on {n} threads; median of {len(times)} runs after 1 warm-up ({med:.2f} s/run, min "
                    f"{min(times):.2f} s, {sum(times):.1f} s timed)",
            **_host_info()}, (x, ref)


def _err_stats(got, ref, bound):
    """max / mean / 99th and 99.9th percentile of |got - ref|, and the largest |d| / bound."""
    import torch

    d = (got.float() - ref.float()).abs().flatten()
    n = d.numel()
    q = lambda f: d.kthvalue(max(1, min(n, int(round(f * n))))).values.item()
    return {"max": d.max().item(), "mean": d.mean().item(), "p99": q(0.99), "p999": q(0.999),
            "max_over_bound": (d / bound(ref).flatten()).max().item(), "max_ref": ref.float().abs().max().item()}


def parity_sample(plan, s, sample, f64_heads: int = 8):
    """The GPU outputs of sequence 0 against the CPU oracle run on the same inputs (the cpu_baseline
    sample is the workload's own sequence 0), with the error distribution: both output streams and
    every state snapshot against the fp32 oracle, and the clean stream's outputs and snapshots of the
    first `f64_heads` value heads against the float64 token recurrence. The bound of each figure is
    the tests' bf16 bound (outputs 2^-6 max|ref| + 2^-7 |ref|, fp32 states 2^-7 max|ref|); a
    max_over_bound at or below 1 is within it."""
    import torch

    sys.path.insert(0, ROOT)
    from oracle import gdn_ref

    u = 2.0 ** -8
    out_b = lambda r: 4 * u * r.float().abs().max() + 2 * u * r.float().abs()
    st_b = lambda r: (2 * u * r.float().abs().max()).expand_as(r.float())
    x, (o0, ot, st, _) = sample
    Ls = o0.shape[1]
    g0, gt, gs = plan.o0[:1, :Ls].cpu(), plan.ot[:1, :Ls].cpu(), plan.states[:1, :Ls // s.block].cpu()
    res = {"sample": f"sequence 0, L={Ls}, all {s.Hv} value heads, against the fp32 CPU oracle; clean stream heads "
                     f"0-{f64_heads - 1} against the float64 token recurrence",
           "o0": _err_stats(g0, o0, out_b), "ot": _err_stats(gt, ot, out_b), "states": _err_stats(gs, st, st_b)}
    y = gdn_ref.causal_conv1d(x["raw0"].transpose(1, 2), x["conv_w"]).transpose(1, 2)
    q, k, v = gdn_ref._split_heads(y, 1, Ls, s.Hk, s.Hv, s.D, s.D)
    hs = slice(0, f64_heads)
    fo, fs = gdn_ref.recurrent_gated_delta_rule_f64(q[:, :, hs], k[:, :, hs], v[:, :, hs], x["g0"][:, :, hs],
                                                    x["beta0"][:, :, hs], chunk_size=s.block)
    fo, fs = torch.from_numpy(fo), torch.from_numpy(fs)
    res["o0_vs_f64"] = _err_stats(g0[:, :, hs], fo, out_b)
    res["states_vs_f64"] = _err_stats(gs[:, :, hs], fs, st_b)
    res["oracle_o0_vs_f64_max"] = (o0[:, :, hs].float() - fo.float()).abs().max().item()
    return res


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=30)
    ap.add_argument("--cpu-sample-L", type=int, default=4096)
    ap.add_argument("--cpu-budget-s", type=float, default=10.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--calibration-copy-gib", type=float, default=0.0,
                    help="after the timed steps, copy this many GiB device-to-device (the reference transfer "
                         "that scales rocprofv3 FETCH_SIZE / WRITE_SIZE readings)")
    ap.add_argument("--pieces", type=int, default=None,
                    help="GDN layer workloads: the step's schedule, the layer cut into this many block ranges "
                         "with the conv of each range beside the fork of the one before (default 1: conv, then "
                         "fork, as gdn_state_fork's default; ranges measured no faster)")
    ap.add_argument("--workload", default="gdn-layer",
                    choices=["gdn-layer", "gdn-layer-08b", "gdn-core", "attention", "stack", "decode"],
                    help="gdn-layer (default, the headline metric); gdn-layer-08b: the same layer at the 0.8B-class "
                         "shape (B=8 L=2048 Hk=Hv=16 D=128); gdn-core: the chunked gated delta rule with "
                         "per-chunk states on the 27B-class clean stream (B=4 T=4096); attention: the "
                         "complementary-mask attention "
                         "layer kernel at B=2 L=4096 Hq=24 Hkv=4 d=256; stack: the 16-layer 27B-class "
                         "two-stream forward at B=1 L=2048; decode: one cached denoising step of that stack "
                         "(a 32-token block over a 2048-token clean prefix)")
    a = ap.parse_args(argv)
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: the state-fork layer shards over (batch, value head) with no "
              "exchange, and bench.py runs and reports the single-GPU share; use --gpus 1", file=sys.stderr)
        return 2
    if a.workload == "attention":
        return bench_attention(a)
    if a.workload == "gdn-core":
        return bench_gdn_core(a)
    if a.workload in ("stack", "decode"):
        # the library GEMMs around the path use the committed TunableOp solution table
        from dllm_qwen38_amd import gemm_tuning

        a.gemm_table = gemm_tuning.enable()
        return bench_stack(a) if a.workload == "stack" else bench_decode(a)

    return bench_gdn_layer(a)


def _host_info():
    """CPU model and torch version of this host, for the cpu_baseline record."""
    import platform

    import torch

    fields = {}
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if not line.strip():
                    break  # the first processor's block
                k, _, v = line.partition(":")
                fields[k.strip()] = v.strip()
    except OSError:
        pass
    model = fields.get("model name") or platform.processor() or ""
    ident = ", ".join(f"{k} {fields[k]}" for k in ("cpu family", "model", "stepping") if k in fields)
    return {"cpu_model": f"{model} ({ident})" if ident else model, "cpu_mhz": fields.get("cpu MHz"),
            "host_logical_cpus": os.cpu_count(), "torch": torch.__version__}


GDN_WORKLOADS = {
    "gdn-layer": ("GDN_27B_BF16", "state-fork GDN layer tokens/s at 27B-class shape; % MFMA/HBM roofline",
                  "state-fork GDN layer, 27B-class: B=4 L=4096 block=chunk=32 Hk=16 Hv=48 Dk=Dv=128 conv width 4, "
                  "bf16 in/out, fp32 state", "gdn_fork_27b_traffic.json", 1),
    "gdn-layer-08b": ("GDN_08B_BF16", "state-fork GDN layer tokens/s at 0.8B-class shape; % MFMA/HBM roofline",
                      "state-fork GDN layer, 0.8B-class: B=8 L=2048 block=chunk=32 Hk=Hv=16 Dk=Dv=128 conv width 4, "
                      "bf16 in/out, fp32 state", "gdn_fork_08b_traffic.json", 1),
}


def bench_gdn_layer(a):
    """One step = one state-fork GDN layer call: the conv of both streams and the fused fork (with
    the v channels' conv inside the fork where that measured faster: the conv launch then covers
    the q and k channels; bit-identical results). With pieces > 1 the step is
    StateForkPlan.run_overlapped (the conv of each block range beside the fork of the range before;
    bit-identical results). The per-kernel roofline comes from a second pass of the two kernels back
    to back, each between HIP events."""
    import torch

    from dllm_qwen38_amd import gdn, inputs

    shape_name, metric, workload, traffic_file, default_pieces = GDN_WORKLOADS[a.workload]
    dev = torch.device("cuda:0")
    s = getattr(inputs, shape_name)
    x = inputs.gdn_layer_inputs(s)
    xd = {k: v.to(dev) for k, v in x.items()}
    plan = gdn.StateForkPlan(xd["raw0"], xd["rawt"], xd["conv_w"], xd["beta0"], xd["betat"], xd["g0"], xd["gt"],
                             num_k_heads=s.Hk, num_v_heads=s.Hv, head_k_dim=s.D, head_v_dim=s.D, block=s.block)
    stream = torch.cuda.current_stream(dev)
    pieces = default_pieces if a.pieces is None else max(1, a.pieces)
    if pieces > 1 and not plan.overlap_supported():
        pieces = 1
    step = (lambda: plan.run_overlapped(pieces)) if pieces > 1 else plan.run
    gdn.kernel_status(reset=True)
    for _ in range(a.warmup):
        step()
    torch.cuda.synchronize(dev)

    # timed region: K steps of the schedule between HIP events on the launch stream (the side
    # stream's conv ranges join it through events before its last fork range)
    # (an event between consecutive steps gives each step's time as well)
    marks = [torch.cuda.Event(enable_timing=True) for _ in range(a.steps + 1)]
    torch.cuda.synchronize(dev)
    t0 = time.perf_counter()
    marks[0].record(stream)
    for i in range(a.steps):
        step()
        marks[i + 1].record(stream)
    torch.cuda.synchronize(dev)
    wall = time.perf_counter() - t0
    step_ms = marks[0].elapsed_time(marks[-1]) / a.steps
    per_step = [m0.elapsed_time(m1) for m0, m1 in zip(marks, marks[1:])]

    # kernels alone: the same K steps as conv, then fork, with HIP events around each kernel
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True),
           torch.cuda.Event(enable_timing=True)) for _ in range(a.steps)]
    for e0, e1, e2 in ev:
        e0.record(stream)
        plan.run_conv()
        e1.record(stream)
        plan.run_core()
        e2.record(stream)
    torch.cuda.synchronize(dev)
    status = gdn.kernel_status(reset=True)
    if status:
        print(f"a bounded wait gave up during the timed steps (status {status}): the outputs are invalid",
              file=sys.stderr)
        return 1
    conv_ms = [e0.elapsed_time(e1) for e0, e1, _ in ev]
    core_ms = [e1.elapsed_time(e2) for _, e1, e2 in ev]
    seq_step_ms = ev[0][0].elapsed_time(ev[-1][2]) / a.steps
    tokens = s.B * s.L
    core_avg = sum(core_ms) / len(core_ms)
    conv_avg = sum(conv_ms) / len(conv_ms)

    # the fork kernel's algorithmic bytes: the q/k/v rows of both streams read once (with the v conv
    # inside the fork, the v rows are the conv's inputs: the same bytes), beta and g of both streams
    # (fp32), both outputs, the fp32 state snapshots, and with the v conv the v channels' conv tails
    Cd, T = s.conv_dim, s.B * s.L
    core_bytes = (2 * T * Cd * 2 + 2 * T * s.Hv * 8 + 2 * T * s.Hv * s.D * 2 + (T // s.block) * s.Hv * s.D * s.D * 4)
    if plan.vconv:
        core_bytes += (T // s.block) * s.Hv * s.D * 3 * 2
    core_flops = gdn.layer_flops(s.B, s.L, s.Hv, s.D, s.D, s.block)
    achieved = core_bytes / (core_avg * 1e-3) / 1e9
    res = {
        "metric": metric,
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
        "config": {"workload": workload, "global_batch": s.B, "seq_len": s.L, "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": _traffic_from_profiles(traffic_file),
                     "kernel": "gdn_fork_pipe_kernel", "algorithmic_bytes": core_bytes},
        "step_ms": _dist(per_step),
        "kernels_ms": {"conv_fork": conv_avg, "gdn_state_fork": core_avg,
                       "conv_fork_dist": _dist(conv_ms), "gdn_state_fork_dist": _dist(core_ms)},
        "schedule": {"pieces": pieces, "vconv": plan.vconv, "ms_per_step_conv_then_fork": seq_step_ms},
        "layer_hbm": {"algorithmic_bytes": gdn.layer_bytes(s.B, s.L, s.Hk, s.Hv, s.D, s.D, s.block),
                      "step_gbs": gdn.layer_bytes(s.B, s.L, s.Hk, s.Hv, s.D, s.D, s.block) / (step_ms * 1e-3) / 1e9},
        "mfma": {"kernel": "gdn_state_fork", "algorithmic_tflops": core_flops / (core_avg * 1e-3) / 1e12,
                 "peak_tflops": BF16_MFMA_PEAK_TFLOPS,
                 "frac": core_flops / (core_avg * 1e-3) / 1e12 / BF16_MFMA_PEAK_TFLOPS},
        "wall_s_timed": wall,
        "cpu_baseline": None,
    }
    _calibration_copy(a, dev)
    if not a.no_cpu_baseline:
        res["cpu_baseline"], sample = cpu_baseline(s, min(a.cpu_sample_L, s.L), a.cpu_budget_s)
        res["speedup_vs_cpu"] = res["value"] / res["cpu_baseline"]["value"]
        res["parity"] = parity_sample(plan, s, sample)
    print(json.dumps(res))
    return 0


def _dist(ms):
    """Median, min and max of per-step (or per-launch) times in ms."""
    return {"median": statistics.median(ms), "min": min(ms), "max": max(ms), "n": len(ms)}


def _timed(fn, steps, warmup, stream):
    """Run fn warmup times, then time exactly `steps` runs between HIP events on `stream`."""
    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record(stream)
    for _ in range(steps):
        fn()
    e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps, time.perf_counter() - t0


def bench_gdn_core(a):
    """chunk_gated_delta_rule_with_states (reference gdn.py:48-123) as the clean pass of the 27B-class
    fork calls it (blockdiff.py:160): B=4 T=4096 chunk 32, Hk=16 Hv=48 Dk=Dv=128, bf16 q/k/v (q and k
    on their 16 key heads, GQA by indexing), fp32 g and beta, the fp32 state after every chunk kept.
    Roofline: HBM, on q, k, v, g and beta read once and the output and states written once."""
    import torch

    from dllm_qwen38_amd import gdn, inputs

    B, T, Hk, Hv, D, C = 4, 4096, 16, 48, 128, 32
    dev = torch.device("cuda:0")
    q, k, v, g, beta = inputs.gdn_core_inputs(B, T, Hk, Hv, D, torch.bfloat16, seed=300, g_shift=1.0)
    qd, kd, vd, gd, bd = (t.to(dev) for t in (q, k, v, g, beta))
    stream = torch.cuda.current_stream(dev)
    ms, wall = _timed(lambda: gdn.chunk_gated_delta_rule_with_states(qd, kd, vd, gd, bd, C), a.steps, a.warmup, stream)
    nbytes = (2 * B * T * Hk * D + B * T * Hv * D) * 2 + 2 * B * T * Hv * 4 + B * T * Hv * D * 2 \
        + B * (T // C) * Hv * D * D * 4
    achieved = nbytes / (ms * 1e-3) / 1e9
    res = {
        "metric": "chunked gated delta rule tokens/s (B*T positions) at the 27B-class shape; % HBM roofline",
        "value": B * T / (ms * 1e-3), "unit": "tokens/s", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
        "ms_per_step": ms, "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) q, k, v; sigmoid beta; g = -softplus(N(0,1) + 1))",
        "config": {"workload": "chunked gated delta rule with per-chunk states, B=4 T=4096 chunk 32 Hk=16 Hv=48 "
                               "Dk=Dv=128, bf16 in/out, fp32 state", "global_batch": B, "seq_len": T,
                   "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": None, "kernel": "gdn_fork_pipe_kernel<.., 1> (one stream)",
                     "algorithmic_bytes": nbytes},
        "wall_s_timed": wall, "cpu_baseline": None,
    }
    if not a.no_cpu_baseline:
        sys.path.insert(0, ROOT)
        from oracle import gdn_ref

        n = len(os.sched_getaffinity(0))
        torch.set_num_threads(n)
        Ts = T
        qs, ks, vs, gs, bs = (t[:1, :Ts] for t in (q, k, v, g, beta))
        # the oracle takes q and k on the value heads, as the reference's mixer expands them (gdn.py:227-229)
        qs, ks = qs.repeat_interleave(Hv // Hk, 2), ks.repeat_interleave(Hv // Hk, 2)
        gdn_ref.chunk_gated_delta_rule_with_states(qs, ks, vs, gs, bs, C)
        times = []
        start = time.perf_counter()
        while len(times) < 3 or time.perf_counter() - start < a.cpu_budget_s:
            t0 = time.perf_counter()
            gdn_ref.chunk_gated_delta_rule_with_states(qs, ks, vs, gs, bs, C)
            times.append(time.perf_counter() - t0)
        med = statistics.median(times)
        res["cpu_baseline"] = {"value": Ts / med, "unit": "tokens/s", "cores": n, "kind": "port",
                               "sample": f"B=1 T={Ts} (one sequence of the workload), same heads, "
                                         f"bf16-rounded inputs, fp32 torch CPU oracle; median of {len(times)} runs "
                                         f"({med:.2f} s/run)", **_host_info()}
        res["speedup_vs_cpu"] = res["value"] / res["cpu_baseline"]["value"]
    print(json.dumps(res))
    return 0


def bench_attention(a):
    """Complementary-mask attention over cat([x_t, x_0]) at B=2 L=4096 block 32, Hq=24 Hkv=4 d=256
    (bf16 Q/K/V ~ N(0,1)/16, rotary already applied). Roofline: MFMA, on the visible pairs only."""
    import torch

    from dllm_qwen38_amd import attention

    B, L, Hq, Hkv, d, block = 2, 4096, 24, 4, 256, 32
    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(407)
    q = (torch.randn(B, 2 * L, Hq, d, generator=g) / 16).to(torch.bfloat16).to(dev)
    k = (torch.randn(B, 2 * L, Hkv, d, generator=g) / 16).to(torch.bfloat16).to(dev)
    v = (torch.randn(B, 2 * L, Hkv, d, generator=g) / 16).to(torch.bfloat16).to(dev)
    out = torch.empty_like(q)
    stream = torch.cuda.current_stream(dev)
    ms, wall = _timed(lambda: attention.bd_attention(q, k, v, block=block, out=out), a.steps, a.warmup, stream)
    fl = attention.attention_flops(B, L, Hq, d, block)
    tf = fl / (ms * 1e-3) / 1e12
    res = {
        "metric": "complementary-mask attention layer tokens/s (B*L clean positions); % bf16 MFMA roofline",
        "value": B * L / (ms * 1e-3), "unit": "tokens/s", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
        "ms_per_step": ms, "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded N(0,1)/16 q, k, v)",
        "config": {"workload": "complementary-mask attention, B=2 L=4096 block 32 Hq=24 Hkv=4 d=256 over "
                               "cat([x_t, x_0]), bf16", "global_batch": B, "seq_len": L, "parallelism": "single GPU"},
        "roofline": {"bound": "mfma", "achieved": tf, "peak": BF16_MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": tf / BF16_MFMA_PEAK_TFLOPS,
                     "traffic": _traffic_from_profiles("attention_27b_traffic.json")},
        "algorithmic_gflop": fl / 1e9, "wall_s_timed": wall, "cpu_baseline": None,
    }
    _calibration_copy(a, dev)
    if not a.no_cpu_baseline:
        sys.path.insert(0, ROOT)
        from oracle import attn_ref

        n = len(os.sched_getaffinity(0))
        torch.set_num_threads(n)
        Ls = 512
        qs, ks, vs = (t[:1].cpu() for t in (q, k, v))
        qs = torch.cat([qs[:, :Ls], qs[:, L:L + Ls]], 1)
        ks = torch.cat([ks[:, :Ls], ks[:, L:L + Ls]], 1)
        vs = torch.cat([vs[:, :Ls], vs[:, L:L + Ls]], 1)
        attn_ref.bd_attention(qs, ks, vs, block=block)
        times = []
        start = time.perf_counter()
        while len(times) < 3 or time.perf_counter() - start < a.cpu_budget_s:
            t = time.perf_counter()
            attn_ref.bd_attention(qs, ks, vs, block=block)
            times.append(time.perf_counter() - t)
        med = statistics.median(times)
        res["cpu_baseline"] = {"value": Ls / med, "unit": "tokens/s", "cores": n, "kind": "port",
                               "sample": f"B=1 L={Ls} (the first {Ls} positions of each half), same heads and d, "
                                         f"fp32 torch CPU oracle; median of {len(times)} runs ({med:.2f} s/run)",
                               **_host_info()}
    print(json.dumps(res))
    return 0


def _stack_flops(model, lm_head, B, L, block):
    """Algorithmic flops of one two-stream forward: every linear layer on 2*B*L token rows, the GDN
    chunk contractions and the attention over visible pairs."""
    from torch import nn

    from dllm_qwen38_amd import attention, gdn

    rows = 2 * B * L
    lin = sum(m.in_features * m.out_features for m in model.modules() if isinstance(m, nn.Linear))
    lin += lm_head.in_features * lm_head.out_features
    c = model.config
    n_gdn = sum(t == "linear_attention" for t in c.layer_types)
    n_att = len(c.layer_types) - n_gdn
    return (2 * rows * lin + n_gdn * gdn.layer_flops(B, L, c.linear_num_value_heads, c.linear_key_head_dim,
                                                      c.linear_value_head_dim, block)
            + n_att * attention.attention_flops(B, L, c.num_attention_heads, c.head_dim, block))


def bench_stack(a):
    """The two-stream block-diffusion forward of a 16-layer 27B-class stack (12 GDN + 4 attention,
    hidden 5120, vocab 151936) at B=1 L=2048 block 32, bf16, seeded N(0, 0.02) weights on the device,
    logits of both streams. Roofline: MFMA over the whole forward's algorithmic flops."""
    import torch

    from dllm_qwen38_amd import blockdiff
    from dllm_qwen38_amd import model as hybrid

    B, L, block = 1, 2048, 32
    dev = torch.device("cuda:0")
    c = hybrid.config_27b_truncated(layers=16)
    model, lm_head = hybrid.build(c, device=dev, dtype=torch.bfloat16, seed=513)
    model.requires_grad_(False)
    lm_head.requires_grad_(False)
    g = torch.Generator().manual_seed(510)
    x0 = torch.randint(0, c.vocab_size, (B, L), generator=g)
    xt = x0.clone()
    tb = torch.rand(B, L // block, generator=g).repeat_interleave(block, 1)
    xt[torch.rand(B, L, generator=g) < tb] = c.vocab_size - 1
    x0, xt = x0.to(dev), xt.to(dev)
    stream = torch.cuda.current_stream(dev)

    def step():
        with torch.inference_mode():
            blockdiff.block_diffusion_forward(model, lm_head, x0, xt, block)

    steps = max(1, min(a.steps, 10))
    ms, wall = _timed(step, steps, max(1, min(a.warmup, 2)), stream)
    fl = _stack_flops(model, lm_head, B, L, block)
    tf = fl / (ms * 1e-3) / 1e12
    res = {
        "metric": "two-stream block-diffusion forward tokens/s (B*L clean positions), 16-layer 27B-class stack",
        "value": B * L / (ms * 1e-3), "unit": "tokens/s", "n_gpus": 1, "steps": steps, "warmup": max(1, min(a.warmup, 2)),
        "ms_per_step": ms, "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded N(0,0.02) weights, uniform ids, per-block masking with mask id V-1)",
        "config": {"workload": "block_diffusion_forward, 16 layers (12 GDN + 4 attention) hidden 5120 MLP 17408 "
                               "vocab 151936, B=1 L=2048 block 32, logits of both streams", "global_batch": B,
                   "seq_len": L, "parallelism": "single GPU"},
        "roofline": {"bound": "mfma", "achieved": tf, "peak": BF16_MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": tf / BF16_MFMA_PEAK_TFLOPS, "traffic": None},
        "algorithmic_tflop": fl / 1e12, "params": hybrid.param_count(model) + lm_head.weight.numel(),
        "gemm_table": getattr(a, "gemm_table", False), "wall_s_timed": wall, "cpu_baseline": None,
    }
    print(json.dumps(res))
    return 0


def bench_decode(a):
    """One denoising step of the prefix-cached decoder on the 16-layer 27B-class stack: a 32-token
    noised block at positions 2048..2079 over a committed 2048-token clean prefix, B=1, bf16, logits
    of the block. At B=1 the step reads every weight once for 32 token rows, so it is bound by HBM:
    the roofline's algorithmic bytes are the weights read (every projection, norm and lm_head; 32
    embedding rows) plus the cached K/V rows and GDN states the step reads. The golden decoder's
    step (the whole two-stream forward over prompt + block) is timed beside it."""
    import torch
    from torch import nn

    from dllm_qwen38_amd import blockdiff, decode
    from dllm_qwen38_amd import model as hybrid

    P, block = 2048, 32
    dev = torch.device("cuda:0")
    c = hybrid.config_27b_truncated(layers=16)
    model, lm_head = hybrid.build(c, device=dev, dtype=torch.bfloat16, seed=513)
    model.requires_grad_(False)
    lm_head.requires_grad_(False)
    g = torch.Generator().manual_seed(511)
    x0 = torch.randint(0, c.vocab_size, (1, P + block), generator=g)
    xt = x0.clone()
    xt[:, P + 3:] = c.vocab_size - 1  # a block with 3 tokens committed, 29 still masked
    x0, xt = x0.to(dev), xt.to(dev)
    stream = torch.cuda.current_stream(dev)
    cache = decode.PrefixCache(model, batch=1, capacity=P + block, block=block)

    def prefill():
        cache.reset()
        decode.forward_segment(model, lm_head, cache, x0[:, :P], commit=True, logits=False)

    prefill_ms, _ = _timed(prefill, 2, 1, stream)

    def step():
        decode.forward_segment(model, lm_head, cache, xt[:, P:], commit=False)

    steps, warm = max(1, a.steps), max(1, a.warmup)
    ms, wall = _timed(step, steps, warm, stream)

    def golden():
        with torch.inference_mode():
            blockdiff.block_diffusion_forward(model, lm_head, x0, xt, block)

    golden_ms, _ = _timed(golden, 2, 1, stream)

    esz = 2
    wbytes = sum(m.weight.numel() * m.weight.element_size() for m in model.modules()
                 if isinstance(m, nn.Linear)) + lm_head.weight.numel() * esz
    wbytes += sum(p.numel() * p.element_size() for n, p in model.named_parameters()
                  if not n.startswith("embed_tokens") and p.dim() == 1)  # norms, conv bias, decay
    wbytes += sum(m.conv1d.weight.numel() * m.conv1d.weight.element_size() for m in model.modules()
                  if hasattr(m, "conv1d"))
    wbytes += block * c.hidden_size * esz  # embedding rows
    kv = sum(2 * t[:, : P + block].numel() * esz for t in cache.k.values())
    st = sum(s.numel() * 4 for s in cache.state.values() if s is not None)
    total = wbytes + kv + st
    gbs = total / (ms * 1e-3) / 1e9
    res = {
        "metric": "cached denoising step of the block-diffusion decoder: block forwards/s (32-token block over "
                  "a 2048-token clean prefix), 16-layer 27B-class stack; % HBM roofline",
        "value": 1e3 / ms, "unit": "forwards/s", "n_gpus": 1, "steps": steps, "warmup": warm,
        "ms_per_step": ms, "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded N(0,0.02) weights, uniform ids, 29 of 32 block positions masked)",
        "config": {"workload": "prefix-cached denoising step, 16 layers (12 GDN + 4 attention) hidden 5120 "
                               "MLP 17408 vocab 151936, B=1, prefix 2048, block 32, logits of the block",
                   "global_batch": 1, "seq_len": P + block, "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": gbs / HBM_PEAK_GBS, "traffic": None},
        "algorithmic_bytes": total, "weight_bytes": wbytes, "kv_cache_bytes": kv, "state_bytes": st,
        "prefill_ms": prefill_ms, "golden_step_ms": golden_ms, "speedup_vs_golden_step": golden_ms / ms,
        "cache_bytes": cache.nbytes(), "gemm_table": getattr(a, "gemm_table", False), "wall_s_timed": wall,
        "cpu_baseline": None,
    }
    print(json.dumps(res))
    return 0


if __name__ == "__main__":
    sys.exit(main())
