"""The 16-layer 27B-class stack (12 GDN + 4 attention layers, hidden 5120, MLP 17408, vocab
151936) on the GPU, against the CPU oracle's two-stream forward in fp32 on the same weights.

This is the stack the benchmark's `stack` workload times (same seeds: weights 513, token ids 510,
per-block masking with mask id V-1, block 32). The oracle is oracle/model_ref.block_diffusion_forward
(pinned against transformers' own modules and the per-block oracle in tests/test_oracle_model.py),
run on an fp32 copy of the bf16 weights.

  * fp32 run: the HIP path in fp32 (fp32 attention kernel, the two-pass fork on the fp32 chunk
    kernel, fp32 GEMMs) on the same weights; bar: the reference harness's fp32 tolerance,
    max |logit difference| <= 1e-3 (src/dllm_qwen38/equivalence.py, --tol default for float32).
  * bf16 run (what the benchmark times): the error against the fp32 oracle is set beside the error
    of the oracle itself run in bf16 on the CPU (the reference's own path in bf16); bar: max and
    mean |logit difference| within twice that of the CPU bf16 run. (The reference's harness
    bf16 tolerance of 0.25 is exceeded by the reference's own bf16 27B run, 0.59 / 0.35 in
    reports/modal/eq-27b-bf16-ref-oracle.log, so it is reported, not asserted.)

Both L = 256 and the workload's full L = 2048 run by default (about 90 s at L = 2048 on 16 host
threads, 45 GB of host memory for the weights); DLLM_STACK_QUICK=1 keeps L = 256 only.
"""

import copy
import os
import time

import pytest
import torch

from dllm_qwen38_amd import blockdiff
from dllm_qwen38_amd import model as hybrid
from oracle import model_ref

pytestmark = pytest.mark.gpu

F32_TOL = 1e-3
LENGTHS = [256] + ([] if os.environ.get("DLLM_STACK_QUICK") == "1" else [2048])


@pytest.fixture(scope="module")
def stack(dev):
    c = hybrid.config_27b_truncated(layers=16)
    model, lm_head = hybrid.build(c, device=dev, dtype=torch.bfloat16, seed=513)
    model.requires_grad_(False)
    lm_head.requires_grad_(False)
    t = time.time()
    with torch.device("meta"):
        cm = hybrid.HybridTextModel(c)
        clm = torch.nn.Linear(c.hidden_size, c.vocab_size, bias=False)
    cm.to_empty(device="cpu")
    clm.to_empty(device="cpu")
    with torch.no_grad():
        for (k, dst), (k2, src) in zip(cm.state_dict().items(), model.state_dict().items()):
            assert k == k2
            dst.copy_(src)
        clm.weight.copy_(lm_head.weight)
        cm.rotary_emb.inv_freq = model.rotary_emb.inv_freq.float().cpu()
    cm.requires_grad_(False)
    clm.requires_grad_(False)
    print(f"fp32 CPU copy of {hybrid.param_count(cm) / 1e9:.2f} G parameters in {time.time() - t:.1f} s", flush=True)
    return c, model, lm_head, cm, clm


def _ids(c, L, block=32):
    g = torch.Generator().manual_seed(510)
    x0 = torch.randint(0, c.vocab_size, (1, L), generator=g)
    xt = x0.clone()
    tb = torch.rand(1, L // block, generator=g).repeat_interleave(block, 1)
    xt[torch.rand(1, L, generator=g) < tb] = c.vocab_size - 1
    return x0, xt


def _stats(name, got, ref):
    d = (got.float() - ref).abs()
    agree = (got.float().argmax(-1) == ref.argmax(-1)).float().mean().item()
    r = {"max": d.max().item(), "mean": d.mean().item(), "argmax": agree}
    print(f"{name}: max|d|={r['max']:.3e} mean|d|={r['mean']:.3e} max|ref|={ref.abs().max().item():.3f} "
          f"argmax agreement {agree:.4f}", flush=True)
    assert torch.isfinite(got).all()
    return r


@pytest.mark.parametrize("L", LENGTHS)
def test_stack27b_vs_fp32_cpu_oracle(stack, dev, L):
    c, model, lm_head, cm, clm = stack
    block = 32
    x0, xt = _ids(c, L, block)
    x0d, xtd = x0.to(dev), xt.to(dev)
    with torch.inference_mode():
        gt16, g016 = (t.float().cpu() for t in blockdiff.block_diffusion_forward(model, lm_head, x0d, xtd, block))
    # the same bf16-rounded weights in fp32 on the device
    m32, h32 = copy.deepcopy(model).float(), copy.deepcopy(lm_head).float()
    with torch.inference_mode():
        gt32, g032 = (t.cpu() for t in blockdiff.block_diffusion_forward(m32, h32, x0d, xtd, block))
    del m32, h32
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    print(f"L={L}: GPU bf16 and fp32 forwards done; CPU oracle in fp32", flush=True)
    torch.set_num_threads(len(os.sched_getaffinity(0)))
    t = time.time()
    with torch.no_grad():
        rt, r0 = model_ref.block_diffusion_forward(cm, clm, x0, xt, block)
    print(f"L={L}: CPU fp32 oracle {time.time() - t:.1f} s; CPU oracle in bf16", flush=True)
    cm16, clm16 = copy.deepcopy(cm).to(torch.bfloat16), copy.deepcopy(clm).to(torch.bfloat16)
    t = time.time()
    with torch.no_grad():
        ct16, c016 = (x.float() for x in model_ref.block_diffusion_forward(cm16, clm16, x0, xt, block))
    del cm16, clm16
    print(f"L={L}: CPU bf16 oracle {time.time() - t:.1f} s", flush=True)
    for name, g32, g16, c16, ref in (("noised", gt32, gt16, ct16, rt), ("clean", g032, g016, c016, r0)):
        s32 = _stats(f"L={L} {name} GPU fp32 vs CPU fp32", g32, ref)
        s16 = _stats(f"L={L} {name} GPU bf16 vs CPU fp32", g16, ref)
        c16s = _stats(f"L={L} {name} CPU bf16 vs CPU fp32", c16, ref)
        assert s32["max"] <= F32_TOL, f"{name}: fp32 run differs by {s32['max']:.3e}"
        assert s16["max"] <= 2 * c16s["max"] and s16["mean"] <= 2 * c16s["mean"], \
            f"{name}: the bf16 run's error exceeds twice the CPU bf16 run's"
