"""Block-diffusion equivalence harness for the HIP forward (command line and `run()`).

The candidate is `blockdiff.block_diffusion_forward` on the ROCm device, with the HIP state fork
and the tile-skipping attention kernel. The oracle is transformers' unmodified model, run in fp32
on the CPU one block at a time under the block-causal mask (for --dtype bfloat16, on weights
rounded to bf16 first), so no kernel of this library sits on both sides of a comparison.

Five checks are measured and reported as numbers:
  * noised-stream-vs-oracle and clean-stream-vs-oracle (max |logit difference|);
  * for each block k >= 1: re-drawing x_t block k-1 or x_0 block k must leave the noised logits
    of block k unchanged, and re-drawing x_0 block k-1 must move them by at least a floor.
Each of the three deliberate faults (concat-causal-gdn, mask-leak, no-conv-prefix) must then push
the noised stream past the tolerance. Exit status: 0 when all checks pass and all faults are
detected, 1 when one does not, 2 when nothing could be measured (no device, no model, bad sizes).
The command-line flags, report keys and output lines follow the reference's harness
(src/dllm_qwen38/equivalence.py) so that its callers and log parsers work unchanged.

    python -m dllm_qwen38_amd.equivalence [--block 32] [--nblocks 4] [--dtype float32|bfloat16]
"""

from __future__ import annotations

import argparse
import copy
import json
import sys
import time

import torch

from . import gdn
from .blockdiff import BreakMode, block_diffusion_forward, reference_block_logits, reference_clean_logits, tiny_text_model

FAULTS = ("concat-causal-gdn", "mask-leak", "no-conv-prefix")


def _maxdiff(a: torch.Tensor, b: torch.Tensor) -> float:
    return float((a.float().cpu() - b.float().cpu()).abs().max())


def oracle_gdn_kernel() -> str:
    """The chunked delta-rule implementation the transformers oracle runs: the flash-linear-attention
    package when it is importable, else transformers' own torch code (the case in this image)."""
    return "fla" if sys.modules.get("fla") is not None else "torch-reference"


def run(cand_model, cand_head, oracle_model, oracle_head, *, block: int, nblocks: int, layers: int | None,
        tol: float, change_floor: float, seed: int, device: str) -> dict:
    """All checks; the candidate runs on `device`, the oracle wherever its model lives."""
    g = torch.Generator().manual_seed(seed)
    L = block * nblocks
    vocab = cand_model.embed_tokens.weight.shape[0]
    x0 = torch.randint(0, vocab, (1, L), generator=g)
    xt = x0.clone()
    xt[torch.rand(1, L, generator=g) < 0.5] = vocab - 1  # mask id: any existing id will do
    odev = oracle_model.embed_tokens.weight.device

    def cand(a, b, fault=None):
        with torch.no_grad():
            out = block_diffusion_forward(cand_model, cand_head, a.to(device), b.to(device), block,
                                          fault=fault, layers=layers)
        # a kernel whose bounded wait gave up wrote invalid logits: stop rather than compare them
        gdn.check_kernel_status("equivalence harness forward")
        return out

    checks: list[dict] = []
    t0 = time.time()
    lt, l0 = cand(x0, xt)
    ref_t = reference_block_logits(oracle_model, oracle_head, x0.to(odev), xt.to(odev), block, layers=layers)
    ref_0 = reference_clean_logits(oracle_model, oracle_head, x0.to(odev), block, layers=layers)
    d = _maxdiff(lt, ref_t)
    checks.append({"name": "noised-stream-vs-oracle", "max_abs_diff": d, "tol": tol, "pass": d <= tol})
    d = _maxdiff(l0, ref_0)
    checks.append({"name": "clean-stream-vs-oracle", "max_abs_diff": d, "tol": tol, "pass": d <= tol})

    if nblocks >= 2:
        worst_xt, worst_x0k, weakest = 0.0, 0.0, float("inf")
        for k in range(1, nblocks):
            sl, prev = slice(k * block, (k + 1) * block), slice((k - 1) * block, k * block)
            xt2 = xt.clone()
            xt2[:, prev] = torch.randint(0, vocab, (1, block), generator=g)
            worst_xt = max(worst_xt, _maxdiff(lt[:, sl], cand(x0, xt2)[0][:, sl]))
            x02 = x0.clone()
            x02[:, sl] = torch.randint(0, vocab, (1, block), generator=g)
            worst_x0k = max(worst_x0k, _maxdiff(lt[:, sl], cand(x02, xt)[0][:, sl]))
            x03 = x0.clone()
            x03[:, prev] = torch.randint(0, vocab, (1, block), generator=g)
            weakest = min(weakest, _maxdiff(lt[:, sl], cand(x03, xt)[0][:, sl]))
        checks.append({"name": "xt-block-k-ignores-xt-block-k-1", "max_abs_diff": worst_xt, "tol": tol,
                       "pass": worst_xt <= tol})
        checks.append({"name": "xt-block-k-ignores-x0-block-k", "max_abs_diff": worst_x0k, "tol": tol,
                       "pass": worst_x0k <= tol})
        checks.append({"name": "xt-block-k-reacts-to-x0-block-k-1", "min_abs_diff": weakest, "floor": change_floor,
                       "pass": weakest >= change_floor})

    faults = []
    for name in FAULTS:
        d = _maxdiff(cand(x0, xt, BreakMode(name))[0], ref_t)
        faults.append({"fault": name, "max_abs_diff": d, "tol": tol, "detected": d > tol})

    return {
        "block": block, "nblocks": nblocks, "seq_len": L,
        "layers": layers if layers is not None else int(cand_model.config.num_hidden_layers),
        "layer_types": list(cand_model.config.layer_types[: layers or None]),
        "dtype": str(cand_model.embed_tokens.weight.dtype), "device": device, "oracle_device": str(odev),
        "seconds": round(time.time() - t0, 2), "checks": checks, "faults": faults,
        "checks_passed": sum(c["pass"] for c in checks), "checks_total": len(checks),
        "faults_detected": sum(f["detected"] for f in faults), "faults_total": len(faults),
    }


def _load(model_id: str | None, seed: int, layers: int | None = None):
    """(text_model, lm_head, vocab) in fp32 on the CPU. model_id None: the tiny random test model
    (vocab None). Otherwise a checkpoint directory on disk (no download). With `layers`, the stack
    is cut to its first `layers` layers BEFORE the fp32 cast: the checkpoint loads in its stored
    dtype (bf16 for the released weights, so a 27B-class stack fits), the tail layers are dropped,
    and only the kept prefix is cast. `vocab` reports the embedding rows against the tokenizer's
    length (the spare rows any id above the tokenizer's range would hit); the tokenizer length is
    None when the directory holds no tokenizer."""
    if model_id is None:
        model, head = tiny_text_model(seed=seed)
        return model, head, None
    from transformers import AutoConfig, AutoModelForCausalLM, AutoModelForImageTextToText

    cfg = AutoConfig.from_pretrained(model_id, local_files_only=True)
    kw = dict(dtype="auto" if layers else torch.float32, attn_implementation="eager", local_files_only=True)
    if getattr(cfg, "text_config", None) is not None:
        m = AutoModelForImageTextToText.from_pretrained(model_id, **kw)
        text_model, head = m.model.language_model, m.lm_head
        if hasattr(m.model, "visual"):
            m.model.visual = None  # the vision tower is never run
    else:
        m = AutoModelForCausalLM.from_pretrained(model_id, **kw)
        text_model, head = m.model, m.lm_head
    if layers:
        if layers > len(text_model.layers):
            raise ValueError(f"--layers {layers} exceeds the model's {len(text_model.layers)} layers")
        del text_model.layers[layers:]
        text_model.config.num_hidden_layers = layers
        text_model.config.layer_types = list(text_model.config.layer_types[:layers])
    text_model.float().eval()
    head.float()
    rows = int(text_model.embed_tokens.weight.shape[0])
    try:
        from transformers import AutoTokenizer

        tok_len = len(AutoTokenizer.from_pretrained(model_id, local_files_only=True))
    except Exception:  # noqa: BLE001 - a checkpoint without tokenizer files still runs
        tok_len = None
    vocab = {"embedding_rows": rows, "tokenizer_len": tok_len,
             "spare_rows": None if tok_len is None else rows - tok_len}
    return text_model, head, vocab


def main(argv: list[str] | None = None) -> int:
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--model", default=None, help="checkpoint directory on disk (no download); default: the tiny "
                   "random test model")
    p.add_argument("--layers", type=int, default=None, help="truncate both models to their first N layers")
    p.add_argument("--block", type=int, default=32)
    p.add_argument("--nblocks", type=int, default=4)
    p.add_argument("--tol", type=float, default=None, help="largest logit difference that still passes "
                   "(1e-3 for float32, 0.25 for bfloat16 unless given)")
    p.add_argument("--change-floor", type=float, default=None, help="smallest logit change that counts as a real "
                   "dependency (ten times the tolerance unless given)")
    p.add_argument("--dtype", default="float32", choices=["float32", "bfloat16"])
    p.add_argument("--attn", default="eager", choices=["eager", "sdpa"], help="attention backend of the "
                   "transformers oracle; the candidate always runs the HIP kernel")
    p.add_argument("--device", default="cuda")
    p.add_argument("--seed", type=int, default=0)
    p.add_argument("--json", default=None, help="write the report here as JSON")
    a = p.parse_args(argv)

    dtype = torch.float32 if a.dtype == "float32" else torch.bfloat16
    tol = a.tol if a.tol is not None else (1e-3 if dtype == torch.float32 else 0.25)
    floor = a.change_floor if a.change_floor is not None else 10 * tol
    if a.nblocks < 1:
        print("COULD-NOT-MEASURE nblocks < 1", file=sys.stderr)
        return 2
    try:
        oracle_model, oracle_head, vocab = _load(a.model, a.seed, a.layers)
    except Exception as e:  # noqa: BLE001 - could not measure is its own exit code
        print(f"COULD-NOT-MEASURE model load failed: {type(e).__name__}: {e}", file=sys.stderr)
        return 2
    if a.layers is not None and a.layers > oracle_model.config.num_hidden_layers:
        print("COULD-NOT-MEASURE --layers exceeds the model", file=sys.stderr)
        return 2
    if not torch.cuda.is_available() or not str(a.device).startswith("cuda"):
        print("COULD-NOT-MEASURE the candidate runs on the HIP kernels and needs a ROCm device", file=sys.stderr)
        return 2
    oracle_model.requires_grad_(False)
    oracle_head.requires_grad_(False)
    oracle_model.set_attn_implementation(a.attn)
    cand_model = copy.deepcopy(oracle_model).to(a.device, dtype)
    cand_head = copy.deepcopy(oracle_head).to(a.device, dtype)
    if dtype != torch.float32:  # the oracle sees the same (rounded) weights, in fp32
        oracle_model.to(dtype).float()
        oracle_head.to(dtype).float()

    rep = run(cand_model, cand_head, oracle_model, oracle_head, block=a.block, nblocks=a.nblocks, layers=a.layers,
              tol=tol, change_floor=floor, seed=a.seed, device=a.device)
    rep["model"] = a.model or "tiny-random"
    rep["attn"] = a.attn
    rep["oracle_gdn_kernel"] = oracle_gdn_kernel()
    if vocab is not None:
        rep["vocab"] = vocab
    if a.json:
        with open(a.json, "w") as f:
            json.dump(rep, f, indent=1)
    for c in rep["checks"]:
        val = c.get("max_abs_diff", c.get("min_abs_diff"))
        print(f"{'PASS' if c['pass'] else 'FAIL'}\t{c['name']}\t{val:.3e}")
    for f in rep["faults"]:
        print(f"{'DETECTED' if f['detected'] else 'UNDETECTED'}\tfault:{f['fault']}\t{f['max_abs_diff']:.3e}")
    print(f"CHECKS\t{rep['checks_passed']}/{rep['checks_total']}\tFAULTS-DETECTED\t{rep['faults_detected']}/"
          f"{rep['faults_total']}\tmodel={rep['model']} layers={rep['layers']} L={rep['seq_len']} dtype={rep['dtype']} "
          f"oracle-gdn={rep['oracle_gdn_kernel']} {rep['seconds']}s")
    if vocab is not None:
        print(f"VOCAB\tembedding_rows={vocab['embedding_rows']}\ttokenizer_len={vocab['tokenizer_len']}\t"
              f"spare_rows={vocab['spare_rows']}")
    ok = rep["checks_passed"] == rep["checks_total"] and rep["faults_detected"] == rep["faults_total"]
    return 0 if ok else 1


if __name__ == "__main__":
    sys.exit(main())
