"""CPU oracle of the block-wise confidence-threshold decoder — TEST INFRASTRUCTURE ONLY.

Restates reference `src/dllm_qwen38/decode.py:36-99` (`generate`, the golden decoder: every
denoising step re-runs the whole two-stream forward) over the oracle's own forward
(`model_ref.block_diffusion_forward`, or any forward passed in), and the block-count helper of
`src/dllm_qwen38/gsm8k_eval.py:207-218` (`blocks_for`).

Per block: x_0 holds every known token, x_t the same with the still-masked positions set to
mask_id; the forward's noised logits at the current block give, per masked position, the argmax
token and its softmax probability (or a sample and its probability at temperature > 0). Every
candidate whose confidence reaches the threshold is committed, and always at least the single
most confident one; with `sub_block`, candidates are limited to the leftmost sub-block that still
holds a mask. The block repeats until clean; decoding stops after the block that produced eos.

How it is pinned (tests/test_oracle_decode.py):
  * the reference's own seam test (tests/test_gsm8k_eval.py:306-333): tiny model seed 0, prompt
    10..14, block 8, threshold 0.9, 24 new tokens -> 4 blocks, 27 generated, 4 step counts;
  * closed forms of the schedule: threshold > 1 commits exactly one position per step (steps =
    masked positions per block), threshold 0 commits every candidate at once (one step per block,
    or one per sub-block with sub_block), generated = room + (n_blocks - 1) * block;
  * at threshold 0 the committed tokens are the argmax of the per-block oracle
    (`model_ref.reference_block_logits`, itself pinned to transformers' model), an independent path;
  * eos ends decoding after the block that holds it; planted mistakes in the schedule fail these.
"""

from __future__ import annotations

import torch

from . import model_ref


def blocks_for(max_new: int, prompt_len: int, block: int) -> int:
    """Blocks needed so that the generated capacity covers max_new: the first block fills the rest
    of the prompt's last block (block - prompt_len % block tokens), later blocks `block` each."""
    first = block - prompt_len % block
    return 1 if max_new <= first else 1 + -(-(max_new - first) // block)


def select(logits: torch.Tensor, masked: torch.Tensor, *, threshold: float, sub_block: int | None,
           temperature: float):
    """One commit decision over a block: logits [C, V] float, masked [C] bool.
    Returns (commit [C] bool, pick [C] token ids)."""
    if temperature > 0:
        probs = torch.softmax(logits / temperature, -1)
        pick = torch.multinomial(probs, 1)[:, 0]
        conf = probs.gather(1, pick[:, None])[:, 0]
    else:
        conf, pick = torch.softmax(logits, -1).max(-1)
    cand = masked.clone()
    if sub_block:
        first = int(torch.nonzero(cand)[0])
        lo = first - first % sub_block
        pos = torch.arange(cand.numel())
        cand &= (pos >= lo) & (pos < lo + sub_block)
    conf = torch.where(cand, conf, torch.full_like(conf, -1.0))
    commit = cand & (conf >= threshold)
    if not bool(commit.any()):
        commit[int(conf.argmax())] = True
    return commit, pick


@torch.no_grad()
def generate(text_model, lm_head, prompt_ids: list[int], *, n_blocks: int, block: int, mask_id: int,
             threshold: float = 0.9, sub_block: int | None = None, eos_id: int | None = None,
             temperature: float = 0.0, layers: int | None = None, forward=None) -> dict:
    """The golden decoder over `forward(text_model, lm_head, x0 [1, L], xt [1, L], block, layers=)`
    -> (logits_t, logits_0), by default the oracle's own fork forward. Returns a dict with the
    reference trace's fields (tokens, forwards, generated, steps_per_block) and `steps`: per step
    (block index, committed positions, their tokens)."""
    forward = forward or model_ref.block_diffusion_forward
    cur = list(prompt_ids)
    forwards, generated, steps_per_block, steps_log = 0, 0, [], []
    for _ in range(n_blocks):
        n = len(cur)
        kb = n // block
        L = (kb + 1) * block
        known = torch.full((L,), mask_id, dtype=torch.long)
        known[:n] = torch.tensor(cur, dtype=torch.long)
        masked = torch.arange(L) >= n
        x0 = known.clone()  # its block kb is invisible to x_t block kb: fixed for the whole block
        steps = 0
        while bool(masked.any()):
            xt = torch.where(masked, torch.full_like(known, mask_id), known)
            lt, _ = forward(text_model, lm_head, x0[None], xt[None], block, layers=layers)
            forwards += 1
            steps += 1
            commit, pick = select(lt[0, kb * block:].float(), masked[kb * block:], threshold=threshold,
                                  sub_block=sub_block, temperature=temperature)
            idx = torch.nonzero(commit)[:, 0]
            known[kb * block + idx] = pick[idx]
            masked[kb * block + idx] = False
            steps_log.append((kb, idx.tolist(), pick[idx].tolist()))
        steps_per_block.append(steps)
        new = known[n:].tolist()
        cur.extend(new)
        generated += len(new)
        if eos_id is not None and eos_id in new:
            break
    return {"tokens": cur, "forwards": forwards, "generated": generated, "steps_per_block": steps_per_block,
            "steps": steps_log}
