"""Pins the decode oracle (oracle/decode_ref.py) and checks the product's host-side commit rule
against it. CPU only."""

import pytest
import torch

from oracle import decode_ref, model_ref
from tests._tiny import tiny_hf_model


def _ref_tiny(seed=0):
    """The reference's unit-test model (blockdiff.py:246-278), built the same way."""
    from dllm_qwen38_amd.blockdiff import tiny_text_model

    m, head = tiny_text_model(seed=seed)
    m.requires_grad_(False)
    head.requires_grad_(False)
    return m, head


def test_blocks_for_closed_form():
    # the reference's seam test: 24 new tokens after a 5-token prompt in blocks of 8 -> 4 blocks
    assert decode_ref.blocks_for(24, 5, 8) == 4
    for plen in range(0, 20):
        for block in (4, 8):
            for max_new in range(1, 40):
                nb = decode_ref.blocks_for(max_new, plen, block)
                cap = lambda k: (block - plen % block) + (k - 1) * block  # noqa: E731
                assert cap(nb) >= max_new and (nb == 1 or cap(nb - 1) < max_new)


def test_reference_seam_known_answer():
    """tests/test_gsm8k_eval.py:306-333 of the reference: seed-0 tiny model, prompt 10..14, block 8,
    threshold 0.9, max_new 24, mask 255, eos 3 -> 4 blocks, 27 generated, 4 step counts."""
    torch.manual_seed(0)
    m, head = _ref_tiny(0)
    nb = decode_ref.blocks_for(24, 5, 8)
    tr = decode_ref.generate(m, head, [10, 11, 12, 13, 14], n_blocks=nb, block=8, mask_id=255, threshold=0.9,
                             eos_id=3)
    assert nb == 4
    assert tr["generated"] == 27
    assert len(tr["steps_per_block"]) == 4
    assert tr["tokens"][:5] == [10, 11, 12, 13, 14] and len(tr["tokens"]) == 32


@pytest.mark.parametrize("plen", [5, 8, 0])
def test_schedule_closed_forms(plen):
    m, head = tiny_hf_model(seed=3, layers=4)
    prompt = list(range(20, 20 + plen))
    block, nb = 8, 3
    room = block - plen % block
    # threshold above 1: exactly one commit per step
    tr = decode_ref.generate(m, head, prompt, n_blocks=nb, block=block, mask_id=255, threshold=1.5)
    assert tr["steps_per_block"] == [room] + [block] * (nb - 1)
    assert all(len(pos) == 1 for _, pos, _ in tr["steps"])
    assert tr["generated"] == room + (nb - 1) * block == tr["forwards"]
    # threshold 0: every candidate commits at once
    tr0 = decode_ref.generate(m, head, prompt, n_blocks=nb, block=block, mask_id=255, threshold=0.0)
    assert tr0["steps_per_block"] == [1] * nb
    # threshold 0 with sub-blocks: one step per sub-block that holds a mask, left to right
    sb = 4
    trs = decode_ref.generate(m, head, prompt, n_blocks=nb, block=block, mask_id=255, threshold=0.0, sub_block=sb)
    first = (block - room) // sb
    assert trs["steps_per_block"] == [block // sb - first] + [block // sb] * (nb - 1)
    for _, pos, _ in trs["steps"]:
        assert len({p // sb for p in pos}) == 1  # one sub-block per step
    kbs = [kb for kb, _, _ in trs["steps"]]
    assert kbs == sorted(kbs)


def test_threshold_zero_tokens_are_the_per_block_oracle_argmax():
    """At threshold 0 block kb's tokens are the argmax of the noised logits of (x_0 = known tokens,
    x_t = known with masks); the per-block oracle computes those from an independent path."""
    m, head = tiny_hf_model(seed=4, layers=4)
    prompt, block = [7, 9, 11, 13, 15, 17, 19, 21, 23, 25, 27], 8
    tr = decode_ref.generate(m, head, prompt, n_blocks=2, block=block, mask_id=255, threshold=0.0)
    toks = tr["tokens"]
    for kb, start in ((1, len(prompt)), (2, 2 * block)):
        L = (kb + 1) * block
        known = torch.full((1, L), 255)
        known[0, :start] = torch.tensor(toks[:start])
        ref = model_ref.reference_block_logits(m, head, known, known, block)[0, kb * block:]
        want = ref.argmax(-1)[start - kb * block:].tolist()
        assert toks[start:L] == want


def test_eos_stops_after_its_block():
    m, head = tiny_hf_model(seed=5, layers=4)
    full = decode_ref.generate(m, head, [1, 2, 3], n_blocks=3, block=8, mask_id=255, threshold=0.0)
    eos = full["tokens"][5]  # produced in the first generated block: decoding ends with that block
    tr = decode_ref.generate(m, head, [1, 2, 3], n_blocks=3, block=8, mask_id=255, threshold=0.0, eos_id=eos)
    assert len(tr["steps_per_block"]) == 1 and tr["generated"] == 5
    assert tr["tokens"] == full["tokens"][:8]
    absent = next(t for t in range(256) if t not in full["tokens"])
    tr = decode_ref.generate(m, head, [1, 2, 3], n_blocks=3, block=8, mask_id=255, threshold=0.0, eos_id=absent)
    assert tr["tokens"] == full["tokens"] and len(tr["steps_per_block"]) == 3


def test_a_planted_sub_block_mistake_fails_the_closed_form(monkeypatch):
    m, head = tiny_hf_model(seed=3, layers=2)
    real = decode_ref.select

    def no_window(logits, masked, **kw):
        kw["sub_block"] = None
        return real(logits, masked, **kw)

    monkeypatch.setattr(decode_ref, "select", no_window)
    trs = decode_ref.generate(m, head, [1, 2, 3, 4, 5], n_blocks=2, block=8, mask_id=255, threshold=0.0, sub_block=4)
    assert trs["steps_per_block"] != [1, 2]  # what the correct schedule gives (first block: 3 masks in one sub-block)


@pytest.mark.parametrize("temperature", [0.0, 0.7])
@pytest.mark.parametrize("sub_block", [None, 4])
@pytest.mark.parametrize("threshold", [0.0, 0.02, 0.9, 1.5])
def test_product_commit_rule_matches_the_oracle(temperature, sub_block, threshold):
    """decode._select (host logic of the product decoders) against the oracle's rule."""
    from dllm_qwen38_amd.decode import _select

    g = torch.Generator().manual_seed(11)
    for trial in range(20):
        logits = torch.randn(8, 50, generator=g) * 3
        masked = torch.rand(8, generator=g) < 0.6
        if not masked.any():
            masked[trial % 8] = True
        torch.manual_seed(trial)
        c1, p1 = _select(logits, masked, threshold=threshold, sub_block=sub_block, temperature=temperature)
        torch.manual_seed(trial)
        c2, p2 = decode_ref.select(logits, masked, threshold=threshold, sub_block=sub_block, temperature=temperature)
        assert torch.equal(c1, c2) and torch.equal(p1[c1], p2[c2])
