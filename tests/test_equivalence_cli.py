"""The equivalence harness's exit codes (reference src/dllm_qwen38/equivalence.py:156-219): 2 when
nothing can be measured. Host-only: every case here stops before any device work."""

import torch

from dllm_qwen38_amd import equivalence


def test_could_not_measure_exit_codes(tmp_path, capsys):
    assert equivalence.main(["--nblocks", "0"]) == 2
    assert equivalence.main(["--model", str(tmp_path / "no-such-checkpoint")]) == 2
    assert equivalence.main(["--layers", "99"]) == 2
    if not torch.cuda.is_available():
        assert equivalence.main([]) == 2  # the candidate needs the HIP device
    assert "COULD-NOT-MEASURE" in capsys.readouterr().err


def test_checkpoint_load_truncates_before_the_fp32_cast(tmp_path):
    """A checkpoint directory on disk (no download): --layers cuts the stack to its first layers
    before the cast to fp32, the config follows the cut, and the vocabulary line reports the
    embedding rows (no tokenizer files here: tokenizer length None)."""
    from transformers.models.qwen3_5.modeling_qwen3_5 import Qwen3_5ForCausalLM

    from _tiny import tiny_hf_model

    model, _ = tiny_hf_model(seed=3, layers=8)
    ckpt = Qwen3_5ForCausalLM(model.config)
    ckpt.to(torch.bfloat16).save_pretrained(tmp_path)
    text, head, vocab = equivalence._load(str(tmp_path), 0, layers=3)
    assert len(text.layers) == 3 and text.config.num_hidden_layers == 3
    assert text.config.layer_types == list(model.config.layer_types[:3])
    assert text.embed_tokens.weight.dtype == torch.float32 and head.weight.dtype == torch.float32
    # the kept layers hold the checkpoint's (bf16-stored) weights exactly
    sd = ckpt.state_dict()
    assert torch.equal(text.layers[2].mlp.down_proj.weight, sd["model.layers.2.mlp.down_proj.weight"].float())
    assert vocab == {"embedding_rows": 256, "tokenizer_len": None, "spare_rows": None}
    full, _, _ = equivalence._load(str(tmp_path), 0)
    assert len(full.layers) == 8 and full.embed_tokens.weight.dtype == torch.float32
    try:
        equivalence._load(str(tmp_path), 0, layers=9)
    except ValueError as e:
        assert "exceeds" in str(e)
    else:
        raise AssertionError("--layers beyond the model must be refused")
