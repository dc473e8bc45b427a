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
