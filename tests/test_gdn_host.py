"""Host-side choices of the state-fork layer that need no GPU."""

from dllm_qwen38_amd import gdn


def test_fork_workgroups_rule():
    """One workgroup per (sequence, value head), or two when twice that fits in the chip; the
    default schedule puts the conv beside the fork only when this leaves compute units free."""
    cus = 256
    assert gdn.fork_workgroups(cus, 4, 48) == 192       # 27B-class layer: 64 CUs free
    assert gdn.fork_workgroups(cus, 8, 16) == 256       # 0.8B-class layer: split, chip full
    assert gdn.fork_workgroups(cus, 1, 48) == 96        # one sequence of the 27B stack: split
    assert gdn.fork_workgroups(cus, 8, 48) == 384       # more heads than CUs: no split
    assert gdn.fork_workgroups(cus, 2, 64) == 256
    assert gdn.fork_workgroups(cus, 3, 43) == 129       # 2 * 129 > 256: one per head


def test_default_pieces_rule():
    """The default schedule is conv then fork, one launch each, at every shape: block ranges beside
    the conv measured no faster at the 27B-class layer once the fork sped up, and slower where the
    column split fills the chip."""
    cus = 256
    for B, Hv, nb in ((4, 48, 128), (4, 48, 32), (1, 48, 64), (8, 16, 64), (8, 48, 128)):
        assert gdn.default_pieces(cus, B, Hv, nb) == 1
