"""Error bounds of the bf16 Gated DeltaNet kernels against the fp32 oracle on the same bf16 inputs.

bf16 carries 8 significant bits: rounding a value x moves it by at most u|x| with u = 2^-8.
The kernels round the MFMA operands (the state S before K S and Q S, the T1/T2/P fragments, V')
and the outputs to bf16 and accumulate in fp32, so every output element is a short chain of
dot products whose operands each carry a relative error of at most u; the chain is
O = e^gamma Q S + P V' with V' = T2 V - T1 (K S). The bound therefore has an absolute part
scaled by the output's own range and a relative part for the final rounding:
  outputs:  |d| <= 4u * max|ref| + 2u * |ref|        (2^-6 max|ref| + 2^-7 |ref|)
  states:   |d| <= 2u * max|ref|                     (2^-7 max|ref|)
The state is fp32; its error comes from the bf16 V' folded into each update and decays with the
gate, so it stays at a few u of the state's range however many blocks are carried.
tests/test_oracle_gdn.py checks that a dropped or a 2% mis-scaled carry, and a fork from the
wrong block, exceed these bounds many times over on the slow-decay inputs.
"""

import torch

U_BF16 = 2.0 ** -8


def out_bound(ref: torch.Tensor) -> torch.Tensor:
    r = ref.float()
    return 4 * U_BF16 * r.abs().max() + 2 * U_BF16 * r.abs()


def state_bound(ref: torch.Tensor) -> torch.Tensor:
    r = ref.float()
    return (2 * U_BF16 * r.abs().max()).expand_as(r)


def excess(got: torch.Tensor, ref: torch.Tensor, bound) -> tuple[float, float]:
    """(max of |d| - bound, max of |d| / bound): <= 0 and <= 1 when within the bound."""
    d = (got.float() - ref.float()).abs()
    b = bound(ref)
    return (d - b).max().item(), (d / b).max().item()
