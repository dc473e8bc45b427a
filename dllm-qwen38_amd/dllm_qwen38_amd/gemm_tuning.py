"""GEMM solution choices for the library GEMMs around the path (the projections, MLP and lm_head of
the 27B-class stack, bf16, both streams), picked on MI355X by PyTorch's TunableOp.

`gemm_tuning_gfx950.csv` is TunableOp's own results table: per GEMM shape the rocBLAS or
hipBLASLt solution that measured fastest, with validator lines for the torch, HIP, hipBLASLt and
rocBLAS versions and the GPU architecture it was made with. `enable()` loads it with run-time
tuning off, so a shape the table lacks keeps the library's default choice. TunableOp rejects the
table when a validator differs (another library build or GPU). The GEMMs stay library calls; the
table only chooses among the library's own solutions (the stack's forward with per-stream MLPs
measured 61.9 -> 56.6 ms on MI355X).
"""

import os

import torch

TABLE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "gemm_tuning_gfx950.csv")


def table_entries(path: str = TABLE) -> dict:
    """The table's validators and GEMM entries: {"validators": {name: value}, "gemms": [(op, shape,
    solution, ms)]}."""
    val, gemms = {}, []
    with open(path) as f:
        for line in f:
            parts = line.strip().split(",")
            if len(parts) == 3 and parts[0] == "Validator":
                val[parts[1]] = parts[2]
            elif len(parts) == 4:
                gemms.append((parts[0], parts[1], parts[2], float(parts[3])))
    return {"validators": val, "gemms": gemms}


def enable(device: int = 0) -> bool:
    """Use the table for torch's GEMMs in this process (no tuning at run time). Returns whether it
    was loaded: False off gfx950, without a GPU, or when TunableOp rejects the table."""
    if not torch.cuda.is_available():
        return False
    arch = torch.cuda.get_device_properties(device).gcnArchName
    if not arch.startswith(table_entries()["validators"].get("GCN_ARCH_NAME", "?").split(":")[0]):
        return False
    from torch.cuda import tunable

    tunable.enable(True)
    tunable.tuning_enable(False)
    tunable.record_untuned_enable(False)
    ok = bool(tunable.read_file(TABLE))
    if not ok:
        tunable.enable(False)
    return ok
