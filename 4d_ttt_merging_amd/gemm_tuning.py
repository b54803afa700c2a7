"""GEMM kernel selection for the block's Linear layers on MI355X.

The qkv, output-projection and MLP Linears stay torch GEMMs (hipBLASLt).  Its
default heuristic picks kernels that are up to ~25% slower than the best
solution for the aggregator's shapes (e.g. qkv, 32,928 x 3,072 x 1,024: 206 us
against 151 us).  `use_tuned_gemms()` switches on PyTorch's TunableOp with
tuning off and loads `tuning/gemm_gfx950.csv`, the solutions TunableOp measured
fastest for these shapes (written by `tuning/tune_gemms.py`).  Shapes missing
from the table keep the default selection.  The chosen kernels are ordinary
hipBLASLt GEMMs: results differ from the default selection only by the
accumulation order of the fp32 sums.

TunableOp is process-wide state: every GEMM torch runs afterwards consults the
table.  The table's validator lines pin the torch / HIP / hipBLASLt / rocBLAS
versions and the GPU; on a mismatch the table is not used.
"""
from __future__ import annotations

from pathlib import Path

import torch

TABLE = Path(__file__).resolve().parent / "tuning" / "gemm_gfx950.csv"


def use_tuned_gemms(path: str | Path | None = None) -> bool:
    """Enable TunableOp with the recorded GEMM selections; True if the table was loaded.

    If the table cannot be read or its validators do not match this process,
    TunableOp is switched off again and torch keeps its default GEMM choice.
    """
    table = Path(path) if path is not None else TABLE
    tunable = torch.cuda.tunable
    if not table.exists():
        return False
    tunable.enable(True)
    tunable.tuning_enable(False)
    loaded = bool(tunable.read_file(str(table)))
    if not loaded:
        tunable.enable(False)
    return loaded


def default_gemms() -> None:
    """Switch TunableOp off again (torch's default hipBLASLt heuristic)."""
    torch.cuda.tunable.enable(False)
