"""GEMM solution table for the decoder projections of the verify forward.

The dense projections (QKV, O, gate/up, down) are plain library GEMMs run by
``F.linear``. PyTorch's TunableOp can pick, per GEMM shape, the fastest of the
hipBLASLt and rocBLAS solutions instead of the library heuristic; the table in
``gemm_mi355x.csv`` holds those picks for the shapes of the benchmark
workloads on MI355X (``make_gemm_table.py`` regenerates it on a GPU). Shapes not
in the table fall back to the library's default choice; a table written for a
different PyTorch / ROCm / hipBLASLt build is ignored by TunableOp's validators.

Set ``FLASHGRPO_AMD_GEMM_TABLE=off`` to leave TunableOp untouched, or to a path to
use another table.
"""
from __future__ import annotations

import os

DEFAULT_TABLE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "gemm_mi355x.csv")
_state = {"done": False, "active": False}


def use_tuned_gemms(path: str | None = None) -> bool:
    """Enable TunableOp in read-only mode with the solution table (once per process).
    Returns whether a table is in use."""
    if _state["done"]:
        return _state["active"]
    _state["done"] = True
    choice = os.environ.get("FLASHGRPO_AMD_GEMM_TABLE", "")
    if choice.lower() == "off":
        return False
    table = path or choice or DEFAULT_TABLE
    if not os.path.exists(table):
        return False
    import torch.cuda.tunable as tunable

    if tunable.is_enabled() and tunable.tuning_is_enabled():  # a caller is tuning: leave it alone
        return False
    tunable.enable(True)
    tunable.tuning_enable(False)  # read-only: with tuning off TunableOp writes nothing back
    tunable.set_filename(table, insert_device_ordinal=False)
    _state["active"] = bool(tunable.read_file(table))
    return _state["active"]
