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

``mlp_mi355x.csv`` (``make_mlp_table.py``) holds, per (rows, intermediate, hidden), the
measured times of the two ways to compute a decoder layer's MLP input -- the tuned
projection followed by ``fg_swiglu``, or the fused ``fg_gate_up_swiglu`` at each tile
height -- and the fastest; ``mlp_table_path`` looks it up
(``FLASHGRPO_AMD_MLP_TABLE=off`` or another path).

``linear_mi355x.csv`` (``make_linear_table.py``) holds, per projection kind (qkv, o, down) and
(rows, columns, hidden), the measured times of the library projection with the op that follows it
(``fg_rope_kv_write``; the residual add and ``fg_rmsnorm``) against the split-K
``fg_linear_parts`` with the kernel that finishes its parts, the best tile and split count of the
latter, and the faster path; ``linear_table_plan`` looks it up
(``FLASHGRPO_AMD_LINEAR_TABLE=off`` or another path). Rows of kind ``qkv_rope`` time the QKV projection
with its rotary epilogue (``fg_linear_rope_kv_write``) in the split-K columns; ``linear_table_times``
returns an entry's times.
"""
from __future__ import annotations

import os

DEFAULT_TABLE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "gemm_mi355x.csv")
DEFAULT_MLP_TABLE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "mlp_mi355x.csv")
DEFAULT_LINEAR_TABLE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "linear_mi355x.csv")
_state = {"done": False, "active": False}
_mlp = {}
_CHOICE = {"pair": 0, "fused64": 64, "fused128": 128, "fused192": 192, "fused256": 256}


def _nearest(cands, rows: int):
    """The value of the (rows, value) entry nearest to ``rows`` on a log scale (ties to the larger count)."""
    import math

    lr = math.log(max(int(rows), 1))
    return min(cands, key=lambda e: (abs(math.log(e[0]) - lr), -e[0]))[1]


def _mlp_read() -> None:
    """Reads the MLP path table once: (inter, hidden) -> sorted [(rows, path)] of the fastest
    path, and -> sorted [(rows, tile height)] of the fastest fused GEMM."""
    entries, fused = {}, {}
    choice = os.environ.get("FLASHGRPO_AMD_MLP_TABLE", "")
    path = DEFAULT_MLP_TABLE if not choice else (None if choice.lower() == "off" else choice)
    if path and os.path.exists(path):
        with open(path) as f:
            header = f.readline().strip().split(",")
            for line in f:
                row = dict(zip(header, line.strip().split(",")))
                if row.get("choice") in _CHOICE:
                    key = (int(row["inter"]), int(row["hidden"]))
                    entries.setdefault(key, []).append((int(row["rows"]), _CHOICE[row["choice"]]))
                    tiles = [(float(row[f"fused{t}_us"]), t) for t in (64, 128, 192, 256) if f"fused{t}_us" in row]
                    if tiles:
                        fused.setdefault(key, []).append((int(row["rows"]), min(tiles)[1]))
    _mlp.setdefault("entries", {k: sorted(v) for k, v in entries.items()})
    _mlp.setdefault("fused", {k: sorted(v) for k, v in fused.items()})


def _mlp_entries() -> dict:
    """(inter, hidden) -> sorted [(rows, path)] from the MLP path table (read once)."""
    if "entries" not in _mlp:
        _mlp_read()
    return _mlp["entries"]


def mlp_table_path(rows: int, inter: int, hidden: int):
    """The measured MLP input path for this shape: 0 (projection + fg_swiglu) or the fused GEMM's
    tile height (64 / 128 / 192 / 256), taken from the table entry of these sizes nearest in row count on a log
    scale (ties to the larger count); None when the table has no entry for (inter, hidden)."""
    cands = _mlp_entries().get((int(inter), int(hidden)))
    return _nearest(cands, rows) if cands else None


def mlp_table_fused_tile(rows: int, inter: int, hidden: int):
    """The fused GEMM's fastest measured tile height for this shape (nearest entry, as
    ``mlp_table_path``), whichever path the table chose; None when the table has no entry."""
    if "fused" not in _mlp:
        _mlp_read()
    cands = _mlp["fused"].get((int(inter), int(hidden)))
    return _nearest(cands, rows) if cands else None


_lin = {}


def _linear_read() -> None:
    """Reads the projection path table once: (kind, cols, hidden) -> sorted [(rows, plan)] with
    plan (tile_m, tile_n, splits, stages) for the split-K kernel or () for the library, and
    -> sorted [(rows, split-K plan)] of the best measured split-K plan whichever path won."""
    entries, split, times = {}, {}, {}
    choice = os.environ.get("FLASHGRPO_AMD_LINEAR_TABLE", "")
    path = DEFAULT_LINEAR_TABLE if not choice else (None if choice.lower() == "off" else choice)
    if path and os.path.exists(path):
        with open(path) as f:
            header = f.readline().strip().split(",")
            for line in f:
                row = dict(zip(header, line.strip().split(",")))
                if row.get("choice") not in ("library", "split_k"):
                    continue
                # a table without a stages column was measured with the 2-stage ring
                sk = (int(row["tile_m"]), int(row["tile_n"]), int(row["splits"]), int(row.get("stages", 2)))
                key = (row["kind"], int(row["cols"]), int(row["hidden"]))
                entries.setdefault(key, []).append((int(row["rows"]), sk if row["choice"] == "split_k" else ()))
                split.setdefault(key, []).append((int(row["rows"]), sk))
                times.setdefault(key, []).append((int(row["rows"]), (float(row["library_us"]),
                                                                     float(row["split_k_us"]), sk)))
    _lin.setdefault("entries", {k: sorted(v) for k, v in entries.items()})
    _lin.setdefault("split", {k: sorted(v) for k, v in split.items()})
    _lin.setdefault("times", {k: sorted(v) for k, v in times.items()})


def _linear_entries() -> dict:
    """(kind, cols, hidden) -> sorted [(rows, plan)] from the projection path table (read once);
    plan is (tile_m, tile_n, splits, stages) for the split-K kernel or () for the library."""
    if "entries" not in _lin:
        _linear_read()
    return _lin["entries"]


def linear_table_plan(kind: str, rows: int, cols: int, hidden: int):
    """The measured projection path for this shape: (tile_m, tile_n, splits, stages) of the split-K kernel,
    () for the library projection, from the table entry of this kind and these sizes nearest in row
    count on a log scale (ties to the larger count); None when the table has no such entry. Row
    counts above twice the largest measured one take the library."""
    cands = _linear_entries().get((kind, int(cols), int(hidden)))
    if not cands:
        return None
    if int(rows) > 2 * cands[-1][0]:
        return ()
    return _nearest(cands, rows)


def linear_table_times(kind: str, rows: int, cols: int, hidden: int):
    """(library_us, split_k_us, split-K plan) of the table entry of this kind and these sizes
    nearest in row count (as ``linear_table_plan``); None when the table has no such entry or the
    row count is above twice the largest measured one. Kind "qkv_rope" holds the q/k/v projection
    with the rotary epilogue (``fg_linear_rope_kv_write``) in the split-K columns."""
    if "times" not in _lin:
        _linear_read()
    cands = _lin["times"].get((kind, int(cols), int(hidden)))
    if not cands or int(rows) > 2 * cands[-1][0]:
        return None
    return _nearest(cands, rows)


def linear_table_split_plan(kind: str, rows: int, cols: int, hidden: int):
    """The best measured split-K plan for this shape (nearest entry, as ``linear_table_plan``),
    whichever path the table chose; None when the table has no such entry."""
    if "split" not in _lin:
        _linear_read()
    cands = _lin["split"].get((kind, int(cols), int(hidden)))
    return _nearest(cands, rows) if cands else None


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
