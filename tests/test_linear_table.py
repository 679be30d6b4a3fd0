"""The projection-path table (tuning/linear_mi355x.csv): format, lookup and coverage (no GPU)."""
import csv
import os

import pytest

from flashgrpo_amd import kernels as K
from flashgrpo_amd import tuning
from flashgrpo_amd.models.target import TargetConfig, default_linear_plan

TABLE = tuning.DEFAULT_LINEAR_TABLE


def rows():
    with open(TABLE) as f:
        return list(csv.DictReader(f))


@pytest.mark.skipif(not os.path.exists(TABLE), reason="no projection path table")
def test_choices_are_the_faster_measured_path_and_plans_are_valid():
    for r in rows():
        lib, sk = float(r["library_us"]), float(r["split_k_us"])
        assert lib > 0 and sk > 0
        fast = "split_k" if sk < lib else "library"
        # one decimal in the file: a choice may tie after rounding but never lose by a step
        assert r["choice"] == fast or abs(lib - sk) < 0.05, r
        tm, tn, s, ns = int(r["tile_m"]), int(r["tile_n"]), int(r["splits"]), int(r["stages"])
        assert tm in K.LINEAR_TILES and tn in K.LINEAR_TILES and ns in (2, 3, 4), r
        assert K.linear_splits(int(r["hidden"]), s) == s, r


@pytest.mark.skipif(not os.path.exists(TABLE), reason="no projection path table")
def test_table_covers_the_bf16_benchmark_models_and_lookup_returns_entries():
    have = {(r["kind"], int(r["cols"]), int(r["hidden"])) for r in rows()}
    for preset in ("qwen25_1p5b", "qwen25_7b", "qwen25_14b", "llama31_8b"):
        c = getattr(TargetConfig, preset)()
        d = c.head_dim
        for key in (("qkv", (c.q_heads + 2 * c.kv_heads) * d, c.hidden), ("o", c.hidden, c.q_heads * d),
                    ("down", c.hidden, c.intermediate)):
            assert key in have, (preset, key)
    for r in rows():
        plan = tuning.linear_table_plan(r["kind"], int(r["rows"]), int(r["cols"]), int(r["hidden"]))
        if r["choice"] == "split_k":
            assert plan == (int(r["tile_m"]), int(r["tile_n"]), int(r["splits"]), int(r["stages"]))
        else:
            assert plan == ()


def test_lookup_nearest_row_count_and_library_beyond_the_measured_range(monkeypatch):
    monkeypatch.setitem(tuning._lin, "entries", {("o", 64, 128): [(64, (64, 64, 2, 4)), (256, ()),
                                                                    (1024, (128, 128, 1, 2))]})
    assert tuning.linear_table_plan("o", 100, 64, 128) == (64, 64, 2, 4)
    assert tuning.linear_table_plan("o", 128, 64, 128) == ()          # equal log distance: the larger count
    assert tuning.linear_table_plan("o", 2048, 64, 128) == (128, 128, 1, 2)
    assert tuning.linear_table_plan("o", 2049, 64, 128) == ()        # beyond twice the largest measured count
    assert tuning.linear_table_plan("qkv", 64, 64, 128) is None       # kind not in the table


def test_default_plan_satisfies_the_kernel_rules():
    for rows_, cols, hidden in ((1, 64, 64), (416, 1536, 8960), (1856, 4608, 3584), (96, 2048, 1536)):
        tm, tn, s, ns = default_linear_plan(rows_, cols, hidden)
        assert tm in K.LINEAR_TILES and tn in K.LINEAR_TILES and ns in (2, 3, 4)
        assert K.linear_splits(hidden, s) == s


@pytest.mark.skipif(not os.path.exists(TABLE), reason="no projection path table")
def test_split_plan_lookup_returns_the_measured_split_k_plan_whichever_path_won():
    for r in rows():
        plan = tuning.linear_table_split_plan(r["kind"], int(r["rows"]), int(r["cols"]), int(r["hidden"]))
        assert plan == (int(r["tile_m"]), int(r["tile_n"]), int(r["splits"]), int(r["stages"]))


def test_split_plan_lookup_nearest_row_count(monkeypatch):
    monkeypatch.setitem(tuning._lin, "split", {("o", 64, 128): [(64, (64, 64, 2, 4)), (256, (128, 64, 1, 4))]})
    assert tuning.linear_table_split_plan("o", 100, 64, 128) == (64, 64, 2, 4)
    assert tuning.linear_table_split_plan("o", 10 ** 6, 64, 128) == (128, 64, 1, 4)  # no library cut-off
    assert tuning.linear_table_split_plan("qkv", 64, 64, 128) is None


@pytest.mark.skipif(not os.path.exists(TABLE), reason="no projection path table")
def test_fused_rotary_rows_pair_with_qkv_rows():
    """Every qkv_rope row (the projection with the rotary epilogue) has a qkv row of the same shape
    measured in the same run (the same library time) and a one-split plan."""
    by = {(r["kind"], r["rows"], r["cols"], r["hidden"]): r for r in rows()}
    fused = [r for r in rows() if r["kind"] == "qkv_rope"]
    assert fused
    for r in fused:
        q = by[("qkv", r["rows"], r["cols"], r["hidden"])]
        assert q["library_us"] == r["library_us"] and r["splits"] == "1", r
        t = tuning.linear_table_times("qkv_rope", int(r["rows"]), int(r["cols"]), int(r["hidden"]))
        assert t[:2] == (float(r["library_us"]), float(r["split_k_us"]))


def test_times_lookup_nearest_row_count_and_none_beyond_the_range(monkeypatch):
    monkeypatch.setitem(tuning._lin, "times", {("qkv_rope", 64, 128): [(64, (10.0, 9.0, (64, 64, 1, 4))),
                                                                       (512, (20.0, 25.0, (128, 64, 1, 2)))]})
    assert tuning.linear_table_times("qkv_rope", 100, 64, 128) == (10.0, 9.0, (64, 64, 1, 4))
    assert tuning.linear_table_times("qkv_rope", 1024, 64, 128)[2] == (128, 64, 1, 2)
    assert tuning.linear_table_times("qkv_rope", 1025, 64, 128) is None
    assert tuning.linear_table_times("qkv", 64, 64, 128) is None
