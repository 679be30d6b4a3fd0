"""The MLP input-path table (tuning/mlp_mi355x.csv): format, lookup and coverage (no GPU)."""
import csv
import math
import os

import pytest

from flashgrpo_amd import tuning
from flashgrpo_amd.models.target import TargetConfig

TABLE = tuning.DEFAULT_MLP_TABLE


def rows():
    with open(TABLE) as f:
        return list(csv.DictReader(f))


@pytest.mark.skipif(not os.path.exists(TABLE), reason="no MLP path table")
def test_table_choices_are_the_fastest_measured_path():
    for r in rows():
        t = {k: float(r[k + "_us"]) for k in ("pair", "fused64", "fused128", "fused192", "fused256")}
        # the generator picks on unrounded times; the file keeps one decimal, so a
        # choice may tie the minimum after rounding but never exceed it by a step
        assert t[r["choice"]] <= min(t.values()) + 0.05, r
        assert all(v > 0 for v in t.values())


@pytest.mark.skipif(not os.path.exists(TABLE), reason="no MLP path table")
def test_table_covers_every_benchmark_model_and_lookup_returns_entries():
    have = {(int(r["inter"]), int(r["hidden"])) for r in rows()}
    for preset in ("tiny", "qwen25_1p5b", "qwen25_7b", "qwen25_14b", "llama31_8b"):
        cfg = getattr(TargetConfig, preset)()
        assert (cfg.intermediate, cfg.hidden) in have, preset
    code = {"pair": 0, "fused64": 64, "fused128": 128, "fused192": 192, "fused256": 256}
    for r in rows():
        assert tuning.mlp_table_path(int(r["rows"]), int(r["inter"]), int(r["hidden"])) == code[r["choice"]]


def test_lookup_takes_the_nearest_row_count_on_a_log_scale(monkeypatch):
    monkeypatch.setitem(tuning._mlp, "entries", {(100, 64): [(64, 0), (256, 192), (1024, 256)]})
    assert tuning.mlp_table_path(100, 100, 64) == 0          # log distance to 64 smaller than to 256
    assert tuning.mlp_table_path(128, 100, 64) == 192         # equal log distance: the larger count
    assert tuning.mlp_table_path(600, 100, 64) == 256
    assert tuning.mlp_table_path(10 ** 6, 100, 64) == 256
    assert tuning.mlp_table_path(1, 100, 64) == 0
    assert tuning.mlp_table_path(64, 101, 64) is None         # sizes not in the table
    assert math.isclose(math.log(128) - math.log(64), math.log(256) - math.log(128))


@pytest.mark.skipif(not os.path.exists(TABLE), reason="no MLP path table")
def test_fused_tile_lookup_is_the_fastest_measured_tile_height():
    for r in rows():
        t = {h: float(r[f"fused{h}_us"]) for h in (64, 128, 192, 256)}
        got = tuning.mlp_table_fused_tile(int(r["rows"]), int(r["inter"]), int(r["hidden"]))
        assert t[got] == min(t.values()), r


def test_fused_tile_lookup_nearest_row_count(monkeypatch):
    monkeypatch.setitem(tuning._mlp, "fused", {(100, 64): [(64, 64), (1024, 256)]})
    assert tuning.mlp_table_fused_tile(100, 100, 64) == 64
    assert tuning.mlp_table_fused_tile(5000, 100, 64) == 256
    assert tuning.mlp_table_fused_tile(64, 101, 64) is None
