"""Pins the oracle's KV extraction on the reference's seed-17 case and the gather closed form."""
import json
import os

import numpy as np
import pytest

from oracle import kv as K

GOLD = os.path.join(os.path.dirname(__file__), "golden")
CASES = json.load(open(os.path.join(GOLD, "reference_cases.json")))
ARR = np.load(os.path.join(GOLD, "reference_arrays.npz"))


def test_seed17_in_place_equals_copy_equals_golden():
    # flashgrpo/tests/test_kv_path_extraction_matches_recompute.py:14-35
    c = CASES["seed17_kv"]
    key, value = ARR["seed17_key"], ARR["seed17_value"]
    old = [(key[:, :, :c["old_len"]].copy(), value[:, :, :c["old_len"]].copy())]
    copied, w1 = K.extract_accepted_path_kv(old, [(key.copy(), value.copy())], c["accepted"], in_place=False)
    compact, w2 = K.extract_accepted_path_kv(old, [(key.copy(), value.copy())], c["accepted"], in_place=True)
    assert w1 == w2 == 3
    assert np.array_equal(compact[0][0], copied[0][0]) and np.array_equal(compact[0][1], copied[0][1])
    assert np.array_equal(copied[0][0], ARR["seed17_expect_key"])
    assert np.array_equal(copied[0][1], ARR["seed17_expect_value"])


def test_aliasing_paths_read_before_write():
    # path [0, 2, 3]: destination slot 1 is written from node 2 while node 2's
    # own slot is later overwritten from node 3 -- sources must be read first.
    t = np.arange(1 * 1 * 6 * 2, dtype=np.float32).reshape(1, 1, 6, 2)
    out = K.extract_layer(t.copy(), np.array([[2, 4, 5]]), 2, 3)
    assert np.array_equal(out[0, 0, 2:5], t[0, 0, [2, 4, 5]])


def test_compact_rows_valid_rows_equal_reference_block():
    rng = np.random.default_rng(4)
    B, H, S, D = 3, 2, 20, 4
    cache = rng.standard_normal((B, H, S, D)).astype(np.float32)
    paths = [[0, 1, 4], [0], [0, 2, 5, 7]]
    old = 6
    ref, width = K.extract_accepted_path_kv([(cache[:, :, :old].copy(),) * 2], [(cache.copy(), cache.copy())], paths)
    seq = np.full(B, old)
    got = K.compact_rows(cache, seq, [p + [0] * (4 - len(p)) for p in paths], [len(p) for p in paths])
    for b, p in enumerate(paths):
        assert np.array_equal(got[b, :, old:old + len(p)], ref[0][0][b, :, old:old + len(p)])
        assert np.array_equal(got[b, :, :old], cache[b, :, :old])


def test_errors_match_reference():
    c = np.zeros((1, 1, 4, 2), np.float32)
    with pytest.raises(ValueError):
        K.extract_accepted_path_kv([(c[:, :, :2], c[:, :, :2])], [(c, c)], [[0, 2]])
    with pytest.raises(ValueError):
        K.extract_accepted_path_kv([(c[:, :, :2], c[:, :, :2])], [(c, c)], [[]])
    with pytest.raises(ValueError):
        K.extract_accepted_path_kv([(c[:, :, :2], c[:, :, :2])], [(c, c)], [])
