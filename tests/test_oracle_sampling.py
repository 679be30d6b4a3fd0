"""Pins the oracle's supplied-noise sampler and the exact_target acceptance walk.

Pins: the weight table against float64 2^x and against the device's generated header,
the weight against float64 exp (accuracy, special values, monotonicity); the exact
per-token probability of the
noise rule against the reference's closed form ``logits_to_probs``; the
reference's distribution tests (50k draws, |dp| < 0.015) and known answers
(greedy, packed == dense, b200 correction token and its emitted-token law).
"""
import json
import os

import numpy as np
import pytest

from oracle import sampling as S
from oracle import tree as T

CASES = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "reference_cases.json")))


def _noise(n, seed=1234, draw=1):
    return np.array([S.counter_noise(seed, 0, i, draw) for i in range(n)], dtype=np.uint64)


HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "ss-grpo_amd", "csrc",
                      "fg_exp2_table.h")


def _header_table():
    import re

    text = open(HEADER).read()
    vals = [int(v, 16) for v in re.findall(r"0x([0-9a-f]{16})ull", text)]
    kt = float(re.search(r"kWeightKt = ([0-9.e+-]+)f", text).group(1))
    zmax = float(re.search(r"kWeightZmax = ([0-9.e+-]+)f", text).group(1))
    return vals, kt, zmax


def test_weight_table_pins():
    t = S._TABLE.astype(np.int64)
    assert t[0] == 2 ** 31 and t[1024] == 2 ** 30 and np.all(np.diff(t) < 0)
    exact = 2.0 ** 31 * np.exp2(-np.arange(1025) / 1024.0)  # float64: ~2e-7 absolute error
    frac = exact - np.floor(exact)
    assert np.all(np.abs(frac - 0.5) > 1e-5)  # no entry near a rounding tie: float64 decides it
    assert np.array_equal(t, np.floor(exact + 0.5).astype(np.int64))
    # 2^(-r/1024) * 2^(-(1024-r)/1024) = 1/2: products of mirrored entries within rounding of 2^61
    prod = t[1:1024].astype(object) * t[1023:0:-1].astype(object)
    assert all(abs(p - 2 ** 61) <= (a + b) // 2 + 1 for p, a, b in zip(prod, t[1:1024], t[1023:0:-1]))
    # the device's generated table packs T[r] | (T[r] - T[r+1]) << 32, and the same constants
    vals, kt, zmax = _header_table()
    assert vals == [int(t[r]) | (int(t[r] - t[r + 1]) << 32) for r in range(1024)]
    assert np.float32(kt) == S.KT_BASE and np.float32(zmax) == S.Z_MAX


def test_weight_scale_is_nearest_float32():
    exact = 2.0 ** 20 / np.log(2.0)
    kt = float(S.KT_BASE)
    ulp = float(np.spacing(S.KT_BASE))
    assert abs(kt - exact) <= ulp / 2
    assert S.weight_scale(1.0) == S.KT_BASE and S.weight_scale(None) == S.KT_BASE
    assert S.weight_scale(0.7) == np.float32(S.KT_BASE / np.float32(0.7))


@pytest.mark.parametrize("T_", [1.0, 0.7, 1.3])
def test_weight_accuracy_against_exp(T_):
    """q / 2^40 against float64 exp((x - m) / T) for 2M logits spread over the range that
    carries weight: within 2.5e-6 relative (fp32 rounding of m - x and of its product with
    kt, 2^-20-octave steps and the linear interpolation), and within one unit of q where
    q is small."""
    x = np.concatenate([[0.0], -np.linspace(0.0, 27.0 * T_, 2_000_001)[1:]]).astype(np.float32)
    q = S.quantized_weights(x, T_).astype(np.float64)
    want = np.exp(x.astype(np.float64) / np.float64(np.float32(T_))) * 2.0 ** 40
    big = want > 2.0 ** 24
    assert np.max(np.abs(q[big] - want[big]) / want[big]) < 2.5e-6
    assert np.max(np.abs(q[~big] - want[~big])) <= 1.0 + 2.5e-6 * 2.0 ** 24
    assert q[0] == 2.0 ** 40


def test_weight_special_values_and_order():
    x = np.array([1.0, np.nan, -np.inf, 1.0 - 30.0, 0.5, 1.0], np.float32)
    q = S.quantized_weights(x)
    assert q[0] == q[5] == 2 ** 40 and q[1] == 0 and q[2] == 0 and q[3] == 0 and 0 < q[4] < 2 ** 40
    assert S.row_max(x) == np.float32(1.0)  # NaN ignored, as the device's fmaxf
    assert S.quantized_weights(np.array([np.inf, 0.0, np.inf], np.float32)).tolist() == [0, 0, 0]
    assert S.quantized_weights(np.full(3, -np.inf, np.float32)).tolist() == [0, 0, 0]
    # a weight never increases as the logit decreases
    grid = -np.sort(np.random.default_rng(1).random(200_000).astype(np.float32) * 30.0)  # 0 down to -30
    grid = np.concatenate([[np.float32(0.0)], grid]).astype(np.float32)
    qg = S.quantized_weights(grid)
    assert np.all(np.diff(qg.astype(np.int64)) <= 0)
    # zeros of either sign weigh the same
    assert S.quantized_weights(np.array([0.0, -0.0], np.float32)).tolist() == [2 ** 40, 2 ** 40]


def test_quantised_max_is_exactly_two_pow_40():
    x = np.random.default_rng(0).standard_normal(1000).astype(np.float32)
    q = S.quantized_weights(x)
    assert q[np.argmax(x)] == 2 ** 40 and q.max() == 2 ** 40


@pytest.mark.parametrize("top_p,top_k,T_", [(1.0, None, 1.0), (0.9, None, 1.0), (1.0, 5, 0.7), (0.8, 12, 1.3), (0.5, None, 0.8)])
def test_exact_rule_probabilities_match_closed_form(top_p, top_k, T_):
    rng = np.random.default_rng(11)
    for _ in range(5):
        x = (rng.standard_normal(64) * 2).astype(np.float32)
        p_rule = S.token_probabilities(x, temperature=T_, top_p=top_p, top_k=top_k)
        p_ref = S.logits_to_probs(x, temperature=T_, top_p=top_p, top_k=top_k)
        assert abs(p_rule.sum() - 1.0) < 1e-12
        assert np.max(np.abs(p_rule - p_ref)) < 2e-6


def test_keep_rule_boundary_equal_mass():
    # Four equal logits at top_p 0.75: the 4th candidate's preceding mass is
    # exactly 0.75, which the reference keeps (cumsum > top_p is false).
    keep = S.kept_mask(np.zeros(4, np.float32), S.quantized_weights(np.zeros(4, np.float32)), top_p=0.75)
    assert keep.all()
    keep = S.kept_mask(np.zeros(4, np.float32), S.quantized_weights(np.zeros(4, np.float32)), top_p=0.74)
    assert keep.tolist() == [True, True, True, False]


def test_reference_nucleus_distribution_tests():
    # flashgrpo/tests/test_exact_acceptance_distribution.py:17-37
    c = CASES["acceptance"]
    for i, case in enumerate(c["nucleus_law"]):
        x = np.array(case["logits"], np.float32)
        draws = S.sample_same_row(x, _noise(c["nucleus_draws"], seed=321 + i), temperature=c["nucleus_temperature"],
                                  top_p=case["top_p"])
        obs = np.bincount(draws, minlength=4) / draws.size
        exp = S.logits_to_probs(x, temperature=c["nucleus_temperature"], top_p=case["top_p"])
        assert np.max(np.abs(obs - exp)) < c["nucleus_tol"]


def test_vectorised_sampler_equals_scalar_sampler():
    rng = np.random.default_rng(2)
    x = (rng.standard_normal(300) * 3).astype(np.float32)
    nz = _noise(200, seed=9)
    for kw in [dict(), dict(top_p=0.9), dict(top_k=7), dict(top_k=20, top_p=0.6, temperature=0.5)]:
        vec = S.sample_same_row(x, nz, **kw)
        sca = [S.sample_row(x, int(u), **kw) for u in nz]
        assert vec.tolist() == sca


def test_inverse_cdf_brute_force_small_vocab():
    x = np.array([0.3, -1.0, 2.0, 0.0, 0.5], np.float32)
    q = S.quantized_weights(x)
    total = int(q.sum(dtype=np.uint64))
    cum = np.cumsum([int(v) for v in q])
    for u in np.linspace(0, 2 ** 32 - 1, 997).astype(np.uint64):
        tgt = (total * int(u)) >> 32
        want = int(np.argmax(cum > tgt))
        assert S.sample_row(x, int(u)) == want
    assert S.sample_row(x, 0) == 0 and S.sample_row(x, 2 ** 32 - 1) == 4


def test_greedy_first_maximum():
    assert S.sample_row(np.array([1.0, 3.0, 3.0], np.float32), 0, do_sample=False) == 1
    assert S.sample_row(np.array([1.0, 3.0, 3.0], np.float32), 0, temperature=0) == 1


def test_counter_noise_is_stable_and_distinct():
    a = S.counter_noise(1, 2, 3, 4)
    assert a == S.counter_noise(1, 2, 3, 4) and 0 <= a < 2 ** 32
    vals = {S.counter_noise(1, s, q, d) for s in range(4) for q in range(8) for d in range(5)}
    assert len(vals) == 4 * 8 * 5
    u = np.array([S.counter_noise(7, 0, i, 0) for i in range(20000)], np.float64) / 2 ** 32
    assert abs(u.mean() - 0.5) < 0.01


def _hot_logits(shape, hot, vocab):
    lg = np.full(shape + (vocab,), -10.0, np.float32)
    for h in hot:
        lg[tuple(h[:-1]) + (h[-1],)] = 10.0
    return lg


def test_greedy_walk_known_answers():
    c = CASES["acceptance"]
    g = c["greedy_single"]
    t = T.Tree(g["tokens"], g["parents"], [1, 2, 2])
    lg = _hot_logits((1, 3), [[0] + h for h in g["hot"]], g["vocab"])
    tok, nodes, _ = S.accept_walk([t], lg, [[0, 0, 0]], do_sample=False, temperature=1.0, top_p=1.0, top_k=None)
    assert tok == [g["expect_tokens"]] and nodes == [g["expect_nodes"]]

    p = c["packed"]
    trees = [T.Tree(x["tokens"], x["parents"], [1, 2, 2, 3]) for x in p["trees"]]
    dense = _hot_logits((2, 4), p["hot"], p["vocab"])
    packed = np.stack([dense[0, 0], dense[0, 1], dense[1, 0], dense[1, 2]])
    nz = [[0] * 4] * 2
    kw = dict(do_sample=False, temperature=1.0, top_p=1.0, top_k=None)
    r_dense = S.accept_walk(trees, dense, nz, **kw)
    r_packed = S.accept_walk(trees, packed, nz, slots=p["slots"], **kw)
    assert r_dense == r_packed
    assert r_dense == (p["expect_tokens"], p["expect_nodes"], p["expect_last"])


def test_b200_correction_known_answer_and_law():
    c = CASES["acceptance"]["correction"]
    t = T.Tree(c["tokens"], c["parents"], [1, 2])
    lg = _hot_logits((1, 2), [[0] + h for h in c["hot"]], c["vocab"])
    tok, nodes, _, corr = S.accept_walk([t], lg, [[0]], do_sample=False, temperature=1.0, top_p=1.0, top_k=None,
                                        emit_correction=True)
    assert tok == [c["expect_tokens"]] and nodes == [c["expect_nodes"]] and corr == [c["expect_correction"]]

    law = CASES["acceptance"]["correction_law"]
    row = np.log(np.array(law["probs"])).astype(np.float32)
    draws = S.sample_same_row(row, _noise(law["draws"], seed=456))
    # child token 0 accepted iff the draw is 0, otherwise the draw is the correction
    emitted = draws
    obs = np.bincount(emitted, minlength=2) / emitted.size
    assert np.max(np.abs(obs - np.array(law["probs"]))) < law["tol"]
    t2 = T.Tree(law["tokens"], law["parents"], [1, 2])
    lg2 = np.broadcast_to(row, (2, 2))
    for u in _noise(50, seed=456):
        tok, _, _, corr = S.accept_walk([t2], lg2[None], [[int(u)]], do_sample=True, temperature=1.0, top_p=1.0,
                                        top_k=None, emit_correction=True)
        d = S.sample_row(row, int(u))
        assert (tok[0][1:] == [d]) if d == 0 else (corr[0] == d and tok[0] == [2])


def test_clamp_accepted():
    toks, nodes, fin, eos = S.clamp_accepted([5, 7, 2, 9], [0, 1, 3, 6], remaining=10, eos_token_id=2, old_len=3,
                                             max_length=100)
    assert toks == [5, 7, 2] and nodes == [0, 1, 3] and fin and eos
    toks, nodes, fin, _ = S.clamp_accepted([5, 7, 8], [0, 1, 3], remaining=2, eos_token_id=2, old_len=98,
                                           max_length=100)
    assert toks == [5, 7] and fin
    toks, _, fin, _ = S.clamp_accepted([5, 7], [0, 1], remaining=0, eos_token_id=2, old_len=100, max_length=100)
    assert toks == [5] and fin
