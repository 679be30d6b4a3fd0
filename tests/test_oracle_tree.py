"""Pins the oracle's planner, canonical top-k, tree builder and attention inputs.

Pins: the reference's own test inputs/known answers (tests/golden, built by
tests/golden/make_golden.py), hand-derived planner tables, the dense-count closed
form, torch.topk on tie-free data, and brute force on tiny trees.
"""
import json
import os

import numpy as np
import pytest

from oracle import tree as T

GOLD = os.path.join(os.path.dirname(__file__), "golden")
CASES = json.load(open(os.path.join(GOLD, "reference_cases.json")))
ARR = np.load(os.path.join(GOLD, "reference_arrays.npz"))


def test_dense_node_count_closed_form():
    rng = np.random.default_rng(0)
    for _ in range(200):
        ks = rng.integers(1, 6, size=rng.integers(0, 5)).tolist()
        brute = 1 + sum(int(np.prod(ks[: i + 1])) for i in range(len(ks)))
        assert T.dense_node_count(ks) == brute
        parents, depths, _ = T.dense_topology(ks, 10 ** 6)
        assert len(parents) == brute


@pytest.mark.parametrize("case", CASES["planner"], ids=lambda c: str(c["kw"]["active_batch_size"]) + c["kw"]["tree_mode"])
def test_plan_tree_matches_hand_derived_table(case):
    p = T.plan_tree(**case["kw"])
    for k, v in case["expect"].items():
        assert getattr(p, k) == v, (k, getattr(p, k), v)


def test_reference_planner_properties():
    # flashgrpo/tests/test_flashgrpo_smoke.py:4-45
    small, large = (T.plan_tree(**c["kw"]) for c in CASES["planner"][:2])
    assert small.actual_nodes >= large.actual_nodes
    adaptive = T.plan_tree(**CASES["planner"][2]["kw"])
    assert adaptive.node_budget_per_seq == 4 and adaptive.active_heads == 3


@pytest.mark.parametrize("case", CASES["fit"])
def test_fit_topk_to_budget(case):
    out = T.fit_topk_to_budget(case["topk"], case["budget"], min_topk_by_depth=case["mins"],
                               depth_weight_decay=case["decay"])
    assert out == case["expect"]
    assert T.dense_node_count(out) <= max(1, case["budget"])


def test_fit_never_exceeds_budget_and_is_maximal_per_depth():
    rng = np.random.default_rng(1)
    for _ in range(300):
        ks = rng.integers(1, 6, size=rng.integers(1, 5)).tolist()
        budget = int(rng.integers(1, 80))
        out = T.fit_topk_to_budget(ks, budget)
        assert T.dense_node_count(out) <= budget
        assert len(out) <= len(ks) and all(1 <= o <= k for o, k in zip(out, ks))


def test_seed7_batched_trees_match_torch_topk_golden():
    # flashgrpo/tests/test_reflex_optimized.py:16-36 (expected from torch.topk + BFS)
    case = CASES["seed7_tree"]
    roots = ARR["seed7_roots"]
    logits = list(ARR["seed7_logits"])
    plan = T.Plan(case["budget"], 2, case["topk"], 10, "fixed", "dense")
    trees = T.build_batch_trees(roots, logits, plan)
    assert [(t.tokens, t.parents) for t in trees] == [(g["tokens"], g["parents"]) for g in case["trees"]]
    per_row = [T.build_dense_tree(roots[b], [lg[b] for lg in logits], plan) for b in range(len(roots))]
    assert [(t.tokens, t.parents) for t in trees] == [(t.tokens, t.parents) for t in per_row]


def test_canonical_topk_tie_order_and_signed_zero():
    x = np.array([1.0, 3.0, 3.0, -0.0, 0.0, 3.0, 2.0], np.float32)
    idx, vals = T.topk_canonical(x, 5)
    assert idx.tolist() == [1, 2, 5, 6, 0]
    idx, _ = T.topk_canonical(np.array([-0.0, 0.0, -1.0], np.float32), 2)
    assert idx.tolist() == [0, 1]
    # bf16-style heavy ties: order must equal a stable descending sort
    rng = np.random.default_rng(3)
    y = np.round(rng.standard_normal(4000) * 4).astype(np.float32)
    ref = np.argsort(-y.astype(np.float64), kind="stable")[:17]
    assert T.topk_canonical(y, 17)[0].tolist() == ref.tolist()


def test_topology_matches_built_trees_and_truncation():
    rng = np.random.default_rng(5)
    for ks, budget in [([4, 2], 16), ([4, 2, 1, 1], 32), ([4, 3, 2], 16), ([3, 3, 3], 20), ([2], 2)]:
        B, V = 3, 50
        logits = [rng.standard_normal((B, V)).astype(np.float32) for _ in ks]
        plan = T.Plan(budget, len(ks), ks, T.dense_node_count(ks), "fixed", "dense")
        trees = T.build_batch_trees(rng.integers(0, V, B), logits, plan)
        parents, depths, ranks = T.dense_topology(ks, budget)
        for b, t in enumerate(trees):
            assert t.parents == parents and t.depths == depths
            assert t.node_count == min(budget, T.dense_node_count(ks))
            for n in range(1, t.node_count):
                cand = T.topk_canonical(logits[depths[n] - 2][b], ks[depths[n] - 2])[0]
                assert t.tokens[n] == cand[ranks[n]]


def test_mask_known_answer():
    # flashgrpo/tests/test_tree_attention_equivalence.py:9-20
    c = CASES["mask"]
    tree = T.Tree(c["tokens"], c["parents"], c["depths"])
    ids, mask, pos, valid = T.tree_attention_inputs([tree], np.ones((1, c["past"]), np.int64),
                                                    np.array([c["logical"]]), pad_token_id=0)
    n, past = c["node"], c["past"]
    assert valid[0, n]
    for a in c["allowed_tree"]:
        assert mask[0, 0, n, past + a] == 0
    for a in c["masked_tree"]:
        assert mask[0, 0, n, past + a] < -1e20
    assert pos[0, n] == c["position"]


def test_mask_brute_force_and_padding_rows():
    trees = [T.Tree([1, 2, 3], [-1, 0, 1], [1, 2, 3]), T.Tree([4, 5, 6, 7, 8], [-1, 0, 0, 1, 2], [1, 2, 2, 3, 3])]
    full = np.array([[0, 1, 1, 1], [1, 1, 1, 1]])
    ids, mask, pos, valid = T.tree_attention_inputs(trees, full, full.sum(-1), pad_token_id=9)
    assert ids[0].tolist() == [1, 2, 3, 9, 9] and valid[0].tolist() == [True] * 3 + [False] * 2
    assert pos[0].tolist() == [3, 4, 5, 0, 0] and pos[1].tolist() == [4, 5, 5, 6, 6]
    for b, t in enumerate(trees):
        for n in range(5):
            for m in range(5):
                if n < t.node_count:
                    want = m < t.node_count and m in t.ancestors_including_self(n)
                else:
                    want = m == n
                assert (mask[b, 0, n, 4 + m] == 0) == want
            assert ((mask[b, 0, n, :4] == 0) == full[b].astype(bool)).all()


def test_internal_slots_match_reference_packed_layout():
    # slot map of flashgrpo/tests/test_exact_acceptance_distribution.py:59-60
    c = CASES["acceptance"]["packed"]
    trees = [T.Tree(t["tokens"], t["parents"], [0] * 4) for t in c["trees"]]
    rows, nodes, slots = T.internal_slots(trees)
    assert slots == c["slots"] and rows == [0, 0, 1, 1] and nodes == [0, 1, 0, 2]


def test_ancestor_bits():
    parents = T.dense_topology([4, 2, 1, 1], 32)[0]
    bits = T.ancestor_bits(parents)
    t = T.Tree([0] * len(parents), parents, [0] * len(parents))
    for n, m in enumerate(bits):
        assert sorted(i for i in range(64) if m >> i & 1) == t.ancestors_including_self(n)


def test_adaptive_confidence_mapping():
    kw = dict(enabled=True, min_topk_by_depth=[1, 1, 1], low=0.15, high=0.45)
    assert T.topk_from_confidence(0.01, 4, 0, **kw) == 4
    assert T.topk_from_confidence(0.9, 4, 0, **kw) == 1
    assert T.topk_from_confidence(0.25, 4, 0, **kw) == 3
    assert T.topk_from_confidence(0.42, 4, 0, **kw) == 1
    assert T.topk_from_confidence(float("nan"), 4, 0, **kw) == 1
    assert T.topk_from_confidence(0.3, 4, 0, **dict(kw, enabled=False)) == 4
    assert T.quantile_linear([0.1, 0.2, 0.3, 0.4], 0.25) == pytest.approx(0.175)


def test_chain_trees_known_answer():
    """Hand-derived chain tree: V=6, k=(2, 2), budget 6. NaN and -inf become -1e9 and
    rank below every finite logit; equal logits resolve to the lower index."""
    nan, inf = float("nan"), float("inf")
    d0 = np.array([[0.1, 0.5, 0.3, nan, -inf, 0.5]], np.float32)           # root -> [1, 5]
    d1 = np.array([[nan, 0.2, 0.9, 0.9, 0.0, -1.0],                        # node 1 -> [2, 3]
                   [inf, 0.0, 0.1, 0.2, 0.3, 0.4]], np.float32)            # node 2 -> [0, 5]
    trees, pidx, toks = T.build_chain_trees([4], [d0, d1], [2, 2], budget=6)
    t = trees[0]
    assert t.tokens == [4, 1, 5, 2, 3, 0]
    assert t.parents == [-1, 0, 0, 1, 1, 2]
    assert t.depths == [1, 2, 2, 3, 3, 3]
    assert pidx == [[0, 0], [0, 0, 1]] and toks == [[1, 5], [2, 3, 0]]
    assert t.scores[5] == 1.0e9  # +inf clamps to 1e9
    # a NaN row ranks every finite logit first
    assert T.build_chain_trees([0], [np.array([[nan, -3.0, nan, -2.0]], np.float32)], [3], 9)[0][0].tokens == [0, 3, 1, 0]


def test_chain_trees_follow_dense_topology():
    rng = np.random.default_rng(8)
    for ks, budget in [([4, 2], 16), ([4, 3, 2], 16), ([2, 2, 2, 2], 12), ([3, 1], 40), ([1, 1, 1], 3)]:
        B, V = 3, 30
        logits, n = [], 1
        for k in ks:
            logits.append(rng.standard_normal((B * n, V)).astype(np.float32))
            n *= k
        trees, pidx, toks = T.build_chain_trees(rng.integers(0, V, B), logits, ks, budget)
        parents, depths, ranks = T.dense_topology(ks, budget)
        first = [depths.index(d) if d in depths else len(depths) for d in range(2, len(ks) + 3)]
        for b, t in enumerate(trees):
            assert t.parents == parents and t.depths == depths
            for node in range(1, t.node_count):
                d = depths[node] - 2
                par = parents[node]
                local = par - (first[d - 1] if d else 0)   # parent's index within its depth
                n_d = first[d] - (first[d - 1] if d else 0)
                row = logits[d][b * n_d + local]
                assert t.tokens[node] == T.topk_canonical(row, ks[d])[0][ranks[node]]
        # creation order is row-major: the parent rows of each depth never decrease
        for p in pidx:
            assert p == sorted(p)


def test_chain_confidence_matches_torch():
    import torch

    from oracle import decode as D

    rng = np.random.default_rng(9)
    x = rng.standard_normal((7, 33)).astype(np.float32) * 3
    x[2, 4] = np.nan
    x[3, :] = -np.inf
    sx = torch.nan_to_num(torch.from_numpy(x).double(), nan=-1e9, posinf=1e9, neginf=-1e9)
    top1 = torch.exp(sx.max(-1).values - torch.logsumexp(sx, -1)).numpy()
    assert np.allclose(D.chain_confidence(x), top1, rtol=1e-12, atol=0)
    v = torch.topk(sx, 2, dim=-1).values
    assert np.allclose(D.chain_confidence(x, "margin"), (v[:, 0] - v[:, 1]).numpy(), rtol=0, atol=0)


# --------------------------------------------------------------------------- sparse asymmetric (b200)
def _sparse_plan(nodes=(4, 3, 2), budget=10, heads=3, min3=1, mode="fixed", **kw):
    """The plan of flashgrpo_b200/tests/test_sparse_asymmetric_hrdcr.py:28-41."""
    return T.plan_tree(active_batch_size=1, num_medusa_heads=heads, tree_mode=mode, tree_layout="sparse_asymmetric",
                       cpeak_nodes=budget, min_tree_nodes_per_seq=1, max_tree_nodes_per_seq=budget,
                       max_tree_depth=4, fixed_tree_topk_by_depth=[4, 3, 2], sparse_nodes_by_head=list(nodes),
                       sparse_min_head3_nodes=min3, sparse_head3_min_budget=8, **kw)


def _proposal_logits(batch=1, vocab=17):
    """flashgrpo_b200/tests/test_sparse_asymmetric_hrdcr.py:44-46: descending logits,
    head i shifted by -0.1 i (float32)."""
    base = np.arange(vocab, dtype=np.float32)[::-1]
    return [np.tile(base - np.float32(i * 0.1), (batch, 1)).astype(np.float32) for i in range(3)]


def test_sparse_allocation_hand_derived():
    """Budget split of flashgrpo_b200/decoding/medusa_tree.py:411-444, worked by hand."""
    assert T.sparse_allocation(10, 3, [4, 3, 2], 1, 8) == [4, 3, 2]      # the reference test's plan
    assert T.sparse_allocation(32, 3, [5, 4, 0], 0, 8) == [5, 4]          # b200 defaults: head 3 dropped
    assert T.sparse_allocation(12, 3, [8, 8, 2], 1, 8) == [8, 2, 1]       # head 2 gives one node to head 3
    assert T.sparse_allocation(12, 3, [8, 8, 2], 3, 8) == [7, 1, 3]       # head 2 keeps one, head 1 gives the rest
    assert T.sparse_allocation(10, 3, [9, 9, 2], 3, 8) == [6, 0, 3]       # an empty head 2 stays in the list
    assert T.sparse_allocation(6, 3, [4, 3, 2], 1, 8) == [4, 1]           # budget below head3_min_budget
    assert T.sparse_allocation(1, 3, [4, 3, 2], 1, 8) == []
    p = _sparse_plan()
    assert (p.active_heads, p.topk_by_depth, p.nodes_by_head, p.actual_nodes, p.layout) == \
        (3, [4, 3, 2], [4, 3, 2], 10, "sparse_asymmetric")
    assert p.diversity_penalty == 0.05 and p.branch_score_temperature == 1.0
    # concurrency-aware: the dense planner's budget floor(cpeak / B), then the split
    q = T.plan_tree(active_batch_size=4, num_medusa_heads=3, tree_mode="concurrency_aware",
                    tree_layout="sparse_asymmetric", cpeak_nodes=64, min_tree_nodes_per_seq=1,
                    max_tree_nodes_per_seq=32, max_tree_depth=4, fixed_tree_topk_by_depth=[4, 3, 2],
                    sparse_nodes_by_head=[8, 6, 4])
    assert q.node_budget_per_seq == 16 and q.nodes_by_head == [8, 6, 1]


def test_sparse_tree_reference_invariants_and_known_answer():
    """flashgrpo_b200/tests/test_sparse_asymmetric_hrdcr.py:50-80, plus the exact trees
    worked by hand from the greedy rule (parent score + candidate score - 0.05 x picks)."""
    plan = _sparse_plan()
    t = T.build_sparse_trees([7], _proposal_logits(), plan, [True])[0]
    assert t.node_count == 10
    assert len({(p, k) for p, k in zip(t.parents, t.tokens)}) == 10
    for n, (p, d) in enumerate(zip(t.parents, t.depths)):
        assert (p == -1) if n == 0 else (0 <= p < n and t.depths[p] == d - 1)
    # head 1: tokens 0..3 (scores 16..13); head 2 picks (node1, 0) 31.9, (node2, 0) 30.9 over
    # (node1, 1) 30.9 - 0.05, then (node1, 1); head 3 picks (node5, 0), then (node6, 0) 46.7
    # over (node5, 1) 46.7 - 0.05.
    assert t.tokens == [7, 0, 1, 2, 3, 0, 0, 1, 0, 0]
    assert t.parents == [-1, 0, 0, 0, 0, 1, 2, 1, 5, 6]
    assert t.depths == [1, 2, 2, 2, 2, 3, 3, 3, 4, 4]
    assert abs(t.scores[8] - (16.0 + 15.9 + 15.8)) < 1e-5
    # head 3 gated off: its two nodes go to head 2 (reference: nodes_by_head + [0] == [4, 5, 0])
    r = T.build_sparse_trees([7], _proposal_logits(), plan, [False])[0]
    assert r.node_count == 10 and [r.depths.count(d) for d in (2, 3, 4)] == [4, 5, 0]
    assert r.parents[5:] == [1, 2, 1, 3, 2] and r.tokens[5:] == [0, 0, 1, 0, 1]


def test_sparse_greedy_without_penalty_is_a_sorted_pool():
    """With no penalty the greedy picks are the pool sorted by (cumulative desc, pair
    index asc): an independent formulation, checked on random tied scores."""
    rng = np.random.default_rng(11)
    for trial in range(200):
        npar, w = int(rng.integers(1, 6)), int(rng.integers(1, 7))
        ps = (rng.integers(-3, 3, npar) / 2).tolist()
        ts = (rng.integers(-3, 3, w) / 2).astype(np.float32).tolist()
        toks = rng.permutation(50)[:w].tolist()
        count = int(rng.integers(0, npar * w + 2))
        got = T.select_sparse_children(list(range(10, 10 + npar)), ps, toks, ts, count, 0.0)
        pool = [(ps[p] + ts[j], p * w + j) for p in range(npar) for j in range(w)]
        want = sorted(pool, key=lambda x: (-x[0], x[1]))[:count]
        assert [(10 + i // w, toks[i % w], c) for c, i in want] == got, trial


def test_sparse_greedy_penalty_spreads_parents_and_skips_nan():
    # equal pools: the penalty alternates parents instead of draining the first one
    got = T.select_sparse_children([1, 2], [0.0, 0.0], [5, 6, 7], [3.0, 2.99, 2.98], 4, 0.05)
    assert [(p, t) for p, t, _ in got] == [(1, 5), (2, 5), (1, 6), (2, 6)]
    # large penalty: every parent gets its best candidate first
    got = T.select_sparse_children([1, 2, 3], [1.0, 0.5, 0.0], [5, 6], [1.0, 0.9], 3, 10.0)
    assert [p for p, _, _ in got] == [1, 2, 3]
    # NaN and -inf values are never picked; an exhausted pool ends the picks
    got = T.select_sparse_children([1], [0.0], [5, 6, 7], [float("nan"), 1.0, float("-inf")], 3, 0.0)
    assert [(p, t) for p, t, _ in got] == [(1, 6)]
    assert T.select_sparse_children([1], [0.0], [5], [1.0], 0, 0.0) == []


def test_sparse_tree_extras_budget_and_widths():
    """Leftover head-1 candidates fill the budget (medusa_tree.py:658-671); heads past
    the third are ignored; widths keep head 3's count in reserve (:569-579)."""
    assert T.sparse_widths([4, 3, 2], 100) == [6, 5, 2] and T.sparse_widths([5, 4], 3) == [3, 3]
    plan = T.Plan(32, 3, [4, 3, 2], 10, "fixed", "sparse_asymmetric", [4, 3, 2], 1, 8, 1.0, 0.05)
    t = T.build_sparse_trees([7], _proposal_logits(), plan)[0]
    assert t.node_count == 12 and t.tokens[10:] == [4, 5] and t.parents[10:] == [0, 0] and t.depths[10:] == [2, 2]
    plan = T.Plan(11, 3, [4, 3, 2], 10, "fixed", "sparse_asymmetric", [4, 3, 2], 1, 8, 1.0, 0.05)
    assert T.build_sparse_trees([7], _proposal_logits(), plan)[0].tokens[10:] == [4]
    plan = T.Plan(8, 3, [4, 3, 2], 10, "fixed", "sparse_asymmetric", [4, 3, 2], 1, 8, 1.0, 0.05)
    t = T.build_sparse_trees([7], _proposal_logits(), plan)[0]
    assert t.node_count == 8 and t.depths == [1, 2, 2, 2, 2, 3, 3, 3]  # cut at the budget
    plan = T.Plan(10, 0, [], 1, "fixed", "sparse_asymmetric", [], 1, 8, 1.0, 0.05)
    assert T.build_sparse_trees([3, 4], _proposal_logits(2), plan)[1].tokens == [4]


def test_native_tree_inputs_from_reference_mask():
    """forward_tree's conversion: the tree block of build_tree_attention_inputs' additive
    mask gives each node its ancestor-or-self word (padded nodes: themselves only), and
    positions become offsets from the committed lengths (depth - 1 on real nodes)."""
    import torch

    from flashgrpo_amd.decoding.medusa_tree import CandidateTree, TreeTopology
    from flashgrpo_amd.decoding.tree_attention import build_tree_attention_inputs, tree_ancestor_bits
    from flashgrpo_amd.models.target import native_tree_inputs

    topo = TreeTopology([4, 3, 2], 40)
    sizes = [topo.num_nodes, 9, 1]
    trees = [CandidateTree(list(range(n)), list(topo.parents[:n]), list(topo.depths[:n])) for n in sizes]
    lens = torch.tensor([50, 7, 0])
    full = torch.zeros(3, 60, dtype=torch.long)
    for b, L in enumerate(lens.tolist()):
        full[b, :L] = 1
    for dtype in (torch.float32, torch.bfloat16):
        ids, mask, pos, valid = build_tree_attention_inputs(trees, full, lens, pad_token_id=0, dtype=dtype)
        anc, off = native_tree_inputs(mask, pos, lens.to(torch.int32))
        assert torch.equal(anc, tree_ancestor_bits(trees, ids.shape[1]))
        depth = torch.tensor([list(t.depths) + [1] * (ids.shape[1] - t.node_count) for t in trees])
        want = torch.where(valid, depth - 1, -lens[:, None])
        assert off.dtype == torch.int32 and torch.equal(off.long(), want)
