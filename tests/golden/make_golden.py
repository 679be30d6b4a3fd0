"""Writes tests/golden/reference_cases.json and reference_arrays.npz.

The cases are the reference's own unit-test inputs and known answers
(ihbkaiser/ss-GRPO ``flashgrpo/tests`` and ``flashgrpo_b200/tests``), rebuilt
here without importing the reference:

* seeded inputs are regenerated with the same torch CPU seeds the reference
  tests use (``torch.manual_seed(7)`` / ``(17)``);
* expected outputs come from the torch library calls the reference makes
  (``torch.topk``, ``Tensor.gather`` + ``copy_``/``torch.cat``) or from the
  known answers asserted in the reference tests;
* planner tables are derived by hand from ``flashgrpo/decoding/medusa_tree.py:102-178``
  (the derivations are written next to each row).

Run: python tests/golden/make_golden.py
"""
from __future__ import annotations

import json
import os

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))


def planner_cases():
    common = dict(tree_layout="dense", min_tree_nodes_per_seq=1)
    return [
        # test_flashgrpo_smoke.py:4-27 -- budget floor(32/1)=32 -> 16; k0=min(4,15)=4 (5 used);
        # k1=min(3, 11//4)=2 (13 used); k2: room 3 < 8 paths -> stop.
        dict(kw=dict(active_batch_size=1, num_medusa_heads=3, tree_mode="concurrency_aware", cpeak_nodes=32,
                     max_tree_nodes_per_seq=16, max_tree_depth=4, fixed_tree_topk_by_depth=[4, 3, 2], **common),
             expect=dict(node_budget_per_seq=16, active_heads=2, topk_by_depth=[4, 2], actual_nodes=13)),
        # budget floor(32/16)=2; k0=1 (2 used); room 0 -> stop.
        dict(kw=dict(active_batch_size=16, num_medusa_heads=3, tree_mode="concurrency_aware", cpeak_nodes=32,
                     max_tree_nodes_per_seq=16, max_tree_depth=4, fixed_tree_topk_by_depth=[4, 3, 2], **common),
             expect=dict(node_budget_per_seq=2, active_heads=1, topk_by_depth=[1], actual_nodes=2)),
        # test_flashgrpo_smoke.py:30-45 -- budget floor(256/64)=4; minimum chain [1,1,1] has 4 nodes <= 4,
        # so all three heads stay with the default branching [4,3,2].
        dict(kw=dict(active_batch_size=64, num_medusa_heads=3, tree_mode="concurrency_aware", cpeak_nodes=256,
                     max_tree_nodes_per_seq=12, max_tree_depth=4, fixed_tree_topk_by_depth=[4, 3, 2],
                     adaptive_tree_enabled=True, adaptive_min_topk_by_depth=[1, 1, 1], **common),
             expect=dict(node_budget_per_seq=4, active_heads=3, topk_by_depth=[4, 3, 2], actual_nodes=41)),
        # Tiny config: fixed, budget 16: [4,3,2]=41 -> [4,3,1]=29 -> [4,3]=17 -> [4,2]=13.
        dict(kw=dict(active_batch_size=8, num_medusa_heads=3, tree_mode="fixed", cpeak_nodes=64,
                     max_tree_nodes_per_seq=16, max_tree_depth=4, fixed_tree_topk_by_depth=[4, 3, 2], **common),
             expect=dict(node_budget_per_seq=16, active_heads=2, topk_by_depth=[4, 2], actual_nodes=13)),
        # Qwen2.5-1.5B: cpeak 512 / 32 = 16 -> same walk as the first row.
        dict(kw=dict(active_batch_size=32, num_medusa_heads=3, tree_mode="concurrency_aware", cpeak_nodes=512,
                     max_tree_nodes_per_seq=16, max_tree_depth=4, fixed_tree_topk_by_depth=[4, 3, 2], **common),
             expect=dict(node_budget_per_seq=16, active_heads=2, topk_by_depth=[4, 2], actual_nodes=13)),
        # Qwen2.5-7B (before adaptation): 2048/64=32; minimum chain of 4 fits; defaults[min(d,2)] -> [4,3,2,2].
        dict(kw=dict(active_batch_size=64, num_medusa_heads=4, tree_mode="concurrency_aware", cpeak_nodes=2048,
                     max_tree_nodes_per_seq=32, max_tree_depth=5, fixed_tree_topk_by_depth=[4, 3, 2],
                     adaptive_tree_enabled=True, adaptive_min_topk_by_depth=[1, 1, 1], **common),
             expect=dict(node_budget_per_seq=32, active_heads=4, topk_by_depth=[4, 3, 2, 2], actual_nodes=89)),
        # Qwen2.5-14B: 8192/128=64; [4 (5), 3 (17), 2 (41)]; depth 4 has room 23 < 24 paths -> stop.
        dict(kw=dict(active_batch_size=128, num_medusa_heads=4, tree_mode="concurrency_aware", cpeak_nodes=8192,
                     max_tree_nodes_per_seq=64, max_tree_depth=5, fixed_tree_topk_by_depth=[4, 3, 2], **common),
             expect=dict(node_budget_per_seq=64, active_heads=3, topk_by_depth=[4, 3, 2], actual_nodes=41)),
    ]


def fit_cases():
    # 7B adaptive refit (base k kept because random-init confidence << low): [4,3,2,2] in budget 32.
    # Greedy: (89) d1 3->2 saves 40; (49) d2 2->1 saves 16... result [4,2,1,1] = 29 nodes.
    return [dict(topk=[4, 3, 2, 2], budget=32, mins=[1, 1, 1], decay=0.5, expect=[4, 2, 1, 1]),
            dict(topk=[4, 3, 2], budget=4, mins=[1, 1, 1], decay=0.5, expect=[1, 1, 1]),
            dict(topk=[2, 2], budget=1, mins=[1, 1], decay=0.5, expect=[])]


def seed7_tree_case(arrays):
    """test_reflex_optimized.py:16-36 inputs; expected trees from torch.topk + BFS."""
    torch.manual_seed(7)
    batch, vocab = 5, 37
    roots = torch.randint(vocab, (batch,))
    logits = [torch.randn(batch, vocab) for _ in range(2)]
    topk, budget = [3, 2], 12
    cands = [torch.topk(lg, k=k, dim=-1) for lg, k in zip(logits, topk)]
    trees = []
    for b in range(batch):
        toks, pars = [int(roots[b])], [-1]
        frontier = [0]
        for d, (vals, idx) in enumerate(cands):
            nxt = []
            for p in frontier:
                for t in idx[b].tolist():
                    toks.append(int(t))
                    pars.append(p)
                    nxt.append(len(toks) - 1)
            frontier = nxt
        trees.append(dict(tokens=toks[:budget], parents=pars[:budget]))
    arrays["seed7_roots"] = roots.numpy()
    arrays["seed7_logits"] = torch.stack(logits).numpy()
    return dict(topk=topk, budget=budget, trees=trees)


def seed17_kv_case(arrays):
    """test_kv_path_extraction_matches_recompute.py:14-35 inputs; expected via gather + cat."""
    torch.manual_seed(17)
    old_len, nodes = 5, 4
    key = torch.randn(2, 2, old_len + nodes, 8)
    value = torch.randn_like(key)
    accepted = [[0, 1, 3], [0, 2]]
    width = max(len(p) for p in accepted)
    pos = torch.tensor([[old_len + n for n in p + [p[-1]] * (width - len(p))] for p in accepted])
    idx = pos[:, None, :, None].expand(2, 2, width, 8)
    exp_k = torch.cat([key[:, :, :old_len], key.gather(2, idx)], dim=2)
    exp_v = torch.cat([value[:, :, :old_len], value.gather(2, idx)], dim=2)
    arrays["seed17_key"] = key.numpy()
    arrays["seed17_value"] = value.numpy()
    arrays["seed17_expect_key"] = exp_k.numpy()
    arrays["seed17_expect_value"] = exp_v.numpy()
    return dict(old_len=old_len, accepted=accepted)


def acceptance_cases():
    return dict(
        # test_exact_acceptance_distribution.py:40-46
        greedy_single=dict(tokens=[5, 7, 9], parents=[-1, 0, 0], hot=[[0, 7]], vocab=16,
                           expect_tokens=[5, 7], expect_nodes=[0, 1]),
        # :49-90 -- rows peak on a child at every internal node, so both walks go to depth 3.
        packed=dict(trees=[dict(tokens=[5, 7, 9, 11], parents=[-1, 0, 0, 1]),
                           dict(tokens=[4, 6, 8, 10], parents=[-1, 0, 0, 2])],
                    hot=[[0, 0, 7], [0, 1, 11], [1, 0, 8], [1, 2, 10]], vocab=16,
                    slots=[[0, 1, -1, -1], [2, -1, 3, -1]],
                    expect_tokens=[[5, 7, 11], [4, 8, 10]], expect_nodes=[[0, 1, 3], [0, 2, 3]],
                    expect_last=[3, 3]),
        # flashgrpo_b200/tests/test_exact_acceptance_distribution.py:57-71
        correction=dict(tokens=[5, 7], parents=[-1, 0], hot=[[0, 9]], vocab=16,
                        expect_tokens=[5], expect_nodes=[0], expect_correction=9),
        # :74-93 -- emitted-token law must stay (0.6, 0.4) within 0.015 over 50k draws.
        correction_law=dict(tokens=[2, 0], parents=[-1, 0], probs=[0.6, 0.4], draws=50000, tol=0.015),
        # flashgrpo/tests/test_exact_acceptance_distribution.py:17-37 (T=0.8, shortlist hint 2).
        nucleus_law=[dict(logits=[5.0, 4.0, 0.0, -1.0], top_p=0.85), dict(logits=[0.0, 0.0, 0.0, 0.0], top_p=0.75)],
        nucleus_temperature=0.8, nucleus_draws=50000, nucleus_tol=0.015,
    )


def mask_case():
    # test_tree_attention_equivalence.py:9-20
    return dict(tokens=[1, 2, 3, 4], parents=[-1, 0, 0, 1], depths=[1, 2, 2, 3], past=5, logical=5,
                node=3, allowed_tree=[0, 1, 3], masked_tree=[2], position=7)


def main():
    arrays = {}
    cases = dict(planner=planner_cases(), fit=fit_cases(), seed7_tree=seed7_tree_case(arrays),
                 seed17_kv=seed17_kv_case(arrays), acceptance=acceptance_cases(), mask=mask_case())
    with open(os.path.join(HERE, "reference_cases.json"), "w") as f:
        json.dump(cases, f, indent=1)
    np.savez(os.path.join(HERE, "reference_arrays.npz"), **arrays)
    print("wrote", sorted(arrays))


if __name__ == "__main__":
    main()
