"""Tree planner, dense candidate trees and their device topology.

Same public names and behaviour as ``flashgrpo/decoding/medusa_tree.py``:
``CandidateTree``, ``TreePlan``, ``dense_node_count``, ``fit_topk_to_budget``,
``plan_tree``, ``build_dense_tree``, ``build_batch_trees``. Candidate ties are
resolved (value desc, index asc), which ``torch.topk`` leaves unspecified.

``TreeTopology`` is the build's device form of a plan: in a dense tree the
parent/depth/candidate-rank of every node depends only on the plan, so it is
computed once per plan on the host (cached) and every row shares it; only the
tokens differ per row and come from ``fg_medusa_topk`` + ``fg_tree_layout``.
"""
from __future__ import annotations

import math
import warnings
from dataclasses import dataclass, field

import numpy as np
import torch

from .. import kernels as K


@dataclass
class CandidateTree:
    tokens: list
    parents: list
    depths: list
    scores: list = field(default_factory=list)

    def __post_init__(self) -> None:
        self.children: dict = {}
        for idx, parent in enumerate(self.parents):
            if parent >= 0:
                self.children.setdefault(parent, []).append(idx)

    def ancestors_including_self(self, node_idx: int) -> list:
        path = [node_idx]
        p = self.parents[node_idx]
        while p >= 0:
            path.append(p)
            p = self.parents[p]
        return path[::-1]

    @property
    def node_count(self) -> int:
        return len(self.tokens)


@dataclass
class TreePlan:
    node_budget_per_seq: int
    active_heads: int
    topk_by_depth: list
    actual_nodes: int
    mode: str
    layout: str
    # sparse_asymmetric layout (flashgrpo_b200/decoding/medusa_tree.py:49-60)
    nodes_by_head: list = field(default_factory=list)
    min_head3_nodes: int = 0
    head3_min_budget: int = 8
    branch_score_temperature: float = 1.0
    diversity_penalty: float = 0.0


def dense_node_count(topk_by_depth) -> int:
    """1 + sum over depths of the product of branching factors (``medusa_tree.py:46-52``)."""
    total, width = 1, 1
    for k in topk_by_depth:
        width *= int(k)
        total += width
    return total


def fit_topk_to_budget(topk_by_depth, node_budget, *, min_topk_by_depth=None, depth_weight_decay=0.5):
    """Greedy budget fit of ``medusa_tree.py:55-99``: shrink the depth with the best
    nodes-saved per discounted log-utility lost; drop the deepest horizon when no
    depth can shrink further."""
    budget = max(1, int(node_budget))
    ks = [max(1, int(k)) for k in topk_by_depth]
    mins = list(min_topk_by_depth or [])
    floor = [max(1, min(ks[i], int(mins[i]) if i < len(mins) else 1)) for i in range(len(ks))]
    base = max(float(depth_weight_decay), 1e-3)
    while ks and dense_node_count(ks) > budget:
        now = dense_node_count(ks)
        best = None
        for d, k in enumerate(ks):
            if k <= floor[d]:
                continue
            saved = now - dense_node_count(ks[:d] + [k - 1] + ks[d + 1:])
            lost = base ** d * (math.log1p(k) - math.log(k))
            cand = (saved / max(lost, 1e-9), saved, d)
            best = cand if best is None or cand > best else best
        if best is None:
            ks.pop()
            floor.pop()
        else:
            ks[best[2]] -= 1
    return ks


def plan_tree(*, active_batch_size, num_medusa_heads, tree_mode, tree_layout, cpeak_nodes, min_tree_nodes_per_seq,
              max_tree_nodes_per_seq, max_tree_depth, fixed_tree_topk_by_depth, adaptive_tree_enabled=False,
              adaptive_min_topk_by_depth=None, sparse_nodes_by_head=None, sparse_min_head3_nodes=1,
              sparse_head3_min_budget=8, sparse_branch_score_temperature=1.0,
              sparse_diversity_penalty=0.05) -> TreePlan:
    """Per-step plan (``medusa_tree.py:102-178``): fixed, or concurrency-aware with a
    ``floor(cpeak_nodes / B)`` node budget clamped to [min, max] nodes per sequence.

    ``tree_layout="sparse_asymmetric"`` (``flashgrpo_b200/decoding/medusa_tree.py:342-458``)
    keeps the dense plan's budget and replaces its branching by per-head node counts
    (``sparse_allocation``); ``"sparse"`` stays the v1 mapping to dense."""
    if tree_layout not in {"dense", "sparse", "sparse_asymmetric"}:
        raise ValueError(f"Unsupported tree_layout={tree_layout}")
    if tree_layout == "sparse_asymmetric":
        dense = plan_tree(active_batch_size=active_batch_size, num_medusa_heads=num_medusa_heads,
                          tree_mode=tree_mode, tree_layout="dense", cpeak_nodes=cpeak_nodes,
                          min_tree_nodes_per_seq=min_tree_nodes_per_seq, max_tree_nodes_per_seq=max_tree_nodes_per_seq,
                          max_tree_depth=max_tree_depth, fixed_tree_topk_by_depth=fixed_tree_topk_by_depth,
                          adaptive_tree_enabled=adaptive_tree_enabled,
                          adaptive_min_topk_by_depth=adaptive_min_topk_by_depth)
        max_heads = min(int(num_medusa_heads), max(0, int(max_tree_depth) - 1))
        requested = list(sparse_nodes_by_head or fixed_tree_topk_by_depth or [4, 3, 2])
        counts = sparse_allocation(dense.node_budget_per_seq, max_heads, requested, sparse_min_head3_nodes,
                                   sparse_head3_min_budget)
        return TreePlan(dense.node_budget_per_seq, len(counts), list(counts), 1 + sum(counts), tree_mode,
                        "sparse_asymmetric", list(counts), max(0, int(sparse_min_head3_nodes)),
                        max(1, int(sparse_head3_min_budget)), max(1e-6, float(sparse_branch_score_temperature)),
                        max(0.0, float(sparse_diversity_penalty)))
    if tree_layout == "sparse":
        warnings.warn("flashgrpo tree_layout='sparse' is a v1 skeleton; falling back to dense.", RuntimeWarning)
        tree_layout = "dense"
    bsz = max(1, int(active_batch_size))
    if tree_mode == "fixed":
        budget = int(max_tree_nodes_per_seq)
        ks = [max(1, int(k)) for k in list(fixed_tree_topk_by_depth)[:num_medusa_heads]]
        while ks and dense_node_count(ks) > budget:
            ks[-1] -= 1
            if ks[-1] <= 0:
                ks.pop()
        ks = ks[:min(len(ks), max(0, int(max_tree_depth) - 1))]
    elif tree_mode == "concurrency_aware":
        budget = max(int(min_tree_nodes_per_seq), min(int(max_tree_nodes_per_seq), int(cpeak_nodes) // bsz))
        max_heads = min(int(num_medusa_heads), max(0, int(max_tree_depth) - 1))
        defaults = list(fixed_tree_topk_by_depth) or [4, 3, 2, 1, 1]
        ks = []
        if adaptive_tree_enabled:
            mins = list(adaptive_min_topk_by_depth or [])
            chain = []
            for d in range(max_heads):
                mk = max(1, int(mins[d]) if d < len(mins) else 1)
                if dense_node_count(chain + [mk]) > budget:
                    break
                chain.append(mk)
                ks.append(max(mk, int(defaults[min(d, len(defaults) - 1)])))
        else:
            paths, used = 1, 1
            for d in range(max_heads):
                room = budget - used
                if room <= 0:
                    break
                k = min(max(1, int(defaults[min(d, len(defaults) - 1)])), max(1, room // paths))
                if used + paths * k > budget:
                    k = room // paths
                if k <= 0:
                    break
                ks.append(int(k))
                paths *= int(k)
                used += paths
    else:
        raise ValueError(f"Unsupported tree_mode={tree_mode}")
    return TreePlan(budget, len(ks), ks, dense_node_count(ks), tree_mode, tree_layout)


def sparse_allocation(budget, max_heads, requested, min_head3_nodes, head3_min_budget) -> list:
    """Per-head node counts of a sparse asymmetric tree
    (``flashgrpo_b200/decoding/medusa_tree.py:411-444``).

    Heads take their requested counts in order out of the ``budget - 1`` non-root
    slots. If head 3 was requested and the budget reaches ``head3_min_budget``,
    head 2 and then head 1 hand over nodes (keeping one each) until head 3 holds
    ``max(1, min_head3_nodes)``. Heads after the last non-empty one are dropped."""
    counts = []
    left = max(0, int(budget) - 1)
    for h in range(max_heads):
        take = min(max(0, int(requested[h]) if h < len(requested) else 0), left)
        counts.append(take)
        left -= take
    if max_heads >= 3 and budget >= int(head3_min_budget) and len(requested) >= 3 and int(requested[2]) > 0:
        short = max(0, max(1, int(min_head3_nodes)) - counts[2])
        for donor in (1, 0):
            give = min(short, max(0, counts[donor] - 1))
            counts[donor] -= give
            counts[2] += give
            short -= give
            if short == 0:
                break
    last = max((h + 1 for h, c in enumerate(counts) if c > 0), default=0)
    return counts[:last]


def sparse_widths(nodes_by_head, vocab) -> list:
    """Top-k candidates taken per head: heads 1 and 2 hold head 3's count in reserve
    (``flashgrpo_b200/decoding/medusa_tree.py:569-579``)."""
    spare = nodes_by_head[2] if len(nodes_by_head) >= 3 else 0
    return [max(1, min(int(c) + (spare if h < 2 else 0), int(vocab))) for h, c in enumerate(nodes_by_head)]


def sparse_max_nodes(plan: TreePlan) -> int:
    """Upper bound of a sparse tree's node count (the verify width): root, the head
    counts of the first three heads, and at most head 3's count of leftover head-1
    candidates, cut at the budget."""
    nodes = list(plan.nodes_by_head or plan.topk_by_depth)[: min(3, plan.active_heads)]
    spare = nodes[2] if len(nodes) >= 3 else 0
    return max(1, min(int(plan.node_budget_per_seq), 1 + sum(nodes) + spare))


def sparse_tree_device(roots: torch.Tensor, cand_tokens: torch.Tensor, cand_scores: torch.Tensor, plan: TreePlan,
                       batch: int, vocab: int, *, head3_gate=None, scores=False) -> dict:
    """Device sparse trees of a batch (``fg_sparse_tree_layout``): tokens, parents,
    depth, pos_offset, anc, n_children [batch, N] and n_nodes [batch] with
    N = ``sparse_max_nodes(plan)``; rows with fewer nodes are padded."""
    nodes = list(plan.nodes_by_head or plan.topk_by_depth)[: plan.active_heads]
    N = sparse_max_nodes(plan)
    if N > 64:
        raise ValueError("tree nodes exceed the 64-node limit of the ancestor bit masks")
    return K.sparse_tree_layout(cand_tokens, cand_scores, batch, roots.to(torch.int32), nodes, vocab=vocab,
                                budget=plan.node_budget_per_seq, num_nodes=N,
                                temperature=plan.branch_score_temperature,
                                diversity_penalty=plan.diversity_penalty, head3_gate=head3_gate, scores=scores)


# ------------------------------------------------------------------ device topology
class TreeTopology:
    """Dense-tree structure of one plan, truncated at its node budget.

    Host lists (``parents``, ``depths``, ``ranks``, ``internal``) plus cached
    device tensors: node depth/rank/position offset [N], ancestor-or-self bit
    masks [N] (int64 bit patterns), and per-batch-size parent/slot maps.
    """

    _cache: dict = {}

    def __init__(self, topk_by_depth, budget):
        parents, depths, ranks = [-1], [1], [0]
        frontier = [0]
        for d, k in enumerate(topk_by_depth):
            if int(k) <= 0:
                break
            nxt, full = [], False
            for p in frontier:
                for r in range(int(k)):
                    parents.append(p)
                    depths.append(d + 2)
                    ranks.append(r)
                    nxt.append(len(parents) - 1)
                    if len(parents) >= budget:
                        full = True
                        break
                if full:
                    break
            frontier = nxt
            if not frontier or len(parents) >= budget:
                break
        self.topk_by_depth = [int(k) for k in topk_by_depth]
        self.parents, self.depths, self.ranks = parents, depths, ranks
        self.num_nodes = len(parents)
        if self.num_nodes > 64:
            raise ValueError("tree nodes exceed the 64-node limit of the ancestor bit masks")
        has_child = [False] * self.num_nodes
        for p in parents[1:]:
            has_child[p] = True
        self.internal = [n for n in range(self.num_nodes) if has_child[n]]
        self.slot_of = [-1] * self.num_nodes
        for i, n in enumerate(self.internal):
            self.slot_of[n] = i
        self.max_depth = max(depths) - 1  # walk steps
        self.depth_counts = {}  # non-root nodes per depth
        for dpt in depths[1:]:
            self.depth_counts[dpt] = self.depth_counts.get(dpt, 0) + 1
        bits = []
        for n in range(self.num_nodes):
            m, p = 1 << n, parents[n]
            while p >= 0:
                m |= 1 << p
                p = parents[p]
            bits.append(m)
        self.anc_bits = bits
        self._dev = {}

    @classmethod
    def for_plan(cls, plan: TreePlan) -> "TreeTopology":
        key = (tuple(int(k) for k in plan.topk_by_depth[: plan.active_heads]), int(plan.node_budget_per_seq))
        topo = cls._cache.get(key)
        if topo is None:
            topo = cls(list(key[0]), key[1])
            cls._cache[key] = topo
        return topo

    def device(self, device, batch: int | None = None) -> dict:
        """Device tensors; batch-sized maps are cached per batch size."""
        key = (str(device), batch)
        d = self._dev.get(key)
        if d is None:
            i32 = dict(dtype=torch.int32, device=device)
            arr = np.array([b & 0xFFFFFFFFFFFFFFFF for b in self.anc_bits], dtype=np.uint64).view(np.int64)
            d = dict(depth=torch.tensor(self.depths, **i32), rank=torch.tensor(self.ranks, **i32),
                     pos_offset=torch.tensor([x - 1 for x in self.depths], **i32),
                     anc=torch.from_numpy(arr).to(device),
                     leaf=torch.tensor([1 if s < 0 else 0 for s in self.slot_of], **i32))
            if batch is not None:
                N, I = self.num_nodes, len(self.internal)
                d["parents"] = torch.tensor([self.parents] * batch, **i32)
                d["n_nodes"] = torch.full((batch,), N, **i32)
                slots = np.full((batch, N), -1, dtype=np.int32)
                rows = np.zeros(batch * I, dtype=np.int32)
                for b in range(batch):
                    for i, n in enumerate(self.internal):
                        slots[b, n] = b * I + i
                        rows[b * I + i] = b * N + n
                d["slot_map"] = torch.from_numpy(slots).to(device)
                d["internal_rows"] = torch.from_numpy(rows).to(device)
            self._dev[key] = d
        return d


# ------------------------------------------------------------------ tree builders
def build_tree_tokens(roots: torch.Tensor, cand_tokens: torch.Tensor, cand_scores: torch.Tensor,
                      topo: TreeTopology, batch: int):
    """Device tokens [B, N] (int32) and scores [B, N] of a dense tree."""
    d = topo.device(roots.device)
    return K.tree_layout(cand_tokens, cand_scores, batch, roots.to(torch.int32), d["depth"], d["rank"],
                         topo.num_nodes)


def _trees_from_device(tokens: torch.Tensor, scores: torch.Tensor, topo: TreeTopology) -> list:
    toks = tokens.cpu().tolist()
    scs = scores.cpu().tolist()
    return [CandidateTree(tokens=t, parents=list(topo.parents), depths=list(topo.depths), scores=s)
            for t, s in zip(toks, scs)]


def build_batch_trees(root_tokens: torch.Tensor, medusa_logits: list, plan: TreePlan, *,
                      head3_gate_mask: torch.Tensor | None = None) -> list:
    """Dense Medusa trees for a batch (``medusa_tree.py:228-278``): one device top-k
    over all depths, one layout launch, then the CandidateTree objects.

    A ``sparse_asymmetric`` plan builds the b200 sparse trees instead
    (``flashgrpo_b200/decoding/medusa_tree.py:731-749``); ``head3_gate_mask``
    [batch] bool switches head 3 off per row (None: every row keeps it)."""
    batch = int(root_tokens.shape[0])
    if plan.layout == "sparse_asymmetric":
        return _sparse_batch_trees(root_tokens, medusa_logits, plan, head3_gate_mask)
    depths = []
    for d, k in enumerate(plan.topk_by_depth[: plan.active_heads]):
        if d >= len(medusa_logits):
            break
        k = min(max(0, int(k)), int(medusa_logits[d].shape[-1]))
        if k <= 0:
            break
        depths.append(k)
    topo = TreeTopology(depths, plan.node_budget_per_seq)
    device = root_tokens.device
    if not depths:
        t = root_tokens.reshape(batch, 1).to(torch.int32)
        return _trees_from_device(t, torch.zeros(batch, 1), topo)
    if device.type != "cuda":
        raise ValueError("build_batch_trees: device tensors required (HIP path)")
    stacked = torch.cat([medusa_logits[d] for d in range(len(depths))], dim=0)
    cand, score, _ = K.medusa_topk(stacked, max(depths))
    tokens, scores = build_tree_tokens(root_tokens, cand, score, topo, batch)
    return _trees_from_device(tokens, scores, topo)


def _sparse_batch_trees(root_tokens, medusa_logits, plan, head3_gate_mask) -> list:
    batch = int(root_tokens.shape[0])
    heads = min(int(plan.active_heads), len(plan.nodes_by_head or plan.topk_by_depth), len(medusa_logits))
    if heads == 0:
        return [CandidateTree(tokens=[int(t)], parents=[-1], depths=[1], scores=[0.0])
                for t in root_tokens.reshape(-1).tolist()]
    if root_tokens.device.type != "cuda":
        raise ValueError("build_batch_trees: device tensors required (HIP path)")
    plan_h = TreePlan(plan.node_budget_per_seq, heads, list(plan.topk_by_depth)[:heads], plan.actual_nodes, plan.mode,
                      plan.layout, list(plan.nodes_by_head or plan.topk_by_depth)[:heads], plan.min_head3_nodes,
                      plan.head3_min_budget, plan.branch_score_temperature, plan.diversity_penalty)
    vocab = int(medusa_logits[0].shape[-1])
    used = min(heads, 3)
    widths = sparse_widths(plan_h.nodes_by_head, vocab)[:used]
    stacked = torch.cat([medusa_logits[h] for h in range(used)], dim=0)
    cand, score, _ = K.medusa_topk(stacked, max(widths))
    d = sparse_tree_device(root_tokens, cand, score, plan_h, batch, vocab, head3_gate=head3_gate_mask, scores=True)
    n = d["n_nodes"].cpu().tolist()
    toks, pars, deps = d["tokens"].cpu().tolist(), d["parents"].cpu().tolist(), d["depth"].cpu().tolist()
    scs = d["scores"].cpu().tolist()
    return [CandidateTree(tokens=toks[b][:n[b]], parents=pars[b][:n[b]], depths=deps[b][:n[b]], scores=scs[b][:n[b]])
            for b in range(batch)]


def build_dense_tree(root_token: int, medusa_logits: list, plan: TreePlan) -> CandidateTree:
    """Single-row tree (``medusa_tree.py:200-225``)."""
    rows = [lg.reshape(1, -1) for lg in medusa_logits]
    device = rows[0].device if rows else torch.device("cuda")
    root = torch.tensor([int(root_token)], dtype=torch.int32, device=device)
    return build_batch_trees(root, rows, plan)[0]
