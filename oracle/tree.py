"""Oracle: tree planner, canonical top-k, dense candidate tree, attention inputs.

Test infrastructure only (see ``oracle/__init__.py``).
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np

MASK_MIN = {np.dtype(np.float32): np.finfo(np.float32).min, np.dtype(np.float64): np.finfo(np.float64).min}


# --------------------------------------------------------------------------- planner
def dense_node_count(topk_by_depth) -> int:
    """Nodes of a dense tree: 1 + sum_d prod_{j<=d} k_j.

    Follows ``flashgrpo/decoding/medusa_tree.py:46-52``.
    """
    total, width = 1, 1
    for k in topk_by_depth:
        width *= int(k)
        total += width
    return total


def fit_topk_to_budget(topk_by_depth, node_budget, *, min_topk_by_depth=None, depth_weight_decay=0.5):
    """Greedy decrement of per-depth branching until the dense tree fits.

    Follows ``flashgrpo/decoding/medusa_tree.py:55-99``: each step removes one
    candidate at the depth with the best (nodes saved / discounted utility loss)
    ratio, ties broken by nodes saved then by the deeper depth; when no depth
    can shrink, the deepest horizon is dropped.
    """
    budget = max(1, int(node_budget))
    ks = [max(1, int(k)) for k in topk_by_depth]
    mins_in = list(min_topk_by_depth or [])
    floor = [max(1, min(ks[i], int(mins_in[i]) if i < len(mins_in) else 1)) for i in range(len(ks))]
    decay = max(float(depth_weight_decay), 1e-3)
    while ks and dense_node_count(ks) > budget:
        best = None
        now = dense_node_count(ks)
        for d, k in enumerate(ks):
            if k <= floor[d]:
                continue
            trial = ks[:d] + [k - 1] + ks[d + 1:]
            saved = now - dense_node_count(trial)
            loss = decay ** d * (math.log1p(k) - math.log(k))
            score = (saved / max(loss, 1e-9), saved, d)
            if best is None or score > best:
                best = score
        if best is not None:
            ks[best[2]] -= 1
        else:
            ks.pop()
            floor.pop()
    return ks


@dataclass
class Plan:
    node_budget_per_seq: int
    active_heads: int
    topk_by_depth: list
    actual_nodes: int
    mode: str
    layout: str
    # sparse_asymmetric layout only (flashgrpo_b200/decoding/medusa_tree.py:49-60)
    nodes_by_head: list = field(default_factory=list)
    min_head3_nodes: int = 0
    head3_min_budget: int = 8
    branch_score_temperature: float = 1.0
    diversity_penalty: float = 0.0


def plan_tree(*, active_batch_size, num_medusa_heads, tree_mode, tree_layout, cpeak_nodes,
              min_tree_nodes_per_seq, max_tree_nodes_per_seq, max_tree_depth,
              fixed_tree_topk_by_depth, adaptive_tree_enabled=False, adaptive_min_topk_by_depth=None,
              sparse_nodes_by_head=None, sparse_min_head3_nodes=1, sparse_head3_min_budget=8,
              sparse_branch_score_temperature=1.0, sparse_diversity_penalty=0.05) -> Plan:
    """Per-step tree plan. Follows ``flashgrpo/decoding/medusa_tree.py:102-178``.

    ``tree_layout="sparse"`` is planned as dense (the reference's v1 mapping,
    ``:118-122``). ``"sparse_asymmetric"`` plans the dense branching first and then
    replaces it with per-head node counts, following
    ``flashgrpo_b200/decoding/medusa_tree.py:342-458``.
    """
    if tree_layout not in ("dense", "sparse", "sparse_asymmetric"):
        raise ValueError(tree_layout)
    if tree_layout == "sparse_asymmetric":
        dense = plan_tree(active_batch_size=active_batch_size, num_medusa_heads=num_medusa_heads,
                          tree_mode=tree_mode, tree_layout="dense", cpeak_nodes=cpeak_nodes,
                          min_tree_nodes_per_seq=min_tree_nodes_per_seq,
                          max_tree_nodes_per_seq=max_tree_nodes_per_seq, max_tree_depth=max_tree_depth,
                          fixed_tree_topk_by_depth=fixed_tree_topk_by_depth,
                          adaptive_tree_enabled=adaptive_tree_enabled,
                          adaptive_min_topk_by_depth=adaptive_min_topk_by_depth)
        max_heads = min(int(num_medusa_heads), max(0, int(max_tree_depth) - 1))
        requested = list(sparse_nodes_by_head or fixed_tree_topk_by_depth or [4, 3, 2])
        alloc = sparse_allocation(dense.node_budget_per_seq, max_heads, requested, sparse_min_head3_nodes,
                                  sparse_head3_min_budget)
        return Plan(dense.node_budget_per_seq, len(alloc), list(alloc), 1 + sum(alloc), tree_mode,
                    "sparse_asymmetric", list(alloc), max(0, int(sparse_min_head3_nodes)),
                    max(1, int(sparse_head3_min_budget)), max(1e-6, float(sparse_branch_score_temperature)),
                    max(0.0, float(sparse_diversity_penalty)))
    layout = "dense"
    bsz = max(1, int(active_batch_size))
    if tree_mode == "fixed":
        budget = int(max_tree_nodes_per_seq)
        ks = [max(1, int(k)) for k in list(fixed_tree_topk_by_depth)[:num_medusa_heads]]
        while ks and dense_node_count(ks) > budget:
            ks[-1] -= 1
            if ks[-1] <= 0:
                ks.pop()
        heads = min(len(ks), max(0, int(max_tree_depth) - 1))
        ks = ks[:heads]
    elif tree_mode == "concurrency_aware":
        budget = int(cpeak_nodes) // bsz
        budget = max(int(min_tree_nodes_per_seq), min(int(max_tree_nodes_per_seq), budget))
        max_heads = min(int(num_medusa_heads), max(0, int(max_tree_depth) - 1))
        defaults = list(fixed_tree_topk_by_depth) or [4, 3, 2, 1, 1]
        ks = []
        if adaptive_tree_enabled:
            mins_in = list(adaptive_min_topk_by_depth or [])
            floor = []
            for d in range(max_heads):
                mk = max(1, int(mins_in[d]) if d < len(mins_in) else 1)
                if dense_node_count(floor + [mk]) > budget:
                    break
                floor.append(mk)
                ks.append(max(mk, int(defaults[min(d, len(defaults) - 1)])))
        else:
            paths, used = 1, 1
            for d in range(max_heads):
                want = int(defaults[min(d, len(defaults) - 1)])
                room = budget - used
                if room <= 0:
                    break
                k = min(max(1, want), max(1, room // paths))
                if used + paths * k > budget:
                    k = room // paths
                if k <= 0:
                    break
                ks.append(int(k))
                paths *= int(k)
                used += paths
        heads = len(ks)
    else:
        raise ValueError(tree_mode)
    return Plan(budget, heads, ks, dense_node_count(ks), tree_mode, layout)


def sparse_allocation(budget, max_heads, requested, min_head3_nodes, head3_min_budget):
    """Per-head node counts of a sparse_asymmetric tree.

    Follows ``flashgrpo_b200/decoding/medusa_tree.py:411-444``: heads take their
    requested counts in order from the ``budget - 1`` non-root slots; when the budget
    reaches ``head3_min_budget`` and head 3 was requested, heads 2 then 1 each give
    up all but one node until head 3 holds ``min_head3_nodes``; trailing zero heads
    are dropped.
    """
    alloc = [0] * max_heads
    remaining = max(0, int(budget) - 1)
    for h in range(max_heads):
        want = max(0, int(requested[h]) if h < len(requested) else 0)
        alloc[h] = min(want, remaining)
        remaining -= alloc[h]
    if max_heads >= 3 and budget >= int(head3_min_budget) and len(requested) >= 3 and int(requested[2]) > 0:
        deficit = max(0, max(1, int(min_head3_nodes)) - alloc[2])
        for donor in (1, 0):
            moved = min(deficit, max(0, alloc[donor] - 1))
            alloc[donor] -= moved
            alloc[2] += moved
            deficit -= moved
            if deficit == 0:
                break
    active = max((h + 1 for h, c in enumerate(alloc) if c > 0), default=0)
    return alloc[:active]


def topk_from_confidence(confidence, base_k, depth_idx, *, enabled, min_topk_by_depth, low, high):
    """Map a confidence to a branching factor.

    Follows ``flashgrpo/decoding/flash_medusa_decoder.py:341-360``.
    """
    base_k = max(1, int(base_k))
    mins = list(min_topk_by_depth) or [1]
    min_k = max(1, min(base_k, int(mins[min(depth_idx, len(mins) - 1)])))
    if (not enabled) or base_k <= min_k:
        return base_k
    if not math.isfinite(float(confidence)):
        return min_k
    if high <= low:
        return min_k if confidence >= high else base_k
    if confidence <= low:
        return base_k
    if confidence >= high:
        return min_k
    ratio = (confidence - low) / (high - low)
    return max(min_k, min(base_k, int(round(base_k - ratio * (base_k - min_k)))))


def quantile_linear(values, q):
    """Linear-interpolation quantile (``torch.quantile`` default), float64."""
    v = np.sort(np.asarray(values, dtype=np.float64))
    if v.size == 0:
        return float("nan")
    pos = q * (v.size - 1)
    lo = int(math.floor(pos))
    hi = min(lo + 1, v.size - 1)
    return float(v[lo] + (v[hi] - v[lo]) * (pos - lo))


# --------------------------------------------------------------------------- canonical top-k
def sort_key32(x) -> np.ndarray:
    """Order-preserving uint32 key of float32 values.

    -0.0 maps to +0.0's key and every NaN to the largest key, so that ranking by
    (key desc, index asc) is a total order that agrees with float comparison.
    """
    x = np.asarray(x, dtype=np.float32)
    bits = x.view(np.uint32).astype(np.uint64)
    neg = (bits >> 31) == 1
    key = np.where(neg, (~bits) & 0xFFFFFFFF, bits | 0x80000000)
    key = np.where(x == 0, np.uint64(0x80000000), key)
    key = np.where(np.isnan(x), np.uint64(0xFFFFFFFF), key)
    return key.astype(np.uint64)


def rank_order(x) -> np.ndarray:
    """Indices of a 1-D row sorted by (value desc, index asc)."""
    key = sort_key32(x)
    idx = np.arange(key.shape[-1], dtype=np.uint64)
    comp = (key << np.uint64(32)) | (np.uint64(0xFFFFFFFF) - idx)
    return np.argsort(~comp, kind="stable")


def topk_canonical(x, k):
    """Top-k of one row, ties broken toward the lower index. Returns (idx, values)."""
    x = np.asarray(x, dtype=np.float32)
    order = rank_order(x)[: int(k)]
    return order.astype(np.int64), x[order]


# --------------------------------------------------------------------------- trees
@dataclass
class Tree:
    tokens: list
    parents: list
    depths: list
    scores: list = field(default_factory=list)

    def children(self, node):
        return [i for i, p in enumerate(self.parents) if p == node]

    def ancestors_including_self(self, node):
        out = [node]
        p = self.parents[node]
        while p >= 0:
            out.append(p)
            p = self.parents[p]
        return out[::-1]

    @property
    def node_count(self):
        return len(self.tokens)


def dense_topology(topk_by_depth, budget):
    """Parent/depth/rank arrays of the dense BFS tree, truncated at ``budget``.

    Node order is parent-major then candidate-rank, as assembled by
    ``flashgrpo/decoding/medusa_tree.py:254-277``. ``rank[n]`` is the index of the
    candidate that node ``n`` takes from its depth's top-k list.
    """
    parents, depths, ranks = [-1], [1], [0]
    frontier = [0]
    for d, k in enumerate(topk_by_depth):
        if k <= 0:
            break
        nxt = []
        stop = False
        for p in frontier:
            for r in range(int(k)):
                parents.append(p)
                depths.append(d + 2)
                ranks.append(r)
                nxt.append(len(parents) - 1)
                if len(parents) >= budget:
                    stop = True
                    break
            if stop:
                break
        frontier = nxt
        if not frontier or len(parents) >= budget:
            break
    return parents, depths, ranks


def build_batch_trees(roots, medusa_logits, plan: Plan):
    """Dense candidate trees for a batch.

    Follows ``flashgrpo/decoding/medusa_tree.py:228-278`` with the canonical
    top-k tie order. ``medusa_logits`` is a list (one per head) of [B, V] arrays.
    """
    roots = [int(r) for r in roots]
    cands = []
    for d, k in enumerate(plan.topk_by_depth[: plan.active_heads]):
        if d >= len(medusa_logits):
            break
        lg = np.asarray(medusa_logits[d], dtype=np.float32)
        k = min(max(0, int(k)), lg.shape[-1])
        if k <= 0:
            break
        cands.append([topk_canonical(lg[b], k) for b in range(lg.shape[0])])
    trees = []
    for b, root in enumerate(roots):
        toks, pars, deps, scs = [root], [-1], [1], [0.0]
        frontier = [0]
        for d, rows in enumerate(cands):
            ids, vals = rows[b]
            nxt = []
            full = False
            for p in frontier:
                for t, s in zip(ids.tolist(), vals.tolist()):
                    toks.append(int(t))
                    pars.append(p)
                    deps.append(d + 2)
                    scs.append(float(s))
                    nxt.append(len(toks) - 1)
                    if len(toks) >= plan.node_budget_per_seq:
                        full = True
                        break
                if full:
                    break
            frontier = nxt
            if not frontier or len(toks) >= plan.node_budget_per_seq:
                break
        trees.append(Tree(toks, pars, deps, scs))
    return trees


def sparse_widths(nodes_by_head, vocab):
    """Candidates taken per head for a sparse tree: heads 1 and 2 keep head 3's count
    in reserve (``flashgrpo_b200/decoding/medusa_tree.py:569-579``)."""
    realloc = nodes_by_head[2] if len(nodes_by_head) >= 3 else 0
    out = []
    for h, c in enumerate(nodes_by_head):
        w = c + realloc if h < 2 else c
        out.append(max(1, min(int(w), int(vocab))))
    return out


def select_sparse_children(parent_nodes, parent_scores, token_ids, token_scores, count, diversity_penalty):
    """Greedy choice of path extensions with a per-parent diversity penalty.

    Follows ``flashgrpo_b200/decoding/medusa_tree.py:509-546``. The pool is every
    (parent, candidate) pair in parent-major order, valued at parent score +
    candidate score (float64). Each pick takes the first pair of strictly largest
    ``cumulative - penalty * picks_of_its_parent`` among the unpicked pairs; a pool
    with no value above -inf ends the picks. Returns (parent node, token, cumulative).
    """
    if count <= 0 or not parent_nodes or len(token_ids) == 0:
        return []
    pool = [(float(parent_scores[p]) + float(s), p, int(t))
            for p in range(len(parent_nodes)) for t, s in zip(token_ids, token_scores)]
    picked = [False] * len(pool)
    uses = [0] * len(parent_nodes)
    pen = float(diversity_penalty)
    out = []
    for _ in range(min(int(count), len(pool))):
        best, best_v = -1, -math.inf
        for i, (cum, p, _t) in enumerate(pool):
            if picked[i]:
                continue
            v = cum - pen * uses[p]
            if v > best_v:
                best_v, best = v, i
        if best < 0:
            break
        cum, p, t = pool[best]
        picked[best] = True
        uses[p] += 1
        out.append((int(parent_nodes[p]), t, cum))
    return out


def build_sparse_trees(roots, medusa_logits, plan: Plan, head3_gate=None):
    """Sparse asymmetric candidate trees for a batch.

    Follows ``flashgrpo_b200/decoding/medusa_tree.py:549-685``. Per row: the root;
    head 1's first ``n1`` candidates under the root; head 2's pairs chosen greedily
    under the head-1 nodes (``n2``, plus head 3's count when head 3 is gated off for
    the row); head 3's pairs under the head-2 nodes; then the remaining head-1
    candidates while the budget allows; truncated to the budget. Candidate scores
    are the top-k logits divided by the branch temperature in float32 (canonical
    top-k order). ``head3_gate`` is a per-row bool list (None = every row).
    """
    B = len(roots)
    nodes = list(plan.nodes_by_head or plan.topk_by_depth)
    heads = min(int(plan.active_heads), len(nodes), len(medusa_logits))
    nodes = nodes[:heads]
    if heads == 0:
        return [Tree([int(r)], [-1], [1], [0.0]) for r in roots]
    V = np.asarray(medusa_logits[0]).shape[-1]
    widths = sparse_widths(nodes, V)
    realloc = nodes[2] if len(nodes) >= 3 else 0
    T = np.float32(max(float(plan.branch_score_temperature), 1e-6))
    cands = []
    for h, w in enumerate(widths):
        lg = np.asarray(medusa_logits[h], dtype=np.float32)
        rows = []
        for b in range(B):
            ids, vals = topk_canonical(lg[b], w)
            rows.append((ids.tolist(), (vals.astype(np.float32) / T).astype(np.float32).tolist()))
        cands.append(rows)
    gate = [True] * B if head3_gate is None else [bool(g) for g in head3_gate]
    budget = int(plan.node_budget_per_seq)
    trees = []
    for b in range(B):
        toks, pars, deps, scs = [int(roots[b])], [-1], [1], [0.0]
        n1 = nodes[0]
        h1_ids, h1_sc = cands[0][b]
        for t, s in zip(h1_ids[:n1], h1_sc[:n1]):
            toks.append(int(t)); pars.append(0); deps.append(2); scs.append(float(s))
        h1_nodes = list(range(1, len(toks)))
        use3 = len(nodes) >= 3 and nodes[2] > 0 and gate[b]
        n2 = (nodes[1] if len(nodes) >= 2 else 0) + (0 if use3 else realloc)
        h2_nodes, h2_sc = [], []
        if n2 > 0 and len(cands) >= 2:
            ids, sc = cands[1][b]
            for p, t, cum in select_sparse_children(h1_nodes, [scs[i] for i in h1_nodes], ids, sc, n2,
                                                    plan.diversity_penalty):
                toks.append(t); pars.append(p); deps.append(3); scs.append(cum)
                h2_nodes.append(len(toks) - 1); h2_sc.append(cum)
        if use3 and len(cands) >= 3 and h2_nodes:
            ids, sc = cands[2][b]
            for p, t, cum in select_sparse_children(h2_nodes, h2_sc, ids, sc, nodes[2], plan.diversity_penalty):
                toks.append(t); pars.append(p); deps.append(4); scs.append(cum)
        seen = {toks[i] for i in h1_nodes}
        for t, s in zip(h1_ids[n1:], h1_sc[n1:]):
            if len(toks) >= budget:
                break
            if int(t) in seen:
                continue
            toks.append(int(t)); pars.append(0); deps.append(2); scs.append(float(s))
            seen.add(int(t))
        trees.append(Tree(toks[:budget], pars[:budget], deps[:budget], scs[:budget]))
    return trees


def build_dense_tree(root, medusa_logits_row, plan: Plan) -> Tree:
    """Single-row tree. Follows ``flashgrpo/decoding/medusa_tree.py:200-225``."""
    return build_batch_trees([root], [np.asarray(r)[None] for r in medusa_logits_row], plan)[0]


def tree_attention_inputs(trees, full_attention_mask, logical_lengths, *, pad_token_id, dtype=np.float32):
    """Flattened ids, additive 4-D mask, positions and node mask.

    Follows ``flashgrpo/decoding/tree_attention.py:6-67``: node n attends to valid
    prefix slots and to its ancestors-or-self; padded query rows attend to
    themselves; position = logical_len + depth - 1 (0 for padding).
    """
    full_attention_mask = np.asarray(full_attention_mask)
    B = len(trees)
    nmax = max(max(t.node_count, 1) for t in trees)
    past = full_attention_mask.shape[1]
    ids = np.full((B, nmax), int(pad_token_id), dtype=np.int64)
    depth = np.ones((B, nmax), dtype=np.int64)
    valid = np.zeros((B, nmax), dtype=bool)
    allowed_tree = np.zeros((B, nmax, nmax), dtype=bool)
    for b, t in enumerate(trees):
        n = t.node_count
        ids[b, :n] = t.tokens
        depth[b, :n] = t.depths
        valid[b, :n] = True
        for i in range(n):
            for a in t.ancestors_including_self(i):
                allowed_tree[b, i, a] = True
        for i in range(n, nmax):
            allowed_tree[b, i, i] = True
    pos = np.asarray(logical_lengths, dtype=np.int64)[:, None] + depth - 1
    pos[~valid] = 0
    prefix = np.broadcast_to(full_attention_mask.astype(bool)[:, None, :], (B, nmax, past))
    allowed = np.concatenate([prefix, allowed_tree], axis=-1)
    dt = np.dtype(dtype)
    mask = np.where(allowed, 0.0, MASK_MIN[dt]).astype(dt)[:, None]
    return ids, mask, pos, valid


def internal_slots(trees):
    """Packed LM-head slot of each node that has children (-1 for leaves).

    Follows ``flashgrpo/decoding/flash_medusa_decoder.py:391-412``: slots are
    numbered row-major over (row, node).
    """
    nmax = max((t.node_count for t in trees), default=1)
    slots = [[-1] * nmax for _ in trees]
    rows, nodes = [], []
    for b, t in enumerate(trees):
        for n in range(t.node_count):
            if t.children(n):
                slots[b][n] = len(rows)
                rows.append(b)
                nodes.append(n)
    return rows, nodes, slots


def ancestor_bits(parents):
    """64-bit ancestor-or-self mask of every node (bit m set if node m is on the path)."""
    out = []
    for n in range(len(parents)):
        m, p = 1 << n, parents[n]
        while p >= 0:
            m |= 1 << p
            p = parents[p]
        out.append(m)
    return out


def nan_to_num_logits(x):
    """The chain-mode sanitising of ``flash_medusa_decoder.py:477-482`` (fp32; NaN -> -1e9,
    +inf -> 1e9, -inf -> -1e9)."""
    return np.nan_to_num(np.asarray(x, np.float32), nan=-1.0e9, posinf=1.0e9, neginf=-1.0e9)


def chain_add_children(trees, cur, logits, k, depth_idx, budget):
    """One depth of the chain builder (``flash_medusa_decoder.py:488-521``).

    cur[b] lists the node ids of row b's current parents; logits[b * n_d + j] is the
    (unsanitised) logits row of parent j of row b, n_d = len(cur[b]). Each parent in
    order receives its top-k children (canonical order) while its row holds fewer than
    `budget` nodes. Returns (next cur, parent_index, tokens): parent_index and tokens
    list the new nodes in creation order (row-major), parent_index as rows of logits.
    """
    lg = nan_to_num_logits(logits)
    B = len(trees)
    n_d = len(cur[0]) if B else 0
    nxt = [[] for _ in range(B)]
    pidx, toks = [], []
    for b in range(B):
        t = trees[b]
        for j, pn in enumerate(cur[b]):
            if t.node_count >= budget:
                break
            ids, vals = topk_canonical(lg[b * n_d + j], min(int(k), lg.shape[-1]))
            for tok, val in zip(ids, vals):
                if t.node_count >= budget:
                    break
                t.tokens.append(int(tok))
                t.parents.append(pn)
                t.depths.append(depth_idx + 2)
                t.scores.append(float(val))
                nxt[b].append(t.node_count - 1)
                pidx.append(b * n_d + j)
                toks.append(int(tok))
    return nxt, pidx, toks


def build_chain_trees(roots, chain_logits, topk_by_depth, budget):
    """Chain-mode candidate trees (``flash_medusa_decoder.py:435-539``) from given
    per-depth logits: chain_logits[d] is [B * n_d, V], the parent states of depth d in
    creation order (row-major over sequences, then node order). Returns
    (trees, parent_index, tokens) with the per-depth lists of chain_add_children.
    """
    trees = [Tree([int(r)], [-1], [1], [0.0]) for r in roots]
    cur = [[0] for _ in roots]
    parent_index, tokens = [], []
    for d, k in enumerate(topk_by_depth):
        if d >= len(chain_logits) or int(k) <= 0:
            break
        cur, pidx, toks = chain_add_children(trees, cur, chain_logits[d], k, d, budget)
        if not pidx:
            break
        parent_index.append(pidx)
        tokens.append(toks)
    return trees, parent_index, tokens
