"""Oracle: one speculative verify round and the generate loop (numpy).

Test infrastructure only (see ``oracle/__init__.py``). Follows the Medusa path
of ``flashgrpo/decoding/flash_medusa_decoder.py:550-1166``: root draw, plan,
Medusa logits, (adaptive) budget fit, dense tree, tree verify, packed
internal-node logits, exact_target walk, clamp/EOS, accepted-path KV
compaction and next-state selection. The cache is held per sequence
(``seq_len[b]`` valid slots), the layout the build uses; the reference's
batch-padded cache has the same valid rows (``oracle.kv.compact_rows``).
Draws use the counter noise of ``oracle.sampling`` with draw 0 for the root
and draw t for walk step t.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

from . import kv as OK
from . import model as OM
from . import sampling as OS
from . import tree as OT


@dataclass
class DecodeSpec:
    num_medusa_heads: int = 3
    tree_mode: str = "concurrency_aware"
    cpeak_nodes: int = 64
    min_tree_nodes_per_seq: int = 1
    max_tree_nodes_per_seq: int = 16
    max_tree_depth: int = 4
    fixed_tree_topk_by_depth: tuple = (4, 3, 2)
    adaptive_tree_enabled: bool = False
    adaptive_confidence_quantile: float = 0.25
    adaptive_confidence_low: float = 0.15
    adaptive_confidence_high: float = 0.45
    adaptive_min_topk_by_depth: tuple = (1, 1, 1)
    adaptive_depth_weight_decay: float = 0.5
    do_sample: bool = True
    temperature: float = 1.0
    top_p: float = 1.0
    top_k: int | None = None
    emit_correction_token: bool = False
    eos_token_id: int = -1
    adaptive_confidence_metric: str = "top1_prob"
    proposal_mode: str = "medusa"
    chain_bootstrap_from_medusa: bool = True
    tree_layout: str = "dense"
    sparse_nodes_by_head: tuple = (5, 4, 0)
    sparse_min_head3_nodes: int = 0
    sparse_head3_min_budget: int = 8
    sparse_branch_score_temperature: float = 1.0
    sparse_diversity_penalty: float = 0.05


def plan_for(spec: DecodeSpec, batch: int) -> OT.Plan:
    return OT.plan_tree(active_batch_size=batch, num_medusa_heads=spec.num_medusa_heads, tree_mode=spec.tree_mode,
                        tree_layout=spec.tree_layout, cpeak_nodes=spec.cpeak_nodes,
                        min_tree_nodes_per_seq=spec.min_tree_nodes_per_seq,
                        max_tree_nodes_per_seq=spec.max_tree_nodes_per_seq, max_tree_depth=spec.max_tree_depth,
                        fixed_tree_topk_by_depth=list(spec.fixed_tree_topk_by_depth),
                        adaptive_tree_enabled=spec.adaptive_tree_enabled,
                        adaptive_min_topk_by_depth=list(spec.adaptive_min_topk_by_depth),
                        sparse_nodes_by_head=list(spec.sparse_nodes_by_head),
                        sparse_min_head3_nodes=spec.sparse_min_head3_nodes,
                        sparse_head3_min_budget=spec.sparse_head3_min_budget,
                        sparse_branch_score_temperature=spec.sparse_branch_score_temperature,
                        sparse_diversity_penalty=spec.sparse_diversity_penalty)


def confidences(spec: DecodeSpec, medusa_logits) -> list:
    """Per-head confidence quantile over the batch (``flash_medusa_decoder.py:320-339``):
    top-1 probability, or the top-1 minus top-2 margin."""
    confs = []
    for lg in medusa_logits:
        x = np.asarray(lg, np.float64)
        if spec.adaptive_confidence_metric == "margin":
            # top-1 minus top-2 value (flash_medusa_decoder.py:326-331)
            part = -np.sort(-x, axis=-1)[:, :2]
            score = part[:, 0] - part[:, 1] if part.shape[1] > 1 else part[:, 0]
        else:
            m = x.max(axis=-1)
            lse = m + np.log(np.exp(x - m[:, None]).sum(axis=-1))
            score = np.exp(m - lse)
        score = np.nan_to_num(score, nan=0.0, posinf=0.0, neginf=0.0)
        confs.append(OT.quantile_linear(score, spec.adaptive_confidence_quantile))
    return confs


def adapt_plan(spec: DecodeSpec, plan: OT.Plan, medusa_logits) -> OT.Plan:
    """Confidence quantile -> branching -> budget fit (``flash_medusa_decoder.py:320-389``)."""
    if not spec.adaptive_tree_enabled or not plan.topk_by_depth:
        return plan
    confs = confidences(spec, medusa_logits[: len(plan.topk_by_depth)])
    ks = [OT.topk_from_confidence(c, k, d, enabled=True, min_topk_by_depth=spec.adaptive_min_topk_by_depth,
                                  low=spec.adaptive_confidence_low, high=spec.adaptive_confidence_high)
          for d, (k, c) in enumerate(zip(plan.topk_by_depth, confs))]
    ks = OT.fit_topk_to_budget(ks, plan.node_budget_per_seq,
                               min_topk_by_depth=list(spec.adaptive_min_topk_by_depth)[: len(ks)],
                               depth_weight_decay=spec.adaptive_depth_weight_decay)
    # a sparse plan takes the fitted list as its per-head node counts
    # (flashgrpo_b200/decoding/flash_medusa_decoder.py:1063-1077)
    sparse = plan.layout == "sparse_asymmetric"
    return OT.Plan(plan.node_budget_per_seq, len(ks), ks, OT.dense_node_count(ks), plan.mode, plan.layout,
                   list(ks) if sparse else [], plan.min_head3_nodes, plan.head3_min_budget,
                   plan.branch_score_temperature, plan.diversity_penalty)


def chain_confidence(logits, metric="top1_prob"):
    """Per-row confidence of sanitised logits (``flash_medusa_decoder.py:317-339``):
    exp(max - logsumexp) or top1 - top2; non-finite scores become 0."""
    x = OT.nan_to_num_logits(logits).astype(np.float64)
    if metric == "margin":
        if x.shape[-1] == 1:
            score = x[:, 0]
        else:
            top2 = -np.sort(-x, axis=-1)[:, :2]
            score = top2[:, 0] - top2[:, 1]
    else:
        m = x.max(axis=-1)
        lse = m + np.log(np.exp(x - m[:, None]).sum(axis=-1))
        score = np.exp(m - lse)
    return np.nan_to_num(score, nan=0.0, posinf=0.0, neginf=0.0)


def chain_proposals(spec: DecodeSpec, plan: OT.Plan, hidden, roots, heads, cell, embed, lm_head, dtype=np.float64,
                    logits_hook=None):
    """Chain-mode trees (``flash_medusa_decoder.py:435-539``).

    The first parent state is Medusa head 0's residual output of the hidden state
    (``chain_bootstrap_from_medusa``) or the chain cell applied to (hidden, root
    embedding). Depth d projects every parent state through the LM head, takes the
    confidence quantile over all of them, maps it to k_d (no budget refit), adds the
    children and advances each child's state with the chain cell on its token's
    embedding. ``logits_hook(d, states)`` may replace the logits computed for depth d
    (the lockstep tests feed in the device's values). Returns
    (trees, chain plan, confidences, per-depth records of states, logits, k,
    parent_index, tokens).
    """
    B = len(roots)
    if spec.chain_bootstrap_from_medusa and heads:
        states = OM.medusa_project(hidden, heads[0], dtype)
    else:
        states = OM.chain_cell(hidden, np.asarray(embed)[np.asarray(roots)], cell, dtype)
    trees = [OT.Tree([int(r)], [-1], [1], [0.0]) for r in roots]
    cur = [[0] for _ in range(B)]
    adapted, confs, recs = [], [], []
    for d, base_k in enumerate(plan.topk_by_depth):
        if states.shape[0] == 0:
            break
        lg = OM.logits(states, lm_head, dtype).astype(np.float32) if logits_hook is None else logits_hook(d, states)
        conf = OT.quantile_linear(chain_confidence(lg, spec.adaptive_confidence_metric),
                                  min(1.0, max(0.0, spec.adaptive_confidence_quantile)))
        confs.append(conf)
        k = OT.topk_from_confidence(conf, base_k, d, enabled=spec.adaptive_tree_enabled,
                                    min_topk_by_depth=spec.adaptive_min_topk_by_depth,
                                    low=spec.adaptive_confidence_low, high=spec.adaptive_confidence_high)
        rec = dict(states=states, logits=lg, k=k)
        recs.append(rec)
        if k <= 0:
            break
        adapted.append(k)
        cur, pidx, toks = OT.chain_add_children(trees, cur, lg, k, d, plan.node_budget_per_seq)
        rec.update(parent_index=pidx, tokens=toks)
        if not toks:
            break
        states = OM.chain_cell(np.asarray(states)[pidx], np.asarray(embed)[toks], cell, dtype)
    ks = [max(1, int(k)) for k in adapted]
    chain_plan = OT.Plan(plan.node_budget_per_seq, len(ks), ks, max(t.node_count for t in trees), plan.mode,
                         plan.layout)
    return trees, chain_plan, confs, recs


@dataclass
class State:
    k: list                  # per layer [B, Hkv, capacity, d]
    v: list
    seq_len: np.ndarray      # [B]
    hidden: np.ndarray       # [B, H]
    logits: np.ndarray       # [B, V]
    seq_ids: np.ndarray      # [B] sequence ids (noise keys)
    pending: np.ndarray = field(default=None)  # [B] forced roots (-1 none)


def prefill_state(cfg, W, prompts, capacity, dtype=np.float64) -> State:
    prompts = np.asarray(prompts)
    B, P = prompts.shape
    hid, ks, vs = OM.prefill(cfg, W, prompts, dtype=dtype)
    k = [np.zeros((B, cfg.kv_heads, capacity, cfg.head_dim), dtype) for _ in ks]
    v = [np.zeros((B, cfg.kv_heads, capacity, cfg.head_dim), dtype) for _ in vs]
    for li in range(len(ks)):
        k[li][:, :, :P] = ks[li]
        v[li][:, :, :P] = vs[li]
    last = hid[:, -1]
    return State(k, v, np.full(B, P, np.int64), last, OM.logits(last, W["lm_head"], dtype), np.arange(B),
                 np.full(B, -1, np.int64))


def verify_round(cfg, W, heads, st: State, spec: DecodeSpec, seed: int, rnd: int, max_length: int,
                 dtype=np.float64, cell=None) -> dict:
    """One round; mutates ``st`` and returns what it decided. ``cell`` holds the chain
    cell weights when ``spec.proposal_mode == "chain"``."""
    B = st.seq_len.shape[0]
    L = cfg.num_layers
    greedy = (not spec.do_sample) or spec.temperature == 0
    kw = dict(do_sample=not greedy, temperature=spec.temperature, top_p=spec.top_p, top_k=spec.top_k)
    roots = np.array([st.pending[b] if spec.emit_correction_token and st.pending[b] >= 0 else
                      OS.sample_row(st.logits[b], OS.counter_noise(seed, rnd, int(st.seq_ids[b]), 0), **kw)
                      for b in range(B)], np.int64)
    plan = plan_for(spec, B)
    if spec.proposal_mode == "chain" and plan.active_heads:
        mlog = []
        trees, plan, _, chain = chain_proposals(spec, plan, st.hidden, roots, heads, cell, W["embed"], W["lm_head"],
                                                dtype)
    else:
        chain = None
        mlog = OM.medusa_logits(st.hidden, heads, W["lm_head"], plan.active_heads, dtype) if plan.active_heads else []
        mlog = [np.asarray(x, np.float32) for x in mlog]
        plan = adapt_plan(spec, plan, mlog)
        if plan.layout == "sparse_asymmetric":
            trees = OT.build_sparse_trees(roots, mlog, plan)
        else:
            trees = OT.build_batch_trees(roots, mlog, plan)
    # Rows are padded to the widest tree: a padding node (token 0, position offset 0)
    # sees only itself (flashgrpo/decoding/tree_attention.py:47-50) and is never walked.
    N = max(t.node_count for t in trees)
    toks = np.zeros((B, N), np.int64)
    allowed = np.zeros((B, N, N), bool)
    depth_off = np.zeros((B, N), np.int64)
    for b, t in enumerate(trees):
        toks[b, :t.node_count] = t.tokens
        for n in range(N):
            if n < t.node_count:
                allowed[b, n, t.ancestors_including_self(n)] = True
                depth_off[b, n] = t.depths[n] - 1
            else:
                allowed[b, n, n] = True
    valid = np.arange(st.k[0].shape[2])[None, :] < st.seq_len[:, None]
    pos = st.seq_len[:, None] + depth_off
    hid, nk, nv = OM.forward(cfg, W, toks, pos, st.k, st.v, valid, allowed, dtype=dtype)
    for li in range(L):
        for b in range(B):
            s = int(st.seq_len[b])
            st.k[li][b, :, s:s + N] = nk[li][b]
            st.v[li][b, :, s:s + N] = nv[li][b]
    out = dict(roots=roots, plan=plan, trees=trees, tree_hidden=hid, medusa_logits=mlog, chain=chain)
    if N > 1:
        rows, nodes, slots = OT.internal_slots(trees)
        packed = OM.logits(hid[rows, nodes], W["lm_head"], dtype).astype(np.float32)
        nz = [[OS.counter_noise(seed, rnd, int(st.seq_ids[b]), 1 + t) for t in range(N)] for b in range(B)]
        acc_t, acc_n, last, corr = OS.accept_walk(trees, packed, nz, slots=slots, emit_correction=True, **kw)
        out.update(tree_logits=packed, slots=slots)
    else:
        acc_t, acc_n, last, corr = [[int(r)] for r in roots], [[0]] * B, [0] * B, [None] * B
    fin = []
    new_len = []
    pend = np.full(B, -1, np.int64)
    for b in range(B):
        raw = len(acc_t[b])
        t, n_, f, _ = OS.clamp_accepted(acc_t[b], acc_n[b], remaining=max_length - st.seq_len[b],
                                         eos_token_id=spec.eos_token_id, old_len=st.seq_len[b], max_length=max_length)
        acc_t[b], acc_n[b] = t, n_
        fin.append(f)
        new_len.append(len(t))
        if corr[b] is not None and len(t) == raw and not f:
            pend[b] = corr[b]
    width = max(new_len)
    nodes_arr = np.array([p + [p[-1]] * (width - len(p)) for p in acc_n])
    for li in range(L):
        OK.compact_rows_in_place(st.k[li], st.seq_len, nodes_arr, new_len)
        OK.compact_rows_in_place(st.v[li], st.seq_len, nodes_arr, new_len)
    lastn = np.array([p[-1] for p in acc_n])
    st.hidden = hid[np.arange(B), lastn]
    st.logits = OM.logits(st.hidden, W["lm_head"], dtype).astype(np.float32)
    st.seq_len = st.seq_len + np.array(new_len)
    st.pending = pend
    out.update(acc_tokens=acc_t, acc_nodes=acc_n, finished=np.array(fin), correction=corr)
    return out


def generate(cfg, W, heads, prompts, spec: DecodeSpec, *, max_length, seed, repeats=1, dtype=np.float64, cell=None):
    """Whole loop for full-length prompts; returns the generated token lists."""
    prompts = np.repeat(np.asarray(prompts), repeats, axis=0)
    B = prompts.shape[0]
    st = prefill_state(cfg, W, prompts, max(max_length, prompts.shape[1] + 1) + 80, dtype)
    st.logits = st.logits.astype(np.float32)
    gen = [[] for _ in range(B)]
    active = np.arange(B)
    rnd = 0
    while active.size:
        out = verify_round(cfg, W, heads, st, spec, seed, rnd, max_length, dtype, cell=cell)
        for i, b in enumerate(active):
            gen[b].extend(out["acc_tokens"][i])
        keep = ~out["finished"]
        active = active[keep]
        st = State([k[keep] for k in st.k], [v[keep] for v in st.v], st.seq_len[keep], st.hidden[keep],
                   st.logits[keep], st.seq_ids[keep], st.pending[keep])
        rnd += 1
    return gen
