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


def plan_for(spec: DecodeSpec, batch: int) -> OT.Plan:
    return OT.plan_tree(active_batch_size=batch, num_medusa_heads=spec.num_medusa_heads, tree_mode=spec.tree_mode,
                        tree_layout="dense", cpeak_nodes=spec.cpeak_nodes,
                        min_tree_nodes_per_seq=spec.min_tree_nodes_per_seq,
                        max_tree_nodes_per_seq=spec.max_tree_nodes_per_seq, max_tree_depth=spec.max_tree_depth,
                        fixed_tree_topk_by_depth=list(spec.fixed_tree_topk_by_depth),
                        adaptive_tree_enabled=spec.adaptive_tree_enabled,
                        adaptive_min_topk_by_depth=list(spec.adaptive_min_topk_by_depth))


def adapt_plan(spec: DecodeSpec, plan: OT.Plan, medusa_logits) -> OT.Plan:
    """Top-1-probability confidence quantile -> branching -> budget fit
    (``flash_medusa_decoder.py:320-389``)."""
    if not spec.adaptive_tree_enabled or not plan.topk_by_depth:
        return plan
    confs = []
    for lg in medusa_logits[: len(plan.topk_by_depth)]:
        x = np.asarray(lg, np.float64)
        m = x.max(axis=-1)
        lse = m + np.log(np.exp(x - m[:, None]).sum(axis=-1))
        confs.append(OT.quantile_linear(np.exp(m - lse), spec.adaptive_confidence_quantile))
    ks = [OT.topk_from_confidence(c, k, d, enabled=True, min_topk_by_depth=spec.adaptive_min_topk_by_depth,
                                  low=spec.adaptive_confidence_low, high=spec.adaptive_confidence_high)
          for d, (k, c) in enumerate(zip(plan.topk_by_depth, confs))]
    ks = OT.fit_topk_to_budget(ks, plan.node_budget_per_seq,
                               min_topk_by_depth=list(spec.adaptive_min_topk_by_depth)[: len(ks)],
                               depth_weight_decay=spec.adaptive_depth_weight_decay)
    return OT.Plan(plan.node_budget_per_seq, len(ks), ks, OT.dense_node_count(ks), plan.mode, plan.layout)


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
                 dtype=np.float64) -> dict:
    """One round; mutates ``st`` and returns what it decided."""
    B = st.seq_len.shape[0]
    L = cfg.num_layers
    greedy = (not spec.do_sample) or spec.temperature == 0
    kw = dict(do_sample=not greedy, temperature=spec.temperature, top_p=spec.top_p, top_k=spec.top_k)
    roots = np.array([st.pending[b] if spec.emit_correction_token and st.pending[b] >= 0 else
                      OS.sample_row(st.logits[b], OS.counter_noise(seed, rnd, int(st.seq_ids[b]), 0), **kw)
                      for b in range(B)], np.int64)
    plan = plan_for(spec, B)
    mlog = OM.medusa_logits(st.hidden, heads, W["lm_head"], plan.active_heads, dtype) if plan.active_heads else []
    mlog = [np.asarray(x, np.float32) for x in mlog]
    plan = adapt_plan(spec, plan, mlog)
    trees = OT.build_batch_trees(roots, mlog, plan)
    N = trees[0].node_count
    parents = trees[0].parents
    depths = trees[0].depths
    toks = np.array([t.tokens for t in trees], np.int64)
    valid = np.arange(st.k[0].shape[2])[None, :] < st.seq_len[:, None]
    allowed = np.zeros((B, N, N), bool)
    for n in range(N):
        for a in trees[0].ancestors_including_self(n):
            allowed[:, n, a] = True
    pos = st.seq_len[:, None] + np.asarray(depths)[None, :] - 1
    hid, nk, nv = OM.forward(cfg, W, toks, pos, st.k, st.v, valid, allowed, dtype=dtype)
    for li in range(L):
        for b in range(B):
            s = int(st.seq_len[b])
            st.k[li][b, :, s:s + N] = nk[li][b]
            st.v[li][b, :, s:s + N] = nv[li][b]
    out = dict(roots=roots, plan=plan, trees=trees, tree_hidden=hid, medusa_logits=mlog)
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
        st.k[li] = OK.compact_rows(st.k[li], st.seq_len, nodes_arr, new_len)
        st.v[li] = OK.compact_rows(st.v[li], st.seq_len, nodes_arr, new_len)
    lastn = np.array([p[-1] for p in acc_n])
    st.hidden = hid[np.arange(B), lastn]
    st.logits = OM.logits(st.hidden, W["lm_head"], dtype).astype(np.float32)
    st.seq_len = st.seq_len + np.array(new_len)
    st.pending = pend
    out.update(acc_tokens=acc_t, acc_nodes=acc_n, finished=np.array(fin), correction=corr)
    return out


def generate(cfg, W, heads, prompts, spec: DecodeSpec, *, max_length, seed, repeats=1, dtype=np.float64):
    """Whole loop for full-length prompts; returns the generated token lists."""
    prompts = np.repeat(np.asarray(prompts), repeats, axis=0)
    B = prompts.shape[0]
    st = prefill_state(cfg, W, prompts, max(max_length, prompts.shape[1] + 1) + 80, dtype)
    st.logits = st.logits.astype(np.float32)
    gen = [[] for _ in range(B)]
    active = np.arange(B)
    rnd = 0
    while active.size:
        out = verify_round(cfg, W, heads, st, spec, seed, rnd, max_length, dtype)
        for i, b in enumerate(active):
            gen[b].extend(out["acc_tokens"][i])
        keep = ~out["finished"]
        active = active[keep]
        st = State([k[keep] for k in st.k], [v[keep] for v in st.v], st.seq_len[keep], st.hidden[keep],
                   st.logits[keep], st.seq_ids[keep], st.pending[keep])
        rnd += 1
    return gen
