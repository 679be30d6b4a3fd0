#!/usr/bin/env python
"""Rollout benchmark of the FlashGRPO speculative verify step on one MI355X.

A step is one verify round of FlashMedusaDecoder over every active sequence:
root draw, Medusa heads + tied LM head, top-k tree, tree-attention verify
forward, lazy walk LM head + exact_target walk and accepted-path KV
compaction. Default workload: the Qwen2.5-7B shape (28 layers, hidden 3584,
28/4 heads, MLP 18944, vocab 152064, bf16), 64 sequences (8 prompts x 8 GRPO
repeats) with a 2048-token uniform-random prefix, 4 tied Medusa heads, adaptive
concurrency-aware tree (cpeak 2048 -> 32-node budget), temperature 1.0.
Weights are seeded random init; the prefix is really prefilled (untimed).

Prints one JSON line: rollout tok/s (emitted tokens over the timed verify
rounds), per-step latency, the roofline of the dominant hand-written kernel
(tree attention: HIP events on its launch stream around its launches inside the
timed rounds), a per-kernel table from a second, fully instrumented run of the
same number of rounds, and the CPU oracle baseline on a bounded sample of the
same workload.

The timed rounds are bracketed by two short spin kernels (outside the timed
region) so a rocprofv3 kernel trace of this command can be cut to exactly those
rounds: `python bench.py --summarize-trace <run>_kernel_trace.csv` prints the
per-kernel table of the dispatches between the markers.
"""
from __future__ import annotations

import argparse
import gc
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "ss-grpo_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
FP32_PEAK_TFLOPS = 157.3

WORKLOADS = {
    "7b": dict(target="qwen25_7b", prompts=8, repeats=8, prefix=2048, heads=4, tree_mode="concurrency_aware",
               cpeak=2048, max_nodes=32, max_depth=5, topk=(4, 3, 2), adaptive=True, temperature=1.0,
               rollout_rounds=512, name="qwen2.5-7b-shape B64 P2048 4 Medusa heads adaptive 32-node tree"),
    "1.5b": dict(target="qwen25_1p5b", prompts=4, repeats=8, prefix=512, heads=3, tree_mode="concurrency_aware",
                 cpeak=512, max_nodes=16, max_depth=4, topk=(4, 3, 2), adaptive=False, temperature=1.0,
                 rollout_rounds=256, name="qwen2.5-1.5b-shape B32 P512 3 Medusa heads 16-node tree"),
    "14b": dict(target="qwen25_14b", prompts=16, repeats=8, prefix=4096, heads=4, tree_mode="concurrency_aware",
                cpeak=8192, max_nodes=64, max_depth=5, topk=(4, 3, 2), adaptive=False, temperature=1.0,
                rollout_rounds=256, name="qwen2.5-14b-shape B128 P4096 4 Medusa heads 64-node tree"),
    "8b": dict(target="llama31_8b", prompts=12, repeats=8, prefix=1024, heads=4, tree_mode="concurrency_aware",
               cpeak=4608, max_nodes=48, max_depth=5, topk=(4, 3, 2), adaptive=True, temperature=0.7,
               proposal="chain", conf_low=0.20, conf_high=0.70,
               rollout_rounds=256, name="llama-3.1-8b-shape B96 P1024 chain proposals (Medusa head 1 + ChainDraftCell) 48-node tree"),
    "tiny": dict(target="tiny", prompts=4, repeats=2, prefix=256, heads=3, tree_mode="fixed", cpeak=64,
                 max_nodes=16, max_depth=4, topk=(4, 3, 2), adaptive=False, temperature=1.0,
                 rollout_rounds=32, name="tiny-qwen2 B8 P256 3 Medusa heads fixed 16-node tree"),
}


class _NoEosTokenizer:
    pad_token_id = 0
    eos_token_id = -1  # synthetic ids: no end-of-sequence token, rows run to max_length


def build(work, dtype, seed=0):
    import torch

    from flashgrpo_amd.decoding import FlashMedusaConfig, FlashMedusaDecoder
    from flashgrpo_amd.models import MedusaHeads, TargetConfig, TargetModel

    cfg = getattr(TargetConfig, work["target"])()
    model = TargetModel.random(cfg, seed=seed, dtype=dtype, device="cuda")
    heads = MedusaHeads.random(cfg.hidden, cfg.vocab, work["heads"], seed=seed + 1, device="cuda")
    dcfg = FlashMedusaConfig(num_medusa_heads=work["heads"], tree_mode=work["tree_mode"], cpeak_nodes=work["cpeak"],
                             max_tree_nodes_per_seq=work["max_nodes"], max_tree_depth=work["max_depth"],
                             fixed_tree_topk_by_depth=tuple(work["topk"]), adaptive_tree_enabled=work["adaptive"],
                             adaptive_min_topk_by_depth=(1, 1, 1), temperature=work["temperature"], top_p=work["top_p"],
                             noise_seed=seed + 2, proposal_mode=work.get("proposal", "medusa"),
                             adaptive_confidence_low=work.get("conf_low", 0.15),
                             adaptive_confidence_high=work.get("conf_high", 0.45))
    return cfg, model, heads, FlashMedusaDecoder(model, heads, _NoEosTokenizer(), dcfg)


def algorithmic_work(cfg, rnd, seq_before, elem):
    """Per-kernel algorithmic bytes / flops of one verify round (the roofline numerators),
    summed over the round's launches of that kernel."""
    B, N, I, nh = rnd["batch"], rnd["num_nodes"], rnd["internal"], rnd["heads"]
    H, V, d, Hq, Hkv, L = cfg.hidden, cfg.vocab, cfg.head_dim, cfg.q_heads, cfg.kv_heads, cfg.num_layers
    keys = sum(int(s) + N for s in seq_before)
    attn_bytes = 2 * Hkv * keys * d * elem + 2 * B * N * Hq * d * elem       # one layer: K, V, Q in, O out
    attn_flops = 4 * Hq * N * d * keys                                          # one layer: QK^T and PV
    draws = int(rnd["walk_draws"].sum())
    chain = rnd.get("chain_rows") or []
    w = {
        "fg_tree_attention": dict(bytes=L * attn_bytes, flops=L * attn_flops, launches=L),
        "fg_lm_head:medusa": dict(flops=2 * nh * B * H * V, bytes=H * V * elem + nh * B * (H + V) * elem, launches=1),
        # the same rows with the top-k in the epilogue (logits not written)
        "fg_lm_head_topk:medusa": dict(flops=2 * nh * B * H * V, bytes=H * V * elem + nh * B * H * elem, launches=1),
        "fg_medusa_heads": dict(flops=2 * nh * B * H * H, bytes=nh * H * H * elem, launches=1),
        "fg_medusa_topk": dict(bytes=nh * B * V * elem, launches=1),
        "fg_sample_tokens": dict(bytes=B * V * elem, launches=1),
        "fg_kv_path_gather": dict(bytes=2 * L * 2 * Hkv * int(rnd["acc_len"].sum()) * d * elem, launches=1),
    }
    if chain:
        # chain proposals: one LM-head launch and one top-k launch per depth over every
        # parent state; the bootstrap state is Medusa head 0 alone
        R = sum(chain)
        del w["fg_lm_head:medusa"], w["fg_lm_head_topk:medusa"]
        w["fg_lm_head:chain"] = dict(flops=2 * R * H * V, bytes=len(chain) * H * V * elem + R * (H + V) * elem,
                                     launches=len(chain))
        w["fg_lm_head_topk:chain"] = dict(flops=2 * R * H * V, bytes=len(chain) * H * V * elem + R * H * elem,
                                          launches=len(chain))
        w["fg_medusa_heads"] = dict(flops=2 * B * H * H, bytes=H * H * elem, launches=1)
        w["fg_medusa_topk"] = dict(bytes=R * V * elem, launches=len(chain))
    if rnd.get("lazy"):
        # one launch per walk step; a step with an active row streams the whole LM-head
        # weight once, a step with none skips every tile
        D = rnd["walk_steps"]
        busy = int(rnd["walk_draws"].max()) if draws else 0
        w["fg_lm_head:tree"] = dict(flops=2 * draws * H * V, bytes=busy * H * V * elem + draws * (H + V) * elem,
                                    launches=D)
        w["fg_lm_head_topk:tree"] = dict(w["fg_lm_head:tree"])
        w["fg_walk_step"] = dict(bytes=draws * V * elem, launches=D)
    else:
        M = B * I
        w["fg_lm_head:tree"] = dict(flops=2 * M * H * V, bytes=H * V * elem + M * H * elem + M * V * elem,
                                    launches=1)
        w["fg_accept_walk"] = dict(bytes=draws * V * elem, launches=1)
    return w


def planted_walk_gather(cfg, r, work, elem, reps=5):
    """Walk and KV gather at their worst-case bytes.

    With random-init weights no candidate is accepted, so the measured rounds walk
    one step and gather one row. Here the walk's logits rows are planted (the first
    child's token is raised by 60) so every sequence accepts a full-depth path of the
    last round's tree shape: D draws over B rows, then D + 1 rows moved per layer,
    K/V and KV head. Runs on the bench's cache after the measured rounds (the gather
    only rewrites tree slots past each committed length, and repeats are idempotent).
    """
    import torch

    from flashgrpo_amd import kernels as K
    from flashgrpo_amd.decoding.medusa_tree import TreeTopology

    plan = r.plan_last
    topo = TreeTopology(list(plan["topk_by_depth"]), int(plan["node_budget_per_seq"]))
    N, D, B, V = topo.num_nodes, topo.max_depth, len(r.active), cfg.vocab
    if N < 2:
        return None
    dev = r.device
    i32 = dict(dtype=torch.int32, device=dev)
    tokens = ((torch.arange(B, **i32)[:, None] * 1009 + torch.arange(N, **i32)[None, :] * 37) % V).contiguous()
    parents = torch.tensor([topo.parents] * B, **i32)
    n_nodes = torch.full((B,), N, **i32)
    path = [0]
    while True:
        kids = [c for c, p in enumerate(topo.parents) if p == path[-1]]
        if not kids:
            break
        path.append(kids[0])
    g = torch.Generator(device="cpu").manual_seed(5)
    logits = torch.randn(D, B, V, generator=g).to(dev, torch.bfloat16 if elem == 2 else torch.float32)
    ar = torch.arange(B, device=dev)
    for t in range(D):
        logits[t, ar, tokens[:, path[t + 1]].long()] += 60.0
    kw = dict(seed=7, step=0, seq_ids=r.row_map, draw0=1, temperature=work["temperature"], greedy=False,
              top_p=work["top_p"], err_flag=r.err)
    # The lazy walk gets each step's row maxima from the LM head that writes the step's logits
    # (fg_lm_head_topk's part_max / part_key), so a decoder walk step is the q-mass and pick
    # launches. Here the planted logits come from torch, so the same maxima are formed once per
    # step outside the timed region (one part per row: the maximum and its first index's rank key).
    parts = []
    for t in range(D):
        lf = logits[t].float()
        mx, arg = lf.max(dim=1)
        bits = mx.view(torch.int32).to(torch.int64) & 0xFFFFFFFF
        key32 = torch.where(mx < 0, (~bits) & 0xFFFFFFFF, bits | 0x80000000)
        key32 = torch.where(mx == 0, torch.full_like(key32, 0x80000000), key32)
        pk = ((key32 << 32) | (0xFFFFFFFF - arg.to(torch.int64))).view(B, 1).contiguous()
        parts.append((mx.view(B, 1).contiguous(), pk))
    ev = lambda: torch.cuda.Event(enable_timing=True)
    # evicts L2 and the 256 MB Infinity Cache between gather launches: each gather then reads
    # its rows from HBM, as it does in a rollout (the rows were written a round earlier)
    flush = torch.empty(1 << 30, dtype=torch.uint8, device=dev)
    walk_ms, walk_max_ms, gather_ms = [], [], []
    # the walk reads logits the LM head has just written (cache-resident, as in the decoder)
    for rep in range(reps):
        for with_parts, out in ((True, walk_ms), (False, walk_max_ms)):
            # a spin kernel first, so the host has queued the launches below before they
            # run and the events time the GPU, not the launch rate
            torch.cuda._sleep(4_000_000)
            walk = K.walk_begin(tokens, parents, n_nodes, acc_stride=D + 1)
            for t in range(D):
                K.walk_rows(walk, N)
                e0, e1 = ev(), ev()
                e0.record()
                K.walk_step(walk, logits[t], tokens, parents, n_nodes, walk_step=t,
                            parts=parts[t] if with_parts else None, **kw)
                e1.record()
                out.append((e0, e1))
    # the gather reads rows the verify forward wrote a round earlier (evicted since)
    for rep in range(reps):
        flush.fill_(rep & 0xFF)
        torch.cuda._sleep(4_000_000)
        e0, e1 = ev(), ev()
        e0.record()
        r.cache.gather_path(r.seq, walk["acc_nodes"], walk["acc_len"], N, row_map=r.row_map, err_flag=r.err)
        e1.record()
        gather_ms.append((e0, e1))
    torch.cuda.synchronize()
    del flush
    if not bool((walk["acc_len"] == D + 1).all()) or int(r.err.max()) != 0:
        raise RuntimeError("planted walk did not accept the full depth")
    # Back-to-back repeats of the last walk's gather between two events: the rows are then
    # resident in L2 / the Infinity Cache, so this is a warm figure, not an HBM rate. Repeats
    # move the same tree slots past the committed lengths again (the committed rows are never
    # written) and take the same time.
    batch_ms = []
    for _ in range(reps):
        torch.cuda._sleep(4_000_000)
        e0, e1 = ev(), ev()
        e0.record()
        for _ in range(GATHER_BATCH):
            r.cache.gather_path(r.seq, walk["acc_nodes"], walk["acc_len"], N, row_map=r.row_map, err_flag=r.err)
        e1.record()
        batch_ms.append((e0, e1))
    torch.cuda.synchronize()
    if int(r.err.max()) != 0:
        raise RuntimeError("planted gather reported an index error")
    mean_us = lambda evs: sum(a.elapsed_time(b) for a, b in evs) / len(evs) * 1e3
    w_us, wm_us = mean_us(walk_ms), mean_us(walk_max_ms)
    g_us = sorted(a.elapsed_time(b) for a, b in gather_ms)[len(gather_ms) // 2] * 1e3
    g_warm = sorted(a.elapsed_time(b) for a, b in batch_ms)[len(batch_ms) // 2] * 1e3 / GATHER_BATCH
    w_bytes = B * V * elem
    # rows a path keeps in place (the root, and node j == j) are not moved: the bytes are
    # the moved rows' reads and writes; ref_bytes also counts the rows left in place (the
    # reference's gather + copy_ reads and writes every accepted row)
    nodes = walk["acc_nodes"][:, :D + 1].long()
    moved = int((nodes != torch.arange(D + 1, device=dev)[None, :]).sum())
    row_bytes = 2 * cfg.num_layers * 2 * cfg.kv_heads * cfg.head_dim * elem
    g_bytes = row_bytes * moved
    g_ref_bytes = row_bytes * B * (D + 1)
    rate = lambda b, us: round(b / us / 1e3, 1)
    return {"depth": D, "sequences": B,
            # walk_step: the decoder's step (row maxima supplied); with_max_us: plus the chunk-maxima
            # launch (a draw whose logits did not come from the LM head)
            "walk_step": {"avg_us": round(w_us, 2), "with_max_us": round(wm_us, 2), "bytes": w_bytes,
                          "GBps": rate(w_bytes, w_us), "hbm_frac": round(w_bytes / w_us / 1e3 / HBM_PEAK_GBS, 4)},
            # avg_us: one launch on cold rows (caches flushed before it; events around the launch
            # add ~2 us). hbm_frac counts the bytes the kernel moves; ref_hbm_frac the algorithmic
            # bytes of the reference's gather + copy_ (every accepted row read and written).
            # warm_batch_us: back-to-back repeats, rows cache-resident (not an HBM rate)
            "kv_path_gather": {"avg_us": round(g_us, 2), "warm_batch_us": round(g_warm, 2),
                               "bytes": g_bytes, "moved_rows": moved, "ref_bytes": g_ref_bytes,
                               "GBps": rate(g_bytes, g_us),
                               "hbm_frac": round(g_bytes / g_us / 1e3 / HBM_PEAK_GBS, 4),
                               "ref_hbm_frac": round(g_ref_bytes / g_us / 1e3 / HBM_PEAK_GBS, 4)}}


GATHER_BATCH = 10


class _PlantedAcceptance:
    """Makes every walk accept a full-depth path, for timing rounds at full acceptance
    (random-init weights accept no candidate). Inside the context, each logits row a walk
    samples from gets +60 on the token of the first child of the node it belongs to (a
    few small torch launches per walk step, counted in the rounds' time), through the
    kernels module the decoder calls: fg_walk_step's step rows (lazy LM head) and
    fg_accept_walk's packed internal-node rows. Planted walk steps take the rows' maxima
    from the planted logits (the chunk-maxima launch) instead of the LM head's."""

    def __init__(self):
        from flashgrpo_amd import kernels as K

        self.K = K
        self.walk_step, self.accept_walk = K.walk_step, K.accept_walk

    def __enter__(self):
        import torch

        K, walk_step, accept_walk = self.K, self.walk_step, self.accept_walk

        def first_child_tokens(tree_tokens, parents, nodes):
            m = parents == nodes[:, None]
            child = m.to(torch.int32).argmax(1)
            return tree_tokens.gather(1, child[:, None].long()).squeeze(1).long(), m.any(1)

        def planted_walk_step(walk, step_logits, tree_tokens, parents, n_nodes, **kw):
            # the planted logits no longer match the row maxima the LM head wrote with them:
            # the step takes its chunk maxima from the logits (one launch more)
            kw.pop("parts", None)
            B = tree_tokens.shape[0]
            cur, active = walk["state"][:B], walk["state"][B:2 * B] != 0
            tok, has = first_child_tokens(tree_tokens, parents, cur)
            rows = torch.arange(B, device=step_logits.device)
            step_logits[rows, tok] += 60.0 * (has & active).to(step_logits.dtype)
            return walk_step(walk, step_logits, tree_tokens, parents, n_nodes, **kw)

        def planted_accept_walk(tree_logits, tree_tokens, parents, n_nodes, *, slot_map=None, **kw):
            B, N = tree_tokens.shape
            if slot_map is not None:
                nodes = torch.arange(N, device=tree_tokens.device, dtype=parents.dtype)
                for n in range(N):
                    tok, has = first_child_tokens(tree_tokens, parents, nodes[n].expand(B))
                    slot = slot_map[:, n].long()
                    ok = has & (slot >= 0)
                    tree_logits[slot.clamp_min(0)[ok], tok[ok]] += 60.0
            return accept_walk(tree_logits, tree_tokens, parents, n_nodes, slot_map=slot_map, **kw)

        K.walk_step, K.accept_walk = planted_walk_step, planted_accept_walk
        return self

    def __exit__(self, *exc):
        self.K.walk_step, self.K.accept_walk = self.walk_step, self.accept_walk


def planted_full_rounds(dec, r, steps, latency_rounds=8):
    """tok/s and verify-step latency of rounds in which every sequence accepts the tree's
    full depth, with the lazy walk LM head and with the packed internal-node LM head."""
    import numpy as np
    import torch

    out = {}
    lazy0 = dec.config.lazy_walk_lm_head
    try:
        with _PlantedAcceptance():
            for lazy in (True, False):
                dec.config.lazy_walk_lm_head = lazy
                for _ in range(3):  # warm-up (graph capture of the unchanged forward shape)
                    dec.step(r)
                torch.cuda.synchronize()
                toks, lens = 0, []
                t0 = time.perf_counter()
                for _ in range(steps):
                    toks += dec.step(r)
                    lens.append(r.last_round["acc_len"].mean())
                torch.cuda.synchronize()
                sec = time.perf_counter() - t0
                r.event_log = []
                for _ in range(latency_rounds):
                    dec.step(r)
                torch.cuda.synchronize()
                ms = np.array([a.elapsed_time(b) for a, b in r.event_log])
                r.event_log = None
                out["lazy" if lazy else "packed"] = {
                    "tok_s": round(toks / sec, 2), "ms_per_step": round(sec / steps * 1e3, 3),
                    "accept_len_mean": round(float(np.mean(lens)), 3),
                    "verify_step_ms": {"median": round(float(np.median(ms)), 3),
                                       "p90": round(float(np.percentile(ms, 90)), 3)}}
    finally:
        dec.config.lazy_walk_lm_head = lazy0
    return out


def measured_rollout(dec, prompts, repeats, rounds):
    """The reference's own rate (generated tokens over the whole generate() time,
    prefill included, flashgrpo_trainer.py:1117) for one rollout of ``rounds`` decode
    rounds, measured end to end."""
    import torch

    P = prompts.shape[1]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    out = dec.generate(prompts, torch.ones_like(prompts), repeated_generate_nums=repeats, max_length=P + rounds)
    torch.cuda.synchronize()
    sec = time.perf_counter() - t0
    toks = sum(len(g) for g in out["generated_token_ids"])
    return {"tok_s": round(toks / sec, 2), "seconds": round(sec, 3), "tokens": int(toks),
            "verify_rounds": int(out["total_verify_rounds"]), "prefill_s": round(out["prefill_time_cost"], 3)}


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(model, heads, r, work, seed, rounds=1):
    """The oracle (numpy, fp32, every layer of the model) running ``rounds`` verify rounds
    of the same workload on the host, from the device's current rollout state (its KV
    cache, hidden states and logits copied to host memory). Nothing is scaled: the
    figure is the tokens those rounds emit over their wall time."""
    import numpy as np

    from oracle import decode as OD
    from oracle import model as OM

    cfg = model.cfg
    f = lambda t: t.detach().float().cpu().numpy()
    qd, kd = cfg.q_heads * cfg.head_dim, cfg.kv_heads * cfg.head_dim
    W = {"embed": f(model.w["embed"]), "final_norm": f(model.w["final_norm"]), "layers": [],
         "inv_freq": model.inv_freq.cpu().numpy()}
    W["lm_head"] = W["embed"] if model.w["lm_head"] is model.w["embed"] else f(model.w["lm_head"])
    for lw in model.w["layers"]:
        qkv = f(lw["qkv_w"])
        b = f(lw["qkv_b"]) if lw["qkv_b"] is not None else None
        gu = f(lw["gate_up_w"])
        W["layers"].append({"input_norm": f(lw["input_norm"]), "q_w": qkv[:qd], "k_w": qkv[qd:qd + kd],
                            "v_w": qkv[qd + kd:], "q_b": None if b is None else b[:qd],
                            "k_b": None if b is None else b[qd:qd + kd], "v_b": None if b is None else b[qd + kd:],
                            "o_w": f(lw["o_w"]), "post_norm": f(lw["post_norm"]), "gate_w": gu[:cfg.intermediate],
                            "up_w": gu[cfg.intermediate:], "down_w": f(lw["down_w"])})
    hd = [{"ln_w": f(h.norm.weight), "ln_b": f(h.norm.bias),
           "fc_w": f(h.fc.weight.to(model.dtype)), "fc_b": f(h.fc.bias.to(model.dtype))} for h in heads.heads]
    cc = heads.chain_cell
    g = lambda t: f(t.to(model.dtype))
    cell = {"sn_w": g(cc.state_norm.weight), "sn_b": g(cc.state_norm.bias), "tn_w": g(cc.token_norm.weight),
            "tn_b": g(cc.token_norm.bias), "sp_w": g(cc.state_proj.weight), "tp_w": g(cc.token_proj.weight),
            "op_w": g(cc.out_proj.weight), "op_b": g(cc.out_proj.bias), "gate": float(cc.gate.detach())}
    ocfg = OM.ModelConfig(cfg.num_layers, cfg.hidden, cfg.q_heads, cfg.kv_heads, cfg.head_dim, cfg.intermediate,
                          cfg.vocab, cfg.rope_theta, cfg.rms_eps, cfg.qkv_bias, cfg.tie_word_embeddings)
    # room for `rounds` rounds of the widest tree after the longest committed row
    cap = int(r.seq_h.max()) + rounds * (int(work["max_nodes"]) + 8) + 8
    rows = r.row_map.long()
    st = OD.State([f(r.cache.kv[l, 0].index_select(0, rows)[:, :, :cap]) for l in range(cfg.num_layers)],
                  [f(r.cache.kv[l, 1].index_select(0, rows)[:, :, :cap]) for l in range(cfg.num_layers)],
                  r.seq_h.copy(), f(r.hidden), f(r.logits), rows.cpu().numpy(),
                  np.full(len(r.active), -1, np.int64))
    spec = OD.DecodeSpec(num_medusa_heads=work["heads"], tree_mode=work["tree_mode"], cpeak_nodes=work["cpeak"],
                         max_tree_nodes_per_seq=work["max_nodes"], max_tree_depth=work["max_depth"],
                         fixed_tree_topk_by_depth=tuple(work["topk"]), adaptive_tree_enabled=work["adaptive"],
                         temperature=work["temperature"], top_p=work["top_p"],
                         proposal_mode=work.get("proposal", "medusa"),
                         adaptive_confidence_low=work.get("conf_low", 0.15),
                         adaptive_confidence_high=work.get("conf_high", 0.45))
    threads = len(os.sched_getaffinity(0))
    try:
        from threadpoolctl import threadpool_info

        blas = [p["num_threads"] for p in threadpool_info() if p.get("user_api") == "blas"]
        threads = max(blas) if blas else threads
    except Exception:
        pass
    tokens = 0
    t0 = time.perf_counter()
    for rnd in range(rounds):
        out = OD.verify_round(ocfg, W, hd, st, spec, seed, rnd, 10 ** 9, dtype=np.float32, cell=cell)
        tokens += sum(len(t) for t in out["acc_tokens"])
    secs = time.perf_counter() - t0
    B, N = len(r.active), out["trees"][0].node_count
    return {"value": round(tokens / secs, 3), "unit": "tok/s", "cores": int(threads), "kind": "port",
            "cpu": cpu_model(),
            "sample": (f"{rounds} verify round(s) of the same workload (B={B}, N={N}, all {cfg.num_layers} layers, "
                       f"vocab {cfg.vocab}) through the numpy oracle in fp32 from the device's rollout state: "
                       f"{tokens} tokens in {secs:.2f} s, no scaling"),
            "seconds": round(secs, 3), "rounds": rounds}


def summarize_trace(path, top=30):
    """Per-kernel table of a rocprofv3 kernel-trace CSV, restricted to the dispatches
    between the first two spin-kernel markers, which bracket the timed rounds (later
    spin kernels belong to the planted measurement)."""
    import csv

    with open(path, newline="") as fh:
        rows = sorted(csv.DictReader(fh), key=lambda r: int(r["Start_Timestamp"]))
    marks = [i for i, r in enumerate(rows) if "spin_kernel" in r["Kernel_Name"]]
    if len(marks) < 2:
        raise SystemExit(f"{path}: no pair of spin_kernel markers around the timed rounds")
    sel = rows[marks[0] + 1:marks[1]]
    agg = {}
    for r in sel:
        name = r["Kernel_Name"]
        dur = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
        a = agg.setdefault(name, [0, 0.0, float("inf"), 0.0])
        a[0] += 1
        a[1] += dur
        a[2] = min(a[2], dur)
        a[3] = max(a[3], dur)
    total = sum(a[1] for a in agg.values())
    span = (int(sel[-1]["End_Timestamp"]) - int(sel[0]["Start_Timestamp"])) / 1e3
    print(f"dispatches between the markers: {len(sel)}; kernel time {total / 1e3:.3f} ms; "
          f"first start to last end {span / 1e3:.3f} ms")
    print("| total ms | % | calls | avg us | min us | max us | kernel |")
    print("|---:|---:|---:|---:|---:|---:|---|")
    for name, (c, t, lo, hi) in sorted(agg.items(), key=lambda kv: -kv[1][1])[:top]:
        short = name if len(name) <= 100 else name[:97] + "..."
        print(f"| {t / 1e3:.3f} | {100 * t / total:.1f} | {c} | {t / c:.1f} | {lo:.1f} | {hi:.1f} | `{short}` |")


# Device symbol of each C-ABI entry point whose launches the roofline can name.
KERNEL_SYMBOLS = {"fg_tree_attention": "tree_attn_bf16_kernel", "fg_lm_head": "gemm_bf16_stream",
                  "fg_lm_head_topk": "lm_stream_kernel",
                  "fg_sample_tokens": "split_", "fg_kv_path_gather": "kv_path_gather_kernel"}


def pmc_traffic(fetch_csv, write_csv, symbol, scale):
    """Mean HBM bytes per dispatch of `symbol` from FETCH_SIZE / WRITE_SIZE counter CSVs
    (KiB per dispatch, each scaled by what the counter reads for a copy of known size)."""
    import csv

    total = 0.0
    for path, counter, k in ((fetch_csv, "FETCH_SIZE", scale[0]), (write_csv, "WRITE_SIZE", scale[1])):
        with open(path, newline="") as fh:
            rows = sorted(csv.DictReader(fh), key=lambda r: int(r["Dispatch_Id"]))
        marks = sorted({int(r["Dispatch_Id"]) for r in rows if "spin_kernel" in r["Kernel_Name"]})
        lo, hi = (marks[0], marks[1]) if len(marks) >= 2 else (-1, 1 << 62)  # the timed rounds
        vals = [float(r["Counter_Value"]) for r in rows
                if lo < int(r["Dispatch_Id"]) < hi and symbol in r["Kernel_Name"] and r["Counter_Name"] == counter]
        if not vals:
            return None
        total += sum(vals) / len(vals) * 1024.0 * k
    return int(total)


def summarize_pmc(path, symbol):
    """Mean value per dispatch of every counter in a rocprofv3 --pmc CSV, over the
    dispatches of kernels whose name contains `symbol` between the timed-round markers."""
    import csv

    with open(path, newline="") as fh:
        rows = sorted(csv.DictReader(fh), key=lambda r: int(r["Dispatch_Id"]))
    # one row per (dispatch, counter): markers are distinct dispatch ids
    marks = sorted({int(r["Dispatch_Id"]) for r in rows if "spin_kernel" in r["Kernel_Name"]})
    lo, hi = (marks[0], marks[1]) if len(marks) >= 2 else (-1, 1 << 62)
    acc = {}
    for r in rows:
        if lo < int(r["Dispatch_Id"]) < hi and symbol in r["Kernel_Name"]:
            acc.setdefault(r["Counter_Name"], []).append(float(r["Counter_Value"]))
    print(f"{path}: kernels matching {symbol!r} between the timed-round markers")
    print("| counter | dispatches | mean per dispatch |")
    print("|---|---:|---:|")
    for name, v in sorted(acc.items()):
        print(f"| {name} | {len(v)} | {sum(v) / len(v):.6g} |")


def attention_only(args, work):
    """fg_tree_attention alone at the config's verify shape: batches of 10 back-to-back
    launches behind a spin kernel, rotating over --cold distinct K/V caches (cold reads),
    HIP events around each batch. Prints one JSON line (us per launch, GB/s, HBM fraction)."""
    import numpy as np
    import torch

    from flashgrpo_amd import kernels as K
    from flashgrpo_amd.decoding.medusa_tree import TreeTopology
    from flashgrpo_amd.models import TargetConfig

    cfg = getattr(TargetConfig, work["target"])()
    B, Hq, Hkv, d = work["prompts"] * work["repeats"], cfg.q_heads, cfg.kv_heads, cfg.head_dim
    P = work["prefix"]
    # the dense tree the config's plan realises with random weights (adaptive plans keep their base k)
    ks = {"7b": [4, 2, 1, 1], "14b": [4, 3, 2], "1.5b": [4, 2], "tiny": [4, 2], "8b": [4, 3, 2, 2]}[args.config]
    topo = TreeTopology(ks, work["max_nodes"])
    N = topo.num_nodes
    cap = P + 64 + 80
    dev, dt = "cuda", torch.bfloat16 if args.config != "tiny" else torch.float32
    g = torch.Generator(device=dev).manual_seed(0)
    kcs = [torch.randn(B, Hkv, cap, d, generator=g, device=dev, dtype=dt) for _ in range(args.cold)]
    vcs = [torch.randn(B, Hkv, cap, d, generator=g, device=dev, dtype=dt) for _ in range(args.cold)]
    q = torch.randn(B, N, Hq, d, generator=g, device=dev, dtype=dt)
    seq = torch.full((B,), P, dtype=torch.int32, device=dev)
    anc = torch.from_numpy(np.array([b & 0xFFFFFFFFFFFFFFFF for b in topo.anc_bits],
                                    dtype=np.uint64).view(np.int64)).to(dev)
    out = torch.empty_like(q)

    def launch(c):
        K.tree_attention(q, kcs[c], vcs[c], seq_len=seq, anc=anc, num_nodes=N, q_heads=Hq, kv_heads=Hkv,
                         head_dim=d, out=out)

    for c in range(args.cold):
        launch(c)
    torch.cuda.synchronize()
    evs = []
    for _ in range(max(args.steps, 1)):
        torch.cuda._sleep(2_000_000)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for j in range(10):
            launch(j % args.cold)
        e1.record()
        evs.append((e0, e1))
    torch.cuda.synchronize()
    us = np.array([a.elapsed_time(b) for a, b in evs]) * 1e3 / 10
    elem = 2 if dt == torch.bfloat16 else 4
    byts = 2 * B * Hkv * (P + N) * d * elem + 2 * B * N * Hq * d * elem
    med = float(np.median(us))
    if getattr(args, "calibrate_copy", False):
        # a device copy of known size in the same run: what FETCH_SIZE / WRITE_SIZE read for it
        # scales the counters of the attention launches into bytes
        src = torch.empty(COPY_BYTES, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(COPY_REPS):
            dst.copy_(src)
        torch.cuda.synchronize()
    print(json.dumps({"kernel": "fg_tree_attention", "config": args.config, "sequences": B, "tree_nodes": N,
                      "prefix": P, "cold_caches": args.cold, "batches": len(us), "us_median": round(med, 2),
                      "us_min": round(float(us.min()), 2), "bytes": byts, "GBps": round(byts / med / 1e3, 1),
                      "hbm_frac": round(byts / med / 1e3 / HBM_PEAK_GBS, 4)}), flush=True)


COPY_BYTES = 256 << 20
COPY_REPS = 3
COPY_SYMBOL = "copyBuffer"


def measure_traffic(args, symbol, timeout_s=240):
    """HBM bytes per launch of the roofline kernel from two rocprofv3 --pmc passes
    (FETCH_SIZE, then WRITE_SIZE, each its own run) over `bench.py --attention-only` at
    the same shape, each counter scaled by what it reads for a 256 MiB device copy in the
    same run. Returns (bytes, detail) or (None, reason)."""
    import csv
    import shutil
    import signal
    import subprocess
    import tempfile

    prof = shutil.which("rocprofv3") or ("/opt/rocm/bin/rocprofv3" if os.path.exists("/opt/rocm/bin/rocprofv3")
                                         else None)
    if prof is None:
        return None, "rocprofv3 not found"
    tmp = os.environ.get("TMPDIR") if os.path.isdir(os.environ.get("TMPDIR", "")) else "/tmp"
    means = {}
    for counter in ("FETCH_SIZE", "WRITE_SIZE"):
        out = tempfile.mkdtemp(prefix="fg_pmc_", dir=tmp)
        cmd = [prof, "--pmc", counter, "--output-format", "csv", "-d", out, "-o", "run", "--", sys.executable,
               os.path.abspath(__file__), "--attention-only", "--config", args.config, "--steps", "2",
               "--calibrate-copy"]
        print(f"bench: traffic pass {counter}", file=sys.stderr, flush=True)
        proc = subprocess.Popen(cmd, stdout=subprocess.DEVNULL, stderr=subprocess.DEVNULL, start_new_session=True,
                                env=dict(os.environ, TMPDIR=tmp))
        try:
            proc.wait(timeout=timeout_s)
        except subprocess.TimeoutExpired:
            os.killpg(proc.pid, signal.SIGKILL)
            proc.wait()
            return None, f"{counter} pass timed out"
        paths = [os.path.join(dp, f) for dp, _, fs in os.walk(out) for f in fs if f.endswith("counter_collection.csv")]
        if not paths:
            return None, f"{counter} pass wrote no counter CSV (exit {proc.returncode})"
        with open(paths[0], newline="") as fh:
            m = counter_means(csv.DictReader(fh), counter, symbol)
        shutil.rmtree(out, ignore_errors=True)
        if m is None:
            return None, f"{counter}: no dispatches of {symbol} or of the calibration copy"
        means[counter] = m
    return traffic_from_means(means)


def counter_means(rows, counter, symbol):
    """(mean KiB per dispatch of `symbol`, KiB per calibration copy) of one counter from the
    rows of a rocprofv3 counter_collection CSV; None if either is missing. The runtime may
    split one copy over several dispatches, so the copy's figure is the sum of its dispatches
    divided by the number of copies."""
    vals = {symbol: [], COPY_SYMBOL: []}
    for row in rows:
        if row.get("Counter_Name") != counter:
            continue
        for key in vals:
            if key in row["Kernel_Name"]:
                vals[key].append(float(row["Counter_Value"]))
    if not vals[symbol] or not vals[COPY_SYMBOL]:
        return None
    return sum(vals[symbol]) / len(vals[symbol]), sum(vals[COPY_SYMBOL]) / COPY_REPS


def traffic_from_means(means):
    """Bytes per launch: each counter's KiB per launch times copy bytes / counted copy bytes."""
    scale = {c: COPY_BYTES / (m[1] * 1024.0) for c, m in means.items()}  # copy bytes per counted byte
    total = sum(m[0] * 1024.0 * scale[c] for c, m in means.items())
    detail = {c: {"KiB_per_launch": round(m[0], 1), "copy_KiB": round(m[1], 1), "scale": round(scale[c], 4)}
              for c, m in means.items()}
    return int(total), detail


def lm_head_only(args, work):
    """The LM-head projection alone at the config's vocabulary and hidden size, for 64, 128,
    192 and 256 bf16 rows: fg_lm_head_topk (logits only; logits + top-k; top-k without the
    logits) against hipBLASLt (F.linear with the tuned table) and hipBLASLt + fg_medusa_topk.
    Batches of 10 launches behind a spin kernel, alternating over two weight copies (cold
    reads), HIP events around each batch. Prints one JSON line per row count."""
    import numpy as np
    import torch
    import torch.nn.functional as F

    from flashgrpo_amd import kernels as K
    from flashgrpo_amd.models import TargetConfig
    from flashgrpo_amd.tuning import use_tuned_gemms

    use_tuned_gemms()
    cfg = getattr(TargetConfig, work["target"])()
    H, V = cfg.hidden, cfg.vocab
    dev, dt = "cuda", torch.bfloat16
    g = torch.Generator(device=dev).manual_seed(0)
    ws = [(torch.randn(V, H, generator=g, device=dev) * 0.02).to(dt) for _ in range(2)]
    kmax = 4

    def timed(fn):
        for i in range(4):
            fn(i)
        torch.cuda.synchronize()
        evs = []
        for _ in range(max(args.steps, 1)):
            torch.cuda._sleep(2_000_000)
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for j in range(10):
                fn(j)
            e1.record()
            evs.append((e0, e1))
        torch.cuda.synchronize()
        return float(np.median(np.array([a.elapsed_time(b) for a, b in evs]) * 1e3 / 10))

    for M in (64, 128, 192, 256):
        x = torch.randn(M, H, generator=g, device=dev).to(dt)
        out = torch.empty(M, V, dtype=dt, device=dev)
        wk = torch.empty(K._lib.load().fg_lm_head_topk_workspace(M, V, kmax), dtype=torch.uint8, device=dev)
        res = {
            "lm_head": timed(lambda i: K.lm_head_topk(x, ws[i % 2], 0, out=out)),
            "lm_head+topk": timed(lambda i: K.lm_head_topk(x, ws[i % 2], kmax, out=out, stats=True, workspace=wk)),
            "topk_only": timed(lambda i: K.lm_head_topk(x, ws[i % 2], kmax, logits=False, stats=True,
                                                        workspace=wk)),
            "hipblaslt": timed(lambda i: F.linear(x, ws[i % 2])),
            "hipblaslt+topk": timed(lambda i: K.medusa_topk(F.linear(x, ws[i % 2]), kmax, stats=True)),
        }
        byts = V * H * 2 + M * H * 2 + M * V * 2
        print(json.dumps({"kernel": "fg_lm_head_topk", "config": args.config, "rows": M, "vocab": V, "hidden": H,
                          "kmax": kmax, "batches": max(args.steps, 1),
                          "us_median": {k: round(v, 1) for k, v in res.items()},
                          "lm_head_hbm_frac": round(byts / res["lm_head"] / 1e3 / HBM_PEAK_GBS, 4),
                          "weight_only_hbm_frac": round(V * H * 2 / res["lm_head"] / 1e3 / HBM_PEAK_GBS, 4)}),
              flush=True)


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=16)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default="7b", choices=sorted(WORKLOADS))
    ap.add_argument("--top-p", type=float, default=1.0, help="1.0 for throughput; 0.95 is the reference default")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-planted-rounds", action="store_true",
                    help="skip the full-acceptance rounds (lazy vs packed tree LM head)")
    ap.add_argument("--no-rollout", action="store_true",
                    help="skip the measured end-to-end rollout (prefill + the config's decode rounds)")
    ap.add_argument("--cpu-rounds", type=int, default=None,
                    help="verify rounds the CPU oracle runs (default: 32 for the tiny config, 1 otherwise)")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--decoder-gemms", default="table", choices=("table", "hand", "library"),
                    help="decoder projections: as the measured path tables choose (default), all on the "
                         "hand-written split-K / fused MLP kernels, or all on hipBLASLt")
    ap.add_argument("--roofline-kernel", default="fg_tree_attention",
                    help="C-ABI entry point whose launches are event-timed in the timed rounds")
    ap.add_argument("--roofline-every", type=int, default=7,
                    help="event-time every launch of the roofline kernel in one timed round in this many "
                         "(those rounds run the verify forward eagerly, the others replay its HIP graph)")
    ap.add_argument("--traffic-from", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"),
                    help="rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE counter_collection CSVs of the roofline kernel")
    ap.add_argument("--traffic-scale", nargs=2, type=float, default=(2.0, 1.0), metavar=("FETCH", "WRITE"),
                    help="copy KiB per counter KiB, measured on a plain copy of known size (FETCH_SIZE, WRITE_SIZE)")
    ap.add_argument("--attention-only", action="store_true",
                    help="time fg_tree_attention alone at the config's verify shape (batches of 10 launches)")
    ap.add_argument("--cold", type=int, default=8, help="--attention-only: distinct K/V caches rotated over")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="--attention-only: also run a 256 MiB device copy (counter calibration)")
    ap.add_argument("--no-traffic", action="store_true",
                    help="skip the two rocprofv3 --pmc passes that measure the roofline kernel's HBM traffic")
    ap.add_argument("--lm-head-only", action="store_true",
                    help="time the LM-head kernel alone against hipBLASLt at 64..256 rows and exit")
    ap.add_argument("--summarize-trace", metavar="CSV", help="summarise a rocprofv3 kernel trace of this command")
    ap.add_argument("--summarize-pmc", nargs=2, metavar=("CSV", "KERNEL"),
                    help="per-dispatch counter means of one kernel from a rocprofv3 --pmc run of this command")
    args = ap.parse_args()
    if args.summarize_trace:
        summarize_trace(args.summarize_trace)
        return
    if args.summarize_pmc:
        summarize_pmc(*args.summarize_pmc)
        return
    if args.gpus != 1:
        print(f"bench.py measures one MI355X: --gpus {args.gpus} is not supported (sequences shard by data "
              "parallelism with no exchange inside the verify step; run one process per GPU)", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    from flashgrpo_amd import timing

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    work = dict(WORKLOADS[args.config], top_p=args.top_p)
    if args.attention_only:
        attention_only(args, work)
        return
    if args.lm_head_only:
        lm_head_only(args, work)
        return
    if args.warmup < 3:
        # the verify forward's HIP graph is captured on its second graph round and the last
        # warm-up round runs eagerly under the kernel timer, so fewer than three warm-up
        # rounds would leave the capture inside the timed rounds
        print(f"bench: warmup raised from {args.warmup} to 3 (graph capture before the timed rounds)",
              file=sys.stderr, flush=True)
        args.warmup = 3
    dtype = torch.float32 if args.config == "tiny" else torch.bfloat16
    elem = 4 if dtype == torch.float32 else 2
    log = lambda msg: print(f"bench: {msg}", file=sys.stderr, flush=True)
    cfg, model, heads, dec = build(work, dtype, seed=args.seed)
    if args.decoder_gemms != "table":
        hand = args.decoder_gemms == "hand"
        model.split_k_linear = hand  # QKV, O, down: fg_linear_parts + its finishing kernels, or the library
        model.fused_mlp = hand       # gate/up: fg_gate_up_swiglu, or the library projection + fg_swiglu
    log(f"built {work['name']} ({dtype})")
    g = torch.Generator().manual_seed(args.seed + 3)
    prompts = torch.randint(0, cfg.vocab, (work["prompts"], work["prefix"]), generator=g)
    # long enough that no row reaches max_length inside the benchmark
    max_length = work["prefix"] + 8 * (args.warmup + 2 * args.steps + 20) + 64
    # one short rollout start first, so the timed prefill excludes one-time library and
    # kernel loading (as in a trainer's later generation steps)
    dec.finish(dec.start(prompts[:1, :64], torch.ones_like(prompts[:1, :64]), max_length=128))
    torch.cuda.synchronize()
    t_pre = time.perf_counter()
    r = dec.start(prompts, torch.ones_like(prompts), repeated_generate_nums=work["repeats"], max_length=max_length)
    torch.cuda.synchronize()
    prefill_s = time.perf_counter() - t_pre
    log(f"prefill {prefill_s:.1f} s")
    for i in range(args.warmup):
        # the last warm-up round runs like a roofline-timed round (eager forward,
        # events on the roofline kernel), after a full collection of Python's cyclic
        # garbage (the collector is then paused for the timed rounds, as timeit does)
        last = i == args.warmup - 1
        if last:
            gc.collect()
            gc.disable()
        with timing.active(timing.KernelTimer(only={args.roofline_kernel}) if last else None):
            dec.step(r)
    torch.cuda.synchronize()
    log("warmup done")
    # Timed rounds: in one round of every --roofline-every, each launch of the
    # roofline kernel is bracketed by HIP events on its stream (that round runs the
    # verify forward launch by launch); the other rounds replay the forward's HIP
    # graph, as the decoder does by default. Nothing else is timed inside.
    every = max(args.roofline_every, 1)
    rtimer = timing.KernelTimer(only={args.roofline_kernel},
                                reserve=cfg.num_layers * ((args.steps + every - 1) // every) + 8)
    torch.cuda.synchronize()
    rounds, seqs = [], []
    tokens = 0
    # (a full collection inside the timed rounds has cost ~40 ms of one round)
    torch.cuda._sleep(1000)  # trace marker: the timed rounds start after this kernel
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    marks = []
    for i in range(args.steps):
        with timing.active(rtimer if i % every == 0 else None):
            seqs.append(r.seq_h.copy())
            tokens += dec.step(r)
            rounds.append(r.last_round)
        marks.append(time.perf_counter())
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    gc.enable()
    log("timed rounds (host ms, each ends at the round's sync): "
        + " ".join(f"{(b - a) * 1e3:.2f}" for a, b in zip([t0] + marks[:-1], marks)))
    torch.cuda._sleep(1000)  # trace marker: end of the timed rounds
    torch.cuda.synchronize()
    log(f"timed {args.steps} steps in {elapsed:.3f} s")
    # Instrumented rounds (same workload, continuing): every hand-written launch
    # timed, for the per-kernel table.
    timer = timing.KernelTimer(reserve=2048)
    rounds_i, seqs_i = [], []
    t1 = time.perf_counter()
    with timing.active(timer):
        for _ in range(args.steps):
            seqs_i.append(r.seq_h.copy())
            dec.step(r)
            rounds_i.append(r.last_round)
    torch.cuda.synchronize()
    elapsed_i = time.perf_counter() - t1
    kstats = timer.summary()
    rstats = rtimer.summary()
    log(f"instrumented {args.steps} steps in {elapsed_i:.3f} s")
    # Latency rounds (continuing): HIP events on the stream around each round's verify
    # step, kept out of the timed rounds.
    r.event_log = []
    for _ in range(max(min(args.steps, 8), 1)):
        dec.step(r)
    torch.cuda.synchronize()
    step_ms = np.array([a.elapsed_time(b) for a, b in r.event_log])
    r.event_log = None
    # Phase rounds (continuing): the decoder's statistical_time mode synchronises
    # at each phase boundary, so the phases add up to slightly more than a round.
    phase_keys = ("medusa_time", "verify_time", "accept_time", "cache_time")
    dec.flush(r)  # the queued round completes outside the phase rounds
    before = {k: r.m[k] for k in phase_keys}
    r.statistical_time = True
    n_phase = max(min(args.steps, 8), 1)
    t2 = time.perf_counter()
    for _ in range(n_phase):
        dec.step(r)
    torch.cuda.synchronize()
    elapsed_p = time.perf_counter() - t2
    r.statistical_time = False
    phases = {k.replace("_time", ""): round((r.m[k] - before[k]) / n_phase * 1e3, 3) for k in phase_keys}
    phases["other"] = round(elapsed_p / n_phase * 1e3 - sum(phases.values()), 3)
    phases["rounds"] = n_phase
    log(f"phases (ms/round) {phases}")
    dec.flush(r)  # the planted walk and gather work on the committed cache state
    planted = planted_walk_gather(cfg, r, work, elem)
    log(f"planted {planted}")
    full_rounds = None
    if not args.no_planted_rounds:
        full_rounds = planted_full_rounds(dec, r, args.steps)
        log(f"planted full-acceptance rounds {full_rounds}")
    rollout = None
    if not args.no_rollout:
        rollout = measured_rollout(dec, prompts, work["repeats"], int(work["rollout_rounds"]))
        log(f"measured rollout {rollout}")

    def work_totals(rnds, sqs):
        totals = {}
        for rnd, sq in zip(rnds, sqs):
            for name, w in algorithmic_work(cfg, rnd, sq, elem).items():
                t = totals.setdefault(name, dict(bytes=0, flops=0, launches=0))
                t["bytes"] += w.get("bytes", 0)
                t["flops"] += w.get("flops", 0)
                t["launches"] += w["launches"]
        return totals

    peak_f = BF16_PEAK_TFLOPS if dtype == torch.bfloat16 else FP32_PEAK_TFLOPS
    # per-kernel table (instrumented rounds): algorithmic work over the measured launch time
    totals_i = work_totals(rounds_i, seqs_i)
    kernels = {}
    for name, t in totals_i.items():
        ks = kstats.get(name)
        if not ks or ks["total_ms"] <= 0:
            continue
        sec = ks["total_ms"] / 1e3
        gbs = t["bytes"] / sec / 1e9
        tfl = t["flops"] / sec / 1e12
        frac = max(gbs / HBM_PEAK_GBS, tfl / peak_f)
        kernels[name] = dict(avg_us=round(ks["avg_ms"] * 1e3, 2), launches=ks["count"],
                             total_ms=round(ks["total_ms"], 3), GBps=round(gbs, 1), TFLOPs=round(tfl, 2),
                             roofline_frac=round(frac, 4))
    mine_ms = sum(v["total_ms"] for k, v in kstats.items())
    # roofline of the named kernel over the timed rounds
    name = args.roofline_kernel
    t = work_totals(rounds, seqs)[name]
    ks = rstats[name]
    per_launch_s = ks["avg_ms"] / 1e3
    n_launch = max(t["launches"], 1)
    bound = "mfma" if t["flops"] / max(t["bytes"], 1) > (peak_f * 1e12) / (HBM_PEAK_GBS * 1e9) else "hbm"
    if bound == "hbm":
        achieved = t["bytes"] / n_launch / per_launch_s / 1e9
        roofline = dict(bound="hbm", achieved=round(achieved, 1), peak=HBM_PEAK_GBS, unit="GB/s",
                        frac=round(achieved / HBM_PEAK_GBS, 4), traffic=None, kernel=name,
                        bytes_per_launch=int(t["bytes"] / n_launch), avg_launch_us=round(ks["avg_ms"] * 1e3, 2),
                        timed_launches=ks["count"], launches=t["launches"])
    else:
        achieved = t["flops"] / n_launch / per_launch_s / 1e12
        roofline = dict(bound="mfma", achieved=round(achieved, 2), peak=peak_f, unit="TFLOP/s",
                        frac=round(achieved / peak_f, 4), traffic=None, kernel=name,
                        flops_per_launch=int(t["flops"] / n_launch), avg_launch_us=round(ks["avg_ms"] * 1e3, 2),
                        timed_launches=ks["count"], launches=t["launches"])

    if args.traffic_from:
        roofline["traffic"] = pmc_traffic(args.traffic_from[0], args.traffic_from[1],
                                          KERNEL_SYMBOLS.get(name, name), args.traffic_scale)
    elif not args.no_traffic and name == "fg_tree_attention" and dtype == torch.bfloat16:
        traffic, detail = measure_traffic(args, KERNEL_SYMBOLS[name])
        roofline["traffic"] = traffic
        roofline["traffic_source"] = ("rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE (one run each) over "
                                      "`bench.py --attention-only` at this shape, scaled by a 256 MiB copy")
        roofline["traffic_detail"] = detail
        log(f"traffic {traffic} {detail}")
    cpu = None
    if not args.no_cpu_baseline:
        log("cpu baseline ...")
        n_cpu = args.cpu_rounds or (32 if args.config == "tiny" else 1)
        dec.flush(r)
        cpu = cpu_baseline(model, heads, r, work, seed=args.seed + 2, rounds=n_cpu)
        log(f"cpu baseline {cpu['seconds']} s")
    res = {
        "metric": "rollout tok/s per MI355X (Qwen2.5-7B shape); verify-step latency; % roofline",
        "value": round(tokens / elapsed, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(elapsed / args.steps * 1e3, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16" if dtype == torch.bfloat16 else "fp32",
        "data": "synthetic (uniform-random prefix tokens, seeded random-init weights and Medusa heads, counter noise)",
        "config": {"workload": work["name"], "sequences": len(r.active), "prefix": work["prefix"],
                   "tree_nodes": rounds[-1]["num_nodes"], "internal_nodes": rounds[-1]["internal"],
                   "topk_by_depth": r.plan_last.get("topk_by_depth"), "temperature": work["temperature"],
                   "top_p": work["top_p"], "parallelism": "single GPU",
                   "verify_forward": "HIP graph replay (eager in the roofline-timed rounds)",
                   "decoder_gemms": args.decoder_gemms},
        "tokens": int(tokens),
        "accept_len_mean": round(tokens / max(sum(x["batch"] for x in rounds), 1), 4),
        "prefill_s": round(prefill_s, 2),
        # The reference's own rate (generated tokens over generation time including the
        # prefill, flashgrpo_trainer.py:1117): one whole rollout of the config's decode
        # rounds timed end to end (generate()).
        "with_prefill": rollout,
        # every sequence accepting the tree's full depth (planted), lazy vs packed tree LM head
        "planted_full_rounds": full_rounds,
        "hand_kernels_ms_per_step": round(mine_ms / args.steps, 3),
        "ms_per_step_instrumented": round(elapsed_i / args.steps * 1e3, 3),
        "phases_ms": phases,
        # HIP events on the stream: verify forward + tree LM head + walk + KV extraction
        "verify_step_ms": {"median": round(float(np.median(step_ms)), 3),
                           "p90": round(float(np.percentile(step_ms, 90)), 3), "rounds": int(step_ms.size)},
        "planted": planted,
        "roofline": roofline,
        "kernels": kernels,
        "cpu_baseline": cpu,
    }
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
