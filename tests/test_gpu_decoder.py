"""End-to-end rollout parity: FlashMedusaDecoder.generate on the GPU in lockstep
with the CPU oracle.

Every verify round is replayed on the oracle from the GPU's own inputs to that
round: decisions (root draw, plan, tree tokens, accepted path and length,
finish flags, b200 forced roots) must be bit-exact given the GPU's logits;
floating-point values (hidden states, Medusa logits, tree hidden states, tree
logits) must be within 1e-5 (fp32) / 2e-2 (bf16) max relative error of an
independent float64 oracle that recomputes the accepted tokens' KV (so the
next round also checks extract == recompute).
"""
import numpy as np
import pytest
import torch

from oracle import decode as OD
from oracle import model as OM
from oracle import sampling as OS
from oracle import tree as OT

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL = {torch.float32: 1e-5, torch.bfloat16: 2e-2}


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30))


class Tok:
    def __init__(self, eos):
        self.eos_token_id = eos
        self.pad_token_id = 0


def build(ocfg, W, heads, dtype, cell=None):
    from flashgrpo_amd.models import MedusaHeads, TargetConfig, TargetModel

    tcfg = TargetConfig(ocfg.num_layers, ocfg.hidden, ocfg.q_heads, ocfg.kv_heads, ocfg.head_dim, ocfg.intermediate,
                        ocfg.vocab, ocfg.rope_theta, ocfg.rms_eps, ocfg.qkv_bias, ocfg.tie_word_embeddings)
    model = TargetModel.from_numpy(tcfg, W, dtype=dtype, device=DEV)
    untied = any(src.get("out_w") is not None for src in heads)
    mh = MedusaHeads(ocfg.hidden, ocfg.vocab, len(heads), tie_lm_head=not untied).to(DEV)
    with torch.no_grad():
        for hd, src in zip(mh.heads, heads):
            hd.fc.weight.copy_(torch.from_numpy(src["fc_w"]))
            hd.fc.bias.copy_(torch.from_numpy(src["fc_b"]))
            hd.norm.weight.copy_(torch.from_numpy(src["ln_w"]))
            hd.norm.bias.copy_(torch.from_numpy(src["ln_b"]))
            if src.get("out_w") is not None:
                hd.output.weight.copy_(torch.from_numpy(src["out_w"]))
            elif untied:
                hd.output = None  # this head stays tied to the LM head
        if cell is not None:
            cc = mh.chain_cell
            for mod_p, key in ((cc.state_norm.weight, "sn_w"), (cc.state_norm.bias, "sn_b"),
                               (cc.token_norm.weight, "tn_w"), (cc.token_norm.bias, "tn_b"),
                               (cc.state_proj.weight, "sp_w"), (cc.token_proj.weight, "tp_w"),
                               (cc.out_proj.weight, "op_w"), (cc.out_proj.bias, "op_b")):
                mod_p.copy_(torch.from_numpy(np.asarray(cell[key], np.float32)))
            cc.gate.fill_(float(cell["gate"]))
    return model, mh


def rounded(W, heads, dtype, cell=None):
    if dtype == torch.float32:
        return W, heads, cell
    r = lambda a: None if a is None else torch.from_numpy(np.asarray(a)).to(torch.bfloat16).float().numpy()
    Wr = {k: r(v) for k, v in W.items() if k not in ("layers", "inv_freq")}
    Wr["inv_freq"] = W["inv_freq"]
    Wr["layers"] = [{k: r(v) for k, v in lw.items()} for lw in W["layers"]]
    hr = [dict(h, fc_w=r(h["fc_w"]), fc_b=r(h["fc_b"]), out_w=r(h.get("out_w"))) for h in heads]
    # the chain cell (and the head that bootstraps it) run in their own fp32 parameters,
    # outside the bf16 autocast of the proposal heads
    return Wr, hr, cell


def _k_near(conf, base_k, d, spec):
    """Branching factors within 1e-6 of a confidence (device and oracle confidences
    differ by rounding; a value on a rounding edge of k may go either way)."""
    return {OT.topk_from_confidence(c, base_k, d, enabled=spec.adaptive_tree_enabled,
                                    min_topk_by_depth=spec.adaptive_min_topk_by_depth,
                                    low=spec.adaptive_confidence_low, high=spec.adaptive_confidence_high)
            for c in (conf - 1e-6, conf, conf + 1e-6)}


def check_chain(rec, spec, Wr, boot_head, cell_r, tol, Bc):
    """Chain proposals of one round from the device's own per-depth states and logits:
    bootstrap state, logits of every state, adapted k, tree tokens (exact given the
    logits) and each next state (cell on the device's parent state)."""
    ch = rec["chain"]
    roots = rec["roots"]
    if spec.chain_bootstrap_from_medusa:
        boot = OM.medusa_project(rec["hidden_in"], boot_head)
    else:
        boot = OM.chain_cell(rec["hidden_in"], Wr["embed"][roots], cell_r)
    assert rel(ch[0]["states"], boot) < tol
    base = OD.plan_for(spec, Bc).topk_by_depth
    budget = rec["chain_budget"]
    trees = [OT.Tree([int(x)], [-1], [1], [0.0]) for x in roots]
    cur = [[0] for _ in range(Bc)]
    ks = []
    for d, c in enumerate(ch):
        assert rel(c["logits"], OM.logits(c["states"], Wr["lm_head"])) < tol, d
        conf = OT.quantile_linear(OD.chain_confidence(c["logits"], spec.adaptive_confidence_metric),
                                  spec.adaptive_confidence_quantile)
        assert c["k"] in _k_near(conf, base[d], d, spec), (d, conf, c["k"])
        ks.append(c["k"])
        cur, pidx, toks = OT.chain_add_children(trees, cur, c["logits"], c["k"], d, budget)
        if not toks:
            break
        if d + 1 < len(ch):
            want = OM.chain_cell(c["states"][pidx], Wr["embed"][toks], cell_r)
            assert rel(ch[d + 1]["states"], want) < tol, d
    assert rec["tree_tokens"].tolist() == [t.tokens for t in trees]
    assert rec["plan"][:len(ks)] == ks
    # a depth reached with the budget already full reports base k (no adaptation)
    assert rec["plan"][len(ks):] == list(base[len(ks):len(rec["plan"])])
    return trees


def cast_weights(W, heads, dt):
    """Weights (and Medusa heads) converted once to the oracle's compute dtype, so the
    oracle's per-call np.asarray(w, dtype) makes no copy."""
    c = lambda a: None if a is None else np.ascontiguousarray(a, dt)
    Wc = {k: c(v) for k, v in W.items() if k not in ("layers", "inv_freq")}
    if W.get("lm_head") is W.get("embed"):
        Wc["lm_head"] = Wc["embed"]
    Wc["inv_freq"] = W["inv_freq"]
    Wc["layers"] = [{k: c(v) for k, v in lw.items()} for lw in W["layers"]]
    hc = [{k: c(v) for k, v in h.items()} for h in heads]
    return Wc, hc


class OracleRow:
    """Per-sequence oracle cache, advanced by recomputing accepted tokens (float64, or
    float32 for the bf16 checks at full-vocabulary geometries)."""

    def __init__(self, ocfg, W, prompt, dtype=np.float64, state=None):
        self.cfg, self.W, self.dt = ocfg, W, dtype
        if state is not None:  # (hidden [H], K list [1, Hkv, P, d], V list, length): a given prefix
            self.hidden, self.k, self.v, self.len = state
            return
        hid, self.k, self.v = OM.prefill(ocfg, W, np.asarray(prompt)[None], dtype=dtype)
        self.hidden = hid[0, -1]
        self.len = len(prompt)

    def append(self, toks):
        n = len(toks)
        hid, nk, nv = OM.forward(self.cfg, self.W, np.asarray(toks)[None], (self.len + np.arange(n))[None], self.k,
                                 self.v, np.ones((1, self.len), bool), np.tril(np.ones((n, n), bool))[None],
                                 dtype=self.dt)
        self.k = [np.concatenate([a, b], axis=2) for a, b in zip(self.k, nk)]
        self.v = [np.concatenate([a, b], axis=2) for a, b in zip(self.v, nv)]
        self.hidden = hid[0, -1]
        self.len += n

    def tree(self, toks, parents, depths):
        N = len(toks)
        allowed = np.zeros((1, N, N), bool)
        for n in range(N):
            a = n
            while a >= 0:
                allowed[0, n, a] = True
                a = parents[a]
        pos = self.len + np.asarray(depths) - 1
        hid, _, _ = OM.forward(self.cfg, self.W, np.asarray(toks)[None], pos[None], self.k, self.v,
                               np.ones((1, self.len), bool), allowed, dtype=self.dt)
        return hid[0]


def lockstep(trace, ocfg, Wr, heads_r, spec, prompts, dtype, seed, max_length, emit_correction=False, cell_r=None,
             odt=np.float64, rows=None, boot_head=None):
    """Replays every traced round on the oracle. ``odt`` is the oracle's compute dtype
    (float32 only for bf16 runs, whose tolerance is 2e-2); ``rows`` optionally gives
    pre-built OracleRows (a prefix taken from the device's cache); ``boot_head`` is the
    head that bootstraps chain proposals in its own parameter dtype (default: head 0 of
    ``heads_r``)."""
    tol = TOL[dtype]
    Wr, heads_r = cast_weights(Wr, heads_r, odt)
    lm = Wr["lm_head"]
    if rows is None:
        rows = {s: OracleRow(ocfg, Wr, prompts[s], odt) for s in range(prompts.shape[0])}
    else:
        for row in rows.values():
            row.W, row.dt = Wr, odt
    kw = dict(do_sample=spec.do_sample and spec.temperature != 0, temperature=spec.temperature, top_p=spec.top_p,
              top_k=spec.top_k)
    stats = dict(rounds=0, deep=0, max_acc=1)
    pending = {}
    for rec in trace:
        rnd, active = rec["round"], rec["active"]
        Bc = len(active)
        want_in = OM.logits(np.stack([rows[s].hidden for s in active]), lm, odt)
        for i, s in enumerate(active):
            assert rel(rec["hidden_in"][i], rows[s].hidden) < tol, (rnd, s)
            assert rel(rec["logits_in"][i], want_in[i]) < tol, (rnd, s)
        want_roots = [pending[s] if s in pending else
                      OS.sample_row(rec["logits_in"][i], OS.counter_noise(seed, rnd, s, 0), **kw)
                      for i, s in enumerate(active)]
        assert rec["roots"].tolist() == want_roots, rnd
        plan = OD.plan_for(spec, Bc)
        if "chain" in rec:
            trees = check_chain(rec, spec, Wr, heads_r[0] if boot_head is None else boot_head, cell_r, tol, Bc)
            stats["chain_rounds"] = stats.get("chain_rounds", 0) + 1
        else:
            if "medusa_logits" in rec:
                nh = plan.active_heads
                ml = rec["medusa_logits"].reshape(nh, Bc, -1)
                want_ml = OM.medusa_logits(rec["hidden_in"], heads_r, lm, nh, dtype=odt)
                for d in range(nh):
                    assert rel(ml[d], want_ml[d]) < tol
                if spec.adaptive_tree_enabled:
                    stats["conf"] = OD.confidences(spec, [ml[d] for d in range(min(nh, len(plan.topk_by_depth)))])
                plan = OD.adapt_plan(spec, plan, [ml[d] for d in range(nh)])
            assert rec["plan"] == list(plan.topk_by_depth), rnd
            heads_logits = []
            if "medusa_logits" in rec:
                ml = rec["medusa_logits"]
                heads_logits = list(ml.reshape(ml.shape[0] // Bc, Bc, -1))
            if plan.layout == "sparse_asymmetric" and plan.active_heads:
                # per-row trees, padded to the widest bound
                trees = OT.build_sparse_trees(rec["roots"], heads_logits, plan)
                sp = rec["sparse"]
                assert rec["sparse_plan"] == list(plan.nodes_by_head), rnd
                for i, t in enumerate(trees):
                    n = t.node_count
                    assert int(sp["n_nodes"][i]) == n, (rnd, i)
                    assert rec["tree_tokens"][i, :n].tolist() == t.tokens, (rnd, i)
                    assert sp["parents"][i, :n].tolist() == t.parents, (rnd, i)
                    assert sp["depth"][i, :n].tolist() == t.depths, (rnd, i)
                stats["sparse_shapes"] = stats.get("sparse_shapes", set()) | {tuple(t.parents) for t in trees}
            else:
                trees = OT.build_batch_trees(rec["roots"], heads_logits, plan)
                assert rec["tree_tokens"].tolist() == [t.tokens for t in trees], rnd
        N = rec["tree_tokens"].shape[1]
        if "tree_hidden" in rec:
            for i, s in enumerate(active):
                want_h = rows[s].tree(trees[i].tokens, trees[i].parents, trees[i].depths)
                assert rel(rec["tree_hidden"][i][:trees[i].node_count], want_h) < tol, (rnd, s)
            nz = [[OS.counter_noise(seed, rnd, s, 1 + t) for t in range(N)] for s in active]
        if "walk_logits" in rec:  # lazy: one projected row per walk step and sequence
            # The walk samples only at the nodes the device projected; those rows are
            # checked against the oracle and packed, every other node maps to a trailing
            # zero row (a walk that left the device's path would read it and mismatch).
            visited = [(i, t, int(rec["acc_nodes"][i, t])) for i in range(Bc)
                       for t in range(int(rec["walk_last"][i]) + 1)]
            if visited:
                want_rows = OM.logits(np.stack([rec["tree_hidden"][i, n] for i, _, n in visited]), lm, odt)
            packed = np.zeros((len(visited) + 1, rec["walk_logits"].shape[-1]), np.float64)
            slots = [[-1] * N for _ in range(Bc)]
            for j, (i, t, node) in enumerate(visited):
                assert rel(rec["walk_logits"][t, i], want_rows[j]) < tol, (rnd, i, t)
                packed[j] = rec["walk_logits"][t, i]
                slots[i][node] = j
            at, an, last, corr = OS.accept_walk(trees, packed, nz, slots=slots, emit_correction=True, **kw)
            for i in range(Bc):  # draws made: one per step until a mismatch or a leaf
                assert int(rec["walk_last"][i]) + 1 == len(at[i]) - (corr[i] is None), (rnd, i)
                assert rec["acc_nodes"][i, :len(an[i])].tolist() == an[i], (rnd, i)
        elif "tree_logits" in rec:
            if rec["slot_map"] is not None:  # packed internal-node rows
                r_, n_, slots = OT.internal_slots(trees)
                want_tl = OM.logits(rec["tree_hidden"][r_, n_], lm, odt)
                assert rec["slot_map"].tolist() == slots
                walk_logits = rec["tree_logits"]
            else:  # every node projected, dense [B, N, V]
                slots = None
                want_tl = OM.logits(rec["tree_hidden"].reshape(Bc * N, -1), lm, odt)
                walk_logits = rec["tree_logits"].reshape(Bc, N, -1)
            assert rel(rec["tree_logits"], want_tl) < tol
            at, an, last, corr = OS.accept_walk(trees, walk_logits, nz, slots=slots, emit_correction=True, **kw)
        else:
            at, an, last, corr = [[int(r)] for r in rec["roots"]], [[0]] * Bc, [0] * Bc, [None] * Bc
        pending = {}
        for i, s in enumerate(active):
            raw = len(at[i])
            t, n, fin, _ = OS.clamp_accepted(at[i], an[i], remaining=max_length - rows[s].len,
                                             eos_token_id=spec.eos_token_id, old_len=rows[s].len,
                                             max_length=max_length)
            L = int(rec["acc_len"][i])
            assert rec["acc_tokens"][i, :L].tolist() == t, (rnd, s)
            assert bool(rec["finished"][i]) == fin
            assert int(rec["last_node"][i]) == n[-1]
            stats["max_acc"] = max(stats["max_acc"], L)
            if emit_correction and corr[i] is not None and len(t) == raw and not fin:
                pending[s] = corr[i]
            rows[s].append(t)
        if emit_correction:
            assert sorted(pending.items()) == sorted((s, int(p)) for s, p in zip(active, rec["pending"]) if p >= 0)
        stats["rounds"] += 1
    return stats


def _run(ocfg, spec, *, dtype, B0, repeats, P, max_length, seed=123, wseed=0, cache_mode="extract_path",
         internal_only=True, lazy=True, untied=(), std=0.05, odt=np.float64, head_autocast=True):
    from flashgrpo_amd.decoding import FlashMedusaConfig, FlashMedusaDecoder

    W = OM.random_weights(ocfg, seed=wseed, std=std)
    heads = OM.random_medusa(ocfg.hidden, spec.num_medusa_heads, seed=wseed + 1, std=std)
    orng = np.random.default_rng(wseed + 3)
    for i in untied:  # these heads get their own output projection
        heads[i]["out_w"] = (orng.standard_normal((ocfg.vocab, ocfg.hidden)) * 0.05).astype(np.float32)
    cell = OM.random_chain_cell(ocfg.hidden, seed=wseed + 2, std=0.05, gate_init=-1.0) \
        if spec.proposal_mode == "chain" else None
    model, mh = build(ocfg, W, heads, dtype, cell)
    cfg = FlashMedusaConfig(num_medusa_heads=spec.num_medusa_heads, tree_mode=spec.tree_mode,
                            cpeak_nodes=spec.cpeak_nodes, max_tree_nodes_per_seq=spec.max_tree_nodes_per_seq,
                            max_tree_depth=spec.max_tree_depth, fixed_tree_topk_by_depth=spec.fixed_tree_topk_by_depth,
                            adaptive_tree_enabled=spec.adaptive_tree_enabled, do_sample=spec.do_sample,
                            temperature=spec.temperature, top_p=spec.top_p, top_k=spec.top_k,
                            emit_correction_token=spec.emit_correction_token, noise_seed=seed,
                            cache_update_mode=cache_mode, project_internal_tree_logits_only=internal_only,
                            lazy_walk_lm_head=lazy, proposal_mode=spec.proposal_mode,
                            chain_bootstrap_from_medusa=spec.chain_bootstrap_from_medusa,
                            adaptive_confidence_metric=spec.adaptive_confidence_metric,
                            adaptive_confidence_quantile=spec.adaptive_confidence_quantile,
                            adaptive_confidence_low=spec.adaptive_confidence_low,
                            adaptive_confidence_high=spec.adaptive_confidence_high,
                            adaptive_min_topk_by_depth=spec.adaptive_min_topk_by_depth,
                            tree_layout=spec.tree_layout, sparse_nodes_by_head=spec.sparse_nodes_by_head,
                            sparse_min_head3_nodes=spec.sparse_min_head3_nodes,
                            sparse_head3_min_budget=spec.sparse_head3_min_budget,
                            sparse_branch_score_temperature=spec.sparse_branch_score_temperature,
                            sparse_diversity_penalty=spec.sparse_diversity_penalty,
                            head_inference_autocast=head_autocast)
    dec = FlashMedusaDecoder(model, mh, Tok(spec.eos_token_id), cfg)
    rng = np.random.default_rng(wseed + 7)
    prompts = rng.integers(0, ocfg.vocab, (B0, P))
    trace = []
    out = dec.generate(torch.from_numpy(prompts), torch.ones(B0, P, dtype=torch.long), repeated_generate_nums=repeats,
                       max_length=max_length, trace=trace)
    Wr, hr, cr = rounded(W, heads, dtype, cell)
    if not head_autocast:
        hr = heads  # the proposal heads run in their own fp32 parameters
    seed_eff = trace[0]["seed"]
    stats = lockstep(trace, ocfg, Wr, hr, spec, np.repeat(prompts, repeats, axis=0), dtype, seed_eff, max_length,
                     emit_correction=spec.emit_correction_token, cell_r=cr, odt=odt, boot_head=heads[0])
    for s, g in enumerate(out["generated_token_ids"]):
        assert len(g) >= 1
    return out, stats


SMALL = OM.ModelConfig(num_layers=2, hidden=256, q_heads=4, kv_heads=2, head_dim=64, intermediate=512, vocab=64)
SMALL16 = OM.ModelConfig(num_layers=2, hidden=256, q_heads=4, kv_heads=2, head_dim=128, intermediate=512, vocab=64)


@pytest.mark.parametrize("top_p,lazy", [(1.0, True), (0.9, True), (0.9, False)])
def test_lockstep_fp32_fixed_tree_small_vocab(top_p, lazy):
    spec = OD.DecodeSpec(tree_mode="fixed", max_tree_nodes_per_seq=16, fixed_tree_topk_by_depth=(4, 2, 1),
                         num_medusa_heads=3, max_tree_depth=4, top_p=top_p)
    out, st = _run(SMALL, spec, dtype=torch.float32, B0=3, repeats=2, P=33, max_length=33 + 24, lazy=lazy)
    assert st["max_acc"] >= 2  # a 64-token vocabulary accepts children: the gather moves real paths
    assert out["kv_extraction_success_count"] == st["rounds"]


def test_lockstep_bf16_concurrency_tree():
    spec = OD.DecodeSpec(tree_mode="concurrency_aware", cpeak_nodes=48, max_tree_nodes_per_seq=16,
                         fixed_tree_topk_by_depth=(4, 3, 2), num_medusa_heads=3, max_tree_depth=4, top_p=0.95,
                         eos_token_id=5)
    _run(SMALL16, spec, dtype=torch.bfloat16, B0=2, repeats=2, P=70, max_length=70 + 20)


def test_lockstep_adaptive_margin_confidence():
    """Adaptive plan from the top-1 minus top-2 margin of each head
    (flash_medusa_decoder.py:326-331), including a plan whose base branching is 1."""
    for ks, low, high in [((3, 2, 2), 0.05, 0.6), ((1, 1, 1), 0.0, 0.1)]:
        spec = OD.DecodeSpec(tree_mode="concurrency_aware", cpeak_nodes=64, max_tree_nodes_per_seq=16,
                             fixed_tree_topk_by_depth=ks, num_medusa_heads=3, max_tree_depth=4,
                             adaptive_tree_enabled=True, adaptive_confidence_metric="margin",
                             adaptive_confidence_low=low, adaptive_confidence_high=high, top_p=1.0)
        out, st = _run(SMALL, spec, dtype=torch.float32, B0=2, repeats=2, P=20, max_length=20 + 16)
        assert st["rounds"] > 0
        conf = out["last_tree_plan"]["adaptive_tree"]["confidence"]
        assert np.allclose(conf, st["conf"], rtol=1e-6, atol=1e-7), (ks, conf, st["conf"])
        assert all(c > 0 for c in conf)  # a real margin, not a top-1 value or 0


def test_lockstep_adaptive_b200_greedy_and_recompute():
    spec = OD.DecodeSpec(tree_mode="concurrency_aware", cpeak_nodes=64, max_tree_nodes_per_seq=32,
                         fixed_tree_topk_by_depth=(4, 3, 2), num_medusa_heads=4, max_tree_depth=5,
                         adaptive_tree_enabled=True, top_p=1.0, emit_correction_token=True)
    out, st = _run(SMALL, spec, dtype=torch.float32, B0=2, repeats=1, P=20, max_length=20 + 16)
    assert out["total_correction_tokens"] >= 0
    spec_g = OD.DecodeSpec(tree_mode="fixed", max_tree_nodes_per_seq=12, fixed_tree_topk_by_depth=(3, 2),
                           num_medusa_heads=2, do_sample=False)
    _run(SMALL, spec_g, dtype=torch.float32, B0=2, repeats=2, P=17, max_length=17 + 12, cache_mode="recompute_accepted")
    _run(SMALL, spec_g, dtype=torch.float32, B0=2, repeats=2, P=17, max_length=17 + 12, internal_only=False,
         lazy=False)
    _run(SMALL, spec, dtype=torch.float32, B0=2, repeats=1, P=20, max_length=20 + 16, lazy=False)


def test_tiny_config_32_rounds_fp32():
    """4 layers, H512, 8/2 heads, d64, F1408, V32000, fixed [4,3,2] in 16 nodes,
    8 sequences (4 prompts x 2 repeats), 256-token prefix, T=1, 32 verify rounds."""
    cfg = OM.ModelConfig(num_layers=4, hidden=512, q_heads=8, kv_heads=2, head_dim=64, intermediate=1408,
                         vocab=32000, rope_theta=1e6, tie_word_embeddings=True)
    spec = OD.DecodeSpec(tree_mode="fixed", max_tree_nodes_per_seq=16, fixed_tree_topk_by_depth=(4, 3, 2),
                         num_medusa_heads=3, max_tree_depth=4, top_p=1.0)
    out, st = _run(cfg, spec, dtype=torch.float32, B0=4, repeats=2, P=256, max_length=256 + 32)
    # one token per round unless a rare Medusa candidate is accepted
    assert 28 <= st["rounds"] == out["total_verify_rounds"] <= 32
    assert out["last_tree_plan"]["topk_by_depth"] == [4, 2]


def test_lockstep_bf16_7b_geometry():
    """The 7B config's attention and vocabulary geometry (28/4 heads of 128, GQA 7,
    vocab 152064, 4 Medusa heads, adaptive concurrency-aware plan with a 32-node
    budget -> 29-node tree) on a 2-layer, 512-wide stack: 4 sequences in lockstep
    with the oracle, bf16."""
    cfg = OM.ModelConfig(num_layers=2, hidden=512, q_heads=28, kv_heads=4, head_dim=128, intermediate=1024,
                         vocab=152064, rope_theta=1e6)
    spec = OD.DecodeSpec(tree_mode="concurrency_aware", cpeak_nodes=128, max_tree_nodes_per_seq=32,
                         fixed_tree_topk_by_depth=(4, 3, 2), num_medusa_heads=4, max_tree_depth=5,
                         adaptive_tree_enabled=True, top_p=1.0)
    out, st = _run(cfg, spec, dtype=torch.bfloat16, B0=2, repeats=2, P=40, max_length=40 + 6)
    assert st["rounds"] == out["total_verify_rounds"] >= 3
    assert out["last_tree_plan"]["node_budget_per_seq"] == 32


@pytest.mark.parametrize("dtype,boot,metric", [(torch.float32, True, "top1_prob"), (torch.float32, False, "margin"),
                                               (torch.bfloat16, True, "top1_prob")])
def test_lockstep_chain_proposals(dtype, boot, metric):
    """proposal_mode="chain": per-depth LM head over every parent state, sanitised
    top-k, adapted k, dense-BFS children under the budget, ChainDraftCell steps."""
    spec = OD.DecodeSpec(tree_mode="concurrency_aware", cpeak_nodes=64, max_tree_nodes_per_seq=16,
                         fixed_tree_topk_by_depth=(4, 3, 2), num_medusa_heads=3, max_tree_depth=4, top_p=1.0,
                         proposal_mode="chain", chain_bootstrap_from_medusa=boot, adaptive_tree_enabled=True,
                         adaptive_confidence_metric=metric,
                         adaptive_confidence_low=0.005 if metric == "top1_prob" else 0.01,
                         adaptive_confidence_high=0.05 if metric == "top1_prob" else 0.3)
    cfg = SMALL if dtype == torch.float32 else SMALL16
    out, st = _run(cfg, spec, dtype=dtype, B0=2, repeats=2, P=24, max_length=24 + 16)
    assert st["chain_rounds"] == st["rounds"] == out["total_verify_rounds"]
    assert out["last_tree_plan"]["proposal_mode"] == "chain"


def test_lockstep_chain_fixed_tree():
    """Non-adaptive chain proposals on a fixed plan ([4, 1] in 12 nodes), top-p 0.9.
    (The adaptive cases above cut their trees inside a depth: a [4, 3, 2] plan in 16
    nodes.)"""
    spec = OD.DecodeSpec(tree_mode="fixed", max_tree_nodes_per_seq=12, fixed_tree_topk_by_depth=(4, 2, 1),
                         num_medusa_heads=3, max_tree_depth=4, top_p=0.9, proposal_mode="chain")
    out, st = _run(SMALL, spec, dtype=torch.float32, B0=2, repeats=2, P=20, max_length=20 + 16)
    assert st["chain_rounds"] == st["rounds"]


def test_lockstep_bf16_8b_chain_geometry():
    """The 8B chain config's geometry (32/8 heads of 128, vocab 128256, theta 5e5, no
    QKV bias, 4 heads, chain proposals, adaptive concurrency-aware plan with a 48-node
    budget) on a 2-layer, 512-wide stack: 4 sequences in lockstep, bf16."""
    cfg = OM.ModelConfig(num_layers=2, hidden=512, q_heads=32, kv_heads=8, head_dim=128, intermediate=1024,
                         vocab=128256, rope_theta=5e5, qkv_bias=False)
    spec = OD.DecodeSpec(tree_mode="concurrency_aware", cpeak_nodes=192, max_tree_nodes_per_seq=48,
                         fixed_tree_topk_by_depth=(4, 3, 2), num_medusa_heads=4, max_tree_depth=5,
                         adaptive_tree_enabled=True, adaptive_confidence_low=0.2, adaptive_confidence_high=0.7,
                         temperature=0.7, top_p=1.0, proposal_mode="chain")
    out, st = _run(cfg, spec, dtype=torch.bfloat16, B0=2, repeats=2, P=40, max_length=40 + 6)
    assert st["chain_rounds"] == st["rounds"] >= 3
    assert out["last_tree_plan"]["node_budget_per_seq"] == 48


@pytest.mark.parametrize("dtype,lazy,b200", [(torch.float32, True, False), (torch.float32, False, True),
                                             (torch.bfloat16, True, False)])
def test_lockstep_sparse_asymmetric_tree(dtype, lazy, b200):
    """b200 sparse_asymmetric trees (per-row parents, rows padded to the widest bound):
    trees, verify hidden states, walk, extraction and next state against the oracle."""
    spec = OD.DecodeSpec(tree_mode="fixed", max_tree_nodes_per_seq=14, fixed_tree_topk_by_depth=(4, 3, 2),
                         num_medusa_heads=3, max_tree_depth=4, top_p=0.95, tree_layout="sparse_asymmetric",
                         sparse_nodes_by_head=(3, 4, 3), sparse_min_head3_nodes=1, sparse_diversity_penalty=0.3,
                         sparse_branch_score_temperature=0.8, emit_correction_token=b200)
    cfg = SMALL16 if dtype == torch.bfloat16 else SMALL  # the bf16 attention takes head_dim 128
    out, st = _run(cfg, spec, dtype=dtype, B0=3, repeats=2, P=33, max_length=33 + 24, lazy=lazy)
    assert st["max_acc"] >= 2
    assert len(st["sparse_shapes"]) > 1  # rows really differ in topology
    assert out["kv_extraction_success_count"] == st["rounds"]
    assert out["last_tree_plan"]["topk_by_depth"] == [3, 4, 3]


def test_lockstep_sparse_adaptive_concurrency():
    """Adaptive sparse plan: the confidence-fitted list becomes the per-head node counts
    (flashgrpo_b200/decoding/flash_medusa_decoder.py:1063-1095)."""
    spec = OD.DecodeSpec(tree_mode="concurrency_aware", cpeak_nodes=96, max_tree_nodes_per_seq=20,
                         fixed_tree_topk_by_depth=(4, 3, 2), num_medusa_heads=3, max_tree_depth=4, top_p=1.0,
                         tree_layout="sparse_asymmetric", sparse_nodes_by_head=(5, 4, 2), sparse_min_head3_nodes=1,
                         adaptive_tree_enabled=True, adaptive_confidence_low=0.05, adaptive_confidence_high=0.2)
    out, st = _run(SMALL, spec, dtype=torch.float32, B0=2, repeats=3, P=20, max_length=20 + 24)
    assert st["rounds"] > 0 and out["kv_extraction_success_count"] == st["rounds"]


def test_graph_replayed_rollouts_equal_eager_rollouts():
    """Two rollouts in a row on one decoder (graphs captured, replayed, dropped with the
    first rollout's cache, captured again for the second) emit exactly the tokens of
    the same rollouts with the eager forward; rows finish at different rounds."""
    from flashgrpo_amd.decoding import FlashMedusaConfig, FlashMedusaDecoder

    W = OM.random_weights(SMALL16, seed=3, std=0.05)
    heads = OM.random_medusa(SMALL16.hidden, 3, seed=4, std=0.05)
    model, mh = build(SMALL16, W, heads, torch.bfloat16)
    rng = np.random.default_rng(9)
    outs = {}
    for graphs in (True, False):
        cfg = FlashMedusaConfig(num_medusa_heads=3, tree_mode="concurrency_aware", cpeak_nodes=48,
                                max_tree_nodes_per_seq=16, fixed_tree_topk_by_depth=(4, 2, 1), top_p=0.9,
                                noise_seed=11, graph_verify_forward=graphs)
        dec = FlashMedusaDecoder(model, mh, Tok(7), cfg)
        res = []
        for P, B, L in ((24, 3, 40), (31, 2, 50)):
            prompts = np.random.default_rng(P).integers(0, SMALL16.vocab, (B, P))
            out = dec.generate(torch.from_numpy(prompts), torch.ones(B, P, dtype=torch.long),
                               repeated_generate_nums=2, max_length=L)
            res.append(out["generated_token_ids"])
        outs[graphs] = res
        assert not model._graphs  # dropped with each rollout
    assert outs[True] == outs[False]
    lens = [len(g) for g in outs[True][0]]
    assert len(set(lens)) > 1 or 7 in sum(outs[True][0], [])  # rows finish apart (EOS) or at max_length


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_lockstep_untied_medusa_heads(dtype):
    """Heads 0 and 2 untied (their own output projection), head 1 tied: every head's
    proposals, trees and the rollout against the oracle (medusa_heads.py:266-276,
    flash_medusa_decoder.py:297-304)."""
    spec = OD.DecodeSpec(tree_mode="fixed", max_tree_nodes_per_seq=16, fixed_tree_topk_by_depth=(4, 2, 1),
                         num_medusa_heads=3, max_tree_depth=4, top_p=1.0)
    cfg = SMALL if dtype == torch.float32 else SMALL16
    out, st = _run(cfg, spec, dtype=dtype, B0=2, repeats=2, P=25, max_length=25 + 12, untied=(0, 2))
    assert st["rounds"] == out["total_verify_rounds"] > 0


def test_lockstep_heads_without_autocast():
    """head_inference_autocast=False: the fp32 heads' residual blocks and head 1's own output
    projection in fp32, the tied heads' rows cast to bf16 for the LM head
    (flash_medusa_decoder.py:268-272 with autocast off, medusa_heads.py:266-276); checked
    against the oracle on the unrounded head weights."""
    spec = OD.DecodeSpec(tree_mode="fixed", max_tree_nodes_per_seq=16, fixed_tree_topk_by_depth=(4, 2, 1),
                         num_medusa_heads=3, max_tree_depth=4, top_p=1.0)
    out, st = _run(SMALL16, spec, dtype=torch.bfloat16, B0=2, repeats=2, P=25, max_length=25 + 12, untied=(1,),
                   head_autocast=False)
    assert st["rounds"] == out["total_verify_rounds"] > 0


def _hf_oracle_weights(hf):
    """The oracle's weight dict (float32 numpy) of a transformers Qwen2 model."""
    f = lambda t: t.detach().float().cpu().numpy().copy()
    body = hf.model
    W = {"embed": f(body.embed_tokens.weight), "final_norm": f(body.norm.weight), "lm_head": f(hf.lm_head.weight),
         "inv_freq": f(body.rotary_emb.inv_freq), "layers": []}
    for layer in body.layers:
        at, mlp = layer.self_attn, layer.mlp
        W["layers"].append({
            "input_norm": f(layer.input_layernorm.weight), "post_norm": f(layer.post_attention_layernorm.weight),
            "q_w": f(at.q_proj.weight), "k_w": f(at.k_proj.weight), "v_w": f(at.v_proj.weight),
            "q_b": f(at.q_proj.bias), "k_b": f(at.k_proj.bias), "v_b": f(at.v_proj.bias), "o_w": f(at.o_proj.weight),
            "gate_w": f(mlp.gate_proj.weight), "up_w": f(mlp.up_proj.weight), "down_w": f(mlp.down_proj.weight)})
    return W


def test_hf_target_resynced_between_rollouts():
    """The reference trainer hands the decoder its live (Hugging Face) policy once and
    steps the optimizer between rollouts (flashgrpo_trainer.py:835,1294). Two rollouts of
    one decoder over a transformers Qwen2 model whose weights are edited in place in
    between: each rollout matches the oracle built from the weights at that moment."""
    transformers = pytest.importorskip("transformers")
    from flashgrpo_amd.decoding import FlashMedusaConfig, FlashMedusaDecoder
    from flashgrpo_amd.models import MedusaHeads

    hc = transformers.Qwen2Config(vocab_size=64, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                                  num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=512,
                                  rope_theta=1.0e6, rms_norm_eps=1e-6, tie_word_embeddings=False)
    torch.manual_seed(0)
    hf = transformers.Qwen2ForCausalLM(hc).to(DEV).float().eval()
    with torch.no_grad():
        for p in hf.parameters():
            p.normal_(0.0, 0.05) if p.dim() > 1 else p.add_(torch.randn_like(p) * 0.05)
    ocfg = OM.ModelConfig(num_layers=2, hidden=256, q_heads=4, kv_heads=2, head_dim=64, intermediate=512, vocab=64,
                          rope_theta=1.0e6, rms_eps=1e-6)
    heads = OM.random_medusa(256, 3, seed=5, std=0.05)
    mh = MedusaHeads(256, 64, 3).to(DEV)
    with torch.no_grad():
        for hd, src in zip(mh.heads, heads):
            hd.fc.weight.copy_(torch.from_numpy(src["fc_w"]))
            hd.fc.bias.copy_(torch.from_numpy(src["fc_b"]))
    spec = OD.DecodeSpec(tree_mode="fixed", max_tree_nodes_per_seq=16, fixed_tree_topk_by_depth=(4, 2, 1),
                         num_medusa_heads=3, max_tree_depth=4, top_p=1.0)
    cfg = FlashMedusaConfig(num_medusa_heads=3, tree_mode="fixed", max_tree_nodes_per_seq=16,
                            fixed_tree_topk_by_depth=(4, 2, 1), max_tree_depth=4, top_p=1.0, noise_seed=3)
    dec = FlashMedusaDecoder(hf, mh, Tok(-1), cfg)
    prompts = np.random.default_rng(1).integers(0, 64, (2, 21))
    outs = []
    for rollout in range(2):
        if rollout == 1:
            with torch.no_grad():  # an optimizer-like in-place step on some parameters
                hf.model.layers[0].self_attn.q_proj.weight.mul_(1.7)
                hf.model.layers[1].mlp.up_proj.weight.add_(torch.randn_like(hf.model.layers[1].mlp.up_proj.weight)
                                                           * 0.05)
                hf.lm_head.weight.mul_(-1.0)
        trace = []
        out = dec.generate(torch.from_numpy(prompts), torch.ones(2, 21, dtype=torch.long), repeated_generate_nums=2,
                           max_length=21 + 10, generation_step=rollout, trace=trace)
        W = _hf_oracle_weights(hf)
        st = lockstep(trace, ocfg, W, heads, spec, np.repeat(prompts, 2, axis=0), torch.float32, trace[0]["seed"],
                      21 + 10)
        assert st["rounds"] == out["total_verify_rounds"] > 0
        outs.append(out["generated_token_ids"])
    assert outs[0] != outs[1]  # the second rollout really sampled the new policy


@pytest.mark.parametrize("mode", ["adaptive", "b200_sparse", "chain"])
def test_pipelined_rounds_equal_sequential_rounds(mode):
    """step() queues the next round (proposals, verify, walk, extraction) before the
    completed round's bookkeeping and reads the next round's adaptive-plan statistics
    back with the current round's results. The rollout emits exactly the tokens and
    metrics of the same rollout run one round at a time (statistical_time) and of the
    traced run, with rows finishing at different rounds (EOS and max_length)."""
    from flashgrpo_amd.decoding import FlashMedusaConfig, FlashMedusaDecoder

    W = OM.random_weights(SMALL16, seed=5, std=0.05)
    heads = OM.random_medusa(SMALL16.hidden, 4, seed=6, std=0.05)
    cell = OM.random_chain_cell(SMALL16.hidden, seed=7, std=0.05, gate_init=-1.0) if mode == "chain" else None
    model, mh = build(SMALL16, W, heads, torch.bfloat16, cell)
    kw = dict(num_medusa_heads=4, tree_mode="concurrency_aware", cpeak_nodes=64, max_tree_nodes_per_seq=24,
              adaptive_tree_enabled=True, adaptive_min_topk_by_depth=(1, 1, 1), adaptive_confidence_low=0.02,
              adaptive_confidence_high=0.1, top_p=0.95, noise_seed=21)
    if mode == "b200_sparse":
        kw.update(tree_layout="sparse_asymmetric", emit_correction_token=True)
    if mode == "chain":
        kw.update(proposal_mode="chain", adaptive_tree_enabled=False)
    prompts = np.random.default_rng(4).integers(0, SMALL16.vocab, (3, 19))
    outs = []
    for how in ("pipelined", "statistical", "traced"):
        dec = FlashMedusaDecoder(model, mh, Tok(5), FlashMedusaConfig(**kw))
        out = dec.generate(torch.from_numpy(prompts), torch.ones(3, 19, dtype=torch.long), repeated_generate_nums=3,
                           max_length=19 + 30, statistical_time=how == "statistical",
                           trace=[] if how == "traced" else None)
        outs.append(out)
    keys = ("total_verify_rounds", "total_accepted_draft_tokens", "total_proposed_draft_tokens",
            "average_active_batch_size", "average_tree_nodes_per_seq", "tree_lm_head_rows", "accept_length_histogram",
            "medusa_proposed_by_depth", "last_tree_plan")
    for o in outs[1:]:
        assert o["generated_token_ids"] == outs[0]["generated_token_ids"]
        for k in keys:
            assert o[k] == outs[0][k], k
    lens = [len(g) for g in outs[0]["generated_token_ids"]]
    assert len(set(lens)) > 1  # rows finished at different rounds
