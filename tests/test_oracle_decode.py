"""Pins the oracle's verify round: extract == recompute, and the loop's bookkeeping.

extract == recompute is the reference's own integration check
(``flashgrpo/scripts/test_kv_extraction.py:29-85``): the cache after accepted-path
extraction must equal the cache of a plain causal forward over prompt + accepted
tokens, and so must the next hidden state.
"""
import numpy as np

from oracle import decode as OD
from oracle import model as OM
from oracle import sampling as OS

CFG = OM.ModelConfig(num_layers=2, hidden=64, q_heads=4, kv_heads=2, head_dim=16, intermediate=96, vocab=40)


def _setup(seed=0):
    W = OM.random_weights(CFG, seed=seed, std=0.3)
    heads = OM.random_medusa(CFG.hidden, 3, seed=seed + 1, std=0.3)
    return W, heads


def test_extract_equals_recompute_over_rounds():
    W, heads = _setup()
    rng = np.random.default_rng(1)
    prompts = rng.integers(0, CFG.vocab, (3, 6))
    spec = OD.DecodeSpec(tree_mode="fixed", max_tree_nodes_per_seq=16, fixed_tree_topk_by_depth=(4, 2, 1),
                         num_medusa_heads=3, max_tree_depth=4, top_p=1.0)
    st = OD.prefill_state(CFG, W, prompts, 64)
    hist = [list(p) for p in prompts]
    deep = 0
    for rnd in range(6):
        out = OD.verify_round(CFG, W, heads, st, spec, seed=5, rnd=rnd, max_length=60)
        for b in range(3):
            hist[b].extend(out["acc_tokens"][b])
            deep = max(deep, len(out["acc_tokens"][b]))
        for b in range(3):
            full = np.array([hist[b]])
            hid, ks, vs = OM.prefill(CFG, W, full)
            L = len(hist[b])
            assert st.seq_len[b] == L
            assert np.allclose(st.hidden[b], hid[0, -1], atol=1e-10)
            for li in range(CFG.num_layers):
                assert np.allclose(st.k[li][b, :, :L], ks[li][0], atol=1e-10)
                assert np.allclose(st.v[li][b, :, :L], vs[li][0], atol=1e-10)
    assert deep >= 2  # a 40-token vocabulary accepts children regularly


def test_generate_loop_lengths_and_eos():
    W, heads = _setup(3)
    prompts = np.random.default_rng(2).integers(0, CFG.vocab, (2, 5))
    spec = OD.DecodeSpec(tree_mode="concurrency_aware", cpeak_nodes=32, max_tree_nodes_per_seq=12, top_p=0.9,
                         eos_token_id=7)
    gen = OD.generate(CFG, W, heads, prompts, spec, max_length=20, seed=11, repeats=2)
    assert len(gen) == 4
    for g in gen:
        assert 1 <= len(g) <= 15
        if 7 in g:
            assert g.index(7) == len(g) - 1
        else:
            assert len(g) == 15
    # same seed -> same rollout; the counter noise is keyed by sequence id
    assert gen == OD.generate(CFG, W, heads, prompts, spec, max_length=20, seed=11, repeats=2)


def test_b200_correction_becomes_next_root():
    W, heads = _setup(4)
    prompts = np.random.default_rng(3).integers(0, CFG.vocab, (4, 5))
    spec = OD.DecodeSpec(tree_mode="fixed", max_tree_nodes_per_seq=8, fixed_tree_topk_by_depth=(2, 1),
                         emit_correction_token=True, top_p=1.0)
    st = OD.prefill_state(CFG, W, prompts, 64)
    seen = 0
    for rnd in range(5):
        before = st.pending.copy()
        out = OD.verify_round(CFG, W, heads, st, spec, seed=9, rnd=rnd, max_length=60)
        for b in range(4):
            if before[b] >= 0:
                assert out["roots"][b] == before[b]
                seen += 1
            c = out["correction"][b]
            assert st.pending[b] == (-1 if c is None else c)
    assert seen > 0
    assert OS.counter_noise(9, 0, 0, 0) != OS.counter_noise(9, 0, 0, 1)


def _greedy_reference(W, prompts, steps):
    """Plain autoregressive greedy decoding (first maximum) by full re-forwards."""
    out = []
    for p in prompts:
        seq = list(p)
        for _ in range(steps):
            hid, _, _ = OM.prefill(CFG, W, np.array([seq]))
            lg = OM.logits(hid[0, -1], W["lm_head"]).astype(np.float32)
            seq.append(int(np.argmax(lg)))
        out.append(seq[len(p):])
    return out


def test_greedy_speculation_equals_greedy_decoding_medusa_and_chain():
    """exact_target acceptance is lossless: with greedy draws, any proposal mode
    emits the target's own greedy continuation."""
    W, heads = _setup(5)
    cell = OM.random_chain_cell(CFG.hidden, seed=6, std=0.3, gate_init=-1.0)
    prompts = np.random.default_rng(4).integers(0, CFG.vocab, (2, 5))
    ref = _greedy_reference(W, prompts, 12)
    for mode, boot, layout in [("medusa", True, "dense"), ("chain", True, "dense"), ("chain", False, "dense"),
                               ("medusa", True, "sparse_asymmetric")]:
        spec = OD.DecodeSpec(tree_mode="fixed", max_tree_nodes_per_seq=12, fixed_tree_topk_by_depth=(3, 2, 1),
                             do_sample=False, proposal_mode=mode, chain_bootstrap_from_medusa=boot,
                             tree_layout=layout, sparse_nodes_by_head=(3, 4, 2), sparse_min_head3_nodes=1)
        gen = OD.generate(CFG, W, heads, prompts, spec, max_length=17, seed=3, cell=cell)
        assert gen == ref, (mode, layout)


def test_sparse_round_extract_equals_recompute_with_row_topologies():
    """Sparse trees differ per row (greedy parent choice, leftover head-1 nodes), so rows
    are padded to the widest tree; extraction must still equal a recompute."""
    W, heads = _setup(8)
    prompts = np.random.default_rng(9).integers(0, CFG.vocab, (4, 6))
    spec = OD.DecodeSpec(tree_mode="fixed", max_tree_nodes_per_seq=14, fixed_tree_topk_by_depth=(4, 3, 2),
                         tree_layout="sparse_asymmetric", sparse_nodes_by_head=(3, 4, 3), sparse_min_head3_nodes=1,
                         sparse_diversity_penalty=0.3, top_p=1.0)
    st = OD.prefill_state(CFG, W, prompts, 96)
    hist = [list(p) for p in prompts]
    shapes, deep = set(), 0
    for rnd in range(5):
        out = OD.verify_round(CFG, W, heads, st, spec, seed=4, rnd=rnd, max_length=90)
        assert out["plan"].nodes_by_head == [3, 4, 3]
        for t in out["trees"]:
            shapes.add(tuple(t.parents))
            assert t.node_count <= 14 and all(0 <= p < n for n, p in enumerate(t.parents) if n)
        for b in range(4):
            hist[b].extend(out["acc_tokens"][b])
            deep = max(deep, len(out["acc_tokens"][b]))
            hid, ks, vs = OM.prefill(CFG, W, np.array([hist[b]]))
            L = len(hist[b])
            assert st.seq_len[b] == L
            assert np.allclose(st.hidden[b], hid[0, -1], atol=1e-10)
            for li in range(CFG.num_layers):
                assert np.allclose(st.k[li][b, :, :L], ks[li][0], atol=1e-10)
                assert np.allclose(st.v[li][b, :, :L], vs[li][0], atol=1e-10)
    assert len(shapes) > 1 and deep >= 2


def test_chain_round_extract_equals_recompute_and_trees():
    W, heads = _setup(6)
    cell = OM.random_chain_cell(CFG.hidden, seed=7, std=0.3, gate_init=-1.0)
    prompts = np.random.default_rng(5).integers(0, CFG.vocab, (3, 6))
    spec = OD.DecodeSpec(tree_mode="fixed", max_tree_nodes_per_seq=10, fixed_tree_topk_by_depth=(3, 2, 2),
                         proposal_mode="chain", adaptive_tree_enabled=True, adaptive_confidence_low=0.05,
                         adaptive_confidence_high=0.3)
    st = OD.prefill_state(CFG, W, prompts, 64)
    hist = [list(p) for p in prompts]
    for rnd in range(4):
        h_in = st.hidden.copy()
        out = OD.verify_round(CFG, W, heads, st, spec, seed=2, rnd=rnd, max_length=60, cell=cell)
        recs = out["chain"]
        plan = out["plan"]
        assert plan.topk_by_depth == [r["k"] for r in recs][:len(plan.topk_by_depth)]
        assert np.array_equal(recs[0]["states"], OM.medusa_project(h_in, heads[0]))
        for b in range(3):
            hist[b].extend(out["acc_tokens"][b])
            full = np.array([hist[b]])
            hid, ks, _ = OM.prefill(CFG, W, full)
            assert np.allclose(st.hidden[b], hid[0, -1], atol=1e-10)
            assert np.allclose(st.k[0][b, :, :len(hist[b])], ks[0][0], atol=1e-10)
        trees = out["trees"]
        assert all(t.parents == trees[0].parents for t in trees)
        assert trees[0].node_count <= 10
