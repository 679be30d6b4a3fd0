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
