"""Parity at the geometries of every BASELINE configuration (the tiny config, the 7B and
8B attention/vocabulary geometries and the sparse layouts are covered in
test_gpu_decoder.py):

* Qwen2.5-1.5B geometry (hidden 1536, 12/2 heads of 128, MLP 8960, vocabulary 151936,
  tied embeddings, 3 Medusa heads, concurrency-aware plan with a 16-node budget ->
  [4, 2], 13 nodes) in lockstep with the oracle;
* Qwen2.5-14B geometry (hidden 5120, 40/8 heads of 128, MLP 13824, vocabulary 152064,
  4 Medusa heads, 64-node budget -> [4, 3, 2], 41 nodes) in lockstep with the oracle;
* Llama-3.1-8B geometry (hidden 4096, 32/8 heads of 128, MLP 14336, vocabulary 128256,
  theta 5e5, RMS eps 1e-5, no QKV bias, untied LM head, chain proposals from Medusa head 1
  and a 4096-wide ChainDraftCell, 48-node budget, temperature 0.7) in lockstep with the oracle;
* one full-size Qwen2.5-7B verify round: 64 sequences (8 prompts x 8 repeats), a
  2048-token prefix, hidden 3584, 28/4 heads of 128, MLP 18944, vocabulary 152064, 4
  Medusa heads, adaptive plan with a 32-node budget (-> [4, 2, 1, 1], 29 nodes), checked
  from the device's post-prefill cache (prefill itself checked on one prompt);
* the accepted-path KV gather at the full 7B and 14B cache shapes with planted
  full-depth paths, bit-exact.

The decoder stacks have one or two layers (the oracle runs on the host); every other
dimension is the configuration's. The oracle computes in float32 for these bf16 runs
(tolerance 2e-2); decisions are compared bit for bit given the device's logits.
"""
import numpy as np
import pytest
import torch

from oracle import decode as OD
from oracle import kv as OK
from oracle import model as OM

from test_gpu_decoder import OracleRow, Tok, _run, lockstep, rel

pytestmark = pytest.mark.gpu
DEV = "cuda"
F32 = np.float32


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def test_lockstep_1p5b_geometry():
    """1.5B geometry, 8 sequences (4 prompts x 2 repeats): cpeak 128 gives the config's
    16-node budget (cpeak 512 at 32 sequences) and the [4, 2] tree."""
    cfg = OM.ModelConfig(num_layers=1, hidden=1536, q_heads=12, kv_heads=2, head_dim=128, intermediate=8960,
                         vocab=151936, rope_theta=1e6, tie_word_embeddings=True)
    spec = OD.DecodeSpec(tree_mode="concurrency_aware", cpeak_nodes=128, max_tree_nodes_per_seq=16,
                         fixed_tree_topk_by_depth=(4, 3, 2), num_medusa_heads=3, max_tree_depth=4, top_p=1.0)
    out, st = _run(cfg, spec, dtype=torch.bfloat16, B0=4, repeats=2, P=48, max_length=48 + 4, std=0.02, odt=F32)
    assert st["rounds"] == out["total_verify_rounds"] >= 3
    plan = out["last_tree_plan"]
    assert plan["node_budget_per_seq"] == 16 and plan["topk_by_depth"] == [4, 2] and plan["actual_nodes"] == 13


def test_lockstep_14b_geometry():
    """14B geometry, 4 sequences (2 prompts x 2 repeats): cpeak 256 gives the config's
    64-node budget (cpeak 8192 at 128 sequences) and the [4, 3, 2] 41-node tree (the
    fourth head gets no room). Embeddings tied to halve the host-side weight setup."""
    cfg = OM.ModelConfig(num_layers=1, hidden=5120, q_heads=40, kv_heads=8, head_dim=128, intermediate=13824,
                         vocab=152064, rope_theta=1e6, tie_word_embeddings=True)
    spec = OD.DecodeSpec(tree_mode="concurrency_aware", cpeak_nodes=256, max_tree_nodes_per_seq=64,
                         fixed_tree_topk_by_depth=(4, 3, 2), num_medusa_heads=4, max_tree_depth=5, top_p=1.0)
    out, st = _run(cfg, spec, dtype=torch.bfloat16, B0=2, repeats=2, P=40, max_length=40 + 3, std=0.02, odt=F32)
    assert st["rounds"] == out["total_verify_rounds"] >= 2
    plan = out["last_tree_plan"]
    assert plan["node_budget_per_seq"] == 64 and plan["topk_by_depth"] == [4, 3, 2] and plan["actual_nodes"] == 41


def test_lockstep_8b_chain_geometry():
    """8B chain config at full width, 4 sequences (2 prompts x 2 repeats): cpeak 192 gives
    the config's 48-node budget (cpeak 4608 at 96 sequences). Every round's proposals come
    from the chain path (Medusa head 1 for depth 2, the recurrent cell after it)."""
    cfg = OM.ModelConfig(num_layers=1, hidden=4096, q_heads=32, kv_heads=8, head_dim=128, intermediate=14336,
                         vocab=128256, rope_theta=5e5, rms_eps=1e-5, qkv_bias=False, tie_word_embeddings=False)
    spec = OD.DecodeSpec(tree_mode="concurrency_aware", cpeak_nodes=192, max_tree_nodes_per_seq=48,
                         fixed_tree_topk_by_depth=(4, 3, 2), num_medusa_heads=4, max_tree_depth=5,
                         adaptive_tree_enabled=True, adaptive_confidence_low=0.2, adaptive_confidence_high=0.7,
                         temperature=0.7, top_p=1.0, proposal_mode="chain")
    out, st = _run(cfg, spec, dtype=torch.bfloat16, B0=2, repeats=2, P=64, max_length=64 + 5, std=0.02, odt=F32)
    assert st["chain_rounds"] == st["rounds"] == out["total_verify_rounds"] >= 2
    plan = out["last_tree_plan"]
    assert plan["proposal_mode"] == "chain" and plan["node_budget_per_seq"] == 48


def _oracle_weights(model, heads):
    """float32 numpy copies of a TargetModel's (bf16) weights and of the Medusa heads as
    the device runs them (in the target's dtype)."""
    cfg = model.cfg
    f = lambda t: t.detach().float().cpu().numpy()
    qd, kd = cfg.q_heads * cfg.head_dim, cfg.kv_heads * cfg.head_dim
    W = {"embed": f(model.w["embed"]), "final_norm": f(model.w["final_norm"]), "layers": [],
         "inv_freq": model.inv_freq.cpu().numpy()}
    W["lm_head"] = W["embed"] if model.w["lm_head"] is model.w["embed"] else f(model.w["lm_head"])
    for lw in model.w["layers"]:
        qkv, b, gu = f(lw["qkv_w"]), f(lw["qkv_b"]), f(lw["gate_up_w"])
        W["layers"].append({"input_norm": f(lw["input_norm"]), "q_w": qkv[:qd], "k_w": qkv[qd:qd + kd],
                            "v_w": qkv[qd + kd:], "q_b": b[:qd], "k_b": b[qd:qd + kd], "v_b": b[qd + kd:],
                            "o_w": f(lw["o_w"]), "post_norm": f(lw["post_norm"]), "gate_w": gu[:cfg.intermediate],
                            "up_w": gu[cfg.intermediate:], "down_w": f(lw["down_w"])})
    hd = [{"ln_w": f(h.norm.weight), "ln_b": f(h.norm.bias), "fc_w": f(h.fc.weight.to(model.dtype)),
           "fc_b": f(h.fc.bias.to(model.dtype))} for h in heads.heads]
    return W, hd


FULL_SIZE = {
    # name: (prefix, prompts, repeats, TargetConfig args after num_layers, Medusa heads, decoder config,
    #        expected plan, expected nodes)
    "7b": (2048, 8, 8, (3584, 28, 4, 128, 18944, 152064, 1e6, 1e-6, True, False), 4,
           dict(tree_mode="concurrency_aware", cpeak_nodes=2048, max_tree_nodes_per_seq=32, max_tree_depth=5,
                fixed_tree_topk_by_depth=(4, 3, 2), adaptive_tree_enabled=True, adaptive_min_topk_by_depth=(1, 1, 1)),
           [4, 2, 1, 1], 29),
    "14b": (4096, 16, 8, (5120, 40, 8, 128, 13824, 152064, 1e6, 1e-6, True, False), 4,
            dict(tree_mode="concurrency_aware", cpeak_nodes=8192, max_tree_nodes_per_seq=64, max_tree_depth=5,
                 fixed_tree_topk_by_depth=(4, 3, 2)),
            [4, 3, 2], 41),
    "1p5b": (512, 4, 8, (1536, 12, 2, 128, 8960, 151936, 1e6, 1e-6, True, True), 3,
             dict(tree_mode="concurrency_aware", cpeak_nodes=512, max_tree_nodes_per_seq=16, max_tree_depth=4,
                  fixed_tree_topk_by_depth=(4, 3, 2)),
             [4, 2], 13),
}


@pytest.mark.parametrize("name", ["7b", "14b", "1p5b"])
def test_full_size_round(name):
    """One verify round at a BASELINE configuration's full batch, prefix, width and
    vocabulary (one decoder layer): 7B (64 sequences = 8 prompts x 8 repeats, 2048-token
    prefix, adaptive 32-node budget -> [4, 2, 1, 1]), 14B (128 = 16 x 8, 4096-token prefix,
    64-node budget -> [4, 3, 2], three Medusa heads x 128 rows = 384 LM-head rows, 1024
    attention workgroups over 65 key tiles) and 1.5B (32 = 4 x 8, 512-token prefix, 16-node
    budget -> [4, 2]). Checked from the device's post-prefill cache (prefill itself checked
    on one prompt), in lockstep with the oracle, then the extraction bit for bit."""
    from flashgrpo_amd.decoding import FlashMedusaConfig, FlashMedusaDecoder
    from flashgrpo_amd.models import MedusaHeads, TargetConfig, TargetModel

    P, B0, R, dims, nh, dkw, want_plan, want_nodes = FULL_SIZE[name]
    H, V = dims[0], dims[5]
    print(f"full-size round {name}: B={B0 * R} P={P} H={H} V={V}", flush=True)
    tcfg = TargetConfig(1, *dims, name=f"{name}-1-layer")
    model = TargetModel.random(tcfg, seed=0, dtype=torch.bfloat16, device=DEV)
    heads = MedusaHeads.random(H, V, nh, seed=1, device=DEV)
    dcfg = FlashMedusaConfig(num_medusa_heads=nh, temperature=1.0, top_p=1.0, noise_seed=2, **dkw)
    dec = FlashMedusaDecoder(model, heads, Tok(-1), dcfg)
    prompts = np.random.default_rng(3).integers(0, V, (B0, P))
    r = dec.start(torch.from_numpy(prompts), torch.ones(B0, P, dtype=torch.long), repeated_generate_nums=R,
                  max_length=P + 64)
    B = B0 * R
    kv0 = r.cache.kv[0].float().cpu().numpy()  # [2, B, Hkv, cap, d] after prefill
    pre_gather = []
    gather = r.cache.gather_path

    def spy(*a, **k):  # the tree cache as the verify forward left it, just before extraction
        pre_gather.append(r.cache.kv.clone())
        return gather(*a, **k)

    r.cache.gather_path = spy
    trace = []
    dec.step(r, trace)
    torch.cuda.synchronize()
    rec = trace[0]
    assert len(rec["active"]) == B and rec["plan"] == want_plan and rec["tree_tokens"].shape == (B, want_nodes)
    W, hd = _oracle_weights(model, heads)
    ocfg = OM.ModelConfig(1, *dims)
    # prefill of prompt 0 (causal tokens through the chunked chain attention)
    hid, pk, pv = OM.prefill(ocfg, W, prompts[:1], dtype=F32)
    assert rel(kv0[0, 0, :, :P], pk[0][0]) < 2e-2 and rel(kv0[1, 0, :, :P], pv[0][0]) < 2e-2
    assert rel(rec["hidden_in"][0], hid[0, -1]) < 2e-2
    # GRPO repeats are exact copies of their prompt's row
    for b in range(B):
        assert np.array_equal(kv0[:, b, :, :P], kv0[:, (b // R) * R, :, :P]), b
    # the round, from the device's post-prefill cache
    rows = {s: OracleRow(ocfg, None, None, F32, state=(rec["hidden_in"][i], [kv0[0, s:s + 1, :, :P]],
                                                       [kv0[1, s:s + 1, :, :P]], P))
            for i, s in enumerate(rec["active"])}
    spec = OD.DecodeSpec(num_medusa_heads=nh, top_p=1.0, **dkw)
    st = lockstep(trace, ocfg, W, hd, spec, None, torch.bfloat16, rec["seed"], P + 64, odt=F32, rows=rows)
    assert st["rounds"] == 1
    # extraction: accepted rows moved bit-exactly, every other slot untouched
    before, after = pre_gather[0], r.cache.kv
    seq = torch.tensor(rec["seq_len"], dtype=torch.long, device=DEV)
    want = before.clone()
    for b in range(B):
        L = int(rec["acc_len"][b])
        src = seq[b] + torch.tensor(rec["acc_nodes"][b, :L], dtype=torch.long, device=DEV)
        want[:, :, b, :, seq[b]:seq[b] + L] = before[:, :, b, :, src]
    assert torch.equal(after, want)


@pytest.mark.parametrize("shape", ["7b", "14b"])
def test_kv_gather_full_cache_shape_planted_paths(shape):
    """fg_kv_path_gather at the configs' cache shape (two of the layers): full-depth
    paths of the config's tree planted in every fourth row (the worst-case bytes), random
    root-to-leaf prefixes elsewhere, bit-exact against the oracle's compaction on the
    window of slots a round can touch, and nothing outside it changed."""
    from flashgrpo_amd import kernels as K
    from flashgrpo_amd.decoding.medusa_tree import TreeTopology

    B, Hkv, P, ks, budget = (64, 4, 2048, [4, 2, 1, 1], 32) if shape == "7b" else (128, 8, 4096, [4, 3, 2], 64)
    topo = TreeTopology(ks, budget)
    N, D, d, L = topo.num_nodes, topo.max_depth, 128, 2
    cap = P + 64 + 80
    g = torch.Generator(device=DEV).manual_seed(1)
    kv = torch.randn(L, 2, B, Hkv, cap, d, generator=g, device=DEV, dtype=torch.bfloat16)
    rng = np.random.default_rng(2)
    seq = rng.integers(P - 64, P + 1, B).astype(np.int32)
    leaves = [n for n in range(N) if n not in set(topo.parents)]
    deepest = max(leaves, key=lambda x: topo.depths[x])
    nodes = np.zeros((B, D + 1), np.int32)
    lens = np.zeros(B, np.int32)
    for b in range(B):
        n = deepest if b % 4 == 0 else int(rng.choice(leaves))
        path = []
        while n >= 0:
            path.append(n)
            n = topo.parents[n]
        path = path[::-1]
        if b % 4:
            path = path[:int(rng.integers(1, len(path) + 1))]
        nodes[b, :len(path)] = path
        nodes[b, len(path):] = path[-1]
        lens[b] = len(path)
    assert (lens == D + 1).sum() >= B // 4
    lo, hi = int(seq.min()), int(seq.max()) + N
    before = kv.clone()
    win = kv[..., lo:hi, :].float().cpu().numpy()
    ptrs = torch.tensor([kv[l, j].data_ptr() for l in range(L) for j in range(2)], dtype=torch.int64, device=DEV)
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    t = kv[0, 0]
    K.kv_path_gather(ptrs, batch=B, kv_heads=Hkv, head_dim=d, elem_bytes=2, strides=(t.stride(0), t.stride(1),
                                                                                       t.stride(2)),
                     capacity=cap, seq_len=torch.from_numpy(seq).to(DEV), acc_nodes=torch.from_numpy(nodes).to(DEV),
                     acc_len=torch.from_numpy(lens).to(DEV), tree_nodes=N, err_flag=err)
    torch.cuda.synchronize()
    assert int(err.item()) == 0
    assert torch.equal(kv[..., :lo, :], before[..., :lo, :]) and torch.equal(kv[..., hi:, :], before[..., hi:, :])
    got = kv[..., lo:hi, :].float().cpu().numpy()
    for l in range(L):
        for j in range(2):
            want = OK.compact_rows(win[l, j], seq - lo, nodes, lens)
            assert np.array_equal(got[l, j], want), (l, j)
