"""Pins the oracle decoder and Medusa heads.

Pins: the installed transformers Qwen2/Llama implementation (float64, tiny
config) for prefill and cached continuation; the tree invariant of
``flashgrpo/decoding/tree_attention.py:14-19`` (node logits equal the
sequential forward of its root path); torch.nn LayerNorm/Linear/SiLU for the
Medusa residual block.
"""
import numpy as np
import pytest
import torch

from oracle import model as M
from oracle import tree as T

CFG = M.ModelConfig(num_layers=2, hidden=64, q_heads=4, kv_heads=2, head_dim=16, intermediate=96, vocab=101,
                    rope_theta=1.0e6, rms_eps=1e-6, qkv_bias=True, tie_word_embeddings=False)


def _hf_model(cfg, W, arch="qwen2"):
    transformers = pytest.importorskip("transformers")
    common = dict(vocab_size=cfg.vocab, hidden_size=cfg.hidden, intermediate_size=cfg.intermediate,
                  num_hidden_layers=cfg.num_layers, num_attention_heads=cfg.q_heads,
                  num_key_value_heads=cfg.kv_heads, rms_norm_eps=cfg.rms_eps, rope_theta=cfg.rope_theta,
                  tie_word_embeddings=cfg.tie_word_embeddings, max_position_embeddings=4096)
    if arch == "qwen2":
        hf = transformers.Qwen2ForCausalLM(transformers.Qwen2Config(**common))
    else:
        hf = transformers.LlamaForCausalLM(transformers.LlamaConfig(attention_bias=False, **common))
    hf = hf.double().eval()
    hf.config._attn_implementation = "eager"
    sd = {"model.embed_tokens.weight": W["embed"], "model.norm.weight": W["final_norm"], "lm_head.weight": W["lm_head"]}
    for i, lw in enumerate(W["layers"]):
        p = f"model.layers.{i}."
        sd.update({p + "input_layernorm.weight": lw["input_norm"], p + "post_attention_layernorm.weight": lw["post_norm"],
                   p + "self_attn.q_proj.weight": lw["q_w"], p + "self_attn.k_proj.weight": lw["k_w"],
                   p + "self_attn.v_proj.weight": lw["v_w"], p + "self_attn.o_proj.weight": lw["o_w"],
                   p + "mlp.gate_proj.weight": lw["gate_w"], p + "mlp.up_proj.weight": lw["up_w"],
                   p + "mlp.down_proj.weight": lw["down_w"]})
        if lw["q_b"] is not None:
            sd.update({p + "self_attn.q_proj.bias": lw["q_b"], p + "self_attn.k_proj.bias": lw["k_b"],
                       p + "self_attn.v_proj.bias": lw["v_b"]})
    hf.load_state_dict({k: torch.from_numpy(np.asarray(v, np.float64)) for k, v in sd.items()}, strict=True)
    hf.model.rotary_emb.inv_freq.copy_(torch.from_numpy(W["inv_freq"].astype(np.float64)))
    return hf


def _biased(W, rng):
    for lw in W["layers"]:
        for k in ("q_b", "k_b", "v_b"):
            if lw[k] is not None:
                lw[k] = (rng.standard_normal(lw[k].shape) * 0.1).astype(np.float32)
        lw["input_norm"] = (1 + 0.1 * rng.standard_normal(lw["input_norm"].shape)).astype(np.float32)
    return W


@pytest.mark.parametrize("arch", ["qwen2", "llama"])
def test_oracle_forward_matches_transformers(arch):
    cfg = CFG if arch == "qwen2" else M.ModelConfig(**{**CFG.__dict__, "qkv_bias": False, "rope_theta": 5e5})
    rng = np.random.default_rng(0)
    W = _biased(M.random_weights(cfg, seed=1, std=0.2), rng)
    hf = _hf_model(cfg, W, arch)
    B, P = 2, 9
    toks = rng.integers(0, cfg.vocab, (B, P))
    with torch.no_grad():
        out = hf.model(input_ids=torch.from_numpy(toks), use_cache=False)
    # transformers rounds the rotary angle to fp32 and takes cos/sin in fp32
    # even in a float64 model; the oracle rounds the angle the same way and
    # takes cos/sin in float64, which leaves ~1e-7 of difference.
    hid, _, _ = M.prefill(cfg, W, toks, fp32_angles=True)
    ref = out.last_hidden_state.numpy()
    assert np.max(np.abs(hid - ref)) / np.max(np.abs(ref)) < 2e-6
    with torch.no_grad():
        logits = hf(input_ids=torch.from_numpy(toks), use_cache=False).logits.numpy()
    assert np.max(np.abs(M.logits(hid, W["lm_head"]) - logits)) / np.max(np.abs(logits)) < 2e-6


def test_tree_logits_equal_sequential_path_forward():
    rng = np.random.default_rng(2)
    W = _biased(M.random_weights(CFG, seed=3, std=0.2), rng)
    B, P = 2, 7
    prompt = rng.integers(0, CFG.vocab, (B, P))
    _, pk, pv = M.prefill(CFG, W, prompt)
    parents, depths, _ = T.dense_topology([3, 2], 16)
    N = len(parents)
    toks = rng.integers(0, CFG.vocab, (B, N))
    hid, tk, tv = M.tree_verify(CFG, W, toks, [depths] * B, [parents] * B, pk, pv, np.full(B, P))
    tree = T.Tree(list(range(N)), parents, depths)
    for n in range(N):
        path = tree.ancestors_including_self(n)
        full = np.concatenate([prompt, toks[:, path]], axis=1)
        seq_hid, _, _ = M.prefill(CFG, W, full)
        assert np.allclose(hid[:, n], seq_hid[:, -1], rtol=0, atol=1e-11)
        # the tree K of node n equals the sequential K at its position
        assert np.allclose(tk[0][:, :, n], M.prefill(CFG, W, full)[1][0][:, :, -1], atol=1e-11)


def test_medusa_block_matches_torch_modules():
    rng = np.random.default_rng(4)
    H = 48
    heads = M.random_medusa(H, 2, seed=5, std=0.3)
    heads[1]["ln_w"] = (1 + 0.2 * rng.standard_normal(H)).astype(np.float32)
    heads[1]["ln_b"] = (0.2 * rng.standard_normal(H)).astype(np.float32)
    h = rng.standard_normal((5, H))
    for hd in heads:
        ln = torch.nn.LayerNorm(H, eps=1e-5).double()
        fc = torch.nn.Linear(H, H).double()
        with torch.no_grad():
            ln.weight.copy_(torch.from_numpy(hd["ln_w"].astype(np.float64)))
            ln.bias.copy_(torch.from_numpy(hd["ln_b"].astype(np.float64)))
            fc.weight.copy_(torch.from_numpy(hd["fc_w"].astype(np.float64)))
            fc.bias.copy_(torch.from_numpy(hd["fc_b"].astype(np.float64)))
            th = torch.from_numpy(h)
            ref = (th + torch.nn.functional.silu(fc(ln(th)))).numpy()
        assert np.allclose(M.medusa_project(h, hd), ref, rtol=0, atol=1e-12)


def test_medusa_logits_untied_heads_use_their_own_output():
    """Head 1 untied (its own nn.Linear output, medusa_heads.py:66-72,266-276), heads 0 and 2
    through the tied LM head: each head's logits equal its torch projection."""
    rng = np.random.default_rng(8)
    H, V = 32, 41
    heads = M.random_medusa(H, 3, seed=9, std=0.3)
    heads[1]["out_w"] = rng.standard_normal((V, H)).astype(np.float32)
    lm = rng.standard_normal((V, H)).astype(np.float32)
    h = rng.standard_normal((4, H))
    got = M.medusa_logits(h, heads, lm)
    for i, hd in enumerate(heads):
        out = torch.nn.Linear(H, V, bias=False).double()
        with torch.no_grad():
            out.weight.copy_(torch.from_numpy(np.asarray(hd.get("out_w", lm), np.float64)))
            want = out(torch.from_numpy(M.medusa_project(h, hd))).numpy()
        assert np.allclose(got[i], want, rtol=0, atol=1e-10), i
    # the tied heads really differ from the untied one
    assert not np.allclose(got[1], M.medusa_project(h, heads[1]) @ lm.T)


def _torch_chain_cell(cell, H):
    """The cell's published structure from torch modules (double): LayerNorm ->
    Linear for state and token, SiLU, Linear with bias, sigmoid-gated residual."""
    mods = dict(sn=torch.nn.LayerNorm(H, eps=1e-5).double(), tn=torch.nn.LayerNorm(H, eps=1e-5).double(),
                sp=torch.nn.Linear(H, cell["sp_w"].shape[0], bias=False).double(),
                tp=torch.nn.Linear(H, cell["tp_w"].shape[0], bias=False).double(),
                op=torch.nn.Linear(cell["op_w"].shape[1], H).double())
    t = lambda a: torch.from_numpy(np.asarray(a, np.float64))
    with torch.no_grad():
        mods["sn"].weight.copy_(t(cell["sn_w"])); mods["sn"].bias.copy_(t(cell["sn_b"]))
        mods["tn"].weight.copy_(t(cell["tn_w"])); mods["tn"].bias.copy_(t(cell["tn_b"]))
        mods["sp"].weight.copy_(t(cell["sp_w"])); mods["tp"].weight.copy_(t(cell["tp_w"]))
        mods["op"].weight.copy_(t(cell["op_w"])); mods["op"].bias.copy_(t(cell["op_b"]))

    def run(s, e):
        with torch.no_grad():
            mixed = mods["sp"](mods["sn"](t(s))) + mods["tp"](mods["tn"](t(e)))
            delta = mods["op"](torch.nn.functional.silu(mixed))
            return (t(s) + torch.sigmoid(torch.tensor(float(cell["gate"]), dtype=torch.float64)) * delta).numpy()
    return run


def test_chain_cell_matches_torch_modules():
    rng = np.random.default_rng(6)
    H = 40
    cell = M.random_chain_cell(H, seed=7, std=0.3, gate_init=-2.0)
    assert cell["sp_w"].shape == (64, H) and cell["op_w"].shape == (H, 64)  # bottleneck max(64, H // 8)
    assert M.random_chain_cell(1024, seed=0)["sp_w"].shape == (128, 1024)
    cell["sn_w"] = (1 + 0.2 * rng.standard_normal(H)).astype(np.float32)
    cell["tn_b"] = (0.2 * rng.standard_normal(H)).astype(np.float32)
    s, e = rng.standard_normal((5, H)), rng.standard_normal((5, H))
    assert np.allclose(M.chain_cell(s, e, cell), _torch_chain_cell(cell, H)(s, e), rtol=0, atol=1e-12)
    # the reference's zero-initialised out_proj makes the cell the identity
    zero = dict(cell, op_w=np.zeros_like(cell["op_w"]), op_b=np.zeros_like(cell["op_b"]))
    assert np.array_equal(M.chain_cell(s, e, zero), s)
    # gate 0 gives half of delta: the output is linear in sigmoid(gate)
    g0 = dict(cell, gate=np.float32(0.0))
    big = dict(cell, gate=np.float32(60.0))
    assert np.allclose(M.chain_cell(s, e, g0) - s, 0.5 * (M.chain_cell(s, e, big) - s), atol=1e-12)
