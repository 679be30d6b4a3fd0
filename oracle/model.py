"""Oracle: Medusa heads and the Qwen2/Llama-architecture tree-verify forward.

Test infrastructure only (see ``oracle/__init__.py``).

The reference runs the target through Hugging Face ``transformers==4.49.0``
(``flashgrpo/models/qwen_flashgrpo_wrapper.py:150-186``, pinned in
``requirements.txt:23``). That package's arithmetic is restated here as a
textbook float64 decoder: RMSNorm, rotary embedding with a caller-supplied fp32
``inv_freq`` table, grouped-query attention under an additive allowed-set mask,
SwiGLU MLP. ``tests/test_oracle_model.py`` pins it against the installed
transformers Qwen2 implementation on a tiny configuration.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

F64 = np.float64


@dataclass
class ModelConfig:
    num_layers: int
    hidden: int
    q_heads: int
    kv_heads: int
    head_dim: int
    intermediate: int
    vocab: int
    rope_theta: float = 1.0e6
    rms_eps: float = 1.0e-6
    qkv_bias: bool = True
    tie_word_embeddings: bool = False

    @property
    def group(self) -> int:
        return self.q_heads // self.kv_heads


def inv_freq_table(head_dim: int, theta: float) -> np.ndarray:
    """fp32 rotary inverse frequencies theta^(-2i/d), computed in float64 then rounded."""
    i = np.arange(0, head_dim, 2, dtype=np.float64)
    return (1.0 / theta ** (i / head_dim)).astype(np.float32)


def random_weights(cfg: ModelConfig, seed: int, std: float = 0.02, dtype=np.float32) -> dict:
    """Seeded N(0, std) weights in the layout the build uses; norm weights 1, biases 0."""
    rng = np.random.default_rng(seed)
    H, d, F = cfg.hidden, cfg.head_dim, cfg.intermediate

    def n(*shape):
        return (rng.standard_normal(shape, dtype=np.float32) * std).astype(dtype)

    W = {"embed": n(cfg.vocab, H), "final_norm": np.ones(H, dtype), "layers": [],
         "inv_freq": inv_freq_table(d, cfg.rope_theta)}
    for _ in range(cfg.num_layers):
        W["layers"].append({
            "input_norm": np.ones(H, dtype),
            "q_w": n(cfg.q_heads * d, H), "k_w": n(cfg.kv_heads * d, H), "v_w": n(cfg.kv_heads * d, H),
            "q_b": np.zeros(cfg.q_heads * d, dtype) if cfg.qkv_bias else None,
            "k_b": np.zeros(cfg.kv_heads * d, dtype) if cfg.qkv_bias else None,
            "v_b": np.zeros(cfg.kv_heads * d, dtype) if cfg.qkv_bias else None,
            "o_w": n(H, cfg.q_heads * d),
            "post_norm": np.ones(H, dtype),
            "gate_w": n(F, H), "up_w": n(F, H), "down_w": n(H, F),
        })
    W["lm_head"] = W["embed"] if cfg.tie_word_embeddings else n(cfg.vocab, H)
    return W


def random_medusa(hidden: int, num_heads: int, seed: int, std: float = 0.02, dtype=np.float32) -> list:
    """Medusa head weights. fc ~ N(0, std) (the reference zero-initialises fc,
    ``flashgrpo/models/medusa_heads.py:64-65``, which would make every head emit
    the same logits); LayerNorm weight 1 and bias 0."""
    rng = np.random.default_rng(seed)
    heads = []
    for _ in range(num_heads):
        heads.append({
            "ln_w": np.ones(hidden, np.float32), "ln_b": np.zeros(hidden, np.float32),
            "fc_w": (rng.standard_normal((hidden, hidden), dtype=np.float32) * std).astype(dtype),
            "fc_b": (rng.standard_normal(hidden, dtype=np.float32) * std).astype(dtype),
        })
    return heads


# --------------------------------------------------------------------------- pieces
def rmsnorm(x, w, eps):
    x = np.asarray(x, F64)
    return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps) * np.asarray(w, F64)


def layernorm(x, w, b, eps=1e-5):
    x = np.asarray(x, F64)
    mu = x.mean(axis=-1, keepdims=True)
    var = ((x - mu) ** 2).mean(axis=-1, keepdims=True)
    return (x - mu) / np.sqrt(var + eps) * np.asarray(w, F64) + np.asarray(b, F64)


def silu(x):
    return x / (1.0 + np.exp(-x))


def rope_cos_sin(positions, inv_freq, fp32_angles=True):
    """cos/sin of angle = pos * inv_freq as float64 [.., d].

    With ``fp32_angles`` the product is rounded to fp32 first, as the build's
    kernels and transformers' fp32/bf16 path do; without it the angle is float64.
    """
    if fp32_angles:
        pos = np.asarray(positions).astype(np.float32)[..., None]
        ang = (pos * np.asarray(inv_freq, np.float32)).astype(np.float32).astype(F64)
    else:
        ang = np.asarray(positions, F64)[..., None] * np.asarray(inv_freq, np.float32).astype(F64)
    ang = np.concatenate([ang, ang], axis=-1)
    return np.cos(ang), np.sin(ang)


def apply_rope(x, cos, sin):
    """x [..., d]; rotate_half convention (first half / second half)."""
    h = x.shape[-1] // 2
    rot = np.concatenate([-x[..., h:], x[..., :h]], axis=-1)
    return x * cos + rot * sin


def medusa_project(hidden, head, dtype=F64):
    """h + SiLU(fc(LayerNorm(h))). Follows ``flashgrpo/models/medusa_heads.py:74-78``."""
    h = np.asarray(hidden, dtype)
    ln = layernorm(h, head["ln_w"], head["ln_b"], 1e-5).astype(dtype)
    z = ln @ np.asarray(head["fc_w"], dtype).T + np.asarray(head["fc_b"], dtype)
    return h + silu(z)


def medusa_logits(hidden, heads, lm_head, max_heads=None, dtype=F64):
    """Per-head logits: through the head's own output projection when it has one
    (``head["out_w"]``, an untied head), else through the tied LM head.

    Follows ``flashgrpo/decoding/flash_medusa_decoder.py:254-304`` and
    ``flashgrpo/models/medusa_heads.py:266-276``.
    """
    n = len(heads) if max_heads is None else min(max_heads, len(heads))
    W = np.asarray(lm_head, dtype)
    return [medusa_project(hidden, heads[i], dtype) @
            (W if heads[i].get("out_w") is None else np.asarray(heads[i]["out_w"], dtype)).T for i in range(n)]


def random_chain_cell(hidden: int, seed: int, std: float = 0.02, bottleneck_ratio: int = 8, gate_init: float = -3.0,
                      dtype=np.float32) -> dict:
    """ChainDraftCell weights (``flashgrpo/models/medusa_heads.py:12-35``): LayerNorms identity,
    projections ~ N(0, std). The reference zero-initialises out_proj, which makes the
    cell the identity; synthetic runs draw it ~ N(0, std) as well."""
    rng = np.random.default_rng(seed)
    bott = max(64, hidden // max(1, bottleneck_ratio))
    n = lambda *shape: (rng.standard_normal(shape, dtype=np.float32) * std).astype(dtype)
    return {"sn_w": np.ones(hidden, dtype), "sn_b": np.zeros(hidden, dtype), "tn_w": np.ones(hidden, dtype),
            "tn_b": np.zeros(hidden, dtype), "sp_w": n(bott, hidden), "tp_w": n(bott, hidden), "op_w": n(hidden, bott),
            "op_b": n(hidden), "gate": np.float32(gate_init)}


def chain_cell(state, token_embedding, cell, dtype=F64):
    """state + sigmoid(gate) * out(SiLU(Ps . LN(state) + Pt . LN(emb))).
    Follows ``flashgrpo/models/medusa_heads.py:37-42`` (LayerNorm eps 1e-5)."""
    s = np.asarray(state, dtype)
    mixed = (layernorm(s, cell["sn_w"], cell["sn_b"]).astype(dtype) @ np.asarray(cell["sp_w"], dtype).T
             + layernorm(token_embedding, cell["tn_w"], cell["tn_b"]).astype(dtype) @ np.asarray(cell["tp_w"], dtype).T)
    delta = silu(mixed) @ np.asarray(cell["op_w"], dtype).T + np.asarray(cell["op_b"], dtype)
    return s + (1.0 / (1.0 + np.exp(-np.float64(cell["gate"])))) * delta


# --------------------------------------------------------------------------- decoder
def forward(cfg: ModelConfig, W: dict, tokens, positions, past_k, past_v, past_valid, self_allowed,
            fp32_angles=True, dtype=F64):
    """Decoder forward of N new tokens per row against a cached prefix.

    tokens/positions [B, N]; past_k/past_v: per layer [B, Hkv, P, d] (P may be 0);
    past_valid [B, P] bool; self_allowed [B, N, N] bool (query n may see new key m).
    Returns (final-normed hidden [B, N, H], new K list, new V list), new K/V
    per layer [B, Hkv, N, d] after rotary embedding. ``dtype`` is the compute
    type (float64 for parity checks; float32 for the timed CPU baseline, with
    weights already in float32 so that no weight copy is made).
    """
    tokens = np.asarray(tokens)
    B, N = tokens.shape
    Hq, Hkv, d, G = cfg.q_heads, cfg.kv_heads, cfg.head_dim, cfg.group
    x = np.asarray(W["embed"], dtype)[tokens]
    cos, sin = rope_cos_sin(positions, W["inv_freq"], fp32_angles)
    cos, sin = cos[:, :, None, :].astype(dtype), sin[:, :, None, :].astype(dtype)
    P = 0 if past_k is None or len(past_k) == 0 else past_k[0].shape[2]
    allowed = np.concatenate([np.broadcast_to(np.asarray(past_valid, bool)[:, None, :], (B, N, P)),
                              np.asarray(self_allowed, bool)], axis=-1)
    scale = 1.0 / np.sqrt(d)
    new_k, new_v = [], []
    for li, lw in enumerate(W["layers"]):
        h = rmsnorm(x, lw["input_norm"], cfg.rms_eps).astype(dtype)

        def proj(w, b):
            y = h @ np.asarray(w, dtype).T
            return y + np.asarray(b, dtype) if b is not None else y

        q = apply_rope(proj(lw["q_w"], lw["q_b"]).reshape(B, N, Hq, d), cos, sin)
        k = apply_rope(proj(lw["k_w"], lw["k_b"]).reshape(B, N, Hkv, d), cos, sin)
        v = proj(lw["v_w"], lw["v_b"]).reshape(B, N, Hkv, d)
        k = k.transpose(0, 2, 1, 3)
        v = v.transpose(0, 2, 1, 3)
        if P:
            keys = np.concatenate([np.asarray(past_k[li], dtype), k], axis=2)
            vals = np.concatenate([np.asarray(past_v[li], dtype), v], axis=2)
        else:
            keys, vals = k, v
        out = np.empty((B, N, Hq, d), dtype=x.dtype)
        for hq in range(Hq):
            kv = hq // G
            s = np.matmul(q[:, :, hq], keys[:, kv].transpose(0, 2, 1)) * scale
            s = np.where(allowed, s, -np.inf)
            s = s - s.max(axis=-1, keepdims=True)
            p = np.exp(s)
            p = p / p.sum(axis=-1, keepdims=True)
            out[:, :, hq] = np.matmul(p, vals[:, kv])
        x = x + out.reshape(B, N, Hq * d) @ np.asarray(lw["o_w"], dtype).T
        h2 = rmsnorm(x, lw["post_norm"], cfg.rms_eps).astype(dtype)
        g = h2 @ np.asarray(lw["gate_w"], dtype).T
        u = h2 @ np.asarray(lw["up_w"], dtype).T
        x = x + ((silu(g) * u) @ np.asarray(lw["down_w"], dtype).T).astype(dtype)
        new_k.append(k)
        new_v.append(v)
    return rmsnorm(x, W["final_norm"], cfg.rms_eps).astype(dtype), new_k, new_v


def prefill(cfg, W, tokens, fp32_angles=True, dtype=F64):
    """Causal forward of full-length prompts [B, P]; returns (hidden, K list, V list)."""
    tokens = np.asarray(tokens)
    B, P = tokens.shape
    pos = np.broadcast_to(np.arange(P), (B, P))
    causal = np.broadcast_to(np.tril(np.ones((P, P), bool)), (B, P, P))
    return forward(cfg, W, tokens, pos, None, None, np.zeros((B, 0), bool), causal, fp32_angles, dtype)


def tree_verify(cfg, W, tree_tokens, depths, parents, past_k, past_v, seq_len, dtype=F64):
    """Tree forward: node n at position seq_len + depth - 1, seeing prefix + ancestors.

    Follows the mask/position construction of ``flashgrpo/decoding/tree_attention.py:6-67``
    feeding ``forward_tree`` (``flashgrpo/models/qwen_flashgrpo_wrapper.py:220-239``),
    for full-length prefixes (every prefix slot valid).
    """
    tree_tokens = np.asarray(tree_tokens)
    B, N = tree_tokens.shape
    allowed = np.zeros((B, N, N), bool)
    for b in range(B):
        for n in range(N):
            a = n
            while a >= 0:
                allowed[b, n, a] = True
                a = parents[b][a]
    pos = np.asarray(seq_len)[:, None] + np.asarray(depths) - 1
    P = past_k[0].shape[2]
    return forward(cfg, W, tree_tokens, pos, past_k, past_v, np.ones((B, P), bool), allowed, dtype=dtype)


def logits(hidden, lm_head, dtype=F64):
    return np.asarray(hidden, dtype) @ np.asarray(lm_head, dtype).T
