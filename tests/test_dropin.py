"""The drop-in boundary at the reference trainer's call sites, on the CPU (no GPU work):

* ``FlashMedusaConfig`` takes exactly the keyword set the trainer's
  ``_make_flash_config`` passes (``flashgrpo/training/flashgrpo_trainer.py:555-633``);
* ``TargetModel.from_hf`` copies every weight of a transformers Qwen2 model (no alias
  of a live parameter), merges LoRA adapters through the module (PEFT layout), and
  ``sync_from_hf`` re-reads the weights in place after an in-place edit;
* Medusa checkpoints round-trip through ``save_pretrained`` / ``from_pretrained``
  with the reference's file and key layout, shape filtering and weights-only loading;
* ``forward_tree`` rejects a mask whose prefix block does not match the cache and a
  tree that does not fit the cache, before any launch.
"""
import json
import pickle

import numpy as np
import pytest
import torch
import torch.nn as nn

# The keyword names _make_flash_config passes (flashgrpo_trainer.py:560-633), in its order.
TRAINER_FIELDS = [
    "num_medusa_heads", "tree_mode", "tree_layout", "acceptance", "cache_update_mode", "allow_recompute_fallback",
    "cpeak_nodes", "min_tree_nodes_per_seq", "max_tree_nodes_per_seq", "max_tree_depth", "fixed_tree_topk_by_depth",
    "do_sample", "temperature", "top_p", "top_k", "clone_tree_cache", "enable_medusa_spec_after", "proposal_mode",
    "chain_enable_after", "chain_bootstrap_from_medusa", "adaptive_tree_enabled", "adaptive_confidence_metric",
    "adaptive_confidence_quantile", "adaptive_confidence_low", "adaptive_confidence_high",
    "adaptive_min_topk_by_depth", "adaptive_depth_weight_decay", "head_inference_autocast",
    "project_internal_tree_logits_only", "inplace_kv_compaction", "reflex_enabled", "reflex_state_space",
    "reflex_fast_state_dim", "reflex_beta", "reflex_eta", "reflex_top_m_feedback", "reflex_feedback_stride",
    "reflex_feedback_stride_min", "reflex_target_topk", "reflex_feedback_union_cap", "reflex_tv_gate_low",
    "reflex_tv_gate_high", "reflex_horizon_weight_decay", "reflex_half_life_tokens", "reflex_feedback_variance_beta",
    "reflex_feedback_rms_clip", "reflex_state_rms_clip", "reflex_numerical_reset_rms",
    "reflex_relative_rms_delta_base", "reflex_warmup_effective_updates", "reflex_magnitude_gate_floor",
    "reflex_guard_calibration_rollouts", "reflex_guard_aal_drop_fraction", "reflex_guard_patience",
    "reflex_guard_disable_rollouts", "reflex_feedback_clip_norm", "reflex_hidden_feedback_clip_norm",
    "reflex_fast_state_clip_norm", "reflex_correction_clip_norm", "reflex_normalize_correction",
    "reflex_feedback_ce_gate", "reflex_feedback_ce_tau", "reflex_feedback_ce_threshold", "reflex_normalize_feedback",
    "reflex_feedback_enabled", "reflex_proposal_injection_enabled", "reflex_proposal_injection_scale",
    "reflex_proposal_injection_after", "reflex_proposal_injection_warmup", "reflex_aux_cache_enabled",
    "reflex_aux_cache_max_records", "reflex_aux_cache_stride", "reflex_aux_store_fast_state",
]


def _trainer_config(**over):
    """The config _make_flash_config builds from an empty yaml (its .get defaults)."""
    from flashgrpo_amd.decoding import FlashMedusaConfig

    defaults = FlashMedusaConfig()
    kw = {k: getattr(defaults, k) for k in TRAINER_FIELDS}
    kw["max_tree_depth"] = kw["num_medusa_heads"] + 1  # flashgrpo_trainer.py:570
    kw["fixed_tree_topk_by_depth"] = tuple([4, 3, 2])
    kw["adaptive_min_topk_by_depth"] = tuple([1, 1, 1])
    kw["reflex_aux_cache_max_records"] = 8192
    kw.update(over)
    return FlashMedusaConfig(**kw)


def test_config_takes_the_trainer_keyword_set():
    from dataclasses import fields

    cfg = _trainer_config()
    names = {f.name for f in fields(cfg)}
    assert set(TRAINER_FIELDS) <= names
    assert cfg.reflex_state_space == "projected" and cfg.reflex_fast_state_dim == 128
    assert cfg.reflex_feedback_ce_tau == 4.0 and cfg.reflex_aux_cache_stride == 1
    assert len(TRAINER_FIELDS) == len(set(TRAINER_FIELDS)) == 73


def _tiny_target():
    from flashgrpo_amd.models import TargetConfig, TargetModel

    cfg = TargetConfig(2, 64, 4, 2, 16, 96, 50)
    return TargetModel.random(cfg, seed=0, dtype=torch.float32, device="cpu")


def test_decoder_accepts_trainer_config_and_rejects_reflex():
    from flashgrpo_amd.decoding import FlashMedusaDecoder
    from flashgrpo_amd.models import MedusaHeads

    model = _tiny_target()
    heads = MedusaHeads(64, 50, 3)

    class Tok:
        pad_token_id, eos_token_id = 0, 1

    dec = FlashMedusaDecoder(model, heads, Tok(), _trainer_config())
    assert dec.model is model
    with pytest.raises(NotImplementedError, match="reflex"):
        FlashMedusaDecoder(model, heads, Tok(), _trainer_config(reflex_enabled=True))
    bad = MedusaHeads(64, 49, 3, tie_lm_head=False)
    with pytest.raises(ValueError, match="untied Medusa head 0"):
        FlashMedusaDecoder(model, bad, Tok(), _trainer_config())


# ------------------------------------------------------------------ Hugging Face target
def _hf_qwen2(seed=0, tie=False, layers=2):
    transformers = pytest.importorskip("transformers")
    cfg = transformers.Qwen2Config(vocab_size=97, hidden_size=64, intermediate_size=112, num_hidden_layers=layers,
                                   num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=256,
                                   rope_theta=10000.0, tie_word_embeddings=tie)
    torch.manual_seed(seed)
    m = transformers.Qwen2ForCausalLM(cfg).eval()
    with torch.no_grad():
        for p in m.parameters():  # norms and biases away from 1 / 0 so a swap would show
            p.add_(torch.randn_like(p) * 0.02)
    return m


def _effective(mod, x):
    """What the module computes on x, as a (weight, bias) pair read back from its output."""
    eye = torch.eye(x.shape[1], dtype=x.dtype)
    zero = torch.zeros(1, x.shape[1], dtype=x.dtype)
    with torch.no_grad():
        b = mod(zero)[0]
        w = (mod(eye) - b).t()
    return w, b


def _check_against_modules(model, hf):
    body = hf.model
    x = torch.zeros(1, 64)
    for i, layer in enumerate(body.layers):
        lw = model.w["layers"][i]
        at, mlp = layer.self_attn, layer.mlp
        qkv = [_effective(m, x) for m in (at.q_proj, at.k_proj, at.v_proj)]
        torch.testing.assert_close(lw["qkv_w"], torch.cat([w for w, _ in qkv]), rtol=1e-6, atol=1e-6)
        torch.testing.assert_close(lw["qkv_b"], torch.cat([b for _, b in qkv]), rtol=1e-6, atol=1e-6)
        torch.testing.assert_close(lw["o_w"], _effective(at.o_proj, torch.zeros(1, 64))[0], rtol=1e-6, atol=1e-6)
        gu = [_effective(m, x)[0] for m in (mlp.gate_proj, mlp.up_proj)]
        torch.testing.assert_close(lw["gate_up_w"], torch.cat(gu), rtol=1e-6, atol=1e-6)
        torch.testing.assert_close(lw["down_w"], _effective(mlp.down_proj, torch.zeros(1, 112))[0], rtol=1e-6,
                                   atol=1e-6)
        assert torch.equal(lw["input_norm"], layer.input_layernorm.weight)
        assert torch.equal(lw["post_norm"], layer.post_attention_layernorm.weight)
    assert torch.equal(model.w["embed"], body.embed_tokens.weight)
    assert torch.equal(model.w["final_norm"], body.norm.weight)
    assert torch.equal(model.w["lm_head"], hf.lm_head.weight)


def _all_tensors(w):
    out = [w["embed"], w["final_norm"], w["lm_head"]]
    for lw in w["layers"]:
        out += [t for t in lw.values() if t is not None]
    return out


@pytest.mark.parametrize("tie", [False, True])
def test_from_hf_copies_and_resyncs(tie):
    from flashgrpo_amd.models import TargetModel

    hf = _hf_qwen2(tie=tie)
    model = TargetModel.from_hf(hf)
    cfg = model.cfg
    assert (cfg.num_layers, cfg.hidden, cfg.q_heads, cfg.kv_heads, cfg.head_dim, cfg.intermediate, cfg.vocab) == \
        (2, 64, 4, 2, 16, 112, 97)
    assert cfg.qkv_bias and cfg.rope_theta == 10000.0 and cfg.tie_word_embeddings == tie
    _check_against_modules(model, hf)
    ptrs = {p.data_ptr() for p in hf.parameters()}
    assert not any(t.data_ptr() in ptrs for t in _all_tensors(model.w))  # copies, never aliases
    assert (model.w["lm_head"] is model.w["embed"]) == tie
    addrs = [t.data_ptr() for t in _all_tensors(model.w)]
    assert not model.sync_from_hf()  # nothing changed
    with torch.no_grad():  # an "optimizer step": in-place updates of a few parameters
        hf.model.layers[1].self_attn.k_proj.weight.mul_(1.5)
        hf.model.layers[0].mlp.down_proj.weight.add_(0.01)
        hf.model.norm.weight.sub_(0.1)
        hf.lm_head.weight.add_(0.02)
    old_k = model.w["layers"][1]["qkv_w"].clone()
    assert model.sync_from_hf()
    assert not torch.equal(old_k, model.w["layers"][1]["qkv_w"])
    _check_against_modules(model, hf)
    assert [t.data_ptr() for t in _all_tensors(model.w)] == addrs  # re-read in place
    assert not model.sync_from_hf()


class FakeLoraLinear(nn.Module):
    """A linear wrapped the way PEFT's LoRA layer stores it (``base_layer``, ``lora_A`` /
    ``lora_B`` module dicts, ``scaling``, ``active_adapters``, ``merged``), with the LoRA
    forward base(x) + scaling * B(A(x)). PEFT itself is not installed here, so the
    merge is pinned against this layout and forward, not against PEFT's own code."""

    def __init__(self, base: nn.Linear, r=4, alpha=8, adapters=("default",), lora_bias=False):
        super().__init__()
        self.base_layer = base
        self.lora_A = nn.ModuleDict({a: nn.Linear(base.in_features, r, bias=False) for a in adapters})
        self.lora_B = nn.ModuleDict({a: nn.Linear(r, base.out_features, bias=lora_bias) for a in adapters})
        self.scaling = {a: alpha / r * (1 + i) for i, a in enumerate(adapters)}
        self.active_adapters = list(adapters)
        self.merged = False
        self.disable_adapters = False
        self.use_dora = {a: False for a in adapters}
        for a in adapters:
            nn.init.normal_(self.lora_A[a].weight, std=0.1)
            nn.init.normal_(self.lora_B[a].weight, std=0.1)  # PEFT starts B at 0; trained B is not
            if lora_bias:
                nn.init.normal_(self.lora_B[a].bias, std=0.1)

    def forward(self, x):
        y = self.base_layer(x)
        if self.merged or self.disable_adapters:
            return y
        for a in self.active_adapters:
            y = y + self.lora_B[a](self.lora_A[a](x)) * self.scaling[a]
        return y


def _wrap_lora(hf, **kw):
    targets = [("self_attn", n) for n in ("q_proj", "k_proj", "v_proj", "o_proj")] + \
              [("mlp", n) for n in ("gate_proj", "up_proj", "down_proj")]
    for layer in hf.model.layers:
        for parent, name in targets:
            owner = getattr(layer, parent)
            setattr(owner, name, FakeLoraLinear(getattr(owner, name), **kw))


class FakePeftModel(nn.Module):
    """get_base_model() as a PEFT wrapper exposes it."""

    def __init__(self, inner):
        super().__init__()
        self.inner = inner

    def get_base_model(self):
        return self.inner


def test_from_hf_merges_lora_adapters_and_follows_their_updates():
    from flashgrpo_amd.models import TargetModel

    hf = _hf_qwen2(seed=1)
    _wrap_lora(hf, adapters=("default", "second"), lora_bias=True)
    peft = FakePeftModel(hf)
    model = TargetModel.from_hf(peft)
    _check_against_modules(model, hf)  # effective weights = what each wrapped module computes
    # an adapter-only update (the LoRA parameters are the trainable ones)
    with torch.no_grad():
        hf.model.layers[0].self_attn.v_proj.lora_B["default"].weight.add_(0.05)
    assert model.sync_from_hf()
    _check_against_modules(model, hf)
    # merged adapters live in the base weight already; disabled adapters contribute nothing
    for layer in hf.model.layers:
        layer.mlp.up_proj.merged = True
        layer.self_attn.q_proj.disable_adapters = True
    model.sync_from_hf(force=True)
    _check_against_modules(model, hf)
    hf.model.layers[1].mlp.down_proj.use_dora["second"] = True
    with pytest.raises(NotImplementedError, match="DoRA"):
        model.sync_from_hf(force=True)


def test_from_hf_native_config_matches_hf_forward_inputs():
    """RoPE inverse frequencies come from the HF rotary module (fp32 copy)."""
    from flashgrpo_amd.models import TargetModel

    hf = _hf_qwen2()
    model = TargetModel.from_hf(hf)
    torch.testing.assert_close(model.inv_freq, hf.model.rotary_emb.inv_freq.float())
    assert model.inv_freq.data_ptr() != hf.model.rotary_emb.inv_freq.data_ptr()


# ------------------------------------------------------------------ Medusa checkpoints
REF_KEYS_PER_HEAD = ["fc.weight", "fc.bias", "norm.weight", "norm.bias"]
REF_CELL_KEYS = ["state_norm.weight", "state_norm.bias", "token_norm.weight", "token_norm.bias",
                 "state_proj.weight", "token_proj.weight", "out_proj.weight", "out_proj.bias", "gate"]


@pytest.mark.parametrize("tie", [True, False])
def test_medusa_checkpoint_round_trip(tmp_path, tie):
    from flashgrpo_amd.models import MedusaHeads

    H = 640  # chain bottleneck max(64, H / ratio): 80 at ratio 8, 160 at ratio 4
    m = MedusaHeads.random(H, 50, 3, seed=4)
    if not tie:
        m = MedusaHeads(H, 50, 3, tie_lm_head=False)
        with torch.no_grad():
            for p in m.parameters():
                p.normal_(0.0, 0.1)
    m.save_pretrained(tmp_path)
    cfg = json.loads((tmp_path / "medusa_config.json").read_text())
    assert cfg == {"hidden_size": H, "vocab_size": 50, "num_heads": 3, "tie_lm_head": tie, "medusa_loss_decay": 0.8,
                   "chain_bottleneck_ratio": 8, "chain_gate_init": -3.0, "reflex_fast_state_dim": 0,
                   "reflex_init_scale": 0.0}
    assert (tmp_path / "medusa_config.yaml").exists()
    want_keys = {f"heads.{i}.{k}" for i in range(3) for k in REF_KEYS_PER_HEAD}
    want_keys |= {f"chain_cell.{k}" for k in REF_CELL_KEYS}
    if not tie:
        want_keys |= {f"heads.{i}.output.weight" for i in range(3)}
    state = torch.load(tmp_path / "medusa_heads.pt", weights_only=True)
    assert set(state) == want_keys
    back = MedusaHeads.from_pretrained(tmp_path, device="cpu")
    assert back.tie_lm_head == tie and back._loaded_compatible_keys == want_keys
    for (k, a), (k2, b) in zip(sorted(m.state_dict().items()), sorted(back.state_dict().items())):
        assert k == k2 and torch.equal(a, b), k
    own = back.output_weights(torch.float32, "cpu")
    assert all((w is None) == tie for w in own)
    # keyword overrides win over the file's config (medusa_heads.py:442-470)
    alt = MedusaHeads.from_pretrained(tmp_path, chain_bottleneck_ratio=4, chain_gate_init=-1.0)
    assert alt.chain_bottleneck_ratio == 4 and alt.chain_gate_init == -1.0
    assert "chain_cell.state_proj.weight" not in alt._loaded_compatible_keys  # shape differs: filtered out
    assert "heads.0.fc.weight" in alt._loaded_compatible_keys


def test_medusa_checkpoint_loading_is_weights_only(tmp_path):
    from flashgrpo_amd.models import MedusaHeads

    MedusaHeads(64, 50, 2).save_pretrained(tmp_path)

    class Payload:
        def __reduce__(self):
            return (print, ("unpickled code ran",))

    state = torch.load(tmp_path / "medusa_heads.pt", weights_only=True)
    state["evil"] = Payload()
    torch.save(state, tmp_path / "medusa_heads.pt")
    with pytest.raises(pickle.UnpicklingError):
        MedusaHeads.from_pretrained(tmp_path)


def test_untied_heads_copy_the_lm_head_module_weight(tmp_path):
    """Heads built as the trainer builds them (``flashgrpo_trainer.py:727-733``:
    ``lm_head=base.lm_head``, an nn.Module) start from the LM head's weight
    (``medusa_heads.py:69-72``), and ``from_pretrained`` keeps that copy for the
    ``output`` keys a checkpoint lacks or that its shape filter drops
    (``flashgrpo_trainer.py:749-753``)."""
    from flashgrpo_amd.models import MedusaHeads

    torch.manual_seed(3)
    lm_head = nn.Linear(16, 40, bias=False)
    m = MedusaHeads(hidden_size=16, vocab_size=40, num_heads=2, dtype=torch.float32, tie_lm_head=False,
                    lm_head=lm_head)
    for hd in m.heads:
        assert torch.equal(hd.output.weight, lm_head.weight)
    # a bare weight tensor is taken too; a mismatched shape leaves nn.Linear's init
    t = MedusaHeads(16, 40, 1, tie_lm_head=False, lm_head=lm_head.weight)
    assert torch.equal(t.heads[0].output.weight, lm_head.weight)
    other = MedusaHeads(16, 40, 1, tie_lm_head=False, lm_head=nn.Linear(16, 41, bias=False))
    assert not torch.equal(other.heads[0].output.weight[:40], lm_head.weight)
    # bf16 heads from an fp32 module: copied with a cast
    b = MedusaHeads(16, 40, 1, dtype=torch.bfloat16, tie_lm_head=False, lm_head=lm_head)
    assert torch.equal(b.heads[0].output.weight, lm_head.weight.to(torch.bfloat16))

    # a tied checkpoint has no output keys: loaded untied with the trainer's lm_head,
    # every head keeps the copy
    MedusaHeads.random(16, 40, 2, seed=1).save_pretrained(tmp_path)
    cfg_path = tmp_path / "medusa_config.json"
    cfg = json.loads(cfg_path.read_text())
    cfg["tie_lm_head"] = False
    cfg_path.write_text(json.dumps(cfg))
    back = MedusaHeads.from_pretrained(tmp_path, map_location="cpu", dtype=torch.float32, lm_head=lm_head)
    assert not any(k.endswith("output.weight") for k in back._loaded_compatible_keys)
    for hd in back.heads:
        assert torch.equal(hd.output.weight, lm_head.weight)


def test_medusa_output_weights_follow_parameter_updates():
    from flashgrpo_amd.models import MedusaHeads

    m = MedusaHeads(8, 11, 2, tie_lm_head=False)
    first = m.output_weights(torch.float64, "cpu")[1].clone()
    with torch.no_grad():
        m.heads[1].output.weight.add_(1.0)
    torch.testing.assert_close(m.output_weights(torch.float64, "cpu")[1], first + 1.0)


# ------------------------------------------------------------------ forward_tree validation
def test_forward_tree_rejects_mismatched_prefix_and_overflow():
    from flashgrpo_amd.decoding.medusa_tree import CandidateTree
    from flashgrpo_amd.decoding.tree_attention import build_tree_attention_inputs
    from flashgrpo_amd.models import forward_tree

    model = _tiny_target()
    cache = model.new_cache(2, 40)
    cache.seq_len.copy_(torch.tensor([5, 9], dtype=torch.int32))
    trees = [CandidateTree([3, 4, 5], [-1, 0, 0], [1, 2, 2]), CandidateTree([6, 7], [-1, 0], [1, 2])]
    full = torch.zeros(2, 12, dtype=torch.long)
    full[0, :5] = 1
    full[1, 3:12] = 1  # a left-padded row: 9 valid slots
    lens = torch.tensor([5, 9])
    ids, mask, pos, _ = build_tree_attention_inputs(trees, full, lens, pad_token_id=0, dtype=torch.float32)
    bad = full.clone()
    bad[0, 4] = 0  # row 0 would see 4 prefix tokens, its cache row holds 5
    _, mask_bad, _, _ = build_tree_attention_inputs(trees, bad, lens, pad_token_id=0, dtype=torch.float32)
    with pytest.raises(ValueError, match="prefix block"):
        forward_tree(model, ids, mask_bad, cache, pos)
    mask_node = mask.clone()
    mask_node[1, 0, 1, 5] = torch.finfo(torch.float32).min  # node 1 of row 1 sees less than node 0
    with pytest.raises(ValueError, match="prefix block"):
        forward_tree(model, ids, mask_node, cache, pos)
    cache.seq_len.copy_(torch.tensor([5, 38], dtype=torch.int32))
    full[1] = 0
    full[1, :12] = 1
    big = torch.zeros(2, 38, dtype=torch.long)
    big[0, :5] = 1
    big[1, :38] = 1
    ids, mask, pos, _ = build_tree_attention_inputs(trees, big, torch.tensor([5, 38]), pad_token_id=0,
                                                    dtype=torch.float32)
    with pytest.raises(ValueError, match="capacity"):
        forward_tree(model, ids, mask, cache, pos)


def test_sync_works_for_weights_made_inside_or_outside_inference_mode():
    """The trainer calls generate under torch.inference_mode: a conversion made there
    (inference tensors) must still re-sync afterwards, and one made outside must sync
    inside it."""
    from flashgrpo_amd.models import TargetModel

    hf = _hf_qwen2(seed=2)
    with torch.inference_mode():
        inside = TargetModel.from_hf(hf)
    outside = TargetModel.from_hf(hf)
    with torch.no_grad():
        hf.model.layers[0].mlp.gate_proj.weight.mul_(0.5)
    assert inside.sync_from_hf()
    with torch.inference_mode():
        assert outside.sync_from_hf()
    for m in (inside, outside):
        _check_against_modules(m, hf)


# ------------------------------------------------------------------ LM-head routing rules
def test_lm_head_routing_predicates():
    """The hand-written LM-head kernels take bf16 operands with K % 64 == 0 and 16-byte
    aligned rows; anything else routes to the library GEMM (host-side decision only)."""
    from flashgrpo_amd.models.target import lm_gemm_ok, lm_stream_ok

    bf = torch.bfloat16
    x = torch.zeros(8, 128, dtype=bf)
    w = torch.zeros(100, 128, dtype=bf)
    assert lm_gemm_ok(x, w) and lm_stream_ok(x, w)
    assert not lm_gemm_ok(torch.zeros(8, 96, dtype=bf), torch.zeros(100, 96, dtype=bf))   # K % 64
    assert not lm_gemm_ok(x.float(), w.float())                                           # dtype
    assert not lm_gemm_ok(torch.zeros(8, 129, dtype=bf)[:, 1:], w)                        # base not 16-byte aligned
    assert not lm_gemm_ok(torch.zeros(8, 132, dtype=bf)[:, :128], w)                      # row stride 132
    assert not lm_gemm_ok(x, torch.zeros(128, 100, dtype=bf).t())                         # weight not K-contiguous
    out = torch.zeros(8, 100, dtype=bf)
    assert lm_stream_ok(x, w, out)
    assert not lm_stream_ok(x, w, torch.zeros(100, 8, dtype=bf).t())                      # output column stride
    assert not lm_stream_ok(x, w, torch.zeros(8, 104, dtype=bf)[:, 1:101])               # 4-column store alignment
    assert lm_stream_ok(x, w, torch.zeros(8, 103, dtype=bf)[:, :100])                     # stride 103: scalar stores
