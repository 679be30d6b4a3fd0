"""The reference wrapper's entry points (models/qwen_flashgrpo_wrapper.py) driven the way
the reference's own extraction check drives them (flashgrpo/scripts/test_kv_extraction.py:
prefill -> build_tree_attention_inputs -> forward_tree(clone_past=True) ->
extract_accepted_path_kv -> forward_tokens), on a transformers Qwen2 model with a
left-padded batch, against the float64 oracle and against recompute."""
import numpy as np
import pytest
import torch

from oracle import model as OM

from test_gpu_decoder import _hf_oracle_weights, rel

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def _hf(vocab=97):
    transformers = pytest.importorskip("transformers")
    hc = transformers.Qwen2Config(vocab_size=vocab, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                                  num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=512,
                                  rope_theta=1.0e6, rms_norm_eps=1e-6, tie_word_embeddings=False)
    torch.manual_seed(4)
    hf = transformers.Qwen2ForCausalLM(hc).to(DEV).float().eval()
    with torch.no_grad():
        for p in hf.parameters():
            p.normal_(0.0, 0.05) if p.dim() > 1 else p.add_(torch.randn_like(p) * 0.05)
    ocfg = OM.ModelConfig(num_layers=2, hidden=256, q_heads=4, kv_heads=2, head_dim=64, intermediate=512,
                          vocab=vocab, rope_theta=1.0e6, rms_eps=1e-6)
    return hf, ocfg


def test_reference_extraction_flow_with_left_padding():
    from flashgrpo_amd.decoding.kv_extraction import extract_accepted_path_kv
    from flashgrpo_amd.decoding.medusa_tree import CandidateTree
    from flashgrpo_amd.decoding.tree_attention import build_tree_attention_inputs
    from flashgrpo_amd.models.qwen_flashgrpo_wrapper import (autocast_dtype, clone_cache, forward_tokens,
                                                             forward_tree, logical_lengths, prefill)

    hf, ocfg = _hf()
    W = _hf_oracle_weights(hf)
    rng = np.random.default_rng(0)
    T, lens = 30, [30, 19]
    ids = torch.zeros(2, T, dtype=torch.long)
    mask = torch.zeros(2, T, dtype=torch.long)
    prompts = [rng.integers(1, 97, n) for n in lens]
    for b, p in enumerate(prompts):  # left padding, as the reference tokenizer pads
        ids[b, T - len(p):] = torch.from_numpy(p)
        mask[b, T - len(p):] = 1
    ids, mask = ids.to(DEV), mask.to(DEV)
    with torch.inference_mode():
        pref = prefill(hf, ids, mask)
        cache = pref["past_key_values"]
        assert cache.seq_len.tolist() == lens
        for b, p in enumerate(prompts):
            want, _, _ = OM.prefill(ocfg, W, p[None])
            got = pref["hidden_states"][b, T - len(p):].cpu().numpy()
            assert rel(got, want[0]) < 1e-5, b
            assert bool((pref["hidden_states"][b, :T - len(p)] == 0).all())  # padding positions
        recompute_cache = clone_cache(cache, clone_tensors=True)  # a deep copy for the recompute path
        logical = logical_lengths(mask)
        trees = [CandidateTree([5, 6, 7, 8], [-1, 0, 0, 1], [1, 2, 2, 3]), CandidateTree([9, 10], [-1, 0], [1, 2])]
        tids, mask4d, pos, _ = build_tree_attention_inputs(trees, mask, logical, pad_token_id=0,
                                                           dtype=autocast_dtype(hf))
        tree_out = forward_tree(hf, tids, mask4d, cache, pos, clone_past=True)
        tree_cache = tree_out["past_key_values"]
        paths = [[0, 1, 3], [0, 1]]
        extracted = extract_accepted_path_kv(cache, tree_cache, paths, causal_lm=hf).past_key_values
        assert cache.seq_len.tolist() == lens  # the past's lengths are untouched
        assert extracted.seq_len.tolist() == [lens[0] + 3, lens[1] + 2]
        # recompute: the accepted tokens appended to the prefix (right-padded row 1)
        acc = torch.tensor([[5, 6, 8], [9, 10, 0]], device=DEV)
        acc_mask = torch.cat([mask, torch.tensor([[1, 1, 1], [1, 1, 0]], device=DEV)], dim=1)
        acc_pos = logical[:, None] + torch.arange(3, device=DEV)[None]
        forward_tokens(hf, acc, acc_mask, recompute_cache, acc_pos)
        assert recompute_cache.seq_len.tolist() == extracted.seq_len.tolist()
        # the next token through both caches
        nxt = torch.tensor([[11], [12]], device=DEV)
        valid = torch.cat([mask, torch.tensor([[1, 1, 1], [1, 1, 0]], device=DEV)], dim=1)
        lens_after = [lens[0] + 3, lens[1] + 2]
        nxt_mask = torch.zeros(2, valid.shape[1] + 1, dtype=torch.long, device=DEV)
        for b, L in enumerate(lens_after):  # committed tokens then the new one
            nxt_mask[b, :L] = 1
            nxt_mask[b, -1] = 1
        nxt_pos = torch.tensor([[lens_after[0]], [lens_after[1]]], device=DEV)
        he = forward_tokens(hf, nxt, nxt_mask, extracted, nxt_pos)["hidden_states"]
        hr = forward_tokens(hf, nxt, nxt_mask, recompute_cache, nxt_pos)["hidden_states"]
    assert rel(he.cpu().numpy(), hr.cpu().numpy()) < 1e-5
    for b, (p, path) in enumerate(zip(prompts, [[5, 6, 8], [9, 10]])):
        seqtoks = np.concatenate([p, path, [11 + b]])
        want, _, _ = OM.prefill(ocfg, W, seqtoks[None])
        assert rel(he[b, 0].cpu().numpy(), want[0, -1]) < 1e-5, b


def test_cache_row_selection_and_repeats():
    from flashgrpo_amd.models.qwen_flashgrpo_wrapper import (cache_seq_length, prefill, repeat_interleave_cache,
                                                             select_cache_batch)

    hf, _ = _hf()
    ids = torch.randint(0, 97, (3, 12), device=DEV)
    mask = torch.ones(3, 12, dtype=torch.long, device=DEV)
    mask[1, :4] = 0
    with torch.inference_mode():
        cache = prefill(hf, ids, mask, capacity=40)["past_key_values"]
    assert cache_seq_length(cache) == 12 and cache.capacity == 40
    sel = select_cache_batch(cache, torch.tensor([2, 0]))
    assert sel.batch == 2 and sel.seq_len.tolist() == [12, 12]
    assert torch.equal(sel.kv, cache.kv[:, :, [2, 0]])
    rep = repeat_interleave_cache(cache, 3)
    assert rep.batch == 9 and rep.seq_len.tolist() == [12] * 3 + [8] * 3 + [12] * 3
    assert torch.equal(rep.kv, cache.kv.repeat_interleave(3, dim=2))
    assert repeat_interleave_cache(cache, 1) is cache
