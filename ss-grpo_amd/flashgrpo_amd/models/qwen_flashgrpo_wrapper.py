"""The reference wrapper's function-level entry points over the native target model.

Same names, arguments and result dicts as ``flashgrpo/models/qwen_flashgrpo_wrapper.py``
(``prefill`` / ``forward_tokens`` / ``forward_tree`` :189-239, ``clone_cache`` /
``select_cache_batch`` / ``repeat_interleave_cache`` / ``cache_seq_length`` :68-147,
``logical_lengths`` / ``position_ids_from_attention_mask`` :29-35), so scripts written
against the reference (``flashgrpo/scripts/test_kv_extraction.py``,
``measure_cpeak.py``) run unchanged. ``causal_lm`` is a ``TargetModel`` or a
transformers Qwen2/Llama causal LM (optionally PEFT-wrapped), converted once by
``TargetModel.from_hf`` and re-read in place whenever its parameters change.

The cache is the native ``KVCache`` ([L, 2, B, Hkv, capacity, d] + committed lengths,
each row's tokens left-aligned) instead of a ``DynamicCache`` over the caller's
left-padded layout. The 2-D attention masks the reference passes are checked against
it: the columns a row marks valid must number exactly the row's committed length.
Differences a caller can see: the cache has a fixed capacity (``prefill``'s
``capacity``, default prompt width + 1024; a write past it raises), and appending
through two containers of one cache past the same committed length (a
``clone_cache(clone_tensors=False)`` copy and its original) overwrites the same
slots, where the reference's ``torch.cat`` would allocate new tensors.
"""
from __future__ import annotations

import numpy as np
import torch

from . import target as _target
from .target import KVCache, TargetModel, unwrap_causal_lm

PREFILL_HEADROOM = 1024  # slots past the prompt width of a cache made by prefill()

__all__ = ["unwrap_causal_lm", "model_device", "autocast_dtype", "position_ids_from_attention_mask",
           "logical_lengths", "as_target_model", "clone_cache", "select_cache_batch", "repeat_interleave_cache",
           "cache_seq_length", "prefill", "forward_tokens", "forward_tree"]


def model_device(model) -> torch.device:
    """``qwen_flashgrpo_wrapper.py:15-19``."""
    if isinstance(model, TargetModel):
        return model.device
    try:
        return next(model.parameters()).device
    except StopIteration:
        return torch.device("cuda" if torch.cuda.is_available() else "cpu")


def autocast_dtype(model) -> torch.dtype:
    """``qwen_flashgrpo_wrapper.py:22-26``: bf16 models run bf16, others fp16 autocast."""
    dtype = model.dtype if isinstance(model, TargetModel) else getattr(unwrap_causal_lm(model), "dtype", None)
    return torch.bfloat16 if dtype == torch.bfloat16 else torch.float16


def position_ids_from_attention_mask(attention_mask: torch.Tensor) -> torch.Tensor:
    """``qwen_flashgrpo_wrapper.py:29-31``: cumulative count of valid tokens minus one,
    0 on padding."""
    pos = attention_mask.long().cumsum(dim=-1) - 1
    return pos.masked_fill(attention_mask == 0, 0)


def logical_lengths(attention_mask: torch.Tensor) -> torch.Tensor:
    """``qwen_flashgrpo_wrapper.py:34-35``."""
    return attention_mask.long().sum(dim=-1)


def as_target_model(causal_lm) -> TargetModel:
    """The native model of ``causal_lm``: itself, or the conversion of a Hugging Face
    model (made once, kept on the module and re-read when its parameters changed)."""
    if isinstance(causal_lm, TargetModel):
        return causal_lm
    native = getattr(causal_lm, "_flashgrpo_amd_target", None)
    if native is None:
        native = TargetModel.from_hf(causal_lm)
        object.__setattr__(causal_lm, "_flashgrpo_amd_target", native)
    else:
        native.sync_from_hf()
    return native


def _need_cache(cache) -> KVCache:
    if not isinstance(cache, KVCache):
        raise TypeError(f"expected a flashgrpo_amd KVCache, got {type(cache).__name__}")
    return cache


def clone_cache(cache, causal_lm=None, *, clone_tensors: bool = False):
    """``qwen_flashgrpo_wrapper.py:68-97``: a new container (sharing storage) or, with
    ``clone_tensors``, a deep copy."""
    if cache is None:
        return None
    c = _need_cache(cache)
    if not clone_tensors:
        return c.container_copy()
    out = c.container_copy()
    out.kv = c.kv.clone()
    out.seq_len = c.seq_len.clone()
    out.tensor_ptrs = torch.tensor([out.kv[l, j].data_ptr() for l in range(c.cfg.num_layers) for j in range(2)],
                                   dtype=torch.int64, device=c.device)
    return out


def select_cache_batch(cache, indices: torch.Tensor, causal_lm=None):
    """``qwen_flashgrpo_wrapper.py:100-118``: a new cache with the rows ``indices``."""
    if cache is None:
        return None
    return _need_cache(cache).select_rows(torch.as_tensor(indices))


def repeat_interleave_cache(cache, repeats: int, causal_lm=None):
    """``qwen_flashgrpo_wrapper.py:121-138``: every row repeated ``repeats`` times in place
    order (row b becomes rows b*repeats .. b*repeats + repeats - 1)."""
    if cache is None or repeats == 1:
        return cache
    c = _need_cache(cache)
    rows = torch.arange(c.batch, device=c.device).repeat_interleave(int(repeats))
    return c.select_rows(rows)


def cache_seq_length(cache) -> int:
    """``qwen_flashgrpo_wrapper.py:141-147``: the longest committed length."""
    if cache is None:
        return 0
    return int(_need_cache(cache).seq_len.max().item())


def _check_prefix(mask2d: torch.Tensor, seq_len: torch.Tensor, what: str):
    valid = mask2d.to(torch.bool)
    if not torch.equal(valid.long().sum(-1).cpu(), seq_len.long().cpu()):
        raise ValueError(f"{what}: the mask's valid prefix columns must equal each row's committed cache length")


def prefill(causal_lm, input_ids: torch.Tensor, attention_mask: torch.Tensor, *, capacity: int | None = None):
    """``qwen_flashgrpo_wrapper.py:189-199``: causal forward of (left-padded) prompts into
    a new cache. Returns ``{"hidden_states": [B, T, H] (the caller's layout, 0 on
    padding), "logits": None, "past_key_values": KVCache}``."""
    model = as_target_model(causal_lm)
    ids_h = input_ids.detach().cpu()
    mask_h = attention_mask.detach().cpu().bool()
    B, T = ids_h.shape
    lens = mask_h.sum(-1).numpy().astype(np.int64)
    if lens.min() < 1:
        raise ValueError("prefill: every row needs at least one valid token")
    packed = torch.zeros((B, int(lens.max())), dtype=torch.int32)
    for b in range(B):
        packed[b, :lens[b]] = ids_h[b][mask_h[b]].to(torch.int32)
    cap = int(capacity) if capacity is not None else T + PREFILL_HEADROOM
    if cap < int(lens.max()):
        raise ValueError(f"prefill: capacity {cap} below the longest prompt {int(lens.max())}")
    cache = model.new_cache(B, cap)
    every = model.prefill(packed.to(model.device), cache, lengths=lens, return_all=True)
    hidden = torch.zeros((B, T, model.cfg.hidden), dtype=model.dtype, device=model.device)
    cols = torch.from_numpy(np.nonzero(mask_h.numpy())[1]).to(model.device)
    rows = torch.from_numpy(np.nonzero(mask_h.numpy())[0]).to(model.device)
    src = torch.cat([torch.arange(int(n), device=model.device) for n in lens])
    hidden[rows, cols] = every[rows, src]
    return {"hidden_states": hidden, "logits": None, "past_key_values": cache}


def forward_tokens(causal_lm, input_ids: torch.Tensor, full_attention_mask: torch.Tensor, past_key_values,
                   position_ids: torch.Tensor):
    """``qwen_flashgrpo_wrapper.py:202-217``: append n tokens per row after its committed
    prefix (a causal chain among them) and commit the valid ones.

    ``full_attention_mask`` [B, S + n]: its first S columns must mark exactly each row's
    committed length valid; of its last n columns, the valid ones must come first
    (right padding, as the reference's recompute path builds them). Positions are taken
    from ``position_ids`` [B, n]. Returns ``{"hidden_states": [B, n, H], "logits": None,
    "past_key_values": cache}`` with the cache's lengths advanced by the valid tokens."""
    model = as_target_model(causal_lm)
    cache = _need_cache(past_key_values)
    B, n = input_ids.shape
    if full_attention_mask.dim() != 2 or full_attention_mask.shape[0] != B or full_attention_mask.shape[1] < n:
        raise ValueError("forward_tokens: full_attention_mask must be [B, past + n]")
    if B != cache.batch:
        raise ValueError(f"forward_tokens: {B} rows for a cache of {cache.batch}")
    mask = full_attention_mask.to(torch.bool)
    _check_prefix(mask[:, :-n], cache.seq_len, "forward_tokens")
    new = mask[:, -n:].cpu()
    counts = new.long().sum(-1)
    if not torch.equal(new, torch.arange(n)[None, :] < counts[:, None]):
        raise ValueError("forward_tokens: valid new tokens must precede padding in each row")
    seq = cache.seq_len.to(torch.int64).cpu()
    if int((seq + n).max()) > cache.capacity:
        raise ValueError(f"forward_tokens: {n} tokens after {int(seq.max())} exceed the cache capacity "
                         f"{cache.capacity}")
    dev = model.device
    offset = (position_ids.to(torch.int64).cpu() - seq[:, None]).to(torch.int32)
    err = torch.zeros(1, dtype=torch.int32, device=dev)
    hidden = model.forward(input_ids.to(device=dev, dtype=torch.int32).contiguous(), cache,
                           pos_offset=offset.to(dev).contiguous(), anc=None, err_flag=err)
    if int(err.item()):
        raise RuntimeError(f"forward_tokens: a cache write fell outside the cache (flag {int(err.item())})")
    cache.seq_len += counts.to(device=dev, dtype=torch.int32)
    return {"hidden_states": hidden, "logits": None, "past_key_values": cache}


def forward_tree(causal_lm, tree_input_ids: torch.Tensor, tree_attention_mask_4d: torch.Tensor, past_key_values,
                 position_ids: torch.Tensor, *, clone_past: bool = True, compute_logits: bool = True):
    """``qwen_flashgrpo_wrapper.py:220-239`` for a TargetModel or a Hugging Face causal LM
    (see ``flashgrpo_amd.models.target.forward_tree``)."""
    return _target.forward_tree(as_target_model(causal_lm), tree_input_ids, tree_attention_mask_4d,
                                _need_cache(past_key_values), position_ids, clone_past=clone_past,
                                compute_logits=compute_logits)
