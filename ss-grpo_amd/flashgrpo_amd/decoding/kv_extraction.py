"""Accepted-path KV extraction (``flashgrpo/decoding/kv_extraction.py:87-218``).

Every layer's K and V move in one ``fg_kv_path_gather`` launch. Supported
cache forms:

* the build's ``KVCache`` (per-sequence ``seq_len``; rows compact to
  ``seq_len[b] + j`` and ``seq_len`` advances by each row's accepted length);
* the reference's tuple-of-(K, V) layers and transformers ``DynamicCache``
  (``key_cache`` lists or ``layers``): rows ``[old_len, old_len + max_len)``
  are written exactly as the reference writes them, shorter paths padded with
  their last node (``kv_extraction.py:34-51``).
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Sequence

import torch

from ..models.target import KVCache


@dataclass
class KvExtractionResult:
    past_key_values: object
    max_accepted_length: int
    cache_format: str


def _path_rows(accepted_node_indices):
    if accepted_node_indices is None or len(accepted_node_indices) == 0:
        raise ValueError("accepted_node_indices is empty")
    width = max(len(p) for p in accepted_node_indices)
    if width <= 0:
        raise ValueError("accepted_node_indices contains an empty path")
    rows = []
    for p in accepted_node_indices:
        if len(p) == 0:
            raise ValueError("accepted path cannot be empty")
        rows.append([int(n) for n in p] + [int(p[-1])] * (width - len(p)))
    return rows, width


def _layers_of(cache):
    if hasattr(cache, "key_cache"):
        return [(k, v) for k, v in zip(cache.key_cache, cache.value_cache)], "dynamic_key_cache"
    if isinstance(cache, (tuple, list)):
        return [(k, v) for k, v in cache], "legacy_tuple"
    if hasattr(cache, "layers"):
        return [(layer.keys, layer.values) for layer in cache.layers], "dynamic_layers"
    raise TypeError(f"Unsupported cache type for KV path extraction: {type(cache)}")


def _seq_length(cache) -> int:
    if isinstance(cache, KVCache):
        raise TypeError("KVCache has per-row lengths")
    if hasattr(cache, "get_seq_length"):
        return int(cache.get_seq_length())
    layers, _ = _layers_of(cache)
    return int(layers[0][0].shape[-2])


def _gather_layers(tensors, rows, width, old_len):
    from .. import kernels as K

    first = tensors[0]
    B, H, S, D = first.shape
    dev = first.device
    for t in tensors:
        if t.shape != first.shape or t.dtype != first.dtype or t.device != dev:
            raise ValueError("all cache tensors must share shape, dtype and device")
        if t.stride(-1) != 1 or t.stride(-2) != D:
            raise ValueError("cache rows must be contiguous")
    if first.stride(0) != tensors[-1].stride(0) or any(t.stride()[:2] != first.stride()[:2] for t in tensors):
        raise ValueError("cache tensors must share strides")
    ptrs = torch.tensor([t.data_ptr() for t in tensors], dtype=torch.int64, device=dev)
    nodes = torch.tensor(rows, dtype=torch.int32, device=dev)
    acc_len = torch.full((B,), width, dtype=torch.int32, device=dev)
    seq = torch.full((B,), old_len, dtype=torch.int32, device=dev)
    err = torch.zeros(1, dtype=torch.int32, device=dev)
    K.kv_path_gather(ptrs, batch=B, kv_heads=H, head_dim=D, elem_bytes=first.element_size(),
                     strides=(first.stride(0), first.stride(1), first.stride(2)), capacity=S, seq_len=seq,
                     acc_nodes=nodes, acc_len=acc_len, tree_nodes=S - old_len, err_flag=err)
    if int(err.item()):
        raise ValueError("accepted node points outside the tree cache")


def extract_accepted_path_kv(old_past_key_values, tree_past_key_values, accepted_node_indices: Sequence, *,
                             causal_lm=None, cache_format: str = "auto",
                             compact_in_place: bool = True) -> KvExtractionResult:
    """Compact the tree-verified cache to prefix + accepted path (see module docstring)."""
    if isinstance(tree_past_key_values, KVCache):
        cache = tree_past_key_values
        rows, width = _path_rows(accepted_node_indices)
        dev = cache.device
        nodes = torch.tensor(rows, dtype=torch.int32, device=dev)
        lens = torch.tensor([len(p) for p in accepted_node_indices], dtype=torch.int32, device=dev)
        err = torch.zeros(1, dtype=torch.int32, device=dev)
        top = int(cache.seq_len.max().item()) + max(max(r) for r in rows)
        if top >= cache.capacity:
            raise ValueError(f"Accepted node points outside tree cache: max_pos={top}, capacity={cache.capacity}")
        cache.gather_path(cache.seq_len, nodes, lens, cache.capacity - int(cache.seq_len.max().item()),
                          err_flag=err)
        if int(err.item()):
            raise ValueError("accepted node points outside the tree cache")
        cache.seq_len += lens
        return KvExtractionResult(cache, width, "kv_cache_in_place")

    if old_past_key_values is None or tree_past_key_values is None:
        raise ValueError("Both old and tree past_key_values are required")
    old_len = _seq_length(old_past_key_values)
    rows, width = _path_rows(accepted_node_indices)
    layers, fmt = _layers_of(tree_past_key_values)
    tree_len = int(layers[0][0].shape[2])
    top = old_len + max(max(r) for r in rows)
    if top >= tree_len:
        raise ValueError(f"Accepted node points outside tree cache: max_pos={top}, tree_seq_len={tree_len}, "
                         f"old_seq_len={old_len}")
    if not compact_in_place:
        layers = [(k.clone(), v.clone()) for k, v in layers]
    flat = [t for kv in layers for t in kv]
    _gather_layers(flat, rows, width, old_len)
    end = old_len + width
    new_layers = [(k[:, :, :end, :], v[:, :, :end, :]) for k, v in layers]
    if not compact_in_place:
        new_layers = [(k.contiguous(), v.contiguous()) for k, v in new_layers]
    suffix = "_in_place" if compact_in_place else ""
    if fmt == "legacy_tuple":
        return KvExtractionResult(tuple(new_layers), width, "legacy_tuple" + suffix)
    if fmt == "dynamic_key_cache":
        target = tree_past_key_values if compact_in_place else type(tree_past_key_values)()
        target.key_cache = [k for k, _ in new_layers]
        target.value_cache = [v for _, v in new_layers]
        return KvExtractionResult(target, width, "dynamic_key_cache" + suffix)
    target = tree_past_key_values
    for layer, (k, v) in zip(target.layers, new_layers):
        layer.keys, layer.values = k, v
    return KvExtractionResult(target, width, "dynamic_layers" + suffix)
