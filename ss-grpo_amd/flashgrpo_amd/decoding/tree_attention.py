"""Tree-attention inputs.

``build_tree_attention_inputs`` keeps the signature and outputs of
``flashgrpo/decoding/tree_attention.py:6-67`` (flattened ids, additive
``[B, 1, N, P+N]`` mask, positions, node mask) for callers that want the
materialised mask. The rollout path does not build that mask: it hands
``fg_tree_attention`` one 64-bit ancestor-or-self word per node
(``tree_ancestor_bits``) and applies it to the scores in registers.
"""
from __future__ import annotations

import numpy as np
import torch


def tree_ancestor_bits(trees, max_nodes: int | None = None) -> torch.Tensor:
    """int64 [B, N] bit patterns: bit m of node n set iff m is n or an ancestor of n.

    Padded nodes (n >= tree.node_count) see only themselves, as in the reference.
    """
    nmax = max_nodes or max(max(t.node_count, 1) for t in trees)
    if nmax > 64:
        raise ValueError("trees larger than 64 nodes are not supported")
    out = np.zeros((len(trees), nmax), dtype=np.uint64)
    for b, t in enumerate(trees):
        for n in range(nmax):
            if n < t.node_count:
                m = 0
                for a in t.ancestors_including_self(n):
                    m |= 1 << a
            else:
                m = 1 << n
            out[b, n] = m
    return torch.from_numpy(out.view(np.int64))


def build_tree_attention_inputs(trees, full_attention_mask: torch.Tensor, logical_lengths: torch.Tensor, *,
                                pad_token_id: int, dtype: torch.dtype):
    """(input_ids [B,N], additive mask [B,1,N,P+N], position_ids [B,N], node_mask [B,N])."""
    device = full_attention_mask.device
    B = len(trees)
    nmax = max(max(t.node_count, 1) for t in trees)
    past = full_attention_mask.shape[1]
    ids = torch.full((B, nmax), int(pad_token_id), dtype=torch.long)
    depth = torch.ones((B, nmax), dtype=torch.long)
    valid = torch.zeros((B, nmax), dtype=torch.bool)
    for b, t in enumerate(trees):
        n = t.node_count
        ids[b, :n] = torch.tensor(t.tokens, dtype=torch.long)
        depth[b, :n] = torch.tensor(t.depths, dtype=torch.long)
        valid[b, :n] = True
    bits = tree_ancestor_bits(trees, nmax)
    shifts = torch.arange(nmax, dtype=torch.int64)
    tree_allowed = ((bits[:, :, None] >> shifts[None, None, :]) & 1).bool()
    ids, depth, valid, tree_allowed = (x.to(device) for x in (ids, depth, valid, tree_allowed))
    pos = logical_lengths.to(device=device, dtype=torch.long)[:, None] + depth - 1
    pos = pos.masked_fill(~valid, 0)
    prefix = full_attention_mask.to(device=device, dtype=torch.bool)[:, None, :].expand(B, nmax, past)
    allowed = torch.cat([prefix, tree_allowed], dim=-1)[:, None]
    mask = torch.zeros((B, 1, nmax, past + nmax), dtype=dtype, device=device)
    mask.masked_fill_(~allowed, torch.finfo(dtype).min)
    return ids, mask, pos, valid
