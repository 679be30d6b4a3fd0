"""Oracle: accepted-path KV extraction.

Test infrastructure only (see ``oracle/__init__.py``).
"""
from __future__ import annotations

import numpy as np


def path_index(accepted_node_indices, old_seq_len):
    """Cache positions of each accepted path, padded with the last node.

    Follows ``flashgrpo/decoding/kv_extraction.py:34-51`` (including its
    ``ValueError`` cases).
    """
    if not accepted_node_indices:
        raise ValueError("accepted_node_indices is empty")
    width = max(len(p) for p in accepted_node_indices)
    if width <= 0:
        raise ValueError("accepted_node_indices contains an empty path")
    rows = []
    for p in accepted_node_indices:
        if not p:
            raise ValueError("accepted path cannot be empty")
        padded = list(p) + [p[-1]] * (width - len(p))
        rows.append([old_seq_len + int(n) for n in padded])
    return np.asarray(rows, dtype=np.int64), width


def extract_layer(tree_tensor, positions, old_seq_len, width, *, in_place=True):
    """Gather the path rows of one [B, H, S, D] tensor into [old, old+width).

    Follows ``flashgrpo/decoding/kv_extraction.py:54-84`` (in place) and
    ``:162-167`` (copy path). Sources are read before any destination is
    written, exactly as ``gather(...).contiguous()`` then ``copy_``.
    """
    t = tree_tensor
    B = t.shape[0]
    if positions.shape[0] != B:
        raise ValueError("accepted path batch != cache batch")
    path = np.stack([t[b][:, positions[b], :] for b in range(B)])  # [B, H, W, D], a copy
    if in_place:
        t[:, :, old_seq_len:old_seq_len + width, :] = path
        return t[:, :, :old_seq_len + width, :]
    return np.concatenate([t[:, :, :old_seq_len, :], path], axis=2)


def extract_accepted_path_kv(old_layers, tree_layers, accepted_node_indices, *, in_place=True):
    """List-of-(K, V) restatement of ``extract_accepted_path_kv``.

    Follows ``flashgrpo/decoding/kv_extraction.py:87-218`` for the legacy
    tuple cache format, including the out-of-range ``ValueError``.
    """
    if old_layers is None or tree_layers is None:
        raise ValueError("Both old and tree past_key_values are required")
    old_len = int(old_layers[0][0].shape[2])
    positions, width = path_index(accepted_node_indices, old_len)
    tree_len = int(tree_layers[0][0].shape[2])
    top = old_len + max(max(int(n) for n in p) for p in accepted_node_indices)
    if top >= tree_len:
        raise ValueError(f"Accepted node points outside tree cache: max_pos={top}, tree_seq_len={tree_len}")
    out = []
    for k, v in tree_layers:
        out.append((extract_layer(k, positions, old_len, width, in_place=in_place),
                    extract_layer(v, positions, old_len, width, in_place=in_place)))
    return out, width


def compact_rows(cache, seq_len, acc_nodes, acc_len):
    """Per-sequence compaction used by the build's contiguous cache.

    ``cache`` is [B, H, S, D]; for each row b the accepted nodes' rows
    ``seq_len[b] + acc_nodes[b][j]`` move to ``seq_len[b] + j`` for j < acc_len[b].
    These are exactly the valid rows of the reference's
    ``[old_len, old_len + max_len)`` block for that sequence.
    """
    return compact_rows_in_place(np.array(cache, copy=True), seq_len, acc_nodes, acc_len)


def compact_rows_in_place(cache, seq_len, acc_nodes, acc_len):
    """``compact_rows`` on ``cache`` itself (only the path rows move, as the reference's
    ``_compact_tree_layer_in_place``, ``kv_extraction.py:70-84``); returns ``cache``."""
    for b in range(cache.shape[0]):
        L = int(acc_len[b])
        src = [int(seq_len[b]) + int(n) for n in acc_nodes[b][:L]]
        rows = cache[b][:, src, :].copy()
        cache[b][:, int(seq_len[b]):int(seq_len[b]) + L, :] = rows
    return cache
