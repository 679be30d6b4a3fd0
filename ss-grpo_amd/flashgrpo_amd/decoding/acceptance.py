"""Target sampling and exact_target acceptance.

Public names follow ``flashgrpo/decoding/acceptance.py``. Draws come from
``fg_sample_tokens`` / ``fg_accept_walk`` and take caller noise: one uint32
per draw (``noise=``), or, when omitted, values drawn from torch's default
generator on the logits' device, so ``torch.manual_seed`` still governs
reproducibility the way it does for the reference's ``torch.multinomial``.
The noise-to-token rule is the integer inverse CDF documented in
``csrc/sample.hip``; for each row it realises exactly the distribution of
``logits_to_probs`` up to the 2^-40 quantisation of the weights.

``emit_correction=True`` selects the correction-token semantics of
``flashgrpo_b200/decoding/acceptance.py:133-267``: the target sample that
matches no child is returned instead of being discarded.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

from .. import kernels as K


def logits_to_probs(logits: torch.Tensor, *, temperature: float = 1.0, top_p: float | None = 1.0,
                    top_k: int | None = None) -> torch.Tensor:
    """Closed-form target distribution (``acceptance.py:7-31``), torch ops."""
    x = logits.float()
    if temperature is not None and temperature > 0:
        x = x / float(temperature)
    if top_k is not None and 0 < top_k < x.shape[-1]:
        vals, idx = torch.topk(x, k=int(top_k), dim=-1)
        x = torch.full_like(x, torch.finfo(x.dtype).min).scatter(-1, idx, vals)
    probs = F.softmax(x, dim=-1)
    if top_p is not None and 0 < float(top_p) < 1.0:
        sp, si = torch.sort(probs, descending=True, dim=-1)
        drop = torch.roll(torch.cumsum(sp, dim=-1) > float(top_p), shifts=1, dims=-1)
        drop[..., 0] = False
        sp = sp.masked_fill(drop, 0.0)
        sp = sp / sp.sum(dim=-1, keepdim=True).clamp_min(1e-12)
        probs = torch.zeros_like(probs).scatter(-1, si, sp)
    return probs


def _noise(noise, shape, device) -> torch.Tensor:
    """uint32 noise as an int32 tensor of `shape` on `device`."""
    if noise is None:
        u = torch.randint(0, 2 ** 32, shape, dtype=torch.int64, device=device)
    else:
        u = torch.as_tensor(noise, device=device).to(torch.int64).reshape(shape)
    return (u & 0xFFFFFFFF).to(torch.int32) if u.dtype != torch.int32 else u


def sample_from_logits(logits: torch.Tensor, *, do_sample: bool = True, temperature: float = 1.0,
                       top_p: float | None = 1.0, top_k: int | None = None, nucleus_topk_hint: int = 2048,
                       noise=None) -> torch.Tensor:
    """Sample one token per row of ``logits`` (``acceptance.py:34-130``).

    The reference's top-2048 shortlist is an exact shortcut to the full nucleus;
    the device sampler computes the full nucleus directly, so the hint is accepted
    and has no effect on the result.
    """
    del nucleus_topk_hint
    V = int(logits.shape[-1])
    out_shape = logits.shape[:-1]
    flat = logits.reshape(-1, V)
    rows = flat.shape[0]
    greedy = (not do_sample) or temperature == 0
    nz = None if greedy else _noise(noise, (rows, 1), flat.device)
    tok = K.sample_tokens(flat, noise=nz, temperature=temperature, greedy=greedy, top_k=top_k, top_p=top_p)
    return tok.to(torch.long).view(out_shape)


def _walk_inputs(trees, tree_logits, node_to_logit, node_to_logit_cpu, device):
    B = len(trees)
    nmax = max(max(t.node_count, 1) for t in trees)
    toks = torch.zeros((B, nmax), dtype=torch.int32)
    pars = torch.full((B, nmax), -2, dtype=torch.int32)
    nn = torch.zeros(B, dtype=torch.int32)
    depth = 0
    for b, t in enumerate(trees):
        n = t.node_count
        toks[b, :n] = torch.tensor([int(x) for x in t.tokens], dtype=torch.int32)
        pars[b, :n] = torch.tensor([int(x) for x in t.parents], dtype=torch.int32)
        nn[b] = n
        depth = max(depth, max((len(t.ancestors_including_self(i)) for i in range(n)), default=1) - 1)
    V = tree_logits.shape[-1]
    if node_to_logit is None and node_to_logit_cpu is None:
        n_l = tree_logits.shape[1]
        slots = torch.full((B, nmax), -1, dtype=torch.int32)
        for b, t in enumerate(trees):
            slots[b, :min(t.node_count, n_l)] = torch.arange(min(t.node_count, n_l), dtype=torch.int32) + b * n_l
        logits2 = tree_logits.reshape(-1, V)
    else:
        src = node_to_logit_cpu if node_to_logit_cpu is not None else node_to_logit.cpu().tolist()
        slots = torch.full((B, nmax), -1, dtype=torch.int32)
        for b in range(B):
            row = [int(x) for x in src[b]][:nmax]
            slots[b, :len(row)] = torch.tensor(row, dtype=torch.int32)
        logits2 = tree_logits.reshape(-1, V)
    return (toks.to(device), pars.to(device), nn.to(device), slots.to(device), logits2, depth)


@torch.no_grad()
def exact_accept_paths_batch(trees, tree_logits: torch.Tensor, *, do_sample: bool, temperature: float,
                             top_p: float | None, top_k: int | None, node_to_logit: torch.Tensor | None = None,
                             node_to_logit_cpu: list | None = None, noise=None, emit_correction: bool = False):
    """Batched exact_target walk (``acceptance.py:179-260``).

    Returns (accepted_tokens, accepted_nodes, last_parent) lists, plus the
    correction tokens (None where every sample matched) with ``emit_correction``.
    ``noise`` [B, max_depth]: column t is the draw of walk step t.
    """
    device = tree_logits.device
    toks, pars, nn, slots, logits2, depth = _walk_inputs(trees, tree_logits, node_to_logit, node_to_logit_cpu, device)
    B = len(trees)
    greedy = (not do_sample) or temperature == 0
    nz = None
    if not greedy and depth > 0:
        nz = _noise(noise, (B, depth), device)
    err = torch.zeros(1, dtype=torch.int32, device=device)
    w = K.accept_walk(logits2, toks, pars, nn, max_walk_steps=depth, slot_map=slots, noise=nz,
                      temperature=temperature, greedy=greedy, top_k=top_k, top_p=top_p, err_flag=err)
    acc_len = w["acc_len"].cpu().tolist()
    at = w["acc_tokens"].cpu().tolist()
    an = w["acc_nodes"].cpu().tolist()
    last = w["last_node"].cpu().tolist()
    corr = w["correction"].cpu().tolist()
    if int(err.item()) & 2:
        raise RuntimeError("acceptance walk reached a node without target logits")
    tokens = [at[b][:acc_len[b]] for b in range(B)]
    nodes = [an[b][:acc_len[b]] for b in range(B)]
    if len(tokens) != B:
        raise RuntimeError("Batched acceptance produced an invalid batch size")
    if emit_correction:
        return tokens, nodes, last, [None if c < 0 else c for c in corr]
    return tokens, nodes, last


def exact_accept_path(tree, tree_logits: torch.Tensor, *, do_sample: bool, temperature: float,
                      top_p: float | None, top_k: int | None, noise=None, emit_correction: bool = False):
    """Single-tree walk (``acceptance.py:133-176``); tree_logits [N, V] dense."""
    res = exact_accept_paths_batch([tree], tree_logits.unsqueeze(0), do_sample=do_sample, temperature=temperature,
                                   top_p=top_p, top_k=top_k, noise=None if noise is None else [noise],
                                   emit_correction=emit_correction)
    return tuple(r[0] for r in res)
