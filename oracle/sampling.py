"""Oracle: supplied-noise target sampler and the exact_target acceptance walk.

Test infrastructure only (see ``oracle/__init__.py``).

The reference draws with ``torch.multinomial`` (``flashgrpo/decoding/acceptance.py:56-60``),
which cannot take caller noise. This build fixes one deterministic
noise-to-token rule that the HIP kernels reproduce bit for bit:

1. ``m = max x`` over the fp32 logits (NaN ignored); ``kt = fp32(2^20 / ln 2)``,
   divided (correctly rounded, once) by T when 0 < T != 1.
2. ``a_i = trunc(min(fp32(fp32(m - x_i) * kt), Z_MAX))``, a fixed-point base-2
   exponent with 20 fraction bits (NaN, -inf and anything 40 octaves below m clamp
   to Z_MAX, whose weight is 0).
3. ``q_i = floor(2^40 * 2^(-a_i / 2^20))`` as uint64, evaluated as
   ``w = T[r] - ((T[r] - T[r+1]) * f >> 10)`` with ``r`` bits 10-19 and ``f`` bits 0-9
   of a_i, ``T[r] = round(2^31 * 2^(-r/1024))``, then ``q = (w << 32) >> (23 + a_i >> 20)``.
   So q_i = 2^40 exp((x_i - m) / T) to within ~1e-6 relative (2^-20 octave steps,
   linear interpolation between 1024 table points); all sums are exact integer sums.
4. Candidate order O = (fp32 key of x_i desc, index asc).  ``top_k`` keeps the
   first k of O.  ``top_p`` keeps O-position j iff the q-mass of the kept
   candidates before j is <= floor(total * tp32 / 2^32), tp32 = floor(top_p * 2^32)
   (the reference rule "keep while preceding cumsum <= top_p",
   ``acceptance.py:62-66``, in exact integers).
5. Draw: ``target = floor(total_kept * u / 2^32)``; the token is the lowest
   vocabulary index among kept candidates whose inclusive q prefix (vocabulary
   order) exceeds ``target``; a row whose kept mass is 0 draws its first maximum.
Greedy (``do_sample`` false or T == 0) is argmax with the first maximum
(``acceptance.py:43-44``).
"""
from __future__ import annotations

from decimal import ROUND_HALF_EVEN, Decimal, localcontext

import numpy as np

from .tree import sort_key32

F32 = np.float32
Q_SHIFT = 40
KT_BASE = F32(1512775.375)           # fp32(2^20 / ln 2)
Z_MAX = F32((41 << 20) - 4)          # a >> 20 = 40: shift 63, weight 0


def exp2_table() -> np.ndarray:
    """T[r] = round(2^31 * 2^(-r / 1024)), r = 0..1024, from 60-digit decimal arithmetic."""
    with localcontext() as ctx:
        ctx.prec = 60
        two = Decimal(2)
        vals = [int((two ** (Decimal(-r) / 1024) * (1 << 31)).to_integral_value(ROUND_HALF_EVEN))
                for r in range(1025)]
    return np.array(vals, dtype=np.uint64)


_TABLE = exp2_table()


def weight_scale(temperature) -> np.float32:
    """kt of step 1: fp32(2^20 / ln 2), divided by T when 0 < T != 1."""
    if temperature is not None and temperature > 0 and F32(temperature) != F32(1.0):
        return F32(KT_BASE / F32(temperature))
    return KT_BASE


def row_max(x) -> np.float32:
    """max x with NaN ignored (-inf for an empty or all-NaN row)."""
    x = np.asarray(x, F32)
    if x.size == 0 or np.all(np.isnan(x)):
        return F32(-np.inf)
    return F32(np.nanmax(x))


def fixed_exponent(x, temperature=None, m=None) -> np.ndarray:
    """a_i of step 2 (uint32)."""
    x = np.asarray(x, F32)
    m = row_max(x) if m is None else F32(m)
    with np.errstate(invalid="ignore", over="ignore"):
        d = (m - x).astype(F32)
        z = np.fmin((d * weight_scale(temperature)).astype(F32), Z_MAX)
    return z.astype(np.uint32)


def quantized_weights(x, temperature=None) -> np.ndarray:
    """q_i of step 3 (uint64) for the logits row x at temperature T."""
    a = fixed_exponent(x, temperature).astype(np.uint64)
    r = (a >> np.uint64(10)) & np.uint64(1023)
    f = a & np.uint64(1023)
    t0 = _TABLE[r]
    w = t0 - (((t0 - _TABLE[r + np.uint64(1)]) * f) >> np.uint64(10))
    return (w << np.uint64(32)) >> ((a >> np.uint64(20)) + np.uint64(23))


def top_p_fixed(top_p) -> int:
    """tp32 = floor(top_p * 2^32); 0 means 'no nucleus cut'."""
    if top_p is None or not (0.0 < float(top_p) < 1.0):
        return 0
    return int(float(top_p) * 4294967296.0)


def kept_mask(x, q, *, top_k=None, top_p=None) -> np.ndarray:
    """Boolean mask of the candidates kept by top-k then top-p (docstring step 4)."""
    x = np.asarray(x, F32)
    V = x.shape[-1]
    key = sort_key32(x)
    idx = np.arange(V, dtype=np.uint64)
    order = np.argsort(~((key << np.uint64(32)) | (np.uint64(0xFFFFFFFF) - idx)), kind="stable")
    n_keep = V
    if top_k is not None and 0 < int(top_k) < V:
        n_keep = int(top_k)
    tp = top_p_fixed(top_p)
    if tp:
        qs = q[order[:n_keep]]
        total = int(qs.sum(dtype=np.uint64))
        thr = (total * tp) >> 32
        before = np.concatenate([[0], np.cumsum(qs, dtype=np.uint64)[:-1]])
        n_keep = int(np.count_nonzero(before <= np.uint64(thr)))
    keep = np.zeros(V, dtype=bool)
    keep[order[:n_keep]] = True
    return keep


def sample_row(x, u32, *, do_sample=True, temperature=1.0, top_p=1.0, top_k=None) -> int:
    """One supplied-noise draw from one logits row (module docstring)."""
    x = np.asarray(x).astype(F32)
    if (not do_sample) or temperature == 0:
        return int(np.argmax(x))
    q = quantized_weights(x, temperature)
    keep = kept_mask(x, q, top_k=top_k, top_p=top_p)
    qk = np.where(keep, q, np.uint64(0))
    total = int(qk.sum(dtype=np.uint64))
    if total == 0:
        return int(np.argmax(np.asarray(x, F32)))
    target = (total * (int(u32) & 0xFFFFFFFF)) >> 32
    cum = np.cumsum(qk, dtype=np.uint64)
    return int(np.argmax(cum > np.uint64(target)))


def sample_rows(logits, noise, **kw) -> np.ndarray:
    logits = np.asarray(logits)
    flat = logits.reshape(-1, logits.shape[-1])
    nz = np.asarray(noise).reshape(-1)
    return np.array([sample_row(flat[i], nz[i], **kw) for i in range(flat.shape[0])], dtype=np.int64)


def token_probabilities(x, *, temperature=1.0, top_p=1.0, top_k=None) -> np.ndarray:
    """Exact probability of each token under the rule, over all 2^32 noise values."""
    x = np.asarray(x).astype(F32)
    q = quantized_weights(x, temperature)
    keep = kept_mask(x, q, top_k=top_k, top_p=top_p)
    qk = [int(v) if k else 0 for v, k in zip(q.tolist(), keep.tolist())]
    total = sum(qk)
    probs = []
    cum = 0
    for w in qk:
        lo = -((-cum << 32) // total)          # ceil(cum * 2^32 / total)
        hi = -((-(cum + w) << 32) // total)
        probs.append((hi - lo) / 4294967296.0)
        cum += w
    return np.array(probs)


def logits_to_probs(logits, *, temperature=1.0, top_p=1.0, top_k=None) -> np.ndarray:
    """Closed-form target distribution, float64.

    Follows ``flashgrpo/decoding/acceptance.py:7-31`` (top-k filter, softmax,
    sorted nucleus with the roll-by-one keep rule, renormalisation).
    """
    x = np.asarray(logits, dtype=np.float64)
    if temperature is not None and temperature > 0:
        x = x / float(temperature)
    if top_k is not None and 0 < top_k < x.shape[-1]:
        kth = np.sort(x, axis=-1)[..., -top_k][..., None]
        x = np.where(x >= kth, x, -np.inf)
    x = x - x.max(axis=-1, keepdims=True)
    p = np.exp(x)
    p = p / p.sum(axis=-1, keepdims=True)
    if top_p is not None and 0 < float(top_p) < 1.0:
        order = np.argsort(-p, axis=-1, kind="stable")
        sp = np.take_along_axis(p, order, -1)
        cum = np.cumsum(sp, axis=-1)
        drop = np.roll(cum > float(top_p), 1, axis=-1)
        drop[..., 0] = False
        sp = np.where(drop, 0.0, sp)
        sp = sp / np.maximum(sp.sum(axis=-1, keepdims=True), 1e-12)
        out = np.zeros_like(p)
        np.put_along_axis(out, order, sp, -1)
        p = out
    return p


# --------------------------------------------------------------------------- counter noise
MASK64 = (1 << 64) - 1


def _mix64(z: int) -> int:
    """SplitMix64 output finalizer (Steele, Lea, Flood 2014)."""
    z &= MASK64
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & MASK64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & MASK64
    return z ^ (z >> 31)


def counter_noise(seed: int, step: int, seq: int, draw: int) -> int:
    """u32 noise keyed by (seed, step, sequence id, draw index)."""
    key = ((int(step) & 0xFFFFFFFF) << 32) | ((int(seq) & 0xFFFFFF) << 8) | (int(draw) & 0xFF)
    h = _mix64(_mix64((int(seed) + 0x9E3779B97F4A7C15) & MASK64) ^ key)
    return h >> 32


def counter_noise_block(seed, step, seq_ids, draws) -> np.ndarray:
    return np.array([[counter_noise(seed, step, s, d) for d in range(draws)] for s in seq_ids], dtype=np.uint64)


# --------------------------------------------------------------------------- acceptance walk
def accept_walk(trees, tree_logits, noise, *, do_sample, temperature, top_p, top_k,
                slots=None, emit_correction=False):
    """exact_target acceptance over a batch of trees with supplied noise.

    Follows ``flashgrpo/decoding/acceptance.py:179-260`` (v1: a sample that
    matches no child is discarded) and, with ``emit_correction``,
    ``flashgrpo_b200/decoding/acceptance.py:184-267`` (it is returned as the
    correction token). ``tree_logits`` is dense [B, N, V] when ``slots`` is None,
    else packed [R, V] addressed by ``slots[b][node]``. ``noise[b][t-1]`` is the
    draw for walk step t (t = 1 for the root's children).
    """
    acc_tok, acc_node, last, corr = [], [], [], []
    for b, t in enumerate(trees):
        toks, nodes, parent, c = [int(t.tokens[0])], [0], 0, None
        step = 0
        while True:
            kids = t.children(parent)
            if not kids:
                break
            row = tree_logits[b][parent] if slots is None else tree_logits[slots[b][parent]]
            tok = sample_row(row, int(noise[b][step]), do_sample=do_sample, temperature=temperature,
                             top_p=top_p, top_k=top_k)
            step += 1
            match = next((k for k in kids if int(t.tokens[k]) == tok), None)
            if match is None:
                c = tok
                break
            toks.append(tok)
            nodes.append(match)
            parent = match
        acc_tok.append(toks)
        acc_node.append(nodes)
        last.append(parent)
        corr.append(c)
    if emit_correction:
        return acc_tok, acc_node, last, corr
    return acc_tok, acc_node, last


def clamp_accepted(tokens, nodes, *, remaining, eos_token_id, old_len, max_length):
    """Length clamp, EOS cut and finished flag for one row.

    Follows ``flashgrpo/decoding/flash_medusa_decoder.py:899-922``.
    """
    keep = max(1, int(remaining))
    tokens = list(tokens)[:keep]
    nodes = list(nodes)[: len(tokens)]
    eos = False
    for i, t in enumerate(tokens):
        if t == eos_token_id:
            tokens, nodes, eos = tokens[: i + 1], nodes[: i + 1], True
            break
    finished = eos or int(old_len) + len(tokens) >= int(max_length)
    return tokens, nodes, finished, eos


def is_finite_row(x) -> bool:
    return bool(np.all(np.isfinite(np.asarray(x, dtype=np.float64))))


def mulhi_u64_u32(total: int, u) -> np.ndarray:
    """floor(total * u / 2^32) for a Python int total < 2^64 and an array of u32, exactly."""
    u = np.asarray(u, dtype=np.uint64)
    hi = np.uint64(int(total) >> 32)
    lo = np.uint64(int(total) & 0xFFFFFFFF)
    return hi * u + ((lo * u) >> np.uint64(32))


def sample_same_row(x, noise, *, temperature=1.0, top_p=1.0, top_k=None) -> np.ndarray:
    """Vectorised ``sample_row`` of one row under many noise values (distribution tests)."""
    x = np.asarray(x).astype(F32)
    q = quantized_weights(x, temperature)
    keep = kept_mask(x, q, top_k=top_k, top_p=top_p)
    qk = np.where(keep, q, np.uint64(0))
    total = int(qk.sum(dtype=np.uint64))
    target = mulhi_u64_u32(total, noise)
    cum = np.cumsum(qk, dtype=np.uint64)
    return np.searchsorted(cum, target, side="right").astype(np.int64)
