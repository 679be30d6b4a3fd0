"""Torch-facing wrappers over the C ABI (one function per entry point).

Each wrapper checks devices, dtypes and shapes on the host, passes raw
pointers plus torch's current HIP stream, and raises on any error code. All
device work happens in the HIP kernels of ``ss-grpo_amd/csrc``.
"""
from __future__ import annotations

import ctypes as C
import math

import torch

from . import _lib, timing

F32, BF16 = 0, 1


def _call(name: str, *args) -> None:
    if timing.idle():  # no timer installed: launch directly (the context manager costs ~3 us)
        _lib.call(name, *args)
        return
    with timing.launch(name):
        _lib.call(name, *args)
_DT = {torch.float32: F32, torch.bfloat16: BF16}


def dtype_code(t: torch.Tensor) -> int:
    try:
        return _DT[t.dtype]
    except KeyError:
        raise TypeError(f"unsupported dtype {t.dtype}; expected float32 or bfloat16") from None


def _ptr(t):
    return None if t is None else t.data_ptr()


_raw_stream = torch._C._cuda_getCurrentRawStream
_cur_device = torch._C._cuda_getDevice


def _stream() -> int:
    """hipStream_t of torch's current stream on the current device (the two direct
    C calls cost ~1 us; torch.cuda.current_stream() costs ~9 us per launch)."""
    return _raw_stream(_cur_device())


_SCRATCH = {}
_SCRATCH_RETIRED = []


def _scratch(name: str, nbytes: int, device) -> torch.Tensor:
    """A cached uint8 device buffer of at least nbytes for one kind of workspace.
    Launches are ordered on the current stream, so successive calls may share it.
    A buffer outgrown is kept alive: a captured graph may still address it."""
    key = (name, str(device))
    buf = _SCRATCH.get(key)
    if buf is None or buf.numel() < nbytes:
        if buf is not None:
            _SCRATCH_RETIRED.append(buf)
        buf = torch.empty(int(nbytes), dtype=torch.uint8, device=device)
        _SCRATCH[key] = buf
    return buf


def _dev(*ts):
    for t in ts:
        if t is not None and not t.is_cuda:
            raise ValueError("flashgrpo_amd kernels take device tensors (got a CPU tensor)")


def _i32(t, name):
    if t is not None and t.dtype != torch.int32:
        raise TypeError(f"{name} must be int32")


def aligned_rows(x: torch.Tensor) -> torch.Tensor:
    """x itself when its rows start 32-byte aligned with a stride that is a
    multiple of 8 elements (what the row kernels load with 16-byte vectors),
    otherwise a padded copy viewed back to x's shape."""
    x2 = x.reshape(-1, x.shape[-1]) if x.dim() != 2 else x
    if x2.stride(-1) == 1 and x2.stride(0) % 8 == 0 and x2.data_ptr() % 32 == 0:
        return x2
    V = x2.shape[-1]
    pad = torch.empty(x2.shape[0], (V + 7) // 8 * 8, dtype=x2.dtype, device=x2.device)
    pad[:, :V].copy_(x2)
    return pad[:, :V]


def top_p_fixed(top_p) -> int:
    """floor(top_p * 2^32) for 0 < top_p < 1, else 0 (no nucleus cut)."""
    if top_p is None or not (0.0 < float(top_p) < 1.0):
        return 0
    return int(float(top_p) * 4294967296.0)


# ------------------------------------------------------------------ contractions
def medusa_heads(hidden, ln_w, ln_b, fc_w, fc_b, *, eps=1e-5, out=None, out_dtype=None, workspace=None):
    """[heads*B, H] = hidden + SiLU(fc(LayerNorm(hidden))) per head (heads stacked)."""
    _dev(hidden, ln_w, ln_b, fc_w, fc_b)
    B, H = hidden.shape
    heads = fc_w.shape[0]
    if hidden.stride(1) != 1 or fc_w.shape[1:] != (H, H) or not fc_w.is_contiguous() or not fc_b.is_contiguous():
        raise ValueError("medusa_heads: expected hidden [B,H] row-major, fc_w [heads,H,H], fc_b [heads,H]")
    if fc_w.dtype != hidden.dtype or fc_b.dtype != hidden.dtype:
        raise TypeError("medusa_heads: fc weights must share the hidden dtype")
    ln_w = ln_w.float().contiguous()
    ln_b = ln_b.float().contiguous()
    od = out_dtype or hidden.dtype
    if out is None:
        out = torch.empty(heads * B, H, dtype=od, device=hidden.device)
    need = _lib.load().fg_medusa_heads_workspace(B, H, heads, dtype_code(hidden))
    if workspace is None or workspace.numel() * workspace.element_size() < need:
        workspace = torch.empty(need, dtype=torch.uint8, device=hidden.device)
    _call("fg_medusa_heads", _ptr(hidden), dtype_code(hidden), B, H, hidden.stride(0), heads, _ptr(ln_w),
              _ptr(ln_b), float(eps), _ptr(fc_w), _ptr(fc_b), _ptr(out), dtype_code(out), _ptr(workspace),
              workspace.numel() * workspace.element_size(), _stream())
    return out


def lm_head(x, weight, *, row_index=None, row_active=None, out=None, out_dtype=None):
    """out[m] = x[row_index[m] if row_index is given else m] @ weight.T

    row_active (int32 [M], optional): output tiles whose rows are all 0 are skipped."""
    _dev(x, weight, row_index, row_active)
    _i32(row_index, "row_index")
    _i32(row_active, "row_active")
    K = x.shape[-1]
    x2 = x.reshape(-1, K)
    if x2.stride(1) != 1 or weight.stride(1) != 1 or weight.shape[1] != K:
        raise ValueError("lm_head: operands must be K-contiguous with matching K")
    if x.dtype != weight.dtype:
        raise TypeError("lm_head: x and weight dtypes differ")
    M = row_index.numel() if row_index is not None else x2.shape[0]
    N = weight.shape[0]
    od = out_dtype or x.dtype
    if out is None:
        out = torch.empty(M, N, dtype=od, device=x.device)
    if M == 0:
        return out
    _call("fg_lm_head", _ptr(x2), dtype_code(x), M, K, x2.stride(0), _ptr(row_index), _ptr(row_active),
          _ptr(weight), weight.stride(0), N, _ptr(out), dtype_code(out), out.stride(0), _stream())
    return out


def lm_head_parts(vocab):
    """Row maxima parts per row that ``lm_head_topk(..., parts=...)`` writes."""
    return int(_lib.load().fg_lm_head_topk_parts(int(vocab)))


def lm_head_topk(x, weight, kmax=0, *, row_index=None, row_active=None, out=None, out_dtype=None,
                 logits=True, stats=False, sanitize=False, workspace=None, parts=None):
    """Tied LM head over <= 256 rows (bf16) on the weight-streaming kernel, with the
    per-row top-kmax candidates fused (``fg_lm_head_topk``).

    Returns (logits [M, N] or None, tokens int32 [M, kmax] or None, scores fp32 [M, kmax]
    or None, stats fp32 [M, 2] or None); the candidates and stats equal
    ``medusa_topk(logits, kmax, stats=..., sanitize=...)`` on the bf16 logits.
    ``parts`` (kmax 0): a (part_max fp32, part_key int64) pair of [M, lm_head_parts(N)]
    tensors that receive each row's per-workgroup maxima (for ``walk_step``).
    """
    _dev(x, weight, row_index, row_active)
    _i32(row_index, "row_index")
    _i32(row_active, "row_active")
    K = x.shape[-1]
    x2 = x.reshape(-1, K)
    if x2.dtype != torch.bfloat16 or weight.dtype != torch.bfloat16:
        raise TypeError("lm_head_topk: x and weight must be bf16")
    if x2.stride(1) != 1 or weight.stride(1) != 1 or weight.shape[1] != K:
        raise ValueError("lm_head_topk: operands must be K-contiguous with matching K")
    if (x2.numel() + x2.storage_offset()) * 2 >= 1 << 32:
        raise ValueError("lm_head_topk: x must span less than 4 GiB")
    M = row_index.numel() if row_index is not None else x2.shape[0]
    N = weight.shape[0]
    dev = x.device
    if logits and out is None:
        out = torch.empty(M, N, dtype=out_dtype or torch.bfloat16, device=dev)
    elif not logits:
        out = None
    elif out is not None:
        _dev(out)
        if out.dtype not in (torch.bfloat16, torch.float32) or (out_dtype is not None and out.dtype != out_dtype):
            raise TypeError("lm_head_topk: out must be bf16 or fp32 (and match out_dtype)")
        if out.dim() != 2 or tuple(out.shape) != (M, N) or out.stride(1) != 1 or out.stride(0) < N:
            raise ValueError(f"lm_head_topk: out must be a [{M}, {N}] view with unit column stride")
        if out.stride(0) % 4 == 0 and out.data_ptr() % (4 * out.element_size()):
            raise ValueError("lm_head_topk: out rows with a stride of 4k elements need a base aligned to 4 columns")
    tok = torch.empty(M, kmax, dtype=torch.int32, device=dev) if kmax else None
    sc = torch.empty(M, kmax, dtype=torch.float32, device=dev) if kmax else None
    st = torch.empty(M, 2, dtype=torch.float32, device=dev) if kmax and stats else None
    if M == 0:
        return out, tok, sc, st
    ws_bytes = 0
    if kmax:
        need = _lib.load().fg_lm_head_topk_workspace(M, N, kmax)
        if workspace is None or workspace.numel() * workspace.element_size() < need:
            workspace = torch.empty(need, dtype=torch.uint8, device=dev)
        ws_bytes = workspace.numel() * workspace.element_size()
    else:
        workspace = None
    pmax = pkey = None
    if parts is not None:
        pmax, pkey = parts
        P = lm_head_parts(N)
        if (kmax or pmax.dtype != torch.float32 or pkey.dtype != torch.int64 or tuple(pmax.shape) != (M, P)
                or tuple(pkey.shape) != (M, P) or not pmax.is_contiguous() or not pkey.is_contiguous()):
            raise ValueError(f"lm_head_topk: parts must be contiguous fp32 / int64 [{M}, {P}] with kmax 0")
    _call("fg_lm_head_topk", _ptr(x2), M, K, x2.stride(0), _ptr(row_index), _ptr(row_active), _ptr(weight),
          weight.stride(0), N, _ptr(out), dtype_code(out) if out is not None else 1,
          out.stride(0) if out is not None else N, int(kmax), int(bool(sanitize)), _ptr(tok), _ptr(sc), _ptr(st),
          _ptr(pmax), _ptr(pkey), _ptr(workspace), ws_bytes, _stream())
    return out, tok, sc, st


# ------------------------------------------------------------------ tree construction
def medusa_topk(logits, kmax, *, stats=False, sanitize=False, workspace=None):
    """Top-kmax candidates per row ranked (value desc, index asc).

    Returns (tokens int32 [R, kmax], scores fp32 [R, kmax], stats fp32 [R, 2] or None)
    where stats holds (row max, row logsumexp). ``sanitize`` ranks
    nan_to_num(logits, nan=-1e9, posinf=1e9, neginf=-1e9) (chain proposals).
    """
    _dev(logits)
    logits = aligned_rows(logits)
    R, V = logits.shape
    tok = torch.empty(R, kmax, dtype=torch.int32, device=logits.device)
    sc = torch.empty(R, kmax, dtype=torch.float32, device=logits.device)
    st = torch.empty(R, 2, dtype=torch.float32, device=logits.device) if stats else None
    need = _lib.load().fg_medusa_topk_workspace(R, V, kmax)
    if workspace is None or workspace.numel() * workspace.element_size() < need:
        workspace = torch.empty(need, dtype=torch.uint8, device=logits.device)
    _call("fg_medusa_topk", _ptr(logits), dtype_code(logits), logits.stride(0), R, V, kmax, int(bool(sanitize)),
          _ptr(tok), _ptr(sc), _ptr(st), _ptr(workspace), workspace.numel() * workspace.element_size(), _stream())
    return tok, sc, st


def tree_layout(cand_tokens, cand_scores, batch, roots, node_depth, node_rank, num_nodes, *, out_tokens=None,
                out_scores=None):
    _dev(cand_tokens, cand_scores, roots, node_depth, node_rank)
    for t, n in ((cand_tokens, "cand_tokens"), (roots, "roots"), (node_depth, "node_depth"), (node_rank, "node_rank")):
        _i32(t, n)
    dev = roots.device
    if out_tokens is None:
        out_tokens = torch.empty(batch, num_nodes, dtype=torch.int32, device=dev)
    if out_scores is None:
        out_scores = torch.empty(batch, num_nodes, dtype=torch.float32, device=dev)
    kstride = cand_tokens.shape[-1] if cand_tokens is not None else 0
    _call("fg_tree_layout", _ptr(cand_tokens), _ptr(cand_scores), kstride, batch, _ptr(roots), _ptr(node_depth),
              _ptr(node_rank), num_nodes, _ptr(out_tokens), _ptr(out_scores), out_tokens.stride(0), _stream())
    return out_tokens, out_scores


def sparse_tree_layout(cand_tokens, cand_scores, batch, roots, nodes_by_head, *, vocab, budget, num_nodes,
                       temperature=1.0, diversity_penalty=0.0, head3_gate=None, scores=False):
    """Sparse asymmetric trees on the device (``fg_sparse_tree_layout``).

    cand_tokens/cand_scores: [heads*batch, kstride] top-k lists (head-major rows).
    Returns a dict of [batch, num_nodes] int32 ``tokens``, ``parents``, ``depth``,
    ``pos_offset``, ``n_children``, int64 ``anc`` bit masks, ``n_nodes`` [batch], and
    with ``scores`` the fp64 path scores [batch, num_nodes].
    """
    _dev(cand_tokens, cand_scores, roots, head3_gate)
    _i32(cand_tokens, "cand_tokens")
    _i32(roots, "roots")
    nodes = [int(n) for n in nodes_by_head]
    if not nodes:
        raise ValueError("sparse_tree_layout: no heads")
    if cand_tokens.shape[0] < min(len(nodes), 3) * batch or cand_scores.shape != cand_tokens.shape:
        raise ValueError("sparse_tree_layout: candidate rows missing")
    if not (cand_tokens.is_contiguous() and cand_scores.is_contiguous() and cand_scores.dtype == torch.float32):
        raise ValueError("sparse_tree_layout: contiguous int32 tokens and fp32 scores required")
    if head3_gate is not None:
        if head3_gate.dtype not in (torch.bool, torch.uint8) or head3_gate.numel() != batch:
            raise ValueError("sparse_tree_layout: head3_gate must be bool/uint8 [batch]")
        head3_gate = head3_gate.contiguous().view(torch.uint8)
    dev = roots.device
    i32 = dict(dtype=torch.int32, device=dev)
    out = dict(tokens=torch.empty(batch, num_nodes, **i32), parents=torch.empty(batch, num_nodes, **i32),
               depth=torch.empty(batch, num_nodes, **i32), pos_offset=torch.empty(batch, num_nodes, **i32),
               anc=torch.empty(batch, num_nodes, dtype=torch.int64, device=dev),
               n_children=torch.empty(batch, num_nodes, **i32), n_nodes=torch.empty(batch, **i32),
               scores=torch.empty(batch, num_nodes, dtype=torch.float64, device=dev) if scores else None)
    nodes_arr = (C.c_int32 * len(nodes))(*nodes)
    _call("fg_sparse_tree_layout", _ptr(cand_tokens), _ptr(cand_scores), cand_tokens.shape[1], batch, int(vocab),
          _ptr(roots), _ptr(head3_gate), C.cast(nodes_arr, C.c_void_p), len(nodes), int(budget), float(temperature),
          float(diversity_penalty), num_nodes, _ptr(out["tokens"]), _ptr(out["parents"]), _ptr(out["depth"]),
          _ptr(out["pos_offset"]), _ptr(out["anc"]), _ptr(out["n_children"]), _ptr(out["n_nodes"]),
          _ptr(out["scores"]), _stream())
    return out


# ------------------------------------------------------------------ verify forward pieces
def rope_kv_write(qkv, *, batch, num_nodes, q_heads, kv_heads, head_dim, seq_len, pos_offset, inv_freq, q_out,
                  k_cache, v_cache, row_map=None, err_flag=None):
    _dev(qkv, seq_len, pos_offset, inv_freq, q_out, k_cache, v_cache, row_map)
    _i32(seq_len, "seq_len")
    _i32(pos_offset, "pos_offset")
    _i32(row_map, "row_map")
    if k_cache.stride(-1) != 1 or k_cache.stride(-2) != head_dim:
        raise ValueError("rope_kv_write: cache rows must be contiguous [.., capacity, d]")
    if v_cache.stride() != k_cache.stride() or v_cache.shape != k_cache.shape or v_cache.dtype != k_cache.dtype:
        raise ValueError("rope_kv_write: v_cache must have k_cache's shape, strides and dtype")
    width = (q_heads + 2 * kv_heads) * head_dim
    if qkv.dtype != k_cache.dtype or qkv.stride(-1) != 1 or qkv.shape[-1] < width or \
            qkv.numel() // qkv.shape[-1] != batch * num_nodes:
        raise ValueError(f"rope_kv_write: qkv must hold {batch * num_nodes} rows of >= {width} unit-stride values "
                         "in the cache dtype")
    if not q_out.is_contiguous() or q_out.numel() != batch * num_nodes * q_heads * head_dim or \
            q_out.dtype != k_cache.dtype:
        raise ValueError("rope_kv_write: q_out must be a contiguous [batch * num_nodes, q_heads, d] tensor")
    if pos_offset.dim() == 2:
        if tuple(pos_offset.shape) != (batch, num_nodes) or not pos_offset.is_contiguous():
            raise ValueError("rope_kv_write: per-sequence pos_offset must be contiguous [batch, num_nodes]")
        pos_stride = num_nodes
    else:
        if pos_offset.numel() < num_nodes:
            raise ValueError("rope_kv_write: pos_offset shorter than num_nodes")
        pos_stride = 0
    _call("fg_rope_kv_write", _ptr(qkv), dtype_code(qkv), qkv.stride(0), batch, num_nodes, q_heads, kv_heads,
              head_dim, _ptr(seq_len), _ptr(pos_offset), pos_stride, _ptr(inv_freq), _ptr(q_out), _ptr(k_cache),
              _ptr(v_cache),
              k_cache.stride(0), k_cache.stride(1), k_cache.shape[-2], _ptr(row_map), _ptr(err_flag), _stream())


def tree_attention(q, k_cache, v_cache, *, seq_len, anc, num_nodes, q_heads, kv_heads, head_dim, out=None,
                   row_map=None, scale=None):
    """q [B, N, Hq, d]; caches [Bc, Hkv, S, d]; anc uint64 as int64 [B, N] or [N], or None for a
    causal chain of new keys (node n sees new keys 0..n)."""
    _dev(q, k_cache, v_cache, seq_len, anc, row_map)
    _i32(seq_len, "seq_len")
    if anc is not None and anc.dtype != torch.int64:
        raise TypeError("anc must be int64 (bit pattern of the uint64 masks)")
    B = q.shape[0]
    if out is None:
        out = torch.empty_like(q)
    anc_stride = 0 if anc is None or anc.dim() == 1 else anc.stride(0)
    scale = 1.0 / math.sqrt(head_dim) if scale is None else scale
    capacity = k_cache.shape[2]
    ws, ws_bytes = None, 0
    if q.dtype == torch.bfloat16:
        need = _lib.load().fg_tree_attention_workspace(B, num_nodes, q_heads, kv_heads, head_dim, capacity)
        if need:
            ws = _scratch("tree_attention", need, q.device)
            ws_bytes = ws.numel()
    _call("fg_tree_attention", _ptr(q), _ptr(out), _ptr(k_cache), _ptr(v_cache), dtype_code(q), B, num_nodes,
          q_heads, kv_heads, head_dim, k_cache.stride(0), k_cache.stride(1), capacity, _ptr(seq_len),
          _ptr(row_map), _ptr(anc), anc_stride, float(scale), _ptr(ws), ws_bytes, _stream())
    return out


def rmsnorm(x, weight, eps, *, delta=None, out=None):
    """RMSNorm(x [+ delta]) * weight over the last dimension (``fg_rmsnorm``); with delta the
    sum is written back to x first. x, delta and out contiguous, one dtype, one shape."""
    _dev(x, weight, delta)
    H = x.shape[-1]
    rows = x.numel() // H
    if not x.is_contiguous() or weight.numel() != H or weight.dtype != x.dtype or not weight.is_contiguous():
        raise ValueError("rmsnorm: x must be contiguous and weight a contiguous [H] tensor of its dtype")
    if delta is not None and (delta.shape != x.shape or delta.dtype != x.dtype or not delta.is_contiguous()):
        raise ValueError("rmsnorm: delta must be a contiguous tensor of x's shape and dtype")
    if out is None:
        out = torch.empty_like(x)
    elif out.shape != x.shape or out.dtype != x.dtype or not out.is_contiguous():
        raise ValueError("rmsnorm: out must be a contiguous tensor of x's shape and dtype")
    if rows == 0:
        return out
    _call("fg_rmsnorm", _ptr(x), _ptr(delta), _ptr(weight), _ptr(out), dtype_code(x), rows, H, float(eps),
              _stream())
    return out


def swiglu(gate_up, *, out=None):
    """SiLU(gate_up[:, :F]) * gate_up[:, F:] (``fg_swiglu``): gate_up a contiguous [rows, 2F]
    tensor (F a multiple of 8), out a contiguous [rows, F] tensor of the same dtype."""
    _dev(gate_up)
    if gate_up.dim() != 2 or gate_up.shape[1] % 16 or not gate_up.is_contiguous():
        raise ValueError("swiglu: gate_up must be a contiguous [rows, 2F] tensor with F a multiple of 8")
    rows, two_f = gate_up.shape
    F = two_f // 2
    if out is None:
        out = torch.empty(rows, F, dtype=gate_up.dtype, device=gate_up.device)
    elif tuple(out.shape) != (rows, F) or out.dtype != gate_up.dtype or not out.is_contiguous():
        raise ValueError(f"swiglu: out must be a contiguous [{rows}, {F}] tensor of the input dtype")
    if rows == 0:
        return out
    _call("fg_swiglu", _ptr(gate_up), _ptr(out), dtype_code(gate_up), rows, F, _stream())
    return out


def chain_cell_norm(state, token, state_w, state_b, token_w, token_b, eps, *, out=None):
    """[rows, 2H] = [LayerNorm(state) * state_w + state_b, LayerNorm(token) * token_w + token_b]
    (``fg_chain_cell_norm``): the ChainDraftCell's two normalised inputs side by side. state and
    token [rows, H] in one dtype (unit column stride), the affine weights [H] in that dtype."""
    _dev(state, token, state_w, state_b, token_w, token_b)
    rows, H = state.shape
    if tuple(token.shape) != (rows, H) or token.dtype != state.dtype or state.stride(1) != 1 or token.stride(1) != 1:
        raise ValueError("chain_cell_norm: state and token must be [rows, H] of one dtype with unit column stride")
    ws = [t.contiguous() for t in (state_w, state_b, token_w, token_b)]
    if any(t.dtype != state.dtype or t.numel() != H for t in ws):
        raise ValueError("chain_cell_norm: affine weights must be [H] in the row dtype")
    if out is None:
        out = torch.empty(rows, 2 * H, dtype=state.dtype, device=state.device)
    elif tuple(out.shape) != (rows, 2 * H) or not out.is_contiguous() or out.dtype != state.dtype:
        raise ValueError("chain_cell_norm: out must be a contiguous [rows, 2H] tensor of the row dtype")
    _call("fg_chain_cell_norm", _ptr(state), state.stride(0), _ptr(token), token.stride(0), dtype_code(state), rows, H,
          *[_ptr(t) for t in ws], float(eps), _ptr(out), _stream())
    return out


def gate_up_swiglu_ok(x, w) -> bool:
    """Whether fg_gate_up_swiglu takes x [rows, hidden] and w [2*inter, hidden] as they are:
    bf16 on the GPU, hidden a multiple of 64, inter a multiple of 4, unit column strides and
    16-byte aligned rows."""
    if not (x.is_cuda and x.dtype == torch.bfloat16 and w.dtype == torch.bfloat16 and x.dim() == 2 and w.dim() == 2):
        return False
    H = x.shape[1]
    if H == 0 or H % 64 or w.shape[1] != H or w.shape[0] % 8 or x.shape[0] == 0:
        return False
    if x.stride(1) != 1 or w.stride(1) != 1 or x.stride(0) % 8 or w.stride(0) % 8:
        return False
    return x.data_ptr() % 16 == 0 and w.data_ptr() % 16 == 0


def gate_up_swiglu(x, w, *, out=None, tile_rows=0):
    """SiLU(x . w[:I]^T) * (x . w[I:]^T) with both projections rounded to bf16 first, as one GEMM
    (``fg_gate_up_swiglu``): x [rows, H] bf16, w [2I, H] bf16 (gate rows, then up rows) ->
    [rows, I] bf16. tile_rows: 0 (the kernel's choice of 192 / 256), 64, 128, 192 or 256."""
    _dev(x, w)
    if not gate_up_swiglu_ok(x, w):
        raise ValueError("gate_up_swiglu: needs bf16 x [rows, H] and w [2I, H] with H % 64 == 0, I % 4 == 0, "
                         "unit column strides and 16-byte aligned rows")
    rows, H = x.shape
    inter = w.shape[0] // 2
    if out is None:
        out = torch.empty(rows, inter, dtype=torch.bfloat16, device=x.device)
    elif out.dtype != torch.bfloat16 or tuple(out.shape) != (rows, inter) or out.stride(1) != 1:
        raise ValueError(f"gate_up_swiglu: out must be bf16 [{rows}, {inter}] with unit column stride")
    _call("fg_gate_up_swiglu", _ptr(x), x.stride(0), _ptr(w), w.stride(0), _ptr(out), out.stride(0), rows, inter, H,
          int(tile_rows), _stream())
    return out


LINEAR_TILES = (64, 128)


def linear_splits(hidden: int, splits: int) -> int:
    """The largest split count <= ``splits`` that gives every split of ``hidden / 64``
    k-steps at least one (the rule fg_linear_parts checks)."""
    nk = hidden // 64
    s = max(1, min(int(splits), nk))
    while s > 1 and -(-nk // -(-nk // s)) != s:
        s -= 1
    return s


def linear_ok(x, w) -> bool:
    """Whether fg_linear_parts takes x [rows, K] and w [N, K] as they are: bf16 on the GPU,
    K a multiple of 64, N a multiple of 4, unit column strides and 16-byte aligned rows."""
    if not (x.is_cuda and x.dtype == torch.bfloat16 and w.dtype == torch.bfloat16 and x.dim() == 2 and w.dim() == 2):
        return False
    K_ = x.shape[1]
    if K_ == 0 or K_ % 64 or w.shape[1] != K_ or w.shape[0] % 4 or x.shape[0] == 0:
        return False
    if x.stride(1) != 1 or w.stride(1) != 1 or x.stride(0) % 8 or w.stride(0) % 8:
        return False
    return x.data_ptr() % 16 == 0 and w.data_ptr() % 16 == 0 and x.stride(0) < (1 << 22) and w.stride(0) < (1 << 22)


def linear_parts(x, w, *, splits=1, tile=(128, 128), stages=0, out=None):
    """Split-K partial products of x [rows, K] . w [N, K]^T (``fg_linear_parts``): fp32
    [splits, rows, N] whose sum over the first dimension (in order) is the projection.
    ``splits`` must satisfy the kernel's rule (see ``linear_splits``); ``stages``: k-steps in
    the kernel's LDS ring (2-4, 0 for 4)."""
    _dev(x, w)
    if not linear_ok(x, w):
        raise ValueError("linear_parts: needs bf16 x [rows, K] and w [N, K] with K % 64 == 0, N % 4 == 0, "
                         "unit column strides and 16-byte aligned rows")
    rows, K_ = x.shape
    N = w.shape[0]
    tm, tn = (int(t) for t in tile)
    if tm not in LINEAR_TILES or tn not in LINEAR_TILES:
        raise ValueError(f"linear_parts: tile sizes must be in {LINEAR_TILES}")
    if int(stages) not in (0, 2, 3, 4):
        raise ValueError("linear_parts: stages must be 0, 2, 3 or 4")
    if linear_splits(K_, splits) != int(splits):
        raise ValueError(f"linear_parts: {splits} splits leave a split of {K_ // 64} k-steps empty")
    shape = (int(splits), rows, N)
    if out is None:
        out = torch.empty(shape, dtype=torch.float32, device=x.device)
    elif out.dtype != torch.float32 or tuple(out.shape) != shape or not out.is_contiguous() or out.data_ptr() % 16:
        raise ValueError(f"linear_parts: out must be a contiguous 16-byte aligned fp32 {list(shape)} tensor")
    _call("fg_linear_parts", _ptr(x), x.stride(0), _ptr(w), w.stride(0), _ptr(out), rows, N, K_, int(splits), tm, tn,
          int(stages), _stream())
    return out


def residual_rmsnorm_parts(parts, x, weight, eps, *, out=None):
    """x <- bf16(x + bf16(parts.sum(0))) in place, then RMSNorm(x) * weight
    (``fg_residual_rmsnorm_parts``): parts fp32 [S, rows, H], x bf16 [rows, H]."""
    _dev(parts, x, weight)
    S, rows, H = parts.shape
    if parts.dtype != torch.float32 or not parts.is_contiguous():
        raise ValueError("residual_rmsnorm_parts: parts must be contiguous fp32 [S, rows, H]")
    if x.dtype != torch.bfloat16 or tuple(x.shape) != (rows, H) or x.stride(1) != 1:
        raise ValueError(f"residual_rmsnorm_parts: x must be bf16 [{rows}, {H}] with unit column stride")
    if weight.dtype != torch.bfloat16 or weight.numel() != H or not weight.is_contiguous():
        raise ValueError("residual_rmsnorm_parts: weight must be a contiguous bf16 [H] tensor")
    if out is None:
        out = torch.empty(rows, H, dtype=torch.bfloat16, device=x.device)
    elif out.dtype != torch.bfloat16 or tuple(out.shape) != (rows, H) or out.stride(1) != 1:
        raise ValueError(f"residual_rmsnorm_parts: out must be bf16 [{rows}, {H}] with unit column stride")
    _call("fg_residual_rmsnorm_parts", _ptr(parts), S, rows, H, _ptr(x), x.stride(0), _ptr(weight), float(eps),
          _ptr(out), out.stride(0), _stream())
    return out


def rope_kv_write_parts(parts, bias, *, batch, num_nodes, q_heads, kv_heads, head_dim, seq_len, pos_offset,
                        inv_freq, q_out, k_cache, v_cache, row_map=None, err_flag=None):
    """``rope_kv_write`` with the qkv rows given as split-K parts fp32 [S, batch*num_nodes,
    (q_heads + 2 kv_heads) * head_dim] plus the projection's bias (or None), each value
    rounded to the cache dtype after the sum (``fg_rope_kv_write_parts``)."""
    _dev(parts, bias, seq_len, pos_offset, inv_freq, q_out, k_cache, v_cache, row_map)
    _i32(seq_len, "seq_len")
    _i32(pos_offset, "pos_offset")
    _i32(row_map, "row_map")
    width = (q_heads + 2 * kv_heads) * head_dim
    if parts.dtype != torch.float32 or not parts.is_contiguous() or tuple(parts.shape[1:]) != (batch * num_nodes,
                                                                                                width):
        raise ValueError(f"rope_kv_write_parts: parts must be contiguous fp32 [S, {batch * num_nodes}, {width}]")
    if bias is not None and (bias.dtype != k_cache.dtype or bias.numel() != width or not bias.is_contiguous()):
        raise ValueError("rope_kv_write_parts: bias must be a contiguous [width] tensor of the cache dtype")
    if k_cache.stride(-1) != 1 or k_cache.stride(-2) != head_dim:
        raise ValueError("rope_kv_write_parts: cache rows must be contiguous [.., capacity, d]")
    if pos_offset.dim() == 2:
        if tuple(pos_offset.shape) != (batch, num_nodes) or not pos_offset.is_contiguous():
            raise ValueError("rope_kv_write_parts: per-sequence pos_offset must be contiguous [batch, num_nodes]")
        pos_stride = num_nodes
    else:
        if pos_offset.numel() < num_nodes:
            raise ValueError("rope_kv_write_parts: pos_offset shorter than num_nodes")
        pos_stride = 0
    _call("fg_rope_kv_write_parts", _ptr(parts), parts.shape[0], _ptr(bias), dtype_code(k_cache), batch, num_nodes,
          q_heads, kv_heads, head_dim, _ptr(seq_len), _ptr(pos_offset), pos_stride, _ptr(inv_freq), _ptr(q_out),
          _ptr(k_cache), _ptr(v_cache), k_cache.stride(0), k_cache.stride(1), k_cache.shape[-2], _ptr(row_map),
          _ptr(err_flag), _stream())


def rope_pair_rows(t, q_heads, kv_heads, head_dim):
    """The rows (dim 0) of a q/k/v projection weight [width, K] or bias [width] in the order
    ``fg_linear_rope_kv_write`` takes: each q and k head's rows pair-interleaved (row 2j holds the
    head's row j, row 2j + 1 its row j + head_dim/2), the v heads' rows in order. A new tensor."""
    d, h = int(head_dim), int(q_heads) + int(kv_heads)
    if d % 2 or t.shape[0] != (h + int(kv_heads)) * d:
        raise ValueError("rope_pair_rows: rows must be (q_heads + 2 kv_heads) * head_dim with an even head_dim")
    qk = t[:h * d].reshape(h, 2, d // 2, *t.shape[1:]).transpose(1, 2).reshape(h * d, *t.shape[1:])
    return torch.cat([qk, t[h * d:]]).contiguous()


def rope_cos_sin(*, batch, num_nodes, head_dim, seq_len, pos_offset, inv_freq, out=None):
    """fp32 [batch*num_nodes, head_dim/2, 2]: (cos, sin) of each row's rotary angles rounded to bf16
    (``fg_rope_cos_sin``), the table ``linear_rope_kv_write`` reads."""
    _dev(seq_len, pos_offset, inv_freq, out)
    _i32(seq_len, "seq_len")
    _i32(pos_offset, "pos_offset")
    pos_stride = _pos_stride(pos_offset, batch, num_nodes, "rope_cos_sin")
    shape = (batch * num_nodes, head_dim // 2, 2)
    if out is None:
        out = torch.empty(shape, dtype=torch.float32, device=seq_len.device)
    elif out.dtype != torch.float32 or tuple(out.shape) != shape or not out.is_contiguous():
        raise ValueError(f"rope_cos_sin: out must be a contiguous fp32 {list(shape)} tensor")
    _call("fg_rope_cos_sin", _ptr(seq_len), _ptr(pos_offset), pos_stride, _ptr(inv_freq), batch, num_nodes, head_dim,
          _ptr(out), _stream())
    return out


def _pos_stride(pos_offset, batch, num_nodes, what):
    if pos_offset.dim() == 2:
        if tuple(pos_offset.shape) != (batch, num_nodes) or not pos_offset.is_contiguous():
            raise ValueError(f"{what}: per-sequence pos_offset must be contiguous [batch, num_nodes]")
        return num_nodes
    if pos_offset.numel() < num_nodes:
        raise ValueError(f"{what}: pos_offset shorter than num_nodes")
    return 0


def linear_rope_kv_write(x, w_pairs, bias_pairs, *, tile=(64, 64), stages=0, batch, num_nodes, q_heads, kv_heads,
                         head_dim, seq_len, q_out, k_cache, v_cache, cos_sin=None, pos_offset=None, inv_freq=None,
                         row_map=None, err_flag=None):
    """The q/k/v projection x [batch*num_nodes, K] . w^T with the bias, rotary embedding and KV-slot
    write in the GEMM epilogue (``fg_linear_rope_kv_write``): the weight and bias given in
    ``rope_pair_rows`` order, the rows' rotary table ``cos_sin`` (``rope_cos_sin``; made here from
    pos_offset and inv_freq when not given); q rows to q_out [batch*num_nodes, q_heads, d], k / v
    rows to their cache slots, bit for bit as ``linear_parts`` (one split) + ``rope_kv_write_parts``."""
    _dev(x, w_pairs, bias_pairs, seq_len, cos_sin, q_out, k_cache, v_cache, row_map)
    _i32(seq_len, "seq_len")
    _i32(row_map, "row_map")
    width = (q_heads + 2 * kv_heads) * head_dim
    if not linear_ok(x, w_pairs) or w_pairs.shape[0] != width or x.shape[0] != batch * num_nodes:
        raise ValueError(f"linear_rope_kv_write: needs bf16 x [{batch * num_nodes}, K] and w [{width}, K] with "
                         "K % 64 == 0, unit column strides and 16-byte aligned rows")
    if bias_pairs is not None and (bias_pairs.dtype != torch.bfloat16 or bias_pairs.numel() != width or
                                   not bias_pairs.is_contiguous()):
        raise ValueError("linear_rope_kv_write: bias must be a contiguous bf16 [width] tensor")
    tm, tn = (int(t) for t in tile)
    if tm not in LINEAR_TILES or tn not in LINEAR_TILES or int(stages) not in (0, 2, 3, 4):
        raise ValueError(f"linear_rope_kv_write: tiles in {LINEAR_TILES}, stages 0, 2, 3 or 4")
    if k_cache.dtype != torch.bfloat16 or k_cache.stride(-1) != 1 or k_cache.stride(-2) != head_dim:
        raise ValueError("linear_rope_kv_write: cache rows must be contiguous bf16 [.., capacity, d]")
    if v_cache.stride() != k_cache.stride() or v_cache.shape != k_cache.shape or v_cache.dtype != k_cache.dtype:
        raise ValueError("linear_rope_kv_write: v_cache must have k_cache's shape, strides and dtype")
    if not q_out.is_contiguous() or q_out.numel() != batch * num_nodes * q_heads * head_dim or \
            q_out.dtype != torch.bfloat16:
        raise ValueError("linear_rope_kv_write: q_out must be a contiguous bf16 [batch * num_nodes, q_heads, d] tensor")
    if cos_sin is None:
        cos_sin = rope_cos_sin(batch=batch, num_nodes=num_nodes, head_dim=head_dim, seq_len=seq_len,
                               pos_offset=pos_offset, inv_freq=inv_freq)
    elif cos_sin.dtype != torch.float32 or cos_sin.numel() != batch * num_nodes * head_dim or \
            not cos_sin.is_contiguous():
        raise ValueError("linear_rope_kv_write: cos_sin must be rope_cos_sin's table of these rows")
    _call("fg_linear_rope_kv_write", _ptr(x), x.stride(0), _ptr(w_pairs), w_pairs.stride(0), _ptr(bias_pairs),
          x.shape[0], x.shape[1], tm, tn, int(stages), batch, num_nodes, q_heads, kv_heads, head_dim, _ptr(seq_len),
          _ptr(cos_sin), _ptr(q_out), _ptr(k_cache), _ptr(v_cache), k_cache.stride(0), k_cache.stride(1),
          k_cache.shape[-2], _ptr(row_map), _ptr(err_flag), _stream())


# ------------------------------------------------------------------ sampling / acceptance
def sample_workspace(rows, device):
    """Scratch that lets unrestricted / greedy draws run split over several workgroups per row."""
    n = _lib.load().fg_sample_workspace(int(rows))
    return torch.empty(n, dtype=torch.uint8, device=device)


def sample_tokens(logits, *, noise=None, noise_col=0, seed=0, step=0, seq_ids=None, draw=0, row_index=None,
                  forced=None, temperature=1.0, greedy=False, top_k=None, top_p=1.0, out=None, split=True):
    """One token per row (see the rule in csrc/sample.hip). noise: uint32 bits as int32 [R, C].
    split=False keeps every row in one workgroup (same tokens; used to cross-check)."""
    _dev(logits, noise, seq_ids, row_index, forced)
    for t, n in ((seq_ids, "seq_ids"), (row_index, "row_index"), (forced, "forced")):
        _i32(t, n)
    if noise is not None and noise.dtype != torch.int32:
        raise TypeError("noise must be int32 holding uint32 bit patterns")
    logits = aligned_rows(logits)
    V = logits.shape[-1]
    rows = row_index.numel() if row_index is not None else logits.shape[0]
    if out is None:
        out = torch.empty(rows, dtype=torch.int32, device=logits.device)
    T = 0.0 if temperature is None else float(temperature)
    use_T = T if T > 0 else (-1.0 if T < 0 or temperature is None else 0.0)
    g = bool(greedy) or (temperature is not None and T == 0.0)
    ws = sample_workspace(rows, logits.device) if split else None
    _call("fg_sample_tokens", _ptr(logits), dtype_code(logits), logits.stride(0), rows,
              V, _ptr(row_index), _ptr(forced), _ptr(noise), noise.stride(0) if noise is not None else 0,
              int(noise_col), int(seed) & (2 ** 64 - 1), int(step), _ptr(seq_ids), int(draw), use_T, int(g),
              int(top_k or 0), top_p_fixed(top_p), _ptr(out), _ptr(ws), 0 if ws is None else ws.numel(), _stream())
    return out


def accept_walk(tree_logits, tree_tokens, parents, n_nodes, *, max_walk_steps, slot_map=None, noise=None,
                noise_col0=0, seed=0, step=0, seq_ids=None, draw0=1, temperature=1.0, greedy=False, top_k=None,
                top_p=1.0, acc_stride=None, err_flag=None, out=None):
    """exact_target walk. Returns dict of int32 device tensors (acc_tokens, acc_nodes, acc_len, last_node, correction)."""
    _dev(tree_logits, tree_tokens, parents, n_nodes, slot_map, noise, seq_ids)
    for t, n in ((tree_tokens, "tree_tokens"), (parents, "parents"), (n_nodes, "n_nodes"), (slot_map, "slot_map"),
                 (seq_ids, "seq_ids")):
        _i32(t, n)
    B, nmax = tree_tokens.shape
    V = tree_logits.shape[-1]
    dev = tree_tokens.device
    acc_stride = acc_stride or (max_walk_steps + 1)
    if out is None:
        out = dict(acc_tokens=torch.zeros(B, acc_stride, dtype=torch.int32, device=dev),
                   acc_nodes=torch.zeros(B, acc_stride, dtype=torch.int32, device=dev),
                   acc_len=torch.empty(B, dtype=torch.int32, device=dev),
                   last_node=torch.empty(B, dtype=torch.int32, device=dev),
                   correction=torch.empty(B, dtype=torch.int32, device=dev),
                   state=torch.empty(3 * B, dtype=torch.int32, device=dev))
    T = 0.0 if temperature is None else float(temperature)
    use_T = T if T > 0 else (-1.0 if T < 0 or temperature is None else 0.0)
    g = bool(greedy) or (temperature is not None and T == 0.0)
    lg = aligned_rows(tree_logits.reshape(-1, V))
    _call("fg_accept_walk", _ptr(lg), dtype_code(lg), lg.stride(0), V, _ptr(slot_map), _ptr(tree_tokens),
              _ptr(parents), _ptr(n_nodes), nmax, B, int(max_walk_steps), _ptr(noise),
              noise.stride(0) if noise is not None else 0, int(noise_col0), int(seed) & (2 ** 64 - 1), int(step),
              _ptr(seq_ids), int(draw0), use_T, int(g), int(top_k or 0), top_p_fixed(top_p), _ptr(out["acc_tokens"]),
              _ptr(out["acc_nodes"]), acc_stride, _ptr(out["acc_len"]), _ptr(out["last_node"]),
              _ptr(out["correction"]), _ptr(out["state"]), _ptr(err_flag), _stream())
    return out


def walk_begin(tree_tokens, parents, n_nodes, *, acc_stride):
    """Initialise a step-at-a-time walk; returns the walk dict (outputs + state)."""
    _dev(tree_tokens, parents, n_nodes)
    B, nmax = tree_tokens.shape
    dev = tree_tokens.device
    w = dict(acc_tokens=torch.empty(B, acc_stride, dtype=torch.int32, device=dev),  # zeroed by fg_walk_begin
             acc_nodes=torch.empty(B, acc_stride, dtype=torch.int32, device=dev),
             acc_len=torch.empty(B, dtype=torch.int32, device=dev),
             last_node=torch.empty(B, dtype=torch.int32, device=dev),
             correction=torch.empty(B, dtype=torch.int32, device=dev),
             state=torch.empty(3 * B, dtype=torch.int32, device=dev),
             row_index=torch.empty(B, dtype=torch.int32, device=dev),
             row_active=torch.empty(B, dtype=torch.int32, device=dev),
             workspace=sample_workspace(B, dev))
    _call("fg_walk_begin", _ptr(tree_tokens), _ptr(parents), _ptr(n_nodes), nmax, B, _ptr(w["acc_tokens"]),
          _ptr(w["acc_nodes"]), acc_stride, _ptr(w["acc_len"]), _ptr(w["last_node"]), _ptr(w["correction"]),
          _ptr(w["state"]), _stream())
    return w


def walk_rows(walk, nmax):
    """Fill walk['row_index'] (b*nmax + parent) and walk['row_active'] for the next step."""
    B = walk["acc_len"].numel()
    _call("fg_walk_rows", _ptr(walk["state"]), B, nmax, _ptr(walk["row_index"]), _ptr(walk["row_active"]), _stream())


def walk_step(walk, step_logits, tree_tokens, parents, n_nodes, *, walk_step, noise=None, noise_col0=0, seed=0,
              step=0, seq_ids=None, draw0=1, temperature=1.0, greedy=False, top_k=None, top_p=1.0, err_flag=None,
              split=True, parts=None, next_rows=False):
    """One walk step: active row b draws from row b of step_logits.

    ``parts``: the (part_max, part_key) row maxima that ``lm_head_topk`` wrote with
    step_logits (an unrestricted / greedy step then needs no chunk-maxima launch). ``next_rows``: also
    fill walk['row_index'] / walk['row_active'] for the next step (as ``walk_rows``)."""
    _dev(step_logits, tree_tokens, parents, n_nodes, noise, seq_ids)
    if parts is not None:
        _dev(*parts)
        pm, pk = parts
        if (pm.dtype != torch.float32 or pk.dtype != torch.int64 or pm.dim() != 2 or pm.shape != pk.shape
                or pm.shape[0] != tree_tokens.shape[0] or not pm.is_contiguous() or not pk.is_contiguous()):
            raise ValueError("walk_step: parts must be contiguous fp32 / int64 [batch, P] pairs")
    B, nmax = tree_tokens.shape
    lg = aligned_rows(step_logits)
    V = lg.shape[-1]
    T = 0.0 if temperature is None else float(temperature)
    use_T = T if T > 0 else (-1.0 if T < 0 or temperature is None else 0.0)
    g = bool(greedy) or (temperature is not None and T == 0.0)
    _call("fg_walk_step", _ptr(lg), dtype_code(lg), lg.stride(0), V, _ptr(tree_tokens), _ptr(parents), _ptr(n_nodes),
          nmax, B, int(walk_step), _ptr(noise), noise.stride(0) if noise is not None else 0, int(noise_col0),
          int(seed) & (2 ** 64 - 1), int(step), _ptr(seq_ids), int(draw0), use_T, int(g), int(top_k or 0),
          top_p_fixed(top_p), _ptr(walk["acc_tokens"]), _ptr(walk["acc_nodes"]), walk["acc_tokens"].stride(0),
          _ptr(walk["acc_len"]), _ptr(walk["last_node"]), _ptr(walk["correction"]), _ptr(walk["state"]),
          _ptr(err_flag), _ptr(parts[0]) if parts is not None else None, _ptr(parts[1]) if parts is not None else None,
          parts[0].shape[1] if parts is not None else 0, _ptr(walk["row_index"]) if next_rows else None,
          _ptr(walk["row_active"]) if next_rows else None, _ptr(walk["workspace"]) if split else None,
          walk["workspace"].numel() if split else 0, _stream())


def accept_finalize(walk, old_len, *, max_length, eos_token_id, finished=None, pending_root=None):
    _dev(old_len)
    _i32(old_len, "old_len")
    B = walk["acc_len"].numel()
    if finished is None:
        finished = torch.empty(B, dtype=torch.int32, device=old_len.device)
    _call("fg_accept_finalize", _ptr(walk["acc_tokens"]), _ptr(walk["acc_nodes"]), walk["acc_tokens"].stride(0),
              _ptr(walk["acc_len"]), _ptr(walk["last_node"]), _ptr(walk["correction"]), _ptr(old_len),
              int(max_length), -1 if eos_token_id is None else int(eos_token_id), _ptr(finished),
              _ptr(pending_root), B, _stream())
    return finished


def kv_path_gather(tensor_ptrs, *, batch, kv_heads, head_dim, elem_bytes, strides, capacity, seq_len, acc_nodes,
                   acc_len, tree_nodes, row_map=None, err_flag=None):
    """tensor_ptrs: int64 device tensor of cache base addresses (K0, V0, K1, V1, ...)."""
    _dev(tensor_ptrs, seq_len, acc_nodes, acc_len, row_map, err_flag)
    for t, n in ((seq_len, "seq_len"), (acc_nodes, "acc_nodes"), (acc_len, "acc_len"), (row_map, "row_map")):
        _i32(t, n)
    bs, hs, rs = strides
    _call("fg_kv_path_gather", _ptr(tensor_ptrs), tensor_ptrs.numel(), batch, kv_heads, head_dim, elem_bytes, bs,
              hs, rs, capacity, _ptr(seq_len), _ptr(row_map), _ptr(acc_nodes), acc_nodes.stride(0), _ptr(acc_len),
              int(tree_nodes), _ptr(err_flag), _stream())
