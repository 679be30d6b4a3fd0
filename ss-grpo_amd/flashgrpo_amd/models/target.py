"""Qwen2/Llama-architecture target model with a per-sequence contiguous KV cache.

Replaces the Hugging Face decoder the reference drives through
``flashgrpo/models/qwen_flashgrpo_wrapper.py:150-239`` (``prefill``,
``forward_tokens``, ``forward_tree``) and its ``DynamicCache``:

* the cache is preallocated once, ``[L, 2, B, Hkv, capacity, d]``, with a
  device ``seq_len[B]``; the tree's K/V go straight into slots
  ``seq_len[b] + n`` (no per-step ``torch.cat`` of the prefix) and the
  accepted path is compacted in place by ``fg_kv_path_gather``;
* attention is ``fg_tree_attention`` (ancestor bitmask in registers) for the
  tree verify and for prefill, which runs as causal 64-token chains;
* RMSNorm, rotary + cache write and SwiGLU are HIP kernels. Each dense
  projection runs, per shape, whichever path the measured tables of
  ``flashgrpo_amd.tuning`` found faster: the split-K MFMA GEMM
  (``fg_linear_parts``) whose fp32 parts are finished by the rotary + cache
  write (QKV) or by the residual add + next RMSNorm (O, down), or the library
  GEMM (``F.linear``: hipBLASLt or rocBLAS with the per-shape solution table;
  the O and down projections add into the residual stream in place, ``addmm_``
  with beta = 1); the MLP input is the fused gate/up + SwiGLU GEMM or the
  library projection + ``fg_swiglu``.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np
import torch
import torch.nn.functional as F

from .. import kernels as K
from .. import timing
from ..tuning import (linear_table_plan, linear_table_split_plan, linear_table_times, mlp_table_fused_tile,
                      mlp_table_path, use_tuned_gemms)

MAX_TREE_NODES = 64      # tree nodes per forward (64-bit ancestor masks)
MAX_CHAIN_TOKENS = 8192  # new tokens per forward without masks (a causal chain)
LM_STREAM_ROWS = 256  # contiguous LM-head rows up to this count run the weight-streaming kernel
PREFILL_CHUNK = 1024     # prompt tokens per prefill forward


@dataclass
class TargetConfig:
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
    name: str = "custom"

    @property
    def group(self) -> int:
        return self.q_heads // self.kv_heads

    # Shapes named by the benchmark configurations.
    @staticmethod
    def tiny():
        return TargetConfig(4, 512, 8, 2, 64, 1408, 32000, 1.0e6, 1e-6, True, True, "tiny-qwen2")

    @staticmethod
    def qwen25_1p5b():
        return TargetConfig(28, 1536, 12, 2, 128, 8960, 151936, 1.0e6, 1e-6, True, True, "qwen2.5-1.5b")

    @staticmethod
    def qwen25_7b():
        return TargetConfig(28, 3584, 28, 4, 128, 18944, 152064, 1.0e6, 1e-6, True, False, "qwen2.5-7b")

    @staticmethod
    def llama31_8b():
        return TargetConfig(32, 4096, 32, 8, 128, 14336, 128256, 5.0e5, 1e-5, False, False, "llama-3.1-8b")

    @staticmethod
    def qwen25_14b():
        return TargetConfig(48, 5120, 40, 8, 128, 13824, 152064, 1.0e6, 1e-6, True, False, "qwen2.5-14b")


def lm_gemm_ok(x: torch.Tensor, w: torch.Tensor) -> bool:
    """Operand rules of the hand-written bf16 LM-head kernels (``fg_lm_head_topk``,
    ``fg_lm_head``): K a multiple of 64, both operands K-contiguous with 16-byte aligned
    rows (base address and row stride), the weight under 4 GiB."""
    K_ = x.shape[-1]
    return (x.dtype == torch.bfloat16 and w.dtype == torch.bfloat16 and K_ % 64 == 0 and w.shape[-1] == K_
            and x.stride(-1) == 1 and w.stride(-1) == 1 and (x.dim() < 2 or x.stride(0) % 8 == 0)
            and w.stride(0) % 8 == 0 and x.data_ptr() % 16 == 0 and w.data_ptr() % 16 == 0
            and w.shape[0] * w.stride(0) * 2 <= 0xFFFFFFFF)


def lm_stream_ok(x: torch.Tensor, w: torch.Tensor, out: torch.Tensor | None = None) -> bool:
    """``lm_gemm_ok`` plus the weight-streaming kernel's own limits: x spans under 4 GiB
    from its first row, and a given output has unit column stride and, when its row stride
    is a multiple of 4 elements, a base aligned for 4-column stores (8 bytes bf16, 16 fp32)."""
    if not lm_gemm_ok(x, w):
        return False
    x2 = x.reshape(-1, x.shape[-1])
    if ((x2.shape[0] - 1) * x2.stride(0) + x2.shape[1]) * 2 >= 1 << 32:
        return False
    if out is not None:
        # 4-column vector stores when the row stride is a multiple of 4 elements
        if out.dim() != 2 or out.stride(1) != 1 or (out.stride(0) % 4 == 0
                                                     and out.data_ptr() % (4 * out.element_size())):
            return False
    return True


def inv_freq_table(head_dim: int, theta: float) -> torch.Tensor:
    """fp32 theta^(-2i/d) computed the way the Hugging Face rotary embedding computes its
    default table (``1 / theta ** (arange(0, d, 2).float() / d)`` in fp32 with torch on the
    host), so the rotation angles match the reference's bit for bit."""
    return 1.0 / (float(theta) ** (torch.arange(0, head_dim, 2, dtype=torch.int64).float() / head_dim))


def chain_bits(n: int) -> list:
    """Ancestor-or-self masks of a causal chain of n nodes."""
    return [(1 << (i + 1)) - 1 if i < 63 else -1 for i in range(n)]


def as_mask_tensor(bits, device) -> torch.Tensor:
    """uint64 bit masks -> int64 tensor with the same bit patterns."""
    arr = np.array([int(b) & 0xFFFFFFFFFFFFFFFF for b in bits], dtype=np.uint64).view(np.int64)
    return torch.from_numpy(arr).to(device)


class KVCache:
    """Contiguous per-sequence KV cache: kv[L, 2, B, Hkv, capacity, d] + seq_len[B].

    ``seq_len`` counts committed (accepted) tokens of each cache row. Tree
    verification writes its nodes after them without advancing ``seq_len``.
    """

    def __init__(self, cfg: TargetConfig, batch: int, capacity: int, *, dtype, device):
        self.cfg = cfg
        self.batch = int(batch)
        self.capacity = int(capacity)
        self.dtype = dtype
        self.device = torch.device(device)
        self.kv = torch.zeros(cfg.num_layers, 2, batch, cfg.kv_heads, capacity, cfg.head_dim, dtype=dtype,
                              device=device)
        self.seq_len = torch.zeros(batch, dtype=torch.int32, device=device)
        ptrs = [self.kv[l, j].data_ptr() for l in range(cfg.num_layers) for j in range(2)]
        self.tensor_ptrs = torch.tensor(ptrs, dtype=torch.int64, device=device)

    def k(self, layer: int) -> torch.Tensor:
        return self.kv[layer, 0]

    def v(self, layer: int) -> torch.Tensor:
        return self.kv[layer, 1]

    @property
    def strides(self):
        t = self.kv[0, 0]
        return t.stride(0), t.stride(1), t.stride(2)

    def gather_path(self, seq_len, acc_nodes, acc_len, tree_nodes, *, row_map=None, err_flag=None):
        K.kv_path_gather(self.tensor_ptrs, batch=seq_len.numel(), kv_heads=self.cfg.kv_heads,
                         head_dim=self.cfg.head_dim, elem_bytes=self.kv.element_size(), strides=self.strides,
                         capacity=self.capacity, seq_len=seq_len, acc_nodes=acc_nodes, acc_len=acc_len,
                         tree_nodes=tree_nodes, row_map=row_map, err_flag=err_flag)

    def repeat_rows(self, src_rows: torch.Tensor, dst_rows: torch.Tensor) -> None:
        """Copy cache rows src -> dst (all layers), e.g. GRPO repeats of one prompt. One layer
        at a time: the gathered temporary holds one layer's source rows (one gather over every
        layer would hold all of them, 91 GiB for the 14B config's 112 repeated rows)."""
        src, dst = src_rows.long(), dst_rows.long()
        for layer in self.kv:  # [2, B, Hkv, capacity, d]
            layer.index_copy_(1, dst, layer.index_select(1, src))
        self.seq_len.index_copy_(0, dst, self.seq_len.index_select(0, src))

    def container_copy(self) -> "KVCache":
        """A second cache object over the same storage with its own committed lengths
        (the reference's clone_cache(clone_tensors=False)). Committed rows are shared
        read-only; the slots past a row's committed length are shared scratch, so two
        containers that append past the same length overwrite each other there."""
        c = KVCache.__new__(KVCache)
        c.__dict__.update(self.__dict__)
        c.seq_len = self.seq_len.clone()
        return c

    def select_rows(self, rows: torch.Tensor, capacity: int | None = None) -> "KVCache":
        """A new cache holding copies of the given rows (in that order)."""
        rows = rows.to(device=self.device, dtype=torch.long)
        cap = self.capacity if capacity is None else int(capacity)
        out = KVCache(self.cfg, int(rows.numel()), cap, dtype=self.dtype, device=self.device)
        keep = min(cap, self.capacity)
        for src, dst in zip(self.kv, out.kv):  # one layer's gathered rows at a time
            dst[..., :keep, :].copy_(src.index_select(1, rows)[..., :keep, :])
        out.seq_len.copy_(self.seq_len.index_select(0, rows).clamp_max(cap))
        return out


# ------------------------------------------------------------------ Hugging Face weights
def unwrap_causal_lm(causal_lm):
    """The causal LM under a PEFT wrapper (``qwen_flashgrpo_wrapper.py:7-12``)."""
    if hasattr(causal_lm, "get_base_model"):
        return causal_lm.get_base_model()
    if hasattr(causal_lm, "base_model") and hasattr(causal_lm.base_model, "model"):
        return causal_lm.base_model.model
    return causal_lm


def hf_target_config(c) -> TargetConfig:
    """TargetConfig of a transformers Qwen2/Llama config."""
    rope = getattr(c, "rope_theta", None) or (getattr(c, "rope_parameters", None) or {}).get("rope_theta", 1e4)
    return TargetConfig(
        num_layers=c.num_hidden_layers, hidden=c.hidden_size, q_heads=c.num_attention_heads,
        kv_heads=getattr(c, "num_key_value_heads", None) or c.num_attention_heads,
        head_dim=getattr(c, "head_dim", None) or c.hidden_size // c.num_attention_heads,
        intermediate=c.intermediate_size, vocab=c.vocab_size, rope_theta=float(rope), rms_eps=float(c.rms_norm_eps),
        qkv_bias=bool(getattr(c, "attention_bias", False) or c.model_type == "qwen2"),
        tie_word_embeddings=bool(getattr(c, "tie_word_embeddings", False)), name=c.model_type)


def hf_parameter_key(model) -> tuple:
    """(address, version counter) of every parameter: changes when an optimizer step,
    an in-place edit or a reassignment touches any of them (adapters included)."""
    return tuple((p.data_ptr(), p._version) for p in model.parameters())


def _active_adapters(mod) -> list:
    act = getattr(mod, "active_adapters", None)
    if act is None:
        act = getattr(mod, "active_adapter", [])
    return [act] if isinstance(act, str) else list(act)


def hf_linear_weight(mod):
    """(weight, bias) a linear module applies, in float32 when an adapter delta is
    merged. A LoRA-wrapped linear (PEFT layout: ``base_layer``, ``lora_A``/``lora_B``
    module dicts, ``scaling``) adds ``scaling[a] * lora_B[a].weight @ lora_A[a].weight``
    (and ``scaling[a] * lora_B[a].bias`` when the adapter has one) for every active
    adapter unless the adapters are merged into the base weight or disabled."""
    base = getattr(mod, "base_layer", None)
    if base is None:
        return mod.weight, getattr(mod, "bias", None)
    while getattr(base, "base_layer", None) is not None:  # nested wrappers
        base = base.base_layer
    w, b = base.weight, getattr(base, "bias", None)
    if getattr(mod, "merged", False) or getattr(mod, "disable_adapters", False):
        return w, b
    lora_a, lora_b = getattr(mod, "lora_A", {}), getattr(mod, "lora_B", {})
    use_dora = getattr(mod, "use_dora", {}) or {}
    out_w, out_b = None, None
    for name in _active_adapters(mod):
        if name not in lora_a:
            continue
        if use_dora.get(name, False):
            raise NotImplementedError(f"DoRA adapter {name!r}: only plain LoRA deltas are merged")
        if getattr(mod, "fan_in_fan_out", False):
            raise NotImplementedError("fan_in_fan_out LoRA layers are not merged")
        scale = float(mod.scaling[name])
        A, B = lora_a[name].weight, lora_b[name].weight
        if out_w is None:
            out_w = w.detach().float().clone()
        out_w += scale * (B.detach().float() @ A.detach().float())
        bb = getattr(lora_b[name], "bias", None)
        if bb is not None:
            if out_b is None:
                out_b = b.detach().float().clone() if b is not None else torch.zeros_like(bb.detach().float())
            out_b += scale * bb.detach().float()
    return (w if out_w is None else out_w), (b if out_b is None else out_b)


def _plain_weight(mod, what):
    if getattr(mod, "base_layer", None) is not None or hasattr(mod, "lora_embedding_A"):
        raise NotImplementedError(f"{what}: adapters on this module are not merged")
    return mod.weight


def _read_hf_weights(base, cfg: TargetConfig, dev, dt, into: dict | None = None) -> dict:
    """The native weight dict of a transformers causal LM, one layer at a time. With
    ``into`` the tensors of an existing dict are overwritten in place (shapes must
    match); otherwise fresh tensors are allocated (never aliases of the parameters)."""

    def put(dst, src):
        src = src.detach()
        if dst is None:
            return src.to(device=dev, dtype=dt, copy=True).contiguous()
        dst.copy_(src.to(device=dev, dtype=dt))
        return dst

    def cat(dst, parts):
        # merged adapter weights are float32: concatenate wide, round to dt once
        wide = any(p.dtype != dt for p in parts)
        t = torch.cat([p.detach().to(device=dev, dtype=torch.float32 if wide else dt) for p in parts]).to(dt)
        if dst is None:
            return t.contiguous()
        dst.copy_(t)
        return dst

    body = base.model
    w = into if into is not None else {"layers": [None] * cfg.num_layers}
    w["embed"] = put(w.get("embed"), _plain_weight(body.embed_tokens, "embed_tokens"))
    w["final_norm"] = put(w.get("final_norm"), body.norm.weight)
    for i, layer in enumerate(body.layers):
        at, mlp = layer.self_attn, layer.mlp
        lw = w["layers"][i] or {}
        q, k, v = (hf_linear_weight(m) for m in (at.q_proj, at.k_proj, at.v_proj))
        lw["qkv_w"] = cat(lw.get("qkv_w"), [q[0], k[0], v[0]])
        lw["qkv_b"] = cat(lw.get("qkv_b"), [q[1], k[1], v[1]]) if q[1] is not None else None
        lw["o_w"] = put(lw.get("o_w"), hf_linear_weight(at.o_proj)[0])
        lw["gate_up_w"] = cat(lw.get("gate_up_w"), [hf_linear_weight(mlp.gate_proj)[0],
                                                    hf_linear_weight(mlp.up_proj)[0]])
        lw["down_w"] = put(lw.get("down_w"), hf_linear_weight(mlp.down_proj)[0])
        lw["input_norm"] = put(lw.get("input_norm"), layer.input_layernorm.weight)
        lw["post_norm"] = put(lw.get("post_norm"), layer.post_attention_layernorm.weight)
        w["layers"][i] = lw
    head = getattr(base, "lm_head", None)
    tied = head is None or head.weight.data_ptr() == body.embed_tokens.weight.data_ptr()
    if tied:
        w["lm_head"] = w["embed"]
    else:
        cur = w.get("lm_head")
        w["lm_head"] = put(None if cur is w["embed"] else cur, _plain_weight(head, "lm_head"))
    return w


_HIP = None


def _graph_memset_nodes(graph: torch.cuda.CUDAGraph) -> int:
    """Memset nodes of a captured (not yet instantiated) graph, counted through the
    HIP runtime torch already loaded. A library call may record a hipMemsetAsync; such
    nodes have given wrong results on replays after the first, so a graph holding one
    is not used."""
    global _HIP
    import ctypes

    if _HIP is None:
        _HIP = ctypes.CDLL("libamdhip64.so.7")
    raw = ctypes.c_void_p(graph.raw_cuda_graph())
    n = ctypes.c_size_t(0)
    if _HIP.hipGraphGetNodes(raw, None, ctypes.byref(n)) != 0:
        raise RuntimeError("hipGraphGetNodes failed")
    nodes = (ctypes.c_void_p * max(n.value, 1))()
    if _HIP.hipGraphGetNodes(raw, nodes, ctypes.byref(n)) != 0:
        raise RuntimeError("hipGraphGetNodes failed")
    kind = ctypes.c_int(0)
    count = 0
    for i in range(n.value):
        if _HIP.hipGraphNodeGetType(ctypes.c_void_p(nodes[i]), ctypes.byref(kind)) != 0:
            raise RuntimeError("hipGraphNodeGetType failed")
        count += kind.value == 2  # hipGraphNodeTypeMemset
    return count


class _ForwardGraph:
    """One captured verify forward: static input buffers and two graphs, the first layer
    and the rest. Launching a graph of ~250 nodes costs ~120 us of host time, and a
    round's GPU idles until its forward's first kernels are queued; with the split, the
    second launch runs on the host while the GPU works through the first layer."""

    FIRST_LAYERS = 1

    def __init__(self, graphs, inputs, out):
        self.graphs, self.inputs, self.out = graphs, inputs, out

    @classmethod
    def capture(cls, model, tokens, cache, pos_offset, anc, seq_len, row_map, err_flag):
        inputs = dict(tokens=tokens.clone(), pos=pos_offset.clone(), anc=anc.clone(), seq=seq_len.clone(),
                      row_map=None if row_map is None else row_map.clone())
        kw = dict(pos_offset=inputs["pos"], anc=inputs["anc"], seq_len=inputs["seq"], row_map=inputs["row_map"],
                  err_flag=err_flag)
        # A warm-up on the current stream allocates every buffer and workspace the
        # launches use outside the graph's pool (it rewrites the same tree slots the
        # caller's forward writes).
        model._forward_eager(inputs["tokens"], cache, **kw)
        if model._graph_pool is None:
            model._graph_pool = torch.cuda.graph_pool_handle()
        L = model.cfg.num_layers
        split = min(cls.FIRST_LAYERS, L)
        g1 = torch.cuda.CUDAGraph(keep_graph=True)
        with torch.cuda.graph(g1, pool=model._graph_pool):
            st = model._forward_begin(inputs["tokens"], cache, **kw)
            model._forward_layers(st, 0, split)
            if split == L:  # no later layer: one graph (the final norm may already be written)
                out = model._forward_end(st)
        graphs = [g1]
        if split < L:
            g2 = torch.cuda.CUDAGraph(keep_graph=True)
            with torch.cuda.graph(g2, pool=model._graph_pool):
                model._forward_layers(st, split, L)
                out = model._forward_end(st)
            graphs.append(g2)
        if any(_graph_memset_nodes(g) for g in graphs):
            return None
        for g in graphs:
            g.instantiate()
        # st["x"] (the residual stream, allocated in the first graph's capture) stays
        # referenced through the second graph, which reads it
        return cls((*graphs, st), inputs, out)

    def run(self, tokens, pos_offset, anc, seq_len, row_map):
        st = self.inputs
        st["tokens"].copy_(tokens)
        st["pos"].copy_(pos_offset)
        st["anc"].copy_(anc)
        st["seq"].copy_(seq_len)
        if row_map is not None:
            st["row_map"].copy_(row_map)
        for g in self.graphs[:-1]:  # the last entry is the capture's forward state
            g.replay()
        return self.out


_CUS = {}


def _cu_count(device) -> int:
    key = str(device)
    if key not in _CUS:
        _CUS[key] = torch.cuda.get_device_properties(torch.device(device)).multi_processor_count
    return _CUS[key]


def mlp_path(rows: int, inter: int, hidden: int, device) -> int:
    """How a decoder layer computes its MLP input for ``rows`` rows: 0 for the hipBLASLt
    projection + fg_swiglu, else the tile height (64, 128, 192 or 256; -1 lets the kernel pick 192
    or 256) of the fused gate/up + SwiGLU GEMM.

    The measured table (``tuning/mlp_mi355x.csv``) decides for the sizes it covers: which path
    is faster depends on the library's solution for the shape (Qwen2.5-7B verify rounds, 1856
    rows: 443 against 457 us, the pair; Qwen2.5-14B, 3712 rows: 957 against 905 us, the fused
    GEMM). Other sizes take the fused GEMM when its tiles make one pass over the compute units,
    where the pass it saves decides (Qwen2.5-1.5B, 512 rows: 58 against 39 us).
    """
    measured = mlp_table_path(rows, inter, hidden)
    if measured is not None:
        return measured
    cols = -(-inter // 128)
    fits = min(-(-rows // bm) * cols for bm in (192, 256)) <= _cu_count(device)
    return -1 if fits else 0  # -1: fused, the kernel picks the tile height


def default_linear_plan(rows: int, cols: int, hidden: int, cus: int = 256) -> tuple:
    """A split-K plan (tile_m, tile_n, splits, stages) for a shape no measurement covers: 128 x 128
    tiles when there are at least a quarter as many as CUs, else 64 x 128; then the split count
    that brings the workgroups nearest to two per CU with at least four k-steps per split; a
    4-stage ring."""
    tm, tn = (128, 128) if -(-rows // 128) * -(-cols // 128) >= cus // 4 else (64, 128)
    tiles = -(-rows // tm) * -(-cols // tn)
    nk = hidden // 64
    best = 1
    for s in range(1, max(1, nk // 4) + 1):
        if K.linear_splits(hidden, s) == s and abs(tiles * s - 2 * cus) < abs(tiles * best - 2 * cus):
            best = s
    return tm, tn, best, 4


def linear_path(kind: str, rows: int, cols: int, hidden: int):
    """How a decoder layer computes projection ``kind`` ("qkv", "o" or "down") for ``rows``
    rows: (tile_m, tile_n, splits, stages) of the split-K GEMM, or None for the library projection.

    The measured table (``tuning/linear_mi355x.csv``) decides for the sizes it covers (split-K at
    the Qwen2.5-1.5B verify rows, where the library's tiles leave most CUs idle; the library at the
    Qwen2.5-7B ones). Other sizes take the library.
    """
    measured = linear_table_plan(kind, rows, cols, hidden)
    return measured or None


class TargetModel:
    """Decoder weights on the device plus the verify / prefill forward."""

    def __init__(self, cfg: TargetConfig, weights: dict, *, dtype, device):
        self.cfg = cfg
        self.dtype = dtype
        self.device = torch.device(device)
        self.w = weights
        self.inv_freq = inv_freq_table(cfg.head_dim, cfg.rope_theta).to(device)
        self._bufs = {}
        self._graphs = {}       # graph key -> _ForwardGraph, or None when the key stays eager
        self._graph_seen = {}   # graph key -> eager calls so far
        self._graph_pool = None
        self._retired = []      # buffers replaced while graphs that address them exist
        self._hf_source = None  # the Hugging Face model the weights were read from (from_hf)
        self._hf_key = None
        # the MLP's gate/up projection and SwiGLU as one GEMM (fg_gate_up_swiglu): None chooses per
        # shape (mlp_path), True wherever the operands allow (at the shape's fastest measured tile
        # height, else the kernel's pick), False never (the hipBLASLt projection, then fg_swiglu);
        # call drop_graphs() after a change
        self.fused_mlp = None
        # the QKV, O and down projections as split-K GEMMs (fg_linear_parts) finished by the rotary
        # + cache write or the residual add + RMSNorm: None chooses per shape (linear_path), True
        # wherever the operands allow (the shape's best measured split-K plan, else
        # default_linear_plan), False never; drop_graphs() after a change
        self.split_k_linear = None
        if self.device.type == "cuda":
            use_tuned_gemms()

    # -------------------------------------------------------------- construction
    @classmethod
    def random(cls, cfg: TargetConfig, *, seed: int = 0, std: float = 0.02, dtype=torch.bfloat16, device="cuda"):
        """Seeded N(0, std) weights generated on the device; norms 1, biases 0."""
        g = torch.Generator(device=device).manual_seed(int(seed))
        H, d, Fi = cfg.hidden, cfg.head_dim, cfg.intermediate
        qkv_rows = (cfg.q_heads + 2 * cfg.kv_heads) * d

        def n(*shape):
            t = torch.empty(*shape, dtype=dtype, device=device)
            t.normal_(0.0, std, generator=g)
            return t

        w = {"embed": n(cfg.vocab, H), "final_norm": torch.ones(H, dtype=dtype, device=device), "layers": []}
        for _ in range(cfg.num_layers):
            w["layers"].append({
                "input_norm": torch.ones(H, dtype=dtype, device=device),
                "qkv_w": n(qkv_rows, H),
                "qkv_b": torch.zeros(qkv_rows, dtype=dtype, device=device) if cfg.qkv_bias else None,
                "o_w": n(H, cfg.q_heads * d),
                "post_norm": torch.ones(H, dtype=dtype, device=device),
                "gate_up_w": n(2 * Fi, H),
                "down_w": n(H, Fi),
            })
        w["lm_head"] = w["embed"] if cfg.tie_word_embeddings else n(cfg.vocab, H)
        return cls(cfg, w, dtype=dtype, device=device)

    @classmethod
    def from_numpy(cls, cfg: TargetConfig, W: dict, *, dtype=torch.float32, device="cuda"):
        """From a dict of numpy arrays with per-projection keys (q_w, k_w, ... gate_w, up_w)."""

        def t(a):
            return None if a is None else torch.from_numpy(np.ascontiguousarray(a)).to(device=device, dtype=dtype)

        w = {"embed": t(W["embed"]), "final_norm": t(W["final_norm"]), "layers": []}
        for lw in W["layers"]:
            bias = None
            if lw.get("q_b") is not None:
                bias = t(np.concatenate([lw["q_b"], lw["k_b"], lw["v_b"]]))
            w["layers"].append({
                "input_norm": t(lw["input_norm"]),
                "qkv_w": t(np.concatenate([lw["q_w"], lw["k_w"], lw["v_w"]])),
                "qkv_b": bias,
                "o_w": t(lw["o_w"]),
                "post_norm": t(lw["post_norm"]),
                "gate_up_w": t(np.concatenate([lw["gate_w"], lw["up_w"]])),
                "down_w": t(lw["down_w"]),
            })
        w["lm_head"] = w["embed"] if cfg.tie_word_embeddings else t(W["lm_head"])
        m = cls(cfg, w, dtype=dtype, device=device)
        if "inv_freq" in W:
            m.inv_freq = torch.from_numpy(np.asarray(W["inv_freq"], np.float32)).to(device)
        return m

    @classmethod
    def from_hf(cls, hf_model, *, dtype=None, device=None):
        """Convert a transformers Qwen2/Llama causal LM, optionally PEFT-wrapped
        (the reference trainer's LoRA target, ``flashgrpo_trainer.py:701-708``).

        Every weight is copied (nothing aliases the live parameters) and each
        projection is read through its module: a LoRA-wrapped linear contributes
        ``base_layer.weight + scaling * lora_B @ lora_A`` for its active, unmerged
        adapters. The model keeps a link to ``hf_model``; ``sync_from_hf`` re-reads
        the weights in place when any parameter changed since the last read (an
        optimizer step between rollouts).
        """
        base = unwrap_causal_lm(hf_model)
        cfg = hf_target_config(base.config)
        dev = torch.device(device) if device is not None else next(base.parameters()).device
        dt = dtype or next(base.parameters()).dtype
        with torch.no_grad():
            w = _read_hf_weights(base, cfg, dev, dt)
        cfg.qkv_bias = w["layers"][0]["qkv_b"] is not None
        m = cls(cfg, w, dtype=dt, device=dev)
        rot = getattr(getattr(base, "model", base), "rotary_emb", None)
        if rot is not None and hasattr(rot, "inv_freq"):
            m.inv_freq = rot.inv_freq.detach().to(device=dev, dtype=torch.float32).clone()
        m._hf_source = hf_model
        m._hf_key = hf_parameter_key(hf_model)
        return m

    def sync_from_hf(self, *, force: bool = False) -> bool:
        """Re-read the linked Hugging Face model's weights into this model's tensors
        (in place, so their device addresses stay valid) when any of its parameters
        changed since the last read. Returns True when weights were copied."""
        src = getattr(self, "_hf_source", None)
        if src is None:
            return False
        key = hf_parameter_key(src)
        if not force and key == self._hf_key:
            return False
        # in-place copies are allowed here whether the weights were made inside or
        # outside inference mode
        with torch.inference_mode():
            _read_hf_weights(unwrap_causal_lm(src), self.cfg, self.device, self.dtype, into=self.w)
            cfg = self.cfg
            for lw in self.w["layers"]:  # derived copies, refreshed in place as well
                if lw.get("qkv_w_pairs") is not None:
                    lw["qkv_w_pairs"].copy_(K.rope_pair_rows(lw["qkv_w"], cfg.q_heads, cfg.kv_heads, cfg.head_dim))
                    if lw.get("qkv_b_pairs") is not None:
                        lw["qkv_b_pairs"].copy_(K.rope_pair_rows(lw["qkv_b"], cfg.q_heads, cfg.kv_heads,
                                                                 cfg.head_dim))
        self._hf_key = key
        return True

    @property
    def lm_head_weight(self) -> torch.Tensor:
        return self.w["lm_head"]

    @property
    def embed_weight(self) -> torch.Tensor:
        return self.w["embed"]

    def new_cache(self, batch: int, capacity: int) -> KVCache:
        return KVCache(self.cfg, batch, capacity, dtype=self.dtype, device=self.device)

    # -------------------------------------------------------------- forward
    def _buf(self, name, shape, dtype=None):
        dtype = dtype or self.dtype
        numel = math.prod(shape)
        b = self._bufs.get(name)
        if b is None or b.numel() < numel or b.dtype != dtype:
            if b is not None and self._graphs:
                self._retired.append(b)  # a captured graph may still address it
            b = torch.empty(max(numel, 1), dtype=dtype, device=self.device)
            self._bufs[name] = b
        return b[:numel].view(*shape)

    def drop_graphs(self, cache: "KVCache | None" = None) -> None:
        """Forget the captured forwards of one cache (None: all of them)."""
        if cache is None:
            self._graphs.clear()
            self._graph_seen.clear()
        else:
            ptr = cache.kv.data_ptr()
            for d in (self._graphs, self._graph_seen):
                for k in [k for k in d if k[4] == ptr]:
                    del d[k]
        if not self._graphs:
            self._retired.clear()
            self._graph_pool = None  # the pool is released with its last graph; the next capture opens a new one

    def forward(self, tokens: torch.Tensor, cache: KVCache, *, pos_offset: torch.Tensor, anc: torch.Tensor,
                seq_len: torch.Tensor | None = None, row_map: torch.Tensor | None = None,
                err_flag: torch.Tensor | None = None, graph: bool = False) -> torch.Tensor:
        """Forward N new tokens per row after each row's committed prefix.

        tokens [B, N] int (device); pos_offset int32 [N] (shared) or [B, N]: position =
        seq_len[b] + pos_offset[(b,) n]; anc: int64 bit masks [N] (shared) or [B, N], or None for a causal
        chain (node n sees new tokens 0..n; up to MAX_CHAIN_TOKENS); node n's K/V land in cache slot
        seq_len[b] + n of cache row row_map[b]. Returns final-normed hidden [B, N, H].
        ``seq_len`` defaults to ``cache.seq_len`` and is not advanced here.

        ``graph=True`` replays a HIP graph of the whole forward (captured on the second
        call with the same shapes, cache and error word): one launch instead of ~9 per
        layer. The returned tensor is then the graph's output buffer, overwritten by
        the next replay of that graph. Calls made while a kernel timer is installed run
        eagerly so every launch stays visible to it.
        """
        seq_len = cache.seq_len if seq_len is None else seq_len
        if graph and anc is not None and timing.idle() and not torch.cuda.is_current_stream_capturing():
            key = (tuple(tokens.shape), tokens.dtype, tuple(pos_offset.shape), tuple(anc.shape), cache.kv.data_ptr(),
                   tuple(cache.kv.shape), tuple(seq_len.shape), None if row_map is None else tuple(row_map.shape),
                   None if err_flag is None else err_flag.data_ptr())
            g = self._graphs.get(key, False)
            if g is False:
                seen = self._graph_seen.get(key, 0)
                self._graph_seen[key] = seen + 1
                if seen >= 1:  # a shape seen twice is worth a capture
                    g = self._graphs[key] = _ForwardGraph.capture(self, tokens, cache, pos_offset, anc, seq_len,
                                                                  row_map, err_flag)
            if g:
                return g.run(tokens, pos_offset, anc, seq_len, row_map)
        return self._forward_eager(tokens, cache, pos_offset=pos_offset, anc=anc, seq_len=seq_len, row_map=row_map,
                                   err_flag=err_flag)

    def _forward_eager(self, tokens, cache, *, pos_offset, anc, seq_len, row_map, err_flag):
        st = self._forward_begin(tokens, cache, pos_offset=pos_offset, anc=anc, seq_len=seq_len, row_map=row_map,
                                 err_flag=err_flag)
        self._forward_layers(st, 0, self.cfg.num_layers)
        return self._forward_end(st)

    def _forward_begin(self, tokens, cache, *, pos_offset, anc, seq_len, row_map, err_flag) -> dict:
        """Shape checks and the embedding rows: the forward's state for _forward_layers."""
        cfg = self.cfg
        B, N = tokens.shape
        if anc is not None and N > MAX_TREE_NODES:
            raise ValueError(f"at most {MAX_TREE_NODES} tree nodes per forward")
        if N > MAX_CHAIN_TOKENS:
            raise ValueError(f"at most {MAX_CHAIN_TOKENS} new tokens per forward")
        d = cfg.head_dim
        x = self.w["embed"].index_select(0, tokens.reshape(-1).long())  # [T, H] residual stream
        return dict(x=x, B=B, N=N, cache=cache, pos_offset=pos_offset, anc=anc, seq_len=seq_len, row_map=row_map,
                    err_flag=err_flag, q=self._buf("q", (B, N, cfg.q_heads, d)),
                    attn=self._buf("attn", (B, N, cfg.q_heads, d)))

    def _forward_layers(self, st: dict, l0: int, l1: int) -> None:
        """Decoder layers [l0, l1) on the residual stream st["x"] (updated in place)."""
        cfg = self.cfg
        x, B, N, cache = st["x"], st["B"], st["N"], st["cache"]
        seq_len, pos_offset, anc, row_map, err_flag = (st["seq_len"], st["pos_offset"], st["anc"], st["row_map"],
                                                       st["err_flag"])
        q, attn = st["q"], st["attn"]
        T = B * N
        H, d = cfg.hidden, cfg.head_dim
        L = cfg.num_layers
        for l in range(l0, l1):
            lw = self.w["layers"][l]
            # the input norm, unless the previous layer's down projection finish wrote it
            h = st.pop("h", None)
            if h is None:
                h = K.rmsnorm(x, lw["input_norm"], cfg.rms_eps, out=self._buf("h", (T, H)))
            plan = self._linear_plan("qkv", h, lw["qkv_w"])
            if plan and len(plan) == 5:  # the projection with the rotary + cache write in its epilogue
                wp, bp = self._rope_pairs(l)
                cs = st.get("rope_cs")
                if cs is None:  # the rows' rotary table, once per forward
                    cs = st["rope_cs"] = K.rope_cos_sin(batch=B, num_nodes=N, head_dim=d, seq_len=seq_len,
                                                        pos_offset=pos_offset, inv_freq=self.inv_freq,
                                                        out=self._buf("rope_cs", (T, d // 2, 2), torch.float32))
                K.linear_rope_kv_write(h, wp, bp, tile=plan[:2], stages=plan[3], batch=B, num_nodes=N,
                                       q_heads=cfg.q_heads, kv_heads=cfg.kv_heads, head_dim=d, seq_len=seq_len,
                                       cos_sin=cs, q_out=q, k_cache=cache.k(l), v_cache=cache.v(l), row_map=row_map,
                                       err_flag=err_flag)
            elif plan:
                parts = self._linear_parts(h, lw["qkv_w"], plan)
                K.rope_kv_write_parts(parts, lw["qkv_b"], batch=B, num_nodes=N, q_heads=cfg.q_heads,
                                      kv_heads=cfg.kv_heads, head_dim=d, seq_len=seq_len, pos_offset=pos_offset,
                                      inv_freq=self.inv_freq, q_out=q, k_cache=cache.k(l), v_cache=cache.v(l),
                                      row_map=row_map, err_flag=err_flag)
            else:
                qkv = F.linear(h, lw["qkv_w"], lw["qkv_b"])
                K.rope_kv_write(qkv, batch=B, num_nodes=N, q_heads=cfg.q_heads, kv_heads=cfg.kv_heads, head_dim=d,
                                seq_len=seq_len, pos_offset=pos_offset, inv_freq=self.inv_freq, q_out=q,
                                k_cache=cache.k(l), v_cache=cache.v(l), row_map=row_map, err_flag=err_flag)
            K.tree_attention(q, cache.k(l), cache.v(l), seq_len=seq_len, anc=anc, num_nodes=N, q_heads=cfg.q_heads,
                             kv_heads=cfg.kv_heads, head_dim=d, out=attn, row_map=row_map)
            a2 = attn.view(T, cfg.q_heads * d)
            plan = self._linear_plan("o", a2, lw["o_w"])
            if plan:
                # bf16(x + bf16(o_proj)) and the post-attention norm from the parts
                h2 = K.residual_rmsnorm_parts(self._linear_parts(a2, lw["o_w"], plan), x, lw["post_norm"],
                                              cfg.rms_eps, out=self._buf("h", (T, H)))
            else:
                # residual adds inside the GEMMs (beta = 1, the residual stream updated in place):
                # the norms then read one tensor instead of two and write one instead of two
                x.addmm_(a2, lw["o_w"].t())
                h2 = K.rmsnorm(x, lw["post_norm"], cfg.rms_eps, out=self._buf("h", (T, H)))
            act = self._buf("act", (T, cfg.intermediate))
            if self.fused_mlp is None:
                path = mlp_path(T, cfg.intermediate, H, h2.device)
            else:
                # forced fused: the fastest measured tile height of the shape, else the kernel's pick
                path = (mlp_table_fused_tile(T, cfg.intermediate, H) or -1) if self.fused_mlp else 0
            if path and K.gate_up_swiglu_ok(h2, lw["gate_up_w"]):
                K.gate_up_swiglu(h2, lw["gate_up_w"], out=act, tile_rows=max(path, 0))
            else:
                K.swiglu(F.linear(h2, lw["gate_up_w"]), out=act)
            plan = self._linear_plan("down", act, lw["down_w"])
            if plan:
                # the residual add and the next norm (the following layer's input norm, or the final
                # norm into the forward's output) from the parts
                last = l == L - 1
                nw = self.w["final_norm"] if last else self.w["layers"][l + 1]["input_norm"]
                out = (torch.empty(T, H, dtype=self.dtype, device=self.device) if last
                       else self._buf("h", (T, H)))
                K.residual_rmsnorm_parts(self._linear_parts(act, lw["down_w"], plan), x, nw, cfg.rms_eps, out=out)
                st["final" if last else "h"] = out
            else:
                x.addmm_(act, lw["down_w"].t())

    def _linear_plan(self, kind: str, x: torch.Tensor, w: torch.Tensor):
        """(tile_m, tile_n, splits, stages) when projection ``kind`` of x by w runs split-K, else None;
        for QKV, (tile_m, tile_n, 1, stages, "rope") when the projection runs with the rotary + cache
        write in its epilogue (``fg_linear_rope_kv_write``), the measured table's fastest path."""
        if self.split_k_linear is False or not K.linear_ok(x, w):
            return None
        rows, hidden = x.shape
        cols = w.shape[0]
        plan = None if self.split_k_linear else linear_path(kind, rows, cols, hidden)
        if self.split_k_linear:  # forced: the best measured split-K plan of the shape, else the default
            plan = (linear_table_split_plan(kind, rows, cols, hidden)
                    or default_linear_plan(rows, cols, hidden, _cu_count(x.device)))
        if kind == "qkv" and x.dtype == torch.bfloat16 and self.cfg.head_dim % 8 == 0:
            rope = linear_table_times("qkv_rope", rows, cols, hidden)
            base = linear_table_times("qkv", rows, cols, hidden)
            if rope is not None and base is not None:
                # the fused epilogue against the faster of the library and the split-K parts path
                # (against the parts path alone when split-K is forced)
                other = base[1] if self.split_k_linear else min(base[0], base[1] if plan else base[0])
                if rope[1] < other:
                    return (*rope[2][:2], 1, rope[2][3], "rope")
        return plan

    def _rope_pairs(self, l: int):
        """Layer l's q/k/v weight and bias with each q and k head's rows pair-interleaved (the order
        fg_linear_rope_kv_write takes), made on first use and kept with the layer's weights."""
        lw = self.w["layers"][l]
        if lw.get("qkv_w_pairs") is None:
            cfg = self.cfg
            lw["qkv_w_pairs"] = K.rope_pair_rows(lw["qkv_w"], cfg.q_heads, cfg.kv_heads, cfg.head_dim)
            b = lw.get("qkv_b")
            lw["qkv_b_pairs"] = None if b is None else K.rope_pair_rows(b, cfg.q_heads, cfg.kv_heads, cfg.head_dim)
        return lw["qkv_w_pairs"], lw["qkv_b_pairs"]

    def _linear_parts(self, x: torch.Tensor, w: torch.Tensor, plan) -> torch.Tensor:
        tm, tn, s, ns = plan
        parts = self._buf("parts", (s, x.shape[0], w.shape[0]), torch.float32)
        return K.linear_parts(x, w, splits=s, tile=(tm, tn), stages=ns, out=parts)

    def _forward_end(self, st: dict) -> torch.Tensor:
        """The final norm: hidden states [B, N, H] (already written when the last down projection
        ran split-K)."""
        B, N, H = st["B"], st["N"], self.cfg.hidden
        out = st.pop("final", None)
        if out is None:
            out = torch.empty(B * N, H, dtype=self.dtype, device=self.device)
            K.rmsnorm(st["x"], self.w["final_norm"], self.cfg.rms_eps, out=out)
        return out.view(B, N, H)

    def walk_parts(self, rows: int, hidden: torch.Tensor):
        """Row maxima buffers (part_max fp32, part_key int64 [rows, P]) for ``logits(...,
        parts=...)`` when gathered rows of ``hidden`` take the weight-streaming LM head
        (which then writes them), else None."""
        x = hidden.reshape(-1, self.cfg.hidden)
        w = self.w["lm_head"]
        if not (0 < rows <= LM_STREAM_ROWS and lm_stream_ok(x, w)):
            return None
        P = K.lm_head_parts(w.shape[0])
        return (torch.empty(rows, P, dtype=torch.float32, device=x.device),
                torch.empty(rows, P, dtype=torch.int64, device=x.device))

    def logits(self, hidden: torch.Tensor, *, row_index=None, row_active=None, out=None, out_dtype=None,
               weight: torch.Tensor | None = None, parts=None) -> torch.Tensor:
        """LM-head rows: hidden rows (optionally gathered by row_index); rows with
        row_active == 0 may be left unwritten. ``weight`` [V, H] replaces the tied LM
        head (an untied Medusa head's own output projection).

        Up to 256 bf16 rows, contiguous or gathered (the lazy walk's rows, skipped as a
        whole when no row is active), run the weight-streaming LM-head kernel
        (``fg_lm_head_topk``, the weight read once). Larger blocks are a square GEMM and go to
        hipBLASLt (gathered ones after an index_select of their rows); larger gathered sets
        with ``row_active`` and fp32 run ``fg_lm_head``. ``parts`` (from ``walk_parts``): the
        streaming kernel also writes each row's maxima parts.
        """
        x = hidden.reshape(-1, self.cfg.hidden)
        w = self.w["lm_head"] if weight is None else weight
        stream = lm_stream_ok(x, w, out)
        if (row_index is None and row_active is None and self.dtype == torch.bfloat16
                and (out_dtype is None or out_dtype == self.dtype)):
            if x.shape[0] <= LM_STREAM_ROWS and stream:
                return K.lm_head_topk(x, w, 0, out=out, parts=parts)[0]
            if parts is not None:
                raise ValueError("logits: row maxima parts need the weight-streaming LM head (see walk_parts)")
            if out is None:
                return F.linear(x, w)
            return torch.matmul(x, w.t(), out=out)
        rows = row_index.numel() if row_index is not None else x.shape[0]
        if (0 < rows <= LM_STREAM_ROWS and stream
                and (out_dtype is None or out_dtype in (torch.bfloat16, torch.float32))):
            return K.lm_head_topk(x, w, 0, row_index=row_index, row_active=row_active, out=out,
                                  out_dtype=out_dtype, parts=parts)[0]
        if parts is not None:
            raise ValueError("logits: row maxima parts need the weight-streaming LM head (see walk_parts)")
        if (self.dtype == torch.bfloat16 and row_index is not None and row_active is None
                and (out_dtype is None or out_dtype == torch.bfloat16)):
            # a gathered block above the streaming kernel's rows (the packed tree's internal
            # nodes) is a square GEMM: gather its rows (rows x H) and run one hipBLASLt GEMM that
            # reads the weight once, instead of one weight stream per 256 rows
            xs = x.index_select(0, row_index.long())
            if out is None:
                return F.linear(xs, w)
            return torch.matmul(xs, w.t(), out=out)
        if self.dtype == torch.bfloat16 and not lm_gemm_ok(x, w):
            # operands the hand-written kernels do not take (hidden size not a multiple of 64,
            # unaligned rows): hipBLASLt over the gathered rows
            xs = x if row_index is None else x.index_select(0, row_index.long())
            y = F.linear(xs, w).to(out_dtype or self.dtype)
            if out is None:
                return y
            if row_active is None:
                return out.copy_(y)
            return torch.where(row_active.view(-1, 1) != 0, y, out, out=out)
        return K.lm_head(x, w, row_index=row_index, row_active=row_active, out=out, out_dtype=out_dtype)

    def logits_masked(self, hidden: torch.Tensor, row_active: torch.Tensor, out: torch.Tensor) -> None:
        """out[m] = LM-head row of hidden[m] where row_active[m] != 0; the other rows of out
        keep their contents (nothing is computed when no row is active). Decided on the
        device, so a caller need not know the active rows."""
        x = hidden.reshape(-1, self.cfg.hidden)
        w = self.w["lm_head"]
        if out.dtype == torch.bfloat16 and 0 < x.shape[0] <= LM_STREAM_ROWS and lm_stream_ok(x, w, out):
            K.lm_head_topk(x, w, 0, row_active=row_active, out=out)  # inactive rows are not written
            return
        tmp = self.logits(x, row_active=row_active, out_dtype=out.dtype)
        torch.where(row_active.view(-1, 1) != 0, tmp, out, out=out)

    def logits_topk(self, hidden: torch.Tensor, kmax: int, *, stats: bool = False, sanitize: bool = False,
                    logits: bool = False, weight: torch.Tensor | None = None, workspace=None):
        """LM-head rows with each row's top-kmax candidates (value desc, index asc) and
        optionally (max, logsumexp): ``(logits or None, tokens [R, kmax], scores [R, kmax],
        stats [R, 2] or None)``, equal to ``medusa_topk(self.logits(hidden), kmax, ...)``.

        Up to 256 bf16 rows the candidates come from the LM-head kernel's epilogue
        (``fg_lm_head_topk``) without the logits being read back; ``logits`` also returns
        them. Other shapes compute the logits and run ``medusa_topk`` on them.
        """
        x = hidden.reshape(-1, self.cfg.hidden)
        w = self.w["lm_head"] if weight is None else weight
        R = x.shape[0]
        if 0 < R <= LM_STREAM_ROWS and (kmax <= 8 or R <= 192) and kmax >= 1 and lm_stream_ok(x, w):
            return K.lm_head_topk(x, w, kmax, logits=logits, stats=stats, sanitize=sanitize, workspace=workspace)
        lg = self.logits(x, weight=weight)
        tok, sc, st = K.medusa_topk(lg, kmax, stats=stats, sanitize=sanitize)
        return (lg if logits else None), tok, sc, st

    def prefill(self, input_ids: torch.Tensor, cache: KVCache, *, lengths=None, chunk: int = PREFILL_CHUNK,
                row_map: torch.Tensor | None = None, return_all: bool = False) -> torch.Tensor:
        """Causal prefill of left-aligned prompts in chains of ``chunk`` tokens (the
        attention runs without masks: each new token sees the prefix and the chunk's
        tokens before it).

        input_ids [B, P] (device or host) holds each row's valid tokens left-aligned
        (row b has ``lengths[b]`` of them, default P). Writes cache slots [0, len) of
        every row, sets ``cache.seq_len`` and returns the hidden state of each row's
        last token [B, H] (``return_all``: of every position, [B, P, H], left-aligned;
        positions past a row's length hold the hidden state of filler tokens).
        """
        B, P = input_ids.shape
        ids = input_ids.to(self.device, dtype=torch.int32)
        lens = np.full(B, P, dtype=np.int64) if lengths is None else np.asarray(lengths, dtype=np.int64)
        if lens.min() < 1:
            raise ValueError("every prompt needs at least one token")
        seq = torch.zeros(B, dtype=torch.int32, device=self.device)
        cache.seq_len.zero_()
        last = torch.empty(B, self.cfg.hidden, dtype=self.dtype, device=self.device)
        every = torch.zeros(B, P, self.cfg.hidden, dtype=self.dtype, device=self.device) if return_all else None
        chunk = max(1, min(int(chunk), MAX_CHAIN_TOKENS))
        offs_full = torch.arange(chunk, dtype=torch.int32, device=self.device)
        for start in range(0, int(lens.max()), chunk):
            n = min(chunk, P - start)
            tok = ids[:, start:start + n].contiguous()
            hid = self.forward(tok, cache, pos_offset=offs_full[:n], anc=None, seq_len=seq, row_map=row_map)
            if every is not None:
                every[:, start:start + n].copy_(hid)
            adv = np.clip(lens - start, 0, n)
            ends = np.nonzero((lens > start) & (lens <= start + n))[0]
            if ends.size:
                e = torch.from_numpy(ends).to(self.device)
                pos = torch.from_numpy(lens[ends] - start - 1).to(self.device)
                last.index_copy_(0, e, hid[e, pos])
            seq += torch.from_numpy(adv.astype(np.int32)).to(self.device)
        if row_map is None:
            cache.seq_len.copy_(seq)
        else:
            cache.seq_len.index_copy_(0, row_map.long(), seq)
        return every if return_all else last


def native_tree_inputs(mask4d: torch.Tensor, pos: torch.Tensor, seq_len: torch.Tensor):
    """(anc int64 [B, N], pos_offset int32 [B, N]) of the native verify forward from the
    reference's additive mask [B, 1, N, P + N] and position ids [B, N]: bit m of node n's
    word is set where the mask's tree block lets n see node m; offsets are positions
    minus each row's committed length. On the device of ``mask4d``."""
    N = mask4d.shape[2]
    allowed = mask4d[:, 0, :, -N:] > torch.finfo(mask4d.dtype).min / 2           # [B, N, N]
    shifts = torch.arange(N, dtype=torch.int64, device=allowed.device)
    anc = (allowed.to(torch.int64) << shifts).sum(-1)                              # distinct bits: sum == or
    offset = pos.to(device=allowed.device, dtype=torch.int64) - seq_len.to(device=allowed.device,
                                                                            dtype=torch.int64)[:, None]
    return anc.contiguous(), offset.to(torch.int32).contiguous()


def forward_tree(causal_lm: TargetModel, ids: torch.Tensor, mask4d: torch.Tensor, pkv: KVCache, pos: torch.Tensor, *,
                 clone_past: bool = True, compute_logits: bool = True) -> dict:
    """Tree-verify forward with the reference's call shape
    (``flashgrpo/models/qwen_flashgrpo_wrapper.py:220-239``).

    ``ids`` [B, N], ``mask4d`` [B, 1, N, P + N] and ``pos`` [B, N] are the outputs of
    ``decoding.tree_attention.build_tree_attention_inputs``. The tree block of the
    additive mask (its last N columns) becomes one ancestor-or-self bit word per node,
    applied in registers by the tree-attention kernel; the prefix a node sees is the
    cache row's committed tokens ``[0, pkv.seq_len[b])`` (the valid prefix slots the
    reference's mask marks), and positions become offsets from ``pkv.seq_len``. Node
    n's K/V land in slot ``seq_len[b] + n``, past the committed tokens, so the past's
    committed rows are never modified. ``clone_past`` (the reference's container copy,
    ``clone_cache(clone_tensors=False)``) returns the tree in a second cache object over
    the same storage with its own lengths, so extracting a path from it leaves ``pkv``'s
    lengths as they were; otherwise ``pkv`` itself is returned. Returns
    ``{"hidden_states": [B, N, H], "logits": [B, N, V] or None, "past_key_values": cache}``.
    """
    B, N = ids.shape
    if mask4d.dim() != 4 or mask4d.shape[0] != B or mask4d.shape[2] != N or mask4d.shape[3] < N:
        raise ValueError(f"forward_tree: mask4d {tuple(mask4d.shape)} does not match ids {tuple(ids.shape)}")
    if N > 64:
        raise ValueError("forward_tree: trees larger than 64 nodes are not supported")
    if B != pkv.batch:
        raise ValueError(f"forward_tree: {B} trees for a cache of {pkv.batch} rows")
    dev = causal_lm.device
    seq = pkv.seq_len.to(mask4d.device, torch.int64)
    # The prefix block (the reference's full_attention_mask, tree_attention.py:61-64) must
    # show every node of row b the same set of exactly seq_len[b] slots: the cache row's
    # committed tokens, which are what the native forward attends.
    P = mask4d.shape[3] - N
    vis = mask4d[:, 0, :, :P] > torch.finfo(mask4d.dtype).min / 2
    if P and (not bool((vis == vis[:, :1]).all()) or not bool((vis[:, 0].sum(-1) == seq).all())):
        raise ValueError("forward_tree: the mask's prefix block must let every node of row b see exactly the "
                         "row's seq_len[b] committed cache tokens")
    if P == 0 and bool((seq != 0).any()):
        raise ValueError("forward_tree: the mask has no prefix block but the cache holds committed tokens")
    if int(seq.max()) + N > pkv.capacity:
        raise ValueError(f"forward_tree: {N} tree nodes after {int(seq.max())} committed tokens exceed the "
                         f"cache capacity {pkv.capacity}")
    anc, offset = native_tree_inputs(mask4d, pos, pkv.seq_len)
    tree_cache = pkv.container_copy() if clone_past else pkv
    err = torch.zeros(1, dtype=torch.int32, device=dev)
    hidden = causal_lm.forward(ids.to(device=dev, dtype=torch.int32), tree_cache, pos_offset=offset.to(dev),
                               anc=anc.to(dev), err_flag=err)
    if int(err.item()):
        raise RuntimeError(f"forward_tree: a cache write fell outside the cache (flag {int(err.item())})")
    logits = causal_lm.logits(hidden.reshape(B * N, -1)).view(B, N, -1) if compute_logits else None
    return {"hidden_states": hidden, "logits": logits, "past_key_values": tree_cache}
