"""FlashMedusaDecoder: the speculative rollout loop on the device.

Same configuration dataclass, constructor and ``generate`` contract as
``flashgrpo/decoding/flash_medusa_decoder.py:41-134,550-1229`` (result keys
included). One verify round, per active sequence:

  root draw            fg_sample_tokens (draw 0; b200 mode: pending correction forced)
  Medusa proposals     fg_medusa_heads -> fg_lm_head_topk (tied LM head with the
                       per-depth top-k and row stats in its epilogue)
  plan / tree          plan_tree (host), adaptive refit from per-head confidence
                       quantiles, cached TreeTopology, fg_tree_layout
  chain proposals      (proposal_mode="chain") per depth: fg_lm_head over every parent
                       state -> fg_medusa_topk (sanitised, + row stats) -> children
                       in dense-BFS order under the budget -> ChainDraftCell step
  tree verify          TargetModel.forward (tree attention with ancestor bit masks)
  acceptance           lazy (default): per walk step t, fg_lm_head_topk over the node
                       each row samples from (with the rows' maxima) -> fg_walk_step
                       (draw 1+t; it also writes the next step's rows);
                       packed: fg_lm_head over internal nodes + fg_accept_walk;
                       then fg_accept_finalize (clamp, EOS)
  cache update         fg_kv_path_gather (extract_path) or a chain re-forward
                       (recompute_accepted)
  next state           hidden at the last accepted node; its logits row from the
                       walk (lazy) or the packed projection, or a fresh LM-head row
                       when it is a leaf

There is one device-to-host copy per round (accepted tokens, lengths, flags),
plus one for the adaptive-plan confidences when that mode is on (one per
depth in chain mode). Draws use counter noise keyed by (seed, round, sequence
id, draw index), so results do not depend on batch composition or on which
rows finished earlier.

Not built here (rejected at construction): reflex fast-state proposals
(``reflex_enabled``).
"""
from __future__ import annotations

import math
import time
import warnings
from dataclasses import dataclass

import numpy as np
import torch

from .. import kernels as K
from .. import timing
from ..models.target import TargetModel, as_mask_tensor, chain_bits
from .medusa_tree import (TreePlan, TreeTopology, dense_node_count, fit_topk_to_budget, plan_tree, sparse_tree_device,
                          sparse_widths)


@dataclass
class FlashMedusaConfig:
    num_medusa_heads: int = 3
    tree_mode: str = "concurrency_aware"
    tree_layout: str = "dense"
    acceptance: str = "exact_target"
    cache_update_mode: str = "extract_path"
    allow_recompute_fallback: bool = True
    cpeak_nodes: int = 64
    min_tree_nodes_per_seq: int = 1
    max_tree_nodes_per_seq: int = 16
    max_tree_depth: int = 4
    fixed_tree_topk_by_depth: tuple = (4, 3, 2)
    do_sample: bool = True
    temperature: float = 1.0
    top_p: float = 0.95
    top_k: int | None = None
    clone_tree_cache: bool = True
    oom_shrink_factor: float = 0.5
    enable_medusa_spec_after: int = 0
    proposal_mode: str = "medusa"
    chain_enable_after: int = 0
    chain_bootstrap_from_medusa: bool = True
    adaptive_tree_enabled: bool = False
    adaptive_confidence_metric: str = "top1_prob"
    adaptive_confidence_quantile: float = 0.25
    adaptive_confidence_low: float = 0.15
    adaptive_confidence_high: float = 0.45
    adaptive_min_topk_by_depth: tuple = (1, 1, 1)
    adaptive_depth_weight_decay: float = 0.5
    head_inference_autocast: bool = True
    project_internal_tree_logits_only: bool = True
    inplace_kv_compaction: bool = True
    reflex_enabled: bool = False
    # Reflex fast-state settings (flash_medusa_decoder.py:74-116). Accepted so that the
    # trainer's config builder (flashgrpo_trainer.py:555-633) constructs this class
    # unchanged; reflex proposals themselves are not built (reflex_enabled=True raises).
    reflex_state_space: str = "projected"
    reflex_fast_state_dim: int = 128
    reflex_beta: float = 0.95
    reflex_eta: float = 0.1
    reflex_top_m_feedback: int = 64
    reflex_feedback_stride: int = 1
    reflex_feedback_stride_min: int = 1
    reflex_target_topk: int = 32
    reflex_feedback_union_cap: int = 96
    reflex_tv_gate_low: float = 0.05
    reflex_tv_gate_high: float = 0.20
    reflex_horizon_weight_decay: float = 0.85
    reflex_half_life_tokens: float = 48.0
    reflex_feedback_variance_beta: float = 0.99
    reflex_feedback_rms_clip: float = 3.0
    reflex_state_rms_clip: float = 2.0
    reflex_numerical_reset_rms: float = 2.5
    reflex_relative_rms_delta_base: float = 0.01
    reflex_warmup_effective_updates: float = 16.0
    reflex_magnitude_gate_floor: float = 0.25
    reflex_guard_calibration_rollouts: int = 20
    reflex_guard_aal_drop_fraction: float = 0.05
    reflex_guard_patience: int = 2
    reflex_guard_disable_rollouts: int = 50
    reflex_feedback_clip_norm: float = 2.0
    reflex_hidden_feedback_clip_norm: float = 0.0
    reflex_fast_state_clip_norm: float = 8.0
    reflex_correction_clip_norm: float = 1.0
    reflex_normalize_correction: bool = True
    reflex_feedback_ce_gate: bool = True
    reflex_feedback_ce_tau: float = 4.0
    reflex_feedback_ce_threshold: float = 0.4
    reflex_normalize_feedback: bool = True
    reflex_feedback_enabled: bool = False
    reflex_proposal_injection_enabled: bool = False
    reflex_proposal_injection_scale: float = 0.0
    reflex_proposal_injection_after: int = 0
    reflex_proposal_injection_warmup: int = 0
    reflex_aux_cache_enabled: bool = False
    reflex_aux_cache_max_records: int = 8192
    reflex_aux_cache_stride: int = 1
    reflex_aux_store_fast_state: bool = False
    # build additions
    emit_correction_token: bool = False  # flashgrpo_b200 acceptance semantics
    noise_seed: int | None = None        # None: drawn from torch's default generator per generate()
    # Project tree LM-head rows lazily, one walk step at a time, for the node each
    # row's walk samples from (at most batch rows per step). Draws, accepted paths
    # and next-round logits are identical to the packed projection; only nodes the
    # walk never reaches are skipped.
    lazy_walk_lm_head: bool = True
    # Replay the verify forward as one HIP graph per (batch, tree width) once that shape
    # repeats; identical results, one launch instead of ~9 per layer.
    graph_verify_forward: bool = True
    # tree_layout="sparse_asymmetric" (flashgrpo_b200/decoding/flash_medusa_decoder.py:65-73);
    # the head-3 quality calibrator and its exploration rounds are not built: every
    # row keeps head 3 (build_batch_trees accepts an explicit per-row gate).
    sparse_nodes_by_head: tuple = (5, 4, 0)
    sparse_min_head3_nodes: int = 0
    sparse_head3_min_budget: int = 8
    sparse_branch_score_temperature: float = 1.0
    sparse_diversity_penalty: float = 0.05


def _quantile(values: np.ndarray, q: float) -> float:
    """Linear-interpolation quantile (torch.quantile's default)."""
    return _quantile_rows(values.reshape(1, -1), q)[0]


def _quantile_rows(values: np.ndarray, q: float) -> list:
    """``_quantile`` of every row of a 2-D array (float64)."""
    v = np.sort(values.astype(np.float64), axis=1)
    pos = q * (v.shape[1] - 1)
    lo = int(math.floor(pos))
    hi = min(lo + 1, v.shape[1] - 1)
    return (v[:, lo] + (v[:, hi] - v[:, lo]) * (pos - lo)).tolist()


class FlashMedusaDecoder:
    def _arange(self, n: int, dev) -> torch.Tensor:
        """arange(n) on dev, made once (one fewer launch per use in the per-round path)."""
        key = (int(n), str(dev))
        t = self._ar_cache.get(key)
        if t is None:
            t = self._ar_cache[key] = torch.arange(int(n), device=dev)
        return t

    def __init__(self, target_model, medusa_heads, tokenizer, config: FlashMedusaConfig):
        self._fit_cache = {}  # (adapted top-k, budget) -> fitted top-k
        self._ar_cache = {}   # (n, device) -> arange(n), read-only
        if config.acceptance != "exact_target":
            raise NotImplementedError("Only exact_target acceptance is implemented in the main FlashGRPO path")
        if config.cache_update_mode not in {"extract_path", "recompute_accepted"}:
            raise ValueError(f"Unsupported cache_update_mode={config.cache_update_mode}")
        if config.proposal_mode not in {"medusa", "chain"}:
            raise ValueError(f"Unsupported proposal_mode={config.proposal_mode}")
        if config.reflex_enabled:
            raise NotImplementedError("reflex fast-state proposals are not built in flashgrpo_amd")
        self.target_model = target_model
        # A Hugging Face target is converted once here and re-read in place at the
        # start of every rollout whose parameters changed since (start()).
        self.model = target_model if isinstance(target_model, TargetModel) else TargetModel.from_hf(target_model)
        self.medusa_heads = medusa_heads
        self.tokenizer = tokenizer
        self.config = config
        for i, hd in enumerate(getattr(medusa_heads, "heads", [])):
            out = getattr(hd, "output", None)
            if out is not None and tuple(out.weight.shape) != (self.model.cfg.vocab, self.model.cfg.hidden):
                raise ValueError(f"untied Medusa head {i}: output {tuple(out.weight.shape)} does not match the "
                                 f"target's (vocab, hidden) = ({self.model.cfg.vocab}, {self.model.cfg.hidden})")

    # ------------------------------------------------------------------ helpers
    def _token_ids(self):
        tok = self.tokenizer
        pad = getattr(tok, "pad_token_id", None)
        eos = getattr(tok, "eos_token_id", None)
        if pad is None:
            pad = eos
        if pad is None:
            pad = 0
        if eos is None:
            eos = pad
        return int(pad), int(eos)

    def _plan(self, active_bsz: int) -> TreePlan:
        cfg = self.config
        return plan_tree(active_batch_size=active_bsz,
                         num_medusa_heads=min(cfg.num_medusa_heads, self.medusa_heads.num_heads),
                         tree_mode=cfg.tree_mode, tree_layout=cfg.tree_layout, cpeak_nodes=cfg.cpeak_nodes,
                         min_tree_nodes_per_seq=cfg.min_tree_nodes_per_seq,
                         max_tree_nodes_per_seq=cfg.max_tree_nodes_per_seq, max_tree_depth=cfg.max_tree_depth,
                         fixed_tree_topk_by_depth=list(cfg.fixed_tree_topk_by_depth),
                         adaptive_tree_enabled=bool(cfg.adaptive_tree_enabled),
                         adaptive_min_topk_by_depth=list(cfg.adaptive_min_topk_by_depth),
                         sparse_nodes_by_head=list(cfg.sparse_nodes_by_head),
                         sparse_min_head3_nodes=int(cfg.sparse_min_head3_nodes),
                         sparse_head3_min_budget=int(cfg.sparse_head3_min_budget),
                         sparse_branch_score_temperature=float(cfg.sparse_branch_score_temperature),
                         sparse_diversity_penalty=float(cfg.sparse_diversity_penalty))

    def _topk_from_confidence(self, confidence: float, base_k: int, depth_idx: int) -> int:
        """``flash_medusa_decoder.py:341-360``."""
        cfg = self.config
        base_k = max(1, int(base_k))
        mins = list(cfg.adaptive_min_topk_by_depth) or [1]
        min_k = max(1, min(base_k, int(mins[min(depth_idx, len(mins) - 1)])))
        if (not cfg.adaptive_tree_enabled) or base_k <= min_k:
            return base_k
        if not math.isfinite(float(confidence)):
            return min_k
        low, high = float(cfg.adaptive_confidence_low), float(cfg.adaptive_confidence_high)
        if high <= low:
            return min_k if confidence >= high else base_k
        if confidence <= low:
            return base_k
        if confidence >= high:
            return min_k
        ratio = (confidence - low) / (high - low)
        return max(min_k, min(base_k, int(round(base_k - ratio * (base_k - min_k)))))

    def _adapt_plan(self, plan: TreePlan, stats: np.ndarray, cand_scores: np.ndarray, batch: int):
        """Confidence quantile per head -> branching -> budget refit (``flash_medusa_decoder.py:320-389``).

        top1_prob confidence = exp(max - logsumexp) of each head's logits row;
        margin = top1 - top2 of the candidate scores.
        """
        cfg = self.config
        heads = min(len(plan.topk_by_depth), plan.active_heads)
        q = min(1.0, max(0.0, float(cfg.adaptive_confidence_quantile)))
        # every head at once (the host time here is on the round's critical path): per row
        # the score, non-finite -> 0, then the linear-interpolation quantile per head
        if cfg.adaptive_confidence_metric == "margin":
            sc = cand_scores[:heads * batch].reshape(heads, batch, -1)
            score = sc[..., 0] - sc[..., 1] if sc.shape[2] > 1 else sc[..., 0]
        else:
            st = stats[:heads * batch].astype(np.float64).reshape(heads, batch, 2)
            score = np.exp(st[..., 0] - st[..., 1])
        score = np.where(np.isfinite(score), score, 0.0).astype(np.float64)
        confs = _quantile_rows(score, q)
        adapted = [self._topk_from_confidence(c, int(k), d) for d, (k, c) in
                   enumerate(zip(plan.topk_by_depth, confs))]
        if adapted:
            key = (tuple(adapted), int(plan.node_budget_per_seq))
            fitted = self._fit_cache.get(key)
            if fitted is None:
                fitted = self._fit_cache[key] = fit_topk_to_budget(
                    adapted, plan.node_budget_per_seq,
                    min_topk_by_depth=list(cfg.adaptive_min_topk_by_depth)[:len(adapted)],
                    depth_weight_decay=float(cfg.adaptive_depth_weight_decay))
            adapted = list(fitted)
        ks = [max(1, int(k)) for k in adapted]
        # a sparse plan takes the fitted list as its per-head node counts
        # (flashgrpo_b200/decoding/flash_medusa_decoder.py:1063-1077)
        new = TreePlan(plan.node_budget_per_seq, len(ks), ks, dense_node_count(ks), plan.mode, plan.layout,
                       list(ks) if plan.layout == "sparse_asymmetric" else [], plan.min_head3_nodes,
                       plan.head3_min_budget, plan.branch_score_temperature, plan.diversity_penalty)
        return new, {"confidence": confs, "topk": list(adapted)}

    def _chain_trees(self, r: "Rollout", roots: torch.Tensor, plan: TreePlan, Bc: int, record: bool):
        """Chain proposals (``flash_medusa_decoder.py:435-539``).

        The first parent state is Medusa head 0's residual output of the hidden state
        (``chain_bootstrap_from_medusa``), else the chain cell on (hidden, root
        embedding). Depth d projects every parent state through the LM head, ranks
        nan_to_num'd logits (value desc, index asc), takes the confidence quantile over
        all parent rows, maps it to k_d (no budget refit) and gives each parent in order
        its top-k_d children while its row holds fewer than the node budget. All rows
        share one topology (the dense BFS of the adapted k list cut at the budget), so
        child c of depth d+1 is rank c % k_d of parent c // k_d and every step is a
        batched gather. Each child's state is the cell applied to its parent's state
        and its token's embedding; the states after the last depth are not computed
        (nothing reads them).

        Returns (tree_tokens [Bc, N] int32, chain plan, info) where info holds the
        adaptive stats, the device confidences still to be read (non-adaptive), the
        LM-head rows of each depth and the per-depth trace records.
        """
        cfg = self.config
        model, heads = self.model, self.medusa_heads
        dev = r.device
        H, V = model.cfg.hidden, model.cfg.vocab
        emb = model.embed_weight
        adaptive = bool(cfg.adaptive_tree_enabled)
        margin = cfg.adaptive_confidence_metric == "margin"
        q = min(1.0, max(0.0, float(cfg.adaptive_confidence_quantile)))
        if cfg.chain_bootstrap_from_medusa and heads.num_heads > 0:
            states = heads.heads[0].project_hidden(r.hidden)
        else:
            states = heads.chain_next_state(r.hidden, roots, emb)
        budget = int(plan.node_budget_per_seq)
        ks = list(plan.topk_by_depth)
        cols = [roots.view(Bc, 1)]
        nodes, n_d = 1, 1
        adapted, confs_host, confs_dev, recs, rows = [], [], [], [], []
        for d, base_k in enumerate(ks):
            base_k = max(1, int(base_k))
            if nodes >= budget and not adaptive:
                # the reference projects these states only to report k_d, which is
                # base_k without adaptation; the tree gets no nodes at this depth
                adapted.append(base_k)
                break
            kq = min(max(base_k, 2 if margin else 1), V)
            with timing.label("chain"):
                # candidates (and confidences) from the LM-head epilogue; the logits
                # themselves only when the round is recorded
                lg, cand, score, st = model.logits_topk(states.to(model.dtype), kq, stats=not margin, sanitize=True,
                                                        logits=record)
            rows.append(int(states.shape[0]))
            if margin:
                row_conf = score[:, 0] - score[:, 1] if kq > 1 else score[:, 0]
            else:
                row_conf = torch.exp(st[:, 0] - st[:, 1])
            if adaptive:
                # k_d decides the next depth's width: one sync per depth, with the
                # quantile taken on the host (torch.quantile's linear rule)
                rc = row_conf.float().cpu().numpy()
                conf = _quantile(np.nan_to_num(rc, nan=0.0, posinf=0.0, neginf=0.0), q)
                confs_host.append(conf)
                k = self._topk_from_confidence(conf, base_k, d)
            else:
                conf_d = torch.quantile(torch.nan_to_num(row_conf, nan=0.0, posinf=0.0, neginf=0.0), q)
                confs_dev.append(conf_d)
                k = base_k
            adapted.append(k)
            kk = min(k, V)
            n_next = min(n_d * kk, budget - nodes)
            rec = dict(k=k, states=states, logits=lg, cand=cand) if record else None
            if n_next <= 0:
                if record:
                    recs.append(rec)
                break
            j = torch.arange(n_next, device=dev)
            par, rank = j // kk, j % kk
            tok = cand.view(Bc, n_d, kq)[:, par, rank]
            cols.append(tok)
            if record:
                rec.update(parent_local=par.cpu().numpy(), rank=rank.cpu().numpy())
                recs.append(rec)
            nodes += n_next
            if d + 1 < len(ks) and (nodes < budget or adaptive):
                ps = states.view(Bc, n_d, H)[:, par].reshape(Bc * n_next, H)
                states = heads.chain_next_state(ps, tok.reshape(-1), emb)
            n_d = n_next
        ks_out = [max(1, int(k)) for k in adapted]
        chain_plan = TreePlan(budget, len(ks_out), ks_out, nodes, plan.mode, plan.layout)
        info = dict(stats={"confidence": confs_host, "topk": list(adapted)}, rows=rows, recs=recs,
                    conf=torch.stack(confs_dev).float() if confs_dev else None)
        return torch.cat(cols, dim=1).contiguous(), chain_plan, info

    def _medusa_candidates(self, proj: torch.Tensor, heads: int, batch: int, kc: int, *, stats: bool,
                           logits: bool):
        """Per-row top-kc candidates of the proposal logits (medusa_tree.py:239-252) and,
        with ``stats``, each row's (max, logsumexp): ``(logits or None, tokens, scores,
        stats)``. Tied heads take them from the LM-head kernel's epilogue in one launch
        over every head's rows; untied heads compute the logits first."""
        own = self.medusa_heads.output_weights(proj.dtype, self.model.device)[:heads]
        if all(w is None for w in own):
            return self.model.logits_topk(proj.to(self.model.dtype), kc, stats=stats, logits=logits)
        mlog = self._medusa_logits(proj, heads, batch)
        cand, score, st = K.medusa_topk(mlog, kc, stats=stats)
        return mlog, cand, score, st

    def _medusa_logits(self, proj: torch.Tensor, heads: int, batch: int) -> torch.Tensor:
        """[heads*B, V] proposal logits (``flash_medusa_decoder.py:281-304``): one LM-head
        GEMM over every head's rows when all heads are tied, otherwise each head's rows
        through its own ``output`` projection (an untied head) or the LM head.

        ``proj`` is in the model's dtype under the heads' autocast, else in the heads'
        parameter dtype (``medusa_heads.py:266-276`` without autocast): the LM head then
        takes the rows cast to the model's dtype and an untied head's own projection runs
        in the heads' dtype, so mixed heads give logits in that dtype (the LM head's bf16
        values held exactly)."""
        model = self.model
        own = self.medusa_heads.output_weights(proj.dtype, model.device)[:heads]
        if all(w is None for w in own):
            return model.logits(proj.to(model.dtype))
        out = torch.empty((heads * batch, model.cfg.vocab), dtype=proj.dtype, device=model.device)
        for h, w in enumerate(own):
            rows = slice(h * batch, (h + 1) * batch)
            if proj.dtype == model.dtype:
                model.logits(proj[rows], out=out[rows], weight=w)
            elif w is None:
                out[rows].copy_(model.logits(proj[rows].to(model.dtype)))
            else:
                torch.matmul(proj[rows], w.t(), out=out[rows])
        return out

    # ------------------------------------------------------------------ rollout
    @torch.no_grad()
    def start(self, input_ids: torch.Tensor, attention_mask: torch.Tensor, *, repeated_generate_nums=None,
              max_length: int = 2048, statistical_time: bool = False, generation_step: int = 0) -> "Rollout":
        """Prefill the prompts (left padding compacted away), repeat rows for GRPO
        groups and return the rollout state before the first verify round."""
        cfg = self.config
        model = self.model
        model.sync_from_hf()  # the policy may have stepped since the last rollout
        dev = model.device
        V = model.cfg.vocab
        repeats = max(1, int(repeated_generate_nums or 1))
        if cfg.noise_seed is None:
            seed = int(torch.randint(0, 2 ** 62, (1,)).item())
        else:
            seed = (int(cfg.noise_seed) * 1000003 + int(generation_step)) & (2 ** 64 - 1)
        r = Rollout(seed=seed, max_length=int(max_length), statistical_time=bool(statistical_time),
                    generation_step=int(generation_step), device=dev)
        r.total_start = time.time()
        ids_h = input_ids.detach().cpu()
        mask_h = attention_mask.detach().cpu().bool()
        B0 = ids_h.shape[0]
        lens = mask_h.sum(-1).numpy().astype(np.int64)
        if lens.min() < 1:
            raise ValueError("every prompt needs at least one unmasked token")
        valid_ids = ids_h[mask_h]
        if int(valid_ids.min()) < 0 or int(valid_ids.max()) >= V:
            raise ValueError(f"input token ids must lie in [0, {V})")
        pmax = int(lens.max())
        # Slots past a row's length are never attended; fill them with token 0.
        packed = torch.zeros((B0, pmax), dtype=torch.int32)
        for b in range(B0):
            packed[b, :lens[b]] = ids_h[b][mask_h[b]].to(torch.int32)
        B = B0 * repeats
        capacity = max(int(max_length), pmax + 1) + 80
        r.cache = model.new_cache(B, capacity)
        first_rows = torch.arange(B0, dtype=torch.int32, device=dev) * repeats
        r.sync()
        t0 = time.time()
        last_hidden = model.prefill(packed.to(dev), r.cache, lengths=lens, row_map=first_rows)
        first_logits = model.logits(last_hidden)
        r.sync()
        r.prefill_time = time.time() - t0
        if repeats > 1:
            src = torch.arange(B0, device=dev).repeat_interleave(repeats) * repeats
            dst = torch.arange(B, device=dev)
            dup = (dst % repeats) != 0
            r.cache.repeat_rows(src[dup].to(torch.int32), dst[dup].to(torch.int32))
            r.hidden = last_hidden.repeat_interleave(repeats, dim=0).contiguous()
            r.logits = first_logits.repeat_interleave(repeats, dim=0).contiguous()
        else:
            r.hidden, r.logits = last_hidden, first_logits
        r.active = list(range(B))
        r.row_map = torch.arange(B, dtype=torch.int32, device=dev)
        r.seq = r.cache.seq_len.clone()
        r.seq_h = np.repeat(lens, repeats).astype(np.int64)
        r.pending = torch.full((B,), -1, dtype=torch.int32, device=dev) if cfg.emit_correction_token else None
        r.generated = [[] for _ in range(B)]
        r.err = torch.zeros(1, dtype=torch.int32, device=dev)
        return r

    def _front(self, r: "Rollout", rnd: int, logits, hidden, row_map, pending, record: bool) -> dict:
        """The device work that opens round ``rnd``: the root draw and, for Medusa
        proposals, the heads and the tied LM head with the per-depth top-k (and row
        stats) over the given next-state rows. Nothing here waits for the host."""
        cfg = self.config
        greedy = (not cfg.do_sample) or cfg.temperature == 0
        Bc = int(row_map.shape[0])
        roots = K.sample_tokens(logits, seed=r.seed, step=rnd, seq_ids=row_map, draw=0, forced=pending,
                                temperature=cfg.temperature, greedy=greedy, top_k=cfg.top_k, top_p=cfg.top_p)
        use_tree = r.generation_step >= int(cfg.enable_medusa_spec_after)
        plan = self._plan(Bc) if use_tree else TreePlan(1, 0, [], 1, cfg.tree_mode, cfg.tree_layout)
        use_chain = use_tree and cfg.proposal_mode == "chain" and r.generation_step >= int(cfg.chain_enable_after)
        f = dict(rnd=rnd, batch=Bc, roots=roots, plan=plan, use_tree=use_tree, use_chain=use_chain, med=None)
        if plan.active_heads > 0 and not use_chain:
            # the heads under bf16 autocast (head_inference_autocast, flash_medusa_decoder.py:
            # 268-272), else in their parameter dtype
            heads_dt = hidden.dtype if cfg.head_inference_autocast else self.medusa_heads.heads[0].norm.weight.dtype
            proj = self.medusa_heads.project_all(hidden.to(heads_dt), plan.active_heads)
            V = self.model.cfg.vocab
            if plan.layout == "sparse_asymmetric":
                # candidate lists of the sparse widths (adaptation only shrinks them)
                kc = max(sparse_widths(list(plan.nodes_by_head or plan.topk_by_depth)[:3], V))
            else:
                kc = max(plan.topk_by_depth)
            if cfg.adaptive_tree_enabled and cfg.adaptive_confidence_metric == "margin":
                kc = max(kc, min(2, V))  # margin = top-1 - top-2 (flash_medusa_decoder.py:327-331)
            with timing.label("medusa"):
                f["med"] = self._medusa_candidates(proj, plan.active_heads, Bc, kc,
                                                   stats=bool(cfg.adaptive_tree_enabled), logits=record)
            if cfg.adaptive_tree_enabled:
                _, _, score, stats = f["med"]
                # what the adaptive plan reads back: (max, logsumexp) and the candidate scores
                f["both_d"] = torch.cat([stats.view(stats.shape[0], -1), score.view(score.shape[0], -1)], 1)
        return f

    def _front_rows(self, f: dict, keep: np.ndarray) -> dict | None:
        """``f`` restricted to the rows that continue (their draws and candidates do not
        depend on the other rows), or None when the plan of the smaller batch differs."""
        Bn = int(keep.size)
        plan = self._plan(Bn) if f["use_tree"] else f["plan"]
        if Bn == 0 or plan != f["plan"]:
            return None
        dev = f["roots"].device
        kt = torch.from_numpy(keep).to(dev)
        g = dict(f, batch=Bn, roots=f["roots"].index_select(0, kt))
        if f["med"] is not None:
            heads = f["plan"].active_heads
            rows_np = (np.arange(heads)[:, None] * f["batch"] + keep[None, :]).reshape(-1)
            rows = torch.from_numpy(rows_np).to(dev)
            g["med"] = tuple(None if t is None else t.index_select(0, rows) for t in f["med"])
            if f.get("both_d") is not None:
                g["both_d"] = f["both_d"].index_select(0, rows)
            if f.get("both_h") is not None:
                g["both_h"] = f["both_h"][rows_np]
        return g

    @torch.no_grad()
    def step(self, r: "Rollout", trace: list | None = None) -> int:
        """One verify round over the active rows; returns the tokens it emitted.

        Rounds are pipelined on the host: a round is queued (``_launch``: proposals, tree,
        verify forward, walk, KV extraction, next state, the next round's proposals, the
        read-back), and a call completes the queued round (``_complete``: its one host
        sync, state update, finished rows dropped), queues the next round at once, and
        only then does the completed round's bookkeeping (``_bookkeep``), so the GPU runs
        the next round while the host works. Without pipelining (``statistical_time``,
        a trace being recorded) a call queues and completes one round."""
        ctx = r.inflight if r.inflight is not None else self._launch(r, trace)
        r.inflight = None
        res = self._complete(r, ctx, trace)
        if r.active and not r.statistical_time and trace is None:
            r.inflight = self._launch(r, None)
        return self._bookkeep(r, ctx, res, trace)

    @torch.no_grad()
    def flush(self, r: "Rollout") -> int:
        """Complete a round queued by ``step`` (returns its tokens; 0 if none is queued).
        Call before reading or changing the rollout's device state directly."""
        ctx, r.inflight = r.inflight, None
        if ctx is None:
            return 0
        return self._bookkeep(r, ctx, self._complete(r, ctx, None), None)

    def _launch(self, r: "Rollout", trace: list | None) -> dict:
        """Queue one verify round; nothing here waits for the GPU except the adaptive
        plan's read-back when the round's proposals were not queued by the previous one."""
        cfg = self.config
        model = self.model
        dev = r.device
        m = r.m
        greedy = (not cfg.do_sample) or cfg.temperature == 0
        b200 = bool(cfg.emit_correction_token)
        _, eos_id = self._token_ids()
        Bc = len(r.active)
        rnd = m["rounds"]
        f, r.front = r.front, None
        if f is None or f["rnd"] != rnd or f["batch"] != Bc:
            r.sync()
            t0 = time.time()
            f = self._front(r, rnd, r.logits, r.hidden, r.row_map, r.pending, trace is not None)
            r.sync()
            m["medusa_time"] += time.time() - t0
        roots, plan, use_tree, use_chain = f["roots"], f["plan"], f["use_tree"], f["use_chain"]
        cand = score = mlog = tree_tokens = chain_conf = sparse = None
        chain_recs, chain_rows = [], []
        adaptive_stats = {}
        if plan.active_heads > 0 and use_chain:
            r.sync()
            t0 = time.time()
            tree_tokens, plan, info = self._chain_trees(r, roots, plan, Bc, trace is not None)
            adaptive_stats, chain_conf = info["stats"], info["conf"]
            chain_recs, chain_rows = info["recs"], info["rows"]
            if chain_conf is not None:
                # confidences reported without adaptation: read after the round's one sync
                conf_h = torch.empty(chain_conf.shape, dtype=torch.float32, pin_memory=True)
                conf_h.copy_(chain_conf, non_blocking=True)
            r.sync()
            m["medusa_time"] += time.time() - t0
        elif plan.active_heads > 0:
            V = self.model.cfg.vocab
            mlog, cand, score, stats = f["med"]
            if cfg.adaptive_tree_enabled:
                # read back with the previous round's results when that round queued this one
                both = f["both_h"] if f.get("both_h") is not None else f["both_d"].cpu().numpy()
                plan, adaptive_stats = self._adapt_plan(plan, both[:, :2], both[:, 2:], Bc)
            if plan.layout == "sparse_asymmetric" and plan.active_heads > 0:
                sparse = sparse_tree_device(roots, cand, score, plan, Bc, V)
        if sparse is not None:
            # per-row topology (b200 sparse_asymmetric): rows padded to the widest bound
            tree_tokens = sparse["tokens"]
            N = tree_tokens.shape[1]
            D = min(3, plan.active_heads)
            tv = dict(pos_offset=sparse["pos_offset"], anc=sparse["anc"], parents=sparse["parents"],
                      n_nodes=sparse["n_nodes"], internal_rows=None, slot_map=None)
        else:
            topo = TreeTopology.for_plan(plan)
            N = topo.num_nodes
            D = topo.max_depth
        plan_last = {"B_cur": Bc, "node_budget_per_seq": plan.node_budget_per_seq,
                     "active_heads": plan.active_heads, "topk_by_depth": plan.topk_by_depth,
                     "actual_nodes": plan.actual_nodes,
                     "proposal_mode": ("chain" if use_chain else "medusa") if use_tree else "target_only",
                     "adaptive_tree": adaptive_stats}
        if sparse is None:
            dshared = topo.device(dev)
            dmap = topo.device(dev, Bc)
            tv = dict(pos_offset=dshared["pos_offset"], anc=dshared["anc"], parents=dmap["parents"],
                      n_nodes=dmap["n_nodes"], internal_rows=dmap["internal_rows"], slot_map=dmap["slot_map"])
            if tree_tokens is not None:
                assert tree_tokens.shape[1] == N, (tree_tokens.shape, N)
            elif N > 1:
                tree_tokens, _ = K.tree_layout(cand, score, Bc, roots, dshared["depth"], dshared["rank"], N)
            else:
                tree_tokens = roots.view(Bc, 1)
        m["active_sum"] += Bc
        m["samples"] += 1
        if sparse is None:
            m["node_sum"] += N
            for dpt, cnt in topo.depth_counts.items():
                r.proposed_by_depth[dpt] = r.proposed_by_depth.get(dpt, 0) + cnt * Bc
        # ---------------- verify forward + tree LM head
        tree_logits = slot_map = hidden_t = walk_logits = walk = None
        lazy = bool(cfg.lazy_walk_lm_head) and N > 1
        if int(r.seq_h.max()) + N > r.cache.capacity:
            raise RuntimeError("KV cache capacity exceeded")  # unreachable: rows finish at max_length
        r.sync()
        t0 = time.time()
        ev_start = None
        if r.event_log is not None:
            ev_start = torch.cuda.Event(enable_timing=True)
            ev_start.record()
        try:
            hidden_t = model.forward(tree_tokens, r.cache, pos_offset=tv["pos_offset"], anc=tv["anc"],
                                     seq_len=r.seq, row_map=r.row_map, err_flag=r.err,
                                     graph=bool(cfg.graph_verify_forward))
            if N > 1:
                m["tree_query_rows"] += Bc * N
                if lazy:
                    walk_logits = torch.empty((D, Bc, model.cfg.vocab), dtype=model.dtype, device=dev)
                else:
                    with timing.label("tree"):
                        if cfg.project_internal_tree_logits_only and tv["internal_rows"] is not None:
                            tree_logits = model.logits(hidden_t, row_index=tv["internal_rows"])
                            slot_map = tv["slot_map"]
                        else:
                            tree_logits = model.logits(hidden_t)
                    m["tree_lm_head_rows"] += tree_logits.shape[0]
        except RuntimeError as exc:
            if "out of memory" not in str(exc).lower():
                raise
            m["oom"] += 1
            torch.cuda.empty_cache()
            hidden_t = tree_logits = walk_logits = None
        r.sync()
        m["verify_time"] += time.time() - t0
        t_acc = time.time()
        # ---------------- acceptance
        walk_kw = dict(seed=r.seed, step=rnd, seq_ids=r.row_map, draw0=1, temperature=cfg.temperature, greedy=greedy,
                       top_k=cfg.top_k, top_p=cfg.top_p, err_flag=r.err)
        if walk_logits is not None:
            # Walk step t samples row b from the node its walk stands on; only those
            # rows are projected (inactive rows' tiles are skipped).
            # With the weight-streaming LM head, each step's launch also leaves the rows' maxima
            # (the draw then needs no chunk-maxima launch) and every step writes the next
            # step's rows.
            walk = K.walk_begin(tree_tokens, tv["parents"], tv["n_nodes"], acc_stride=D + 1)
            parts = model.walk_parts(Bc, hidden_t)
            K.walk_rows(walk, N)
            for t in range(D):
                with timing.label("tree"):
                    model.logits(hidden_t, row_index=walk["row_index"], row_active=walk["row_active"],
                                 out=walk_logits[t], parts=parts)
                K.walk_step(walk, walk_logits[t], tree_tokens, tv["parents"], tv["n_nodes"], walk_step=t,
                            parts=parts, next_rows=True, **walk_kw)
        elif tree_logits is not None:
            walk = K.accept_walk(tree_logits, tree_tokens, tv["parents"], tv["n_nodes"], max_walk_steps=D,
                                 slot_map=slot_map, **walk_kw)
        else:
            zeros = torch.zeros(Bc, dtype=torch.int32, device=dev)
            walk = dict(acc_tokens=roots.view(Bc, 1).clone(), acc_nodes=zeros.view(Bc, 1).clone(),
                        acc_len=torch.ones(Bc, dtype=torch.int32, device=dev), last_node=zeros.clone(),
                        correction=torch.full((Bc,), -1, dtype=torch.int32, device=dev))
        new_pending = torch.empty(Bc, dtype=torch.int32, device=dev) if b200 else None
        finished_d = K.accept_finalize(walk, r.seq, max_length=r.max_length, eos_token_id=eos_id,
                                       pending_root=new_pending)
        # ---------------- cache update + next state, queued before the round's host sync (they
        # need only device data, so the GPU has work while the host reads the round's results)
        extracted = False
        leaf_d = None
        state_in = (r.logits, r.hidden)  # the round's inputs, for the trace
        if cfg.cache_update_mode == "extract_path" and (tree_logits is not None or walk_logits is not None):
            r.sync()
            t0 = time.time()
            r.cache.gather_path(r.seq, walk["acc_nodes"], walk["acc_len"], N, row_map=r.row_map, err_flag=r.err)
            ar = self._arange(Bc, dev)
            last = walk["last_node"].long()
            # row gathers as index_select over flattened leading dims (one vectorised gather
            # launch; two-index advanced indexing ran 34 us for the 7B walk logits)
            r.hidden = hidden_t.flatten(0, 1).index_select(0, torch.add(last, ar, alpha=hidden_t.shape[1]))
            if walk_logits is None and slot_map is None:
                r.logits = tree_logits.index_select(0, torch.add(last, ar, alpha=N))
            else:
                if walk_logits is not None:
                    # the last accepted node at position acc_len-1 was sampled from at that
                    # walk step unless it is a leaf (then it has no projected row)
                    tpos = (walk["acc_len"].long() - 1).clamp(0, D - 1)
                    r.logits = walk_logits.flatten(0, 1).index_select(0, torch.add(ar, tpos, alpha=walk_logits.shape[1]))
                else:
                    slots = slot_map[ar, last]
                    r.logits = tree_logits.index_select(0, slots.clamp_min(0).long())
                # rows whose last node is a leaf get their LM-head row here (no launch when none is)
                if sparse is not None:
                    leaf_d = (sparse["n_children"].gather(1, last.view(-1, 1)) == 0).view(-1).to(torch.int32)
                else:
                    leaf_d = dshared["leaf"].index_select(0, last)
                with timing.label("leaf"):
                    model.logits_masked(r.hidden, leaf_d, r.logits)
            r.sync()
            dt_ = time.time() - t0
            m["extract_time"] += dt_
            m["cache_time"] += dt_
            m["extract_ok"] += 1
            extracted = True
        elif cfg.cache_update_mode == "extract_path" and plan.active_heads > 0:
            m["extract_fallback"] += 1
            if not cfg.allow_recompute_fallback:
                raise RuntimeError("KV extraction was requested but no tree cache was available")
        # ---------------- the one host sync of the round
        W = walk["acc_tokens"].shape[1]
        cols = [walk["acc_tokens"], walk["acc_len"].view(-1, 1), finished_d.view(-1, 1),
                walk["last_node"].view(-1, 1), r.err.expand(Bc).view(-1, 1)]
        if walk_logits is not None:
            cols += [walk["state"][2 * Bc:3 * Bc].view(-1, 1), walk["acc_nodes"]]
        if b200:
            cols.append(new_pending.view(-1, 1))
        if sparse is not None:
            # last node is a leaf; nodes per row; non-root nodes per depth 2..D+1
            per_depth = (sparse["depth"].unsqueeze(2) == torch.arange(2, D + 2, device=dev, dtype=torch.int32)).sum(1)
            leaf_s = sparse["n_children"].gather(1, walk["last_node"].long().view(-1, 1)) == 0
            cols += [leaf_s.to(torch.int32), sparse["n_nodes"].view(-1, 1), per_depth.to(torch.int32)]
        if leaf_d is not None:
            cols.append(leaf_d.view(-1, 1))
        pack_d = torch.cat(cols, dim=1)
        nxt = None
        if extracted and not r.statistical_time:
            # The next round's opening work, queued before the read-back for every row (rows
            # that finish this round are dropped from it afterwards).
            # Its adaptive-plan statistics come back with this round's results: one host
            # sync per round, and the GPU works while the host reads them.
            # medusa_time gets the host time of queuing it (the GPU runs it overlapped with
            # this round's read-back; statistical_time rounds are timed phase by phase)
            t_front = time.time()
            nxt = self._front(r, rnd + 1, r.logits, r.hidden, r.row_map, new_pending if b200 else r.pending,
                              trace is not None)
            m["medusa_time"] += time.time() - t_front
        seq_next = r.seq + walk["acc_len"]  # committed lengths after this round (device)
        pack_h = torch.empty(pack_d.shape, dtype=pack_d.dtype, pin_memory=True)
        pack_h.copy_(pack_d, non_blocking=True)
        both_h = None
        if nxt is not None and nxt.get("both_d") is not None:
            both_h = torch.empty(nxt["both_d"].shape, dtype=nxt["both_d"].dtype, pin_memory=True)
            both_h.copy_(nxt["both_d"], non_blocking=True)
        done = torch.cuda.Event()
        done.record()
        return dict(rnd=rnd, Bc=Bc, N=N, D=D, W=W, plan=plan, use_tree=use_tree, use_chain=use_chain,
                    sparse=sparse, topo=None if sparse is not None else topo, roots=roots, mlog=mlog, cand=cand,
                    tree_tokens=tree_tokens, tree_logits=tree_logits, slot_map=slot_map, hidden_t=hidden_t,
                    walk_logits=walk_logits, walk=walk, new_pending=new_pending, extracted=extracted,
                    leaf_d=leaf_d, state_in=state_in, seq_in=r.seq, active_in=list(r.active), ev_start=ev_start,
                    chain_recs=chain_recs, chain_rows=chain_rows, chain_conf=chain_conf,
                    conf_h=conf_h if chain_conf is not None else None, adaptive_stats=adaptive_stats,
                    plan_last=plan_last, nxt=nxt, pack_h=pack_h, both_h=both_h, done=done, t_acc=t_acc,
                    seq_next=seq_next)

    def _complete(self, r: "Rollout", c: dict, trace: list | None) -> dict:
        """Wait for a queued round's read-back and bring the rollout's state up to date:
        committed lengths, the b200 pending roots, the next round's queued proposals,
        and the rows that finished dropped. Returns the round's host arrays."""
        cfg = self.config
        model = self.model
        dev = r.device
        m = r.m
        b200 = bool(cfg.emit_correction_token)
        Bc, N, D, W, plan = c["Bc"], c["N"], c["D"], c["W"], c["plan"]
        walk, walk_logits, hidden_t = c["walk"], c["walk_logits"], c["hidden_t"]
        # spin on the event: a blocking wait adds its wake-up latency to the GPU's idle time
        done = c["done"]
        while not done.query():
            pass
        pack = c["pack_h"].numpy()
        m["accept_time"] += time.time() - c["t_acc"]
        # only what the next round needs before it is queued; the rest is read in _bookkeep
        acc_len_h = pack[:, W]
        fin_h = pack[:, W + 1].astype(bool)
        if int(pack[0, W + 3]):
            raise RuntimeError(f"flashgrpo_amd kernel reported an index error (flag {int(pack[0, W + 3])})")
        nxt = c["nxt"]
        if nxt is not None:
            nxt["both_h"] = None if c["both_h"] is None else c["both_h"].numpy()
            r.front = self._front_rows(nxt, np.nonzero(~fin_h)[0]) if fin_h.any() else nxt
        # ---------------- next state when the cache is recomputed (extraction ran before the sync)
        if not c["extracted"]:
            r.sync()
            t0 = time.time()
            if N == 1 and hidden_t is not None:
                # root-only round: the forward already wrote the root's K/V at slot seq_len
                r.hidden = hidden_t[:, 0].contiguous()
            else:
                wmax = int(acc_len_h.max())
                cols_ = torch.arange(wmax, device=dev)[None, :]
                # entries past a row's accepted length are padding: use token 0
                chain = torch.where(cols_ < walk["acc_len"][:, None], walk["acc_tokens"][:, :wmax],
                                    torch.zeros((), dtype=torch.int32, device=dev)).contiguous()
                h = model.forward(chain, r.cache, pos_offset=torch.arange(wmax, dtype=torch.int32, device=dev),
                                  anc=as_mask_tensor(chain_bits(wmax), dev), seq_len=r.seq, row_map=r.row_map,
                                  err_flag=r.err)
                r.hidden = h[torch.arange(Bc, device=dev), (walk["acc_len"] - 1).long()].contiguous()
            with timing.label("next"):
                r.logits = model.logits(r.hidden)
            r.sync()
            dt_ = time.time() - t0
            m["cache_time"] += dt_
            if cfg.cache_update_mode == "extract_path" and plan.active_heads > 0:
                m["recompute_time"] += dt_
        if c["ev_start"] is not None and r.event_log is not None:
            ev_end = torch.cuda.Event(enable_timing=True)
            ev_end.record()
            r.event_log.append((c["ev_start"], ev_end))
        r.seq = c["seq_next"]
        r.seq_h = r.seq_h + acc_len_h
        if b200:
            r.pending = c["new_pending"]
        m["rounds"] += 1
        if fin_h.any():
            keep = np.nonzero(~fin_h)[0]
            if keep.size == 0:
                r.active = []
            else:
                kt = torch.from_numpy(keep).to(dev)
                r.active = [r.active[i] for i in keep]
                r.row_map = r.row_map.index_select(0, kt)
                r.seq = r.seq.index_select(0, kt)
                r.seq_h = r.seq_h[keep]
                r.hidden = r.hidden.index_select(0, kt)
                r.logits = r.logits.index_select(0, kt)
                if b200:
                    r.pending = r.pending.index_select(0, kt)
        return dict(pack=pack, fin_h=fin_h)

    def _parse_round(self, r: "Rollout", c: dict, h: dict) -> dict:
        """The completed round's host arrays from its read-back (and the metrics in it)."""
        m = r.m
        b200 = bool(self.config.emit_correction_token)
        D, W, walk_logits, sparse = c["D"], c["W"], c["walk_logits"], c["sparse"]
        pack = h["pack"]
        if c["chain_conf"] is not None:
            c["adaptive_stats"]["confidence"] = c["conf_h"].tolist()
        acc_tok_h, acc_len_h = pack[:, :W], pack[:, W]
        last_h = pack[:, W + 2]
        if c["leaf_d"] is not None:
            m["tree_lm_head_rows"] += int(pack[:, -1].sum())
        col = W + 4
        walk_last_h = acc_nodes_h = None
        if walk_logits is not None:
            walk_last_h, acc_nodes_h = pack[:, col], pack[:, col + 1:col + 1 + W]
            col += 1 + W
            m["tree_lm_head_rows"] += int(np.sum(walk_last_h + 1))
        if b200:
            m["corrections"] += int(np.count_nonzero(pack[:, col] >= 0))
        sparse_leaf_h = None
        sparse = c["sparse"]
        proposed_before = sum(r.proposed_by_depth.get(j + 2, 0) for j in range(D))
        if sparse is not None:
            c0 = col + (1 if b200 else 0)
            sparse_leaf_h = pack[:, c0].astype(bool)
            m["node_sum"] += float(pack[:, c0 + 1].mean())
            for j in range(D):
                r.proposed_by_depth[j + 2] = r.proposed_by_depth.get(j + 2, 0) + int(pack[:, c0 + 2 + j].sum())
        proposed_sparse = sum(r.proposed_by_depth.get(j + 2, 0) for j in range(D)) - proposed_before
        return dict(pack=pack, acc_tok_h=acc_tok_h, acc_len_h=acc_len_h, fin_h=h["fin_h"], last_h=last_h,
                    walk_last_h=walk_last_h, acc_nodes_h=acc_nodes_h, sparse_leaf_h=sparse_leaf_h,
                    proposed_sparse=proposed_sparse, col=col)

    def _bookkeep(self, r: "Rollout", c: dict, h: dict, trace: list | None) -> int:
        """Host-only accounting of a completed round (tokens, histograms, metrics, the
        trace record); returns the tokens it emitted."""
        h = self._parse_round(r, c, h)
        m = r.m
        b200 = bool(self.config.emit_correction_token)
        Bc, N, D, plan, sparse, topo = c["Bc"], c["N"], c["D"], c["plan"], c["sparse"], c["topo"]
        pack, acc_tok_h, acc_len_h, fin_h, last_h = h["pack"], h["acc_tok_h"], h["acc_len_h"], h["fin_h"], h["last_h"]
        walk_last_h, acc_nodes_h, sparse_leaf_h, col = h["walk_last_h"], h["acc_nodes_h"], h["sparse_leaf_h"], h["col"]
        rnd = c["rnd"]
        roots, mlog, cand, tree_tokens = c["roots"], c["mlog"], c["cand"], c["tree_tokens"]
        tree_logits, slot_map, hidden_t, walk_logits = c["tree_logits"], c["slot_map"], c["hidden_t"], c["walk_logits"]
        chain_recs, chain_rows, state_in = c["chain_recs"], c["chain_rows"], c["state_in"]
        r.plan_last = c["plan_last"]
        if trace is not None:
            rec = dict(round=rnd, active=list(c["active_in"]), plan=list(plan.topk_by_depth),
                       budget=plan.node_budget_per_seq, seq_len=c["seq_in"].cpu().numpy().copy(),
                       logits_in=state_in[0].float().cpu().numpy(), hidden_in=state_in[1].float().cpu().numpy(),
                       roots=roots.cpu().numpy(), tree_tokens=tree_tokens.cpu().numpy(), acc_tokens=acc_tok_h.copy(),
                       acc_len=acc_len_h.copy(), finished=fin_h.copy(), last_node=last_h.copy(), seed=r.seed)
            if mlog is not None:
                rec["medusa_logits"] = mlog.float().cpu().numpy()
                rec["cand"] = cand.cpu().numpy()
            if chain_recs:
                rec["chain"] = [dict(k=c["k"], states=c["states"].float().cpu().numpy(),
                                     logits=c["logits"].float().cpu().numpy(), cand=c["cand"].cpu().numpy(),
                                     parent_local=c.get("parent_local"), rank=c.get("rank")) for c in chain_recs]
                rec["chain_budget"] = plan.node_budget_per_seq
            if sparse is not None:
                rec["sparse"] = {k: sparse[k].cpu().numpy() for k in ("parents", "depth", "n_nodes", "n_children",
                                                                       "pos_offset", "anc")}
                rec["sparse_plan"] = list(plan.nodes_by_head)
            if tree_logits is not None:
                rec["tree_logits"] = tree_logits.float().cpu().numpy()
                rec["slot_map"] = None if slot_map is None else slot_map.cpu().numpy()
            if walk_logits is not None:
                # rows[t, b] is valid for t <= walk_last[b]; it is the node acc_nodes[b, t]
                rec["walk_logits"] = walk_logits.float().cpu().numpy()
                rec["walk_last"] = walk_last_h.copy()
                rec["acc_nodes"] = acc_nodes_h.copy()
            if hidden_t is not None and N > 1:
                rec["tree_hidden"] = hidden_t.float().cpu().numpy()
            if b200:
                rec["pending"] = pack[:, col].copy()
            trace.append(rec)
        if walk_last_h is not None:
            draws = walk_last_h.astype(np.int64) + 1
        elif N > 1 and sparse_leaf_h is not None:
            draws = acc_len_h.astype(np.int64) - sparse_leaf_h.astype(np.int64)
        elif N > 1:
            draws = np.array([int(a) - (1 if topo.slot_of[int(n)] < 0 else 0) for a, n in zip(acc_len_h, last_h)])
        else:
            draws = np.zeros(Bc, dtype=np.int64)
        # internal = LM-head rows per sequence of the packed projection (all N for sparse trees)
        r.last_round = dict(num_nodes=N, internal=N if sparse is not None else len(topo.internal),
                            acc_len=acc_len_h.copy(),
                            last_node=last_h.copy(), walk_draws=draws, heads=plan.active_heads, batch=Bc,
                            lazy=walk_last_h is not None, walk_steps=D if walk_last_h is not None else 0,
                            chain_rows=list(chain_rows))
        # ---------------- bookkeeping
        lens = acc_len_h.astype(np.int64)
        emitted = int(lens.sum())
        toks = acc_tok_h.tolist()
        active_in = c["active_in"]
        for i, L in enumerate(lens.tolist()):
            r.generated[active_in[i]].extend(toks[i][:L])
        for L, c in enumerate(np.bincount(lens).tolist()):
            if c:
                r.accept_hist[L] = r.accept_hist.get(L, 0) + c
        for dpt in range(2, int(lens.max()) + 1):
            r.accept_by_depth[dpt] = r.accept_by_depth.get(dpt, 0) + int(np.count_nonzero(lens >= dpt))
        m["total_acc_length"] += emitted
        m["total_decoded_steps"] += Bc
        m["accepted"] += int(np.maximum(lens - 1, 0).sum())
        if sparse is not None:
            m["proposed"] += h["proposed_sparse"]
        else:
            m["proposed"] += max(N - 1, 0) * Bc
        return emitted

    def finish(self, r: "Rollout") -> dict:
        """Result dict with the keys of ``flash_medusa_decoder.py:1189-1229``."""
        cfg = self.config
        m = r.m
        self.flush(r)
        if r.cache is not None:
            self.model.drop_graphs(r.cache)  # the rollout's cache goes with it
        r.front = None
        total_time = time.time() - r.total_start
        accept_rate = m["accepted"] / max(m["proposed"], 1)
        avg_accept = m["total_acc_length"] / max(m["total_decoded_steps"], 1)
        reflex = {"enabled": False, "feedback_enabled": False, "proposal_injection_enabled": False,
                  "fast_state_norm_mean": 0.0, "fast_state_norm_p95": 0.0}
        return {
            "generated_token_ids": r.generated,
            "max_sequence_length": max((len(s) for s in r.generated), default=0),
            "total_acc_length": int(m["total_acc_length"]),
            "average_accept_length": float(avg_accept),
            "accepted_tokens_per_medusa_step": float(avg_accept),
            "total_decoded_token_num": int(m["total_decoded_steps"]),
            "total_accepted_draft_tokens": int(m["accepted"]),
            "total_proposed_draft_tokens": int(m["proposed"]),
            "total_accepted_medusa_tokens": int(m["accepted"]),
            "total_proposed_medusa_tokens": int(m["proposed"]),
            "draft_acceptance_rate": float(accept_rate),
            "medusa_acceptance_rate": float(accept_rate),
            "total_verify_rounds": int(m["rounds"]),
            "average_active_batch_size": m["active_sum"] / max(m["rounds"], 1),
            "average_tree_nodes_per_seq": m["node_sum"] / max(m["samples"], 1),
            "tree_query_rows": int(m["tree_query_rows"]),
            "tree_lm_head_rows": int(m["tree_lm_head_rows"]),
            "tree_lm_head_row_ratio": m["tree_lm_head_rows"] / max(m["tree_query_rows"], 1),
            "accept_length_histogram": r.accept_hist,
            "medusa_accept_by_depth": r.accept_by_depth,
            "medusa_proposed_by_depth": r.proposed_by_depth,
            "last_tree_plan": r.plan_last,
            "cache_update_mode": cfg.cache_update_mode,
            "kv_extraction_success_count": int(m["extract_ok"]),
            "kv_extraction_fallback_count": int(m["extract_fallback"]),
            "kv_extraction_time": m["extract_time"],
            "recompute_fallback_time": m["recompute_time"],
            "oom_count": int(m["oom"]),
            "total_time_cost": total_time,
            "prefill_time_cost": r.prefill_time,
            "target_time_cost": r.prefill_time + m["verify_time"] + m["cache_time"],
            "tree_verify_time_cost": m["verify_time"],
            "cache_update_time_cost": m["cache_time"],
            "medusa_head_time_cost": m["medusa_time"],
            "draft_time_cost": m["medusa_time"],
            "check_time_cost": 0.0,
            # walk + finalize + the round's one sync (lazy walks project their LM-head rows here)
            "accept_time_cost": m["accept_time"],
            "noise_seed": r.seed,
            "total_correction_tokens": int(m["corrections"]),
            "reflex_metrics": reflex,
            "reflex_head_metrics": {},
            "reflex_aux_records": {},
        }

    @torch.no_grad()
    def generate(self, input_ids: torch.Tensor, attention_mask: torch.Tensor, *, repeated_generate_nums=None,
                 max_length: int = 2048, statistical_time: bool = False, generation_step: int = 0,
                 collect_reflex_aux_cache=None, trace: list | None = None) -> dict:
        """Reference contract of ``flash_medusa_decoder.py:550-1229``. ``trace``
        (optional list) receives one dict of host copies per verify round; it adds
        copies and synchronisation and is meant for parity tests."""
        del collect_reflex_aux_cache
        r = self.start(input_ids, attention_mask, repeated_generate_nums=repeated_generate_nums,
                       max_length=max_length, statistical_time=statistical_time, generation_step=generation_step)
        while r.active:
            self.step(r, trace)
        return self.finish(r)


class Rollout:
    """Device state of one generate() call between verify rounds (compact over active rows)."""

    def __init__(self, *, seed, max_length, statistical_time, generation_step, device):
        self.seed = seed
        self.max_length = max_length
        self.statistical_time = statistical_time
        self.generation_step = generation_step
        self.device = device
        # when a list: (start, end) HIP events of each round's verify step (verify
        # forward + tree LM head + walk + KV extraction), recorded on the stream
        self.event_log = None
        self.cache = None
        self.active = []
        self.row_map = self.seq = self.hidden = self.logits = self.pending = self.err = None
        self.seq_h = None
        self.front = None  # the next round's queued opening work (FlashMedusaDecoder._front)
        self.inflight = None  # a queued round not yet completed (FlashMedusaDecoder.step)
        self.generated = []
        self.prefill_time = 0.0
        self.total_start = time.time()
        self.m = dict(total_acc_length=0, total_decoded_steps=0, accepted=0, proposed=0, rounds=0, active_sum=0,
                      node_sum=0.0, samples=0, tree_query_rows=0, tree_lm_head_rows=0, medusa_time=0.0,
                      verify_time=0.0, accept_time=0.0, cache_time=0.0, extract_time=0.0, recompute_time=0.0, extract_ok=0,
                      extract_fallback=0, oom=0, corrections=0)
        self.accept_hist, self.accept_by_depth, self.proposed_by_depth = {}, {}, {}
        self.plan_last = {}

    def sync(self):
        if self.statistical_time:
            torch.cuda.synchronize(self.device)
