"""Medusa heads with the reference's module layout and a fused device forward.

Module and parameter names follow ``flashgrpo/models/medusa_heads.py:12-142``
(``heads.{i}.fc``, ``heads.{i}.norm``, ``heads.{i}.output``, ``chain_cell.*``)
so ``medusa_heads.pt`` checkpoints written by the reference load unchanged
(``from_pretrained`` reads them with ``torch.load(weights_only=True)``). The
forward of all active heads is one ``fg_medusa_heads`` call (LayerNorm, MFMA
GEMM, bias, SiLU and residual fused) instead of one module call per head.
"""
from __future__ import annotations

import json
from pathlib import Path

import torch
import torch.nn as nn
import torch.nn.functional as F

from .. import kernels as K


class ChainDraftCell(nn.Module):
    """Recurrent proposal state (chain mode); layout of ``medusa_heads.py:12-42``."""

    def __init__(self, hidden_size, *, bottleneck_ratio=8, gate_init=-3.0, dtype=None):
        super().__init__()
        bottleneck = max(64, int(hidden_size) // max(1, int(bottleneck_ratio)))
        self.state_norm = nn.LayerNorm(hidden_size, dtype=dtype)
        self.token_norm = nn.LayerNorm(hidden_size, dtype=dtype)
        self.state_proj = nn.Linear(hidden_size, bottleneck, bias=False, dtype=dtype)
        self.token_proj = nn.Linear(hidden_size, bottleneck, bias=False, dtype=dtype)
        self.out_proj = nn.Linear(bottleneck, hidden_size, bias=True, dtype=dtype)
        self.act = nn.SiLU()
        self.gate = nn.Parameter(torch.tensor(float(gate_init), dtype=dtype or torch.float32))
        nn.init.zeros_(self.out_proj.weight)
        nn.init.zeros_(self.out_proj.bias)
        self._cast = None
        self._cast_key = None

    def forward(self, state, token_embedding):
        dt = self.state_norm.weight.dtype
        s = state.to(dt)
        mixed = self.state_proj(self.state_norm(s)) + self.token_proj(self.token_norm(token_embedding.to(dt)))
        return s + torch.sigmoid(self.gate) * self.out_proj(self.act(mixed))

    def _weights(self, dtype, device):
        params = list(self.parameters())
        key = (dtype, str(device), tuple(p._version for p in params), tuple(p.data_ptr() for p in params))
        if self._cast_key != key:
            with torch.no_grad():
                c = lambda t: t.detach().to(device=device, dtype=dtype).contiguous()
                self._cast = dict(
                    sn_w=c(self.state_norm.weight), sn_b=c(self.state_norm.bias),
                    tn_w=c(self.token_norm.weight), tn_b=c(self.token_norm.bias),
                    sp_w=c(self.state_proj.weight), tp_w=c(self.token_proj.weight),
                    out_w=c(self.out_proj.weight), out_b=c(self.out_proj.bias),
                    # sigmoid in the gate's own dtype, as the module's forward takes it
                    gate=torch.sigmoid(self.gate.detach()).to(device=device),
                    eps=float(self.state_norm.eps))
            self._cast_key = key
        return self._cast

    def step(self, state, token_embedding):
        """The cell in its parameters' dtype, as ``medusa_heads.py:36-42`` runs it (the
        rollout calls it outside autocast, ``flash_medusa_decoder.py:435-539``): the state
        and the embedding are cast to that dtype and the new state keeps it. On the GPU the
        two LayerNorms are one HIP launch (``fg_chain_cell_norm``); the two projections,
        their sum, SiLU, the output projection and the gated residual are the module's
        own torch calls, so every intermediate is rounded where the module rounds it."""
        dt = self.state_norm.weight.dtype
        w = self._weights(dt, state.device)
        H = state.shape[-1]
        s = state.to(dt)
        tok = token_embedding.to(dt)
        if s.is_cuda:
            # both LayerNorms in one launch, written side by side (fg_chain_cell_norm)
            from .. import kernels as K

            rows = lambda t: t.reshape(-1, H) if t.is_contiguous() else t.reshape(-1, H).contiguous()
            x = K.chain_cell_norm(rows(s), rows(tok), w["sn_w"], w["sn_b"], w["tn_w"], w["tn_b"], w["eps"])
            xs, xt = x[:, :H].view(*s.shape), x[:, H:].view(*s.shape)
        else:
            xs = F.layer_norm(s, (H,), w["sn_w"], w["sn_b"], w["eps"])
            xt = F.layer_norm(tok, (H,), w["tn_w"], w["tn_b"], w["eps"])
        mixed = F.linear(xs, w["sp_w"]) + F.linear(xt, w["tp_w"])
        delta = F.linear(F.silu(mixed), w["out_w"], w["out_b"])
        return s + w["gate"] * delta


class MedusaPredictionHead(nn.Module):
    """h + SiLU(fc(LayerNorm(h))); layout of ``medusa_heads.py:45-87``."""

    def __init__(self, hidden_size, vocab_size, *, dtype=None, tie_lm_head=True, lm_head=None):
        super().__init__()
        self.hidden_size = int(hidden_size)
        self.vocab_size = int(vocab_size)
        self.tie_lm_head = bool(tie_lm_head)
        self.fc = nn.Linear(hidden_size, hidden_size, bias=True, dtype=dtype)
        self.act = nn.SiLU()
        self.norm = nn.LayerNorm(hidden_size, dtype=dtype)
        nn.init.zeros_(self.fc.weight)
        nn.init.zeros_(self.fc.bias)
        if self.tie_lm_head:
            self.output = None
        else:
            self.output = nn.Linear(hidden_size, vocab_size, bias=False, dtype=dtype)
            # the reference copies ``lm_head.weight`` of an nn.Module LM head
            # (``medusa_heads.py:69-72``, built so by ``flashgrpo_trainer.py:727-733``);
            # a bare [V, H] weight tensor is taken as well
            src = lm_head.weight if isinstance(getattr(lm_head, "weight", None), torch.Tensor) else lm_head
            if isinstance(src, torch.Tensor) and tuple(src.shape) == tuple(self.output.weight.shape):
                with torch.no_grad():
                    self.output.weight.copy_(src.detach().to(self.output.weight.dtype))

    def project_hidden(self, hidden_states):
        """Single-head residual block on the device (fg_medusa_heads with one head), in the
        head's parameter dtype as ``medusa_heads.py:74-78`` computes it outside autocast
        (the chain bootstrap, ``flash_medusa_decoder.py:455-456``)."""
        h = hidden_states
        lead = h.shape[:-1]
        flat = h.reshape(-1, self.hidden_size).to(self.norm.weight.dtype).contiguous()
        out = K.medusa_heads(flat, self.norm.weight.detach()[None], self.norm.bias.detach()[None],
                             self.fc.weight.detach().to(flat.dtype)[None].contiguous(),
                             self.fc.bias.detach().to(flat.dtype)[None].contiguous(), eps=self.norm.eps)
        return out.view(*lead, self.hidden_size)


class MedusaHeads(nn.Module):
    def __init__(self, hidden_size, vocab_size, num_heads=3, *, dtype=None, tie_lm_head=True, lm_head=None,
                 medusa_loss_decay=0.8, chain_bottleneck_ratio=8, chain_gate_init=-3.0, reflex_fast_state_dim=0,
                 reflex_init_scale=0.0):
        super().__init__()
        self.hidden_size = int(hidden_size)
        self.vocab_size = int(vocab_size)
        self.num_heads = int(num_heads)
        self.tie_lm_head = bool(tie_lm_head)
        self.medusa_loss_decay = float(medusa_loss_decay)
        self.chain_bottleneck_ratio = int(chain_bottleneck_ratio)
        self.chain_gate_init = float(chain_gate_init)
        self.reflex_fast_state_dim = int(reflex_fast_state_dim or 0)
        self.reflex_init_scale = float(reflex_init_scale)
        self.heads = nn.ModuleList([MedusaPredictionHead(hidden_size, vocab_size, dtype=dtype, tie_lm_head=tie_lm_head,
                                                         lm_head=lm_head) for _ in range(num_heads)])
        self.chain_cell = ChainDraftCell(hidden_size, bottleneck_ratio=chain_bottleneck_ratio,
                                         gate_init=chain_gate_init, dtype=dtype)
        self._fused = None
        self._fused_key = None

    # -------------------------------------------------------------- device forward
    def _fused_weights(self, dtype, device):
        params = [p for hd in self.heads for p in (hd.fc.weight, hd.fc.bias, hd.norm.weight, hd.norm.bias)]
        key = (dtype, str(device), tuple(p._version for p in params), tuple(p.data_ptr() for p in params))
        if self._fused_key != key:
            with torch.no_grad():
                self._fused = dict(
                    fc_w=torch.stack([hd.fc.weight.to(device=device, dtype=dtype) for hd in self.heads]).contiguous(),
                    fc_b=torch.stack([hd.fc.bias.to(device=device, dtype=dtype) for hd in self.heads]).contiguous(),
                    ln_w=torch.stack([hd.norm.weight.to(device=device, dtype=torch.float32) for hd in self.heads]),
                    ln_b=torch.stack([hd.norm.bias.to(device=device, dtype=torch.float32) for hd in self.heads]),
                    eps=float(self.heads[0].norm.eps))
            self._fused_key = key
        return self._fused

    def project_all(self, hidden: torch.Tensor, max_heads: int | None = None, *, out=None, workspace=None):
        """[n*B, H] residual-block outputs of the first n heads, heads stacked (one launch)."""
        n = self.num_heads if max_heads is None else max(0, min(int(max_heads), self.num_heads))
        if n == 0:
            return hidden.new_empty(0, self.hidden_size)
        fw = self._fused_weights(hidden.dtype, hidden.device)
        return K.medusa_heads(hidden.contiguous(), fw["ln_w"][:n], fw["ln_b"][:n], fw["fc_w"][:n], fw["fc_b"][:n],
                              eps=fw["eps"], out=out, workspace=workspace)

    def output_weights(self, dtype, device) -> list:
        """Per head: its own output projection [V, H] (an untied head, cast once to
        ``dtype`` and cached until the parameter changes) or None (tied to the LM head)."""
        outs = [hd.output.weight if hd.output is not None else None for hd in self.heads]
        key = (dtype, str(device), tuple(None if w is None else (w._version, w.data_ptr()) for w in outs))
        if getattr(self, "_out_key", None) != key:
            with torch.no_grad():
                self._out = [None if w is None else w.detach().to(device=device, dtype=dtype).contiguous()
                             for w in outs]
            self._out_key = key
        return self._out

    def logits_for_last_hidden(self, last_hidden, lm_head_weight, *, max_heads=None):
        """Per-head logits [B, V]: an untied head through its own ``output``, the others
        through the LM head (``medusa_heads.py:241-277``)."""
        if last_hidden.dim() == 3:
            last_hidden = last_hidden[:, -1, :]
        B = last_hidden.shape[0]
        proj = self.project_all(last_hidden, max_heads)
        if proj.numel() == 0:
            return []
        own = self.output_weights(proj.dtype, proj.device)
        n = proj.shape[0] // B
        if all(w is None for w in own[:n]):
            return list(F.linear(proj, lm_head_weight.to(proj.dtype)).split(B, dim=0))
        return [F.linear(proj[h * B:(h + 1) * B], (lm_head_weight if own[h] is None else own[h]).to(proj.dtype))
                for h in range(n)]

    def chain_next_state(self, state, token_ids, embedding_weight):
        """Next chain state from the parent state and the path token's embedding
        (``medusa_heads.py:279-286``), computed in the cell's parameter dtype."""
        emb = embedding_weight.index_select(0, token_ids.to(embedding_weight.device).long())
        return self.chain_cell.step(state, emb)

    # -------------------------------------------------------------- checkpoint I/O
    def _config(self):
        return {"hidden_size": self.hidden_size, "vocab_size": self.vocab_size, "num_heads": self.num_heads,
                "tie_lm_head": self.tie_lm_head, "medusa_loss_decay": self.medusa_loss_decay,
                "chain_bottleneck_ratio": self.chain_bottleneck_ratio, "chain_gate_init": self.chain_gate_init,
                "reflex_fast_state_dim": self.reflex_fast_state_dim, "reflex_init_scale": self.reflex_init_scale}

    def save_pretrained(self, save_directory):
        """Same files as ``medusa_heads.py:424-440``."""
        import yaml

        d = Path(save_directory)
        d.mkdir(parents=True, exist_ok=True)
        cfg = self._config()
        (d / "medusa_config.json").write_text(json.dumps(cfg, indent=2), encoding="utf-8")
        (d / "medusa_config.yaml").write_text(yaml.safe_dump(cfg, sort_keys=False), encoding="utf-8")
        torch.save(self.state_dict(), d / "medusa_heads.pt")

    @classmethod
    def from_pretrained(cls, load_directory, *, map_location="cpu", dtype=None, lm_head=None,
                        chain_bottleneck_ratio=None, chain_gate_init=None, reflex_fast_state_dim=None,
                        reflex_init_scale=None, device=None):
        """Shape-filtered load of a directory written by ``save_pretrained``, as
        ``medusa_heads.py:442-480``: ``medusa_config.json`` gives the architecture (the
        keyword arguments that are not None win), ``medusa_heads.pt`` is read with
        weights-only unpickling and every tensor whose name and shape match is loaded;
        the others keep their initial values (``_loaded_state_keys`` /
        ``_loaded_compatible_keys`` record what the file held and what was taken).
        ``device`` (not in the reference) moves the module after loading."""
        d = Path(load_directory)
        cfg = json.loads((d / "medusa_config.json").read_text(encoding="utf-8"))

        def pick(arg, key, default):
            return arg if arg is not None else cfg.get(key, default)

        model = cls(cfg["hidden_size"], cfg["vocab_size"], cfg["num_heads"], dtype=dtype,
                    tie_lm_head=cfg.get("tie_lm_head", True), lm_head=lm_head,
                    medusa_loss_decay=cfg.get("medusa_loss_decay", 0.8),
                    chain_bottleneck_ratio=pick(chain_bottleneck_ratio, "chain_bottleneck_ratio", 8),
                    chain_gate_init=pick(chain_gate_init, "chain_gate_init", -3.0),
                    reflex_fast_state_dim=pick(reflex_fast_state_dim, "reflex_fast_state_dim", 0),
                    reflex_init_scale=pick(reflex_init_scale, "reflex_init_scale", 0.0))
        state = torch.load(d / "medusa_heads.pt", map_location=map_location, weights_only=True)
        current = model.state_dict()
        compatible = {k: v for k, v in state.items() if k in current and tuple(current[k].shape) == tuple(v.shape)}
        model.load_state_dict(compatible, strict=False)
        model._loaded_state_keys = set(state.keys())
        model._loaded_compatible_keys = set(compatible.keys())
        if device is not None:
            model = model.to(device)
        return model

    @classmethod
    def random(cls, hidden_size, vocab_size, num_heads, *, seed=0, std=0.02, dtype=torch.float32, device="cpu"):
        """Random-init heads for synthetic benchmarks: fc ~ N(0, std), LayerNorm identity."""
        m = cls(hidden_size, vocab_size, num_heads, dtype=dtype).to(device)
        g = torch.Generator(device=device).manual_seed(int(seed))
        with torch.no_grad():
            for hd in m.heads:
                hd.fc.weight.normal_(0.0, std, generator=g)
                hd.fc.bias.normal_(0.0, std, generator=g)
            # the reference zero-initialises out_proj (the cell starts as the identity);
            # synthetic runs draw it too so that chain depths differ
            cc = m.chain_cell
            for p in (cc.state_proj.weight, cc.token_proj.weight, cc.out_proj.weight, cc.out_proj.bias):
                p.normal_(0.0, std, generator=g)
        return m
