"""A small decoder around the attention module: the reference's forward glue, so the
attention and its cache can be exercised the way generate(), the speculative decoder
and CUDA-graph decoding use them.

Follows sleuth/forge/model/transformer.py: pre-norm blocks (75-99, SwiGLU MLP), one
RoPE table per layer kind (151-164), offset = cache.pos and the max_seq_len check
(257-277), static positions through index_select(pos_t) + new_step() (278-284), RoPE
rows sliced by offset (285-288), cache.advance(T) after all layers (299-300).
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch
import torch.nn.functional as F
from torch import nn

from .attention import Attention
from .config import ModelConfig
from .norm import RMSNorm
from .rope import rope_tables
from .taps import make_tap, name_taps


class SwiGLU(nn.Module):
    def __init__(self, d: int, hidden: int):
        super().__init__()
        self.gate = nn.Linear(d, hidden, bias=False)
        self.up = nn.Linear(d, hidden, bias=False)
        self.down = nn.Linear(hidden, d, bias=False)

    def forward(self, x):
        return self.down(F.silu(self.gate(x)) * self.up(x))


class Block(nn.Module):
    def __init__(self, cfg: ModelConfig, i: int):
        super().__init__()
        self.kind = cfg.layer_type(i)
        self.norm1 = RMSNorm(cfg.d_model, cfg.norm_eps)
        self.attn = Attention(cfg, i)
        self.norm2 = RMSNorm(cfg.d_model, cfg.norm_eps)
        self.mlp = SwiGLU(cfg.d_model, cfg.hidden)
        self.tap_attn_out = make_tap()
        self.tap_resid_post = make_tap()

    def forward(self, x, cos, sin, cache=None, same_doc=None):
        x = x + self.tap_attn_out(self.attn(self.norm1(x), cos, sin, cache, same_doc))
        return self.tap_resid_post(x + self.mlp(self.norm2(x)))


@dataclass
class ModelOutput:
    logits: torch.Tensor
    hidden: torch.Tensor | None = None


class Transformer(nn.Module):
    def __init__(self, cfg: ModelConfig):
        super().__init__()
        if not cfg.vocab_size:
            raise ValueError("vocab_size must be set")
        self.cfg = cfg
        self.tok_emb = nn.Embedding(cfg.vocab_size, cfg.d_model)
        self.blocks = nn.ModuleList(Block(cfg, i) for i in range(cfg.n_layers))
        self.norm_f = RMSNorm(cfg.d_model, cfg.norm_eps)
        self.lm_head = nn.Linear(cfg.d_model, cfg.vocab_size, bias=False)
        if cfg.tie_embeddings:
            self.lm_head.weight = self.tok_emb.weight
        for kind, (cos, sin) in self._rope().items():
            self.register_buffer(f"rope_cos_{kind}", cos, persistent=False)
            self.register_buffer(f"rope_sin_{kind}", sin, persistent=False)
        self.apply(self._init)
        for name, p in self.named_parameters():
            if name.endswith(("o_proj.weight", "down.weight")):
                nn.init.normal_(p, 0.0, cfg.init_std / math.sqrt(2 * cfg.n_layers))
        self._share_layers()
        name_taps(self)

    def _share_layers(self) -> None:
        """cfg.shared_layers: block i takes block j's Linear Parameters (the same objects),
        norms stay per block; each application keeps its own cache slot (layer index i)."""
        for i, j in enumerate(self.cfg.shared_layers):
            if i == j:
                continue
            linears = {n: m for n, m in self.blocks[j].named_modules() if isinstance(m, nn.Linear)}
            for n, m in self.blocks[i].named_modules():
                if n in linears:
                    m.weight = linears[n].weight
                    m.bias = linears[n].bias

    def _init(self, m):
        if isinstance(m, (nn.Linear, nn.Embedding)):
            nn.init.normal_(m.weight, 0.0, self.cfg.init_std)
            if getattr(m, "bias", None) is not None:
                nn.init.zeros_(m.bias)

    def _rope(self):
        cfg, out = self.cfg, {}
        for i in range(cfg.n_layers):
            spec = cfg.attn_spec(i)
            if spec.kind in out:
                continue
            if cfg.pos_type == "rope":
                out[spec.kind] = rope_tables(min(cfg.rope_dim or spec.head_dim, spec.head_dim),
                                             cfg.max_seq_len, spec.rope_theta)
            else:
                z = torch.zeros(cfg.max_seq_len, spec.head_dim)
                out[spec.kind] = (z, z)
        return out

    def _rope_kinds(self):
        return sorted({b.kind for b in self.blocks})

    def rope_rows(self, offset, T, cache=None):
        """cos/sin per layer kind for this pass: index_select(pos) in static mode, a slice
        at offset otherwise, per-row rows [B, T, hd] for a ragged cache."""
        if getattr(cache, "static", False):
            pos = cache.positions
            return {k: (getattr(self, f"rope_cos_{k}").index_select(0, pos),
                        getattr(self, f"rope_sin_{k}").index_select(0, pos)) for k in self._rope_kinds()}
        if getattr(cache, "ragged", False):
            idx = cache.seq_lens.long()[:, None] + torch.arange(T, device=cache.seq_lens.device)[None, :]
            return {k: (getattr(self, f"rope_cos_{k}")[idx], getattr(self, f"rope_sin_{k}")[idx])
                    for k in self._rope_kinds()}
        return {k: (getattr(self, f"rope_cos_{k}")[offset:offset + T],
                    getattr(self, f"rope_sin_{k}")[offset:offset + T]) for k in self._rope_kinds()}

    def forward(self, idx: torch.Tensor, cache=None, return_hidden: bool = False) -> ModelOutput:
        B, T = idx.shape
        offset = cache.pos if cache is not None else 0
        if offset + T > self.cfg.max_seq_len:
            raise ValueError(f"sequence length {offset + T} exceeds max_seq_len {self.cfg.max_seq_len}")
        if getattr(cache, "static", False):
            cache.new_step()
        rope = self.rope_rows(offset, T, cache)
        x = self.tok_emb(idx)
        for block in self.blocks:
            x = block(x, *rope[block.kind], cache)
        if cache is not None:
            cache.advance(T)
        h = self.norm_f(x)
        return ModelOutput(self.lm_head(h), h if return_hidden else None)
