"""Gated attention of the Qwen3.5 family: the drop-in for sleuth/formats/qwen35.py:187-216.

Same constructor (cfg, layer_idx) with the norms built in it and the projections (q_proj,
k_proj, v_proj, o_proj) attached by the loader, and the same forward(x, cos, sin, cache=None):
  q_proj gives per head [q | gate] (2·head_dim), q and k get RMSNorm and NEOX RoPE on their
  first n_rot channels, the cache is updated at cache.pos, causal attention over the cache
  (no mask for one token), and the output is multiplied by sigmoid(gate) before o_proj.

On the GPU without autograd, the cache write and the attention run in the HIP kernels
(forge_kv_append, forge_attn_prefill / forge_attn_decode); the norm and the partial RoPE stay
in torch, as in the reference, which rounds after each. Everything else runs the reference's
eager code. cfg needs n_heads, n_kv_heads, head_dim, n_rot and norm_eps (Qwen35Config,
qwen35.py:60-65).
"""

from __future__ import annotations

import torch
import torch.nn.functional as F
from torch import nn

from .attention import DECODE_MAX_T, _hip_ready, causal_mask, hip_shape_ok, hip_disabled
from .norm import RMSNorm
from .rope import apply_rope


class GatedAttention(nn.Module):
    def __init__(self, cfg, layer_idx: int):
        super().__init__()
        self.cfg, self.layer_idx = cfg, layer_idx
        self.q_norm = RMSNorm(cfg.head_dim, cfg.norm_eps)
        self.k_norm = RMSNorm(cfg.head_dim, cfg.norm_eps)
        self.last_path = ""

    def _use_hip(self, q: torch.Tensor, cache) -> bool:
        if not q.is_cuda or hip_disabled() or (torch.is_grad_enabled() and q.requires_grad):
            return False
        if not hip_shape_ok(q.dtype, self.cfg.head_dim):
            return False
        if cache is not None and (getattr(cache, "static", False) or getattr(cache, "ragged", False)):
            return False  # the reference model drives this layer with a plain cache only
        if cache is not None and cache.k[self.layer_idx].dtype != q.dtype:
            return False
        _hip_ready(q.device, q.dtype)
        return True

    def forward(self, x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, cache=None) -> torch.Tensor:
        c = self.cfg
        B, T, _ = x.shape
        qg = self.q_proj(x).view(B, T, c.n_heads, 2 * c.head_dim)
        qv, gate = qg[..., :c.head_dim], qg[..., c.head_dim:]
        qv = self.q_norm(qv).transpose(1, 2)
        k = self.k_norm(self.k_proj(x).view(B, T, c.n_kv_heads, c.head_dim)).transpose(1, 2)
        v = self.v_proj(x).view(B, T, c.n_kv_heads, c.head_dim).transpose(1, 2)
        # NEOX RoPE on the first n_rot channels (tables narrower than the head: partial RoPE)
        cos, sin = cos[..., :c.n_rot], sin[..., :c.n_rot]
        qv, k = apply_rope(qv, cos, sin), apply_rope(k, cos, sin)
        if self._use_hip(qv, cache):
            y = self._attend_hip(qv, k, v, cache)          # [B, T, H, hd]
            self.last_path = "hip"
        else:
            y = self._attend_torch(qv, k, v, cache).transpose(1, 2)
            self.last_path = "torch"
        y = y.reshape(B, T, c.n_heads * c.head_dim)
        return self.o_proj(y * torch.sigmoid(gate.reshape(B, T, -1)))

    def _attend_hip(self, q, k, v, cache) -> torch.Tensor:
        from . import ops

        B, H, T, hd = q.shape
        K = self.cfg.n_kv_heads
        if cache is None:
            kc = torch.empty(B, K, T, hd, device=q.device, dtype=q.dtype)
            vc = torch.empty_like(kc)
            offset, chunk = 0, 0
        else:
            if cache.pos + T > cache.max_len:  # as KVCache.update (kv_cache.py:56-57)
                raise ValueError(f"KV cache full: pos {cache.pos} + {T} > max_len {cache.max_len}")
            kc, vc = cache.k[self.layer_idx], cache.v[self.layer_idx]
            offset = cache.pos
            chunk = ops.decode_chunk(q.dtype, B, 1, H, K, hd, cache.max_len, 0, uniform=True)
        ops.kv_append(k, v, kc, vc, pos=offset)
        scale = hd ** -0.5
        if T > DECODE_MAX_T and ops.prefill_supported(q):
            return ops.attn_prefill(q, kc, vc, scale=scale, offset=offset)
        return ops.attn_decode(q, kc, vc, scale=scale, pos=offset, max_kv_len=offset + T, chunk=chunk)

    def _attend_torch(self, q, k, v, cache) -> torch.Tensor:
        """qwen35.py:202-214: [B, H, T, hd]."""
        c = self.cfg
        T = q.shape[2]
        offset = 0
        if cache is not None:
            offset = cache.pos
            k, v = cache.update(self.layer_idx, k, v)
        # one token sees the whole cache: no mask
        mask = None if T == 1 else causal_mask(T, k.shape[2], offset, 0, q.device)
        return F.scaled_dot_product_attention(q, k.to(q.dtype), v.to(q.dtype), attn_mask=mask,
                                              enable_gqa=c.n_kv_heads != c.n_heads)
