"""Attention of the MTP drafter onto the target model's KV cache: the drop-in for the
attention part of AssistantLayer.forward (sleuth/forge/infer/mtp.py:73-92) and of its
graph form forward_static (mtp.py:169-188).

The drafter has no K/V projections of its own: it attends with one new query per row onto
the keys the target has stored (positions 0 .. n_past-1), its query sitting at position
n_past; a sliding layer sees only the last window-1 of them (llama.cpp's rule q - k < window,
mtp.py:83-86). Scale 1.0, GQA over the target layer's KV heads (mtp.py:87-88).

Same submodule names as the reference layer's attention part (the loader's contract,
mtp.py:130-133): q_proj, q_norm, o_proj. forward(h, k, v, cos, sin, n_past) -> [B, 1, d]
where h is the layer's normed input [B, 1, d], k/v the target layer's cache [B, K, >=n_past,
hd], cos/sin the RoPE rows of position n_past, and n_past either a host int (eager,
mtp.py:73-92) or an int64 device tensor holding it (the graph form, where the position
lives on the device: nothing of the call then depends on a host number).

On the GPU without autograd the q norm + RoPE and the attention run in one
forge_attn_decode call (ops.attn_drafter); otherwise the reference's eager code runs.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F
from torch import nn

from .attention import _hip_ready, hip_shape_ok, hip_disabled
from .norm import RMSNorm
from .rope import apply_rope


class DrafterAttention(nn.Module):
    def __init__(self, d_model: int, n_heads: int, head_dim: int, sliding: bool, window: int,
                 eps: float = 1e-6, bias: bool = False):
        super().__init__()
        if sliding and window < 2:
            raise ValueError("a sliding drafter layer needs window >= 2")
        self.sliding, self.n_heads, self.hd, self.window, self.eps = sliding, n_heads, head_dim, window, eps
        self.q_proj = nn.Linear(d_model, n_heads * head_dim, bias=bias)
        self.q_norm = RMSNorm(head_dim, eps)
        self.o_proj = nn.Linear(n_heads * head_dim, d_model, bias=bias)
        self.last_path = ""

    def _use_hip(self, q: torch.Tensor, k: torch.Tensor) -> bool:
        if not q.is_cuda or hip_disabled() or (torch.is_grad_enabled() and q.requires_grad):
            return False
        if not hip_shape_ok(q.dtype, self.hd) or k.dtype != q.dtype:
            return False
        _hip_ready(q.device, q.dtype)
        return True

    def forward(self, h: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cos: torch.Tensor,
                sin: torch.Tensor, n_past: int | torch.Tensor) -> torch.Tensor:
        B, T, _ = h.shape
        if T != 1:
            raise ValueError("the drafter attends with one query per row")
        q = self.q_proj(h).view(B, T, self.n_heads, self.hd).transpose(1, 2)   # [B, H, 1, hd]
        window = self.window if self.sliding else 0
        if self._use_hip(q, k):
            from . import ops

            where = dict(n_past_dev=n_past) if torch.is_tensor(n_past) else dict(n_past=int(n_past))
            y = ops.attn_drafter(q, k, v, window=window, scale=1.0, q_weight=self.q_norm.weight_f32(),
                                 eps=self.eps, norm_q=True, cos=cos.float(), sin=sin.float(), **where)
            self.last_path = "hip"
        else:
            y = self._attend_torch(q, k, v, cos, sin, n_past, window).transpose(1, 2)
            self.last_path = "torch"
        return self.o_proj(y.reshape(B, T, self.n_heads * self.hd))

    def _attend_torch(self, q, k, v, cos, sin, n_past, window):
        """The reference's eager attention (mtp.py:79-88): RMSNorm then RoPE, each rounded;
        the first n_past keys (sliding: the last window-1 of them), or with a device n_past the
        same set as a mask over the whole view (mtp.py:180-183). Returns [B, H, 1, hd]."""
        q = apply_rope(self.q_norm(q), cos, sin)
        gqa = k.shape[1] != self.n_heads
        if torch.is_tensor(n_past):
            kpos = torch.arange(k.shape[2], device=k.device)
            seen = kpos < n_past
            if window:
                seen &= n_past - kpos < window
            return F.scaled_dot_product_attention(q, k.to(q.dtype), v.to(q.dtype), attn_mask=seen.view(1, 1, 1, -1),
                                                  scale=1.0, enable_gqa=gqa)
        lo = max(0, n_past - (window - 1)) if window else 0
        k, v = k[:, :, lo:n_past], v[:, :, lo:n_past]
        return F.scaled_dot_product_attention(q, k.to(q.dtype), v.to(q.dtype), scale=1.0, enable_gqa=gqa)
