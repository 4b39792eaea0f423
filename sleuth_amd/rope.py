"""RoPE tables and the torch form of NEOX rotate-half RoPE.

The tables are the model's buffers (sleuth/forge/model/rope.py:21-38): inv_freq =
1/theta^(arange(0, d, 2)/d) in fp32, angles = outer(pos, inv_freq) with the two halves
duplicated, cos/sin [max_len, d] fp32. The HIP kernels read rows of these tables; the
torch form (rope.py:41-55) serves the explicit/training path and partial RoPE.
"""

from __future__ import annotations

import torch


def rope_tables(head_dim: int, max_len: int, theta: float,
                freq_factors: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    half = torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim
    inv_freq = 1.0 / (theta ** half)
    if freq_factors is not None:
        if freq_factors.numel() != head_dim // 2:
            raise ValueError(f"{freq_factors.numel()} RoPE frequency factors for head_dim {head_dim}")
        inv_freq = inv_freq / freq_factors.float().cpu()
    angles = torch.outer(torch.arange(max_len, dtype=torch.float32), inv_freq)
    angles = torch.cat([angles, angles], dim=-1)
    return angles.cos(), angles.sin()


def rotate_half(x: torch.Tensor) -> torch.Tensor:
    x1, x2 = x.chunk(2, dim=-1)
    return torch.cat([-x2, x1], dim=-1)


def apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """x [B,H,T,d]; cos/sin [T, rd] (or [B,T,rd] per row). fp32 math, x's dtype out.
    rd < d: only the first rd channels rotate (partial RoPE)."""
    rd = cos.shape[-1]
    if rd < x.shape[-1]:
        return torch.cat([apply_rope(x[..., :rd], cos, sin), x[..., rd:]], dim=-1)
    if cos.dim() == 3:
        cos, sin = cos[:, None], sin[:, None]
    return (x.float() * cos + rotate_half(x.float()) * sin).to(x.dtype)
