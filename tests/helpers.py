"""Seeded inputs for the BASELINE configs and small helpers shared by the tests."""

from __future__ import annotations

import math

import torch

import oracle


def gen(seed: int) -> torch.Generator:
    return torch.Generator().manual_seed(seed)


def randn(g, *shape, dtype=torch.float32):
    return torch.randn(*shape, generator=g).to(dtype)


def qkv_proj_views(g, B, T, H, K, D, dtype):
    """Raw q/k/v laid out as Attention.forward makes them: q_proj(x).view(B,T,H,hd)
    .transpose(1,2) -- a [B,H,T,hd] view of a [B,T,H,hd] buffer (attention.py:106-108)."""
    q = randn(g, B, T, H, D, dtype=dtype).transpose(1, 2)
    k = randn(g, B, T, K, D, dtype=dtype).transpose(1, 2)
    v = randn(g, B, T, K, D, dtype=dtype).transpose(1, 2)
    return q, k, v


def tables(D, max_len, theta):
    return oracle.rope_tables(D, max_len, theta)


def max_abs(a: torch.Tensor, b: torch.Tensor) -> float:
    return (a.float().cpu() - b.float().cpu()).abs().max().item()


def tol(dtype) -> float:
    """fp32 1e-4, bf16/fp16 2e-2 (max-abs)."""
    return 1e-4 if dtype == torch.float32 else 2e-2


def scale_of(D: int) -> float:
    return 1.0 / math.sqrt(D)
