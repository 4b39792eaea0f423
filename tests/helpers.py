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


ARGMAX_VOCAB = 128     # width of the stand-in downstream projection
ARGMAX_MARGIN = 0.01   # near-tie threshold: fraction of the reference logits' RMS


def downstream_argmax(got: torch.Tensor, ref: torch.Tensor, vocab: int = ARGMAX_VOCAB,
                      margin: float = ARGMAX_MARGIN, seed: int = 0) -> dict:
    """Argmax agreement of downstream logits, the north star's bf16 criterion.

    Each token's attention output (got/ref [B, T, ...], flattened per (b, t) row) goes
    through one fixed random projection W ~ N(0, 1/d) [d, vocab], the stand-in for the
    layers above attention. A row whose reference top-2 margin is below
    margin * RMS(reference logits) is a near-tie that bf16 rounding may legitimately flip:
    such rows are counted, not compared. Every other row must give the same argmax.
    The threshold is fixed in advance, not derived from the observed error.
    Returns {"rows", "near_ties", "mismatched"}."""
    rows = got.shape[0] * got.shape[1]
    yg = got.reshape(rows, -1).double().cpu()
    yr = ref.reshape(rows, -1).double().cpu()
    g = torch.Generator().manual_seed(seed)
    W = torch.randn(yr.shape[1], vocab, generator=g, dtype=torch.float64) / math.sqrt(yr.shape[1])
    lg, lr = yg @ W, yr @ W
    top2 = lr.topk(2, dim=1).values
    tie = (top2[:, 0] - top2[:, 1]) < margin * lr.pow(2).mean().sqrt()
    bad = (lg.argmax(1) != lr.argmax(1)) & ~tie
    return {"rows": rows, "near_ties": int(tie.sum()), "mismatched": int(bad.sum())}
