"""First-use self-check of the HIP kernels on a device, like the reference's
fused_ops._self_check (fused_ops.py:144-173), but failing loudly: a wrong or missing
kernel raises instead of quietly falling back.

The checks compare each kernel with the torch formulas (computed in fp32 on the same
device) on small random inputs: head norm + RoPE, the cache append, split-K attention
(decode and a 3-token verify) and, for bf16/fp16, the MFMA prefill.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

from ._lib import ForgeError
from .rope import apply_rope, rope_tables


def _close(a: torch.Tensor, b: torch.Tensor, tol: float) -> bool:
    return bool(torch.allclose(a.float(), b.float(), atol=tol, rtol=tol))


def _ref_attention(q, k, v, offset, window, scale):
    """fp32 masked softmax attention, q [B,H,T,D], k/v [B,K,S,D] -> [B,T,H,D]."""
    B, H, T, D = q.shape
    rep = H // k.shape[1]
    kk = k.float().repeat_interleave(rep, 1)
    vv = v.float().repeat_interleave(rep, 1)
    s = (q.float() @ kk.transpose(-1, -2).contiguous()) * scale
    S = k.shape[2]
    qpos = torch.arange(T, device=q.device)[:, None] + offset
    kpos = torch.arange(S, device=q.device)[None, :]
    ok = kpos <= qpos
    if window:
        ok &= qpos - kpos < window
    p = s.masked_fill(~ok, float("-inf")).softmax(-1)
    return (p @ vv).transpose(1, 2)


def self_check(device: torch.device, dtype: torch.dtype) -> None:
    from . import ops

    tol = 1e-4 if dtype == torch.float32 else 3e-2
    g = torch.Generator().manual_seed(0)
    try:
        B, H, K, D, T, L = 2, 4, 2, 64, 3, 40
        dev = device
        x = torch.randn(B, T, H, D, generator=g).to(dtype).to(dev).transpose(1, 2)
        w = (1 + 0.1 * torch.randn(D, generator=g)).to(dev)
        cos, sin = (t.to(dev) for t in rope_tables(D, L, 1e4))
        c, s = cos[10:10 + T], sin[10:10 + T]
        want = apply_rope(F.rms_norm(x.float(), (D,), w, 1e-6), c, s)
        if not _close(ops.head_norm_rope(x, w, 1e-6, c, s), want, tol):
            raise ForgeError("head_norm_rope disagrees with the torch formula")

        kc = torch.randn(B, K, L, D, generator=g).to(dtype).to(dev)
        vc = torch.randn(B, K, L, D, generator=g).to(dtype).to(dev)
        knew = torch.randn(B, T, K, D, generator=g).to(dtype).to(dev).transpose(1, 2)
        vnew = torch.randn(B, T, K, D, generator=g).to(dtype).to(dev).transpose(1, 2)
        ops.kv_append(knew, vnew, kc, vc, pos=10, k_weight=w, eps=1e-6, norm_k=True, cos=c, sin=s)
        kn = apply_rope(F.rms_norm(knew.float(), (D,), w, 1e-6), c, s)
        if not (_close(kc[:, :, 10:13], kn, tol) and _close(vc[:, :, 10:13], vnew, 0)):
            raise ForgeError("kv_append wrote the wrong values")

        q = torch.randn(B, H, T, D, generator=g).to(dtype).to(dev)
        for t_q, window in ((1, 0), (T, 5)):
            qq = q[:, :, :t_q]
            got = ops.attn_decode(qq, kc, vc, scale=0.125, pos=13 - t_q, window=window)
            want = _ref_attention(qq, kc[:, :, :13], vc[:, :, :13], 13 - t_q, window, 0.125)
            if not _close(got, want, tol):
                raise ForgeError(f"split-K attention disagrees with torch (T={t_q}, window={window})")
        if dtype != torch.float32:
            qp = torch.randn(1, H, 40, D, generator=g).to(dtype).to(dev)
            got = ops.attn_prefill(qp, kc[:1], vc[:1], scale=0.125, offset=0)
            want = _ref_attention(qp, kc[:1], vc[:1], 0, 0, 0.125)
            if not _close(got, want, tol):
                raise ForgeError("MFMA prefill disagrees with torch")
        torch.cuda.synchronize(device)
    except ForgeError as e:
        raise ForgeError(f"HIP attention self-check failed on {device} ({dtype}): {e}") from e
