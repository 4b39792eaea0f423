"""The allocation-free decode entry point (forge_attn_decode_noalloc, through the C ABI)
against the entry point it mirrors (forge_attn_decode with a caller workspace): the same
output bit for bit, on two calls in a row, the second smaller than the first (the library's
scratch array keeps the first call's partials and work ticket, which the second must not
pick up). Sizes beyond the scratch array are rejected before anything is launched."""

from __future__ import annotations

import math

import pytest
import torch

import oracle
from conftest import gpu_available
from helpers import max_abs

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not gpu_available(), reason="needs a GPU")]
DEV = "cuda"


def ops():
    from sleuth_amd import ops as o

    return o


def _case(seed, B, H, K, D, T, lens, window, dtype, host_pos):
    """Cache rows of N(0,1) up to each row's length (new tokens included), raw q with the
    norm + RoPE fused; returns keyword arguments shared by both entry points."""
    max_len = max(lens)
    g = torch.Generator(device=DEV).manual_seed(seed)
    kc = torch.randn(B, K, max_len, D, generator=g, device=DEV, dtype=dtype)
    vc = torch.randn(B, K, max_len, D, generator=g, device=DEV, dtype=dtype)
    q = torch.randn(B, T, H, D, generator=g, device=DEV, dtype=dtype).transpose(1, 2)
    w = (1 + 0.1 * torch.randn(D, generator=g, device=DEV)).to(dtype)
    cos, sin = oracle.rope_tables(D, max_len, 1e6)
    base = torch.tensor([L - T for L in lens])
    idx = base[:, None] + torch.arange(T)[None, :]
    kw = dict(scale=1.0 / math.sqrt(D), window=window, q_weight=w, eps=1e-6, norm_q=True, max_kv_len=max_len)
    if host_pos:
        assert len(set(lens)) == 1
        kw.update(pos=int(base[0]), cos=cos[idx[0]].to(DEV), sin=sin[idx[0]].to(DEV))
    else:
        kw.update(row_pos=base.to(torch.int32).to(DEV), cos=cos[idx].to(DEV), sin=sin[idx].to(DEV))
    return q, kc, vc, kw


CASES = {
    # C4 shape: 64 ragged rows up to 32k keys, persistent grid + combine (~32.5 MB of partials)
    "c4": dict(B=64, H=16, K=8, D=128, T=1, lens=torch.randint(1024, 32769, (64,),
               generator=torch.Generator().manual_seed(0)).tolist(), window=0, dtype=torch.bfloat16,
               host_pos=False),
    # C5 shape, smaller: MQA verify on the MFMA kernel, window 1024, one host position
    "c5": dict(B=8, H=8, K=1, D=256, T=4, lens=[8196] * 8, window=1024, dtype=torch.bfloat16, host_pos=True),
    # fp32, G = 3 (VALU kernel), T = 5, ragged rows
    "f32": dict(B=3, H=12, K=4, D=64, T=5, lens=[70, 900, 2049], window=0, dtype=torch.float32, host_pos=False),
}


@pytest.mark.parametrize("order", [("c4", "c5", "f32"), ("c5", "f32")])
def test_noalloc_equals_the_workspace_entry_point(order):
    """Calls in a row, each smaller than the one before: forge_attn_decode_noalloc gives
    forge_attn_decode's output bit for bit, and both match the oracle on a row."""
    for i, name in enumerate(order):
        c = CASES[name]
        q, kc, vc, kw = _case(50 + i, c["B"], c["H"], c["K"], c["D"], c["T"], c["lens"], c["window"],
                              c["dtype"], c["host_pos"])
        want = ops().attn_decode(q, kc, vc, **kw)
        out = torch.full_like(want, float("nan"))
        got = ops().attn_decode_noalloc(q, kc, vc, out=out, **kw)
        torch.cuda.synchronize()
        assert got is out and torch.equal(got, want), name
        b, L, T = 0, c["lens"][0], c["T"]
        cos_b = kw["cos"] if c["host_pos"] else kw["cos"][b]
        sin_b = kw["sin"] if c["host_pos"] else kw["sin"][b]
        qn = oracle.head_norm_rope(q[b:b + 1].cpu(), kw["q_weight"].cpu(), 1e-6, cos_b.cpu(), sin_b.cpu())
        ref = oracle.sdpa(qn.float(), kc[b:b + 1, :, :L].float().cpu(), vc[b:b + 1, :, :L].float().cpu(),
                          L - T, c["window"], kw["scale"]).transpose(1, 2)
        assert max_abs(got[b:b + 1], ref) <= (1e-4 if c["dtype"] == torch.float32 else 2e-2), name


def test_noalloc_rejects_calls_beyond_the_scratch_array():
    from sleuth_amd import _lib

    B, H, K, D, T, S = 64, 16, 8, 128, 16, 4096   # about 545 MB of partials at 64-key chunks
    need = ops().decode_workspace_bytes(torch.bfloat16, B, T, H, K, D, S, 64)
    assert need > _lib.NOALLOC_SCRATCH_BYTES
    kc = torch.zeros(B, K, S, D, device=DEV, dtype=torch.bfloat16)
    q = torch.zeros(B, H, T, D, device=DEV, dtype=torch.bfloat16)
    out = torch.full((B, T, H, D), 7.0, device=DEV, dtype=torch.bfloat16)
    with pytest.raises(_lib.ForgeError, match="scratch"):
        ops().attn_decode_noalloc(q, kc, kc, scale=0.1, out=out, pos=S - T, chunk=64)
    torch.cuda.synchronize()
    assert torch.all(out == 7.0)   # nothing was launched
