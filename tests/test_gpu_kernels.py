"""Parity of each HIP kernel, called through the C ABI (sleuth_amd.ops), with the CPU
oracle on identical seeded inputs. Tolerances: fp32 max-abs <= 1e-4, bf16/fp16 <= 2e-2."""

from __future__ import annotations

import random

import pytest
import torch

import oracle
from conftest import gpu_available
from helpers import gen, max_abs, qkv_proj_views, randn, scale_of, tables, tol

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not gpu_available(), reason="needs a GPU")]

DEV = "cuda"
DTYPES = [torch.float32, torch.bfloat16, torch.float16]


def ops():
    from sleuth_amd import ops as o

    return o


# ------------------------------------------------------------------ head_norm_rope
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("D", [16, 32, 48, 64, 96, 128, 256])
def test_head_norm_rope(dtype, D):
    """fused_ops.head_norm_rope semantics (fused_ops.py:101-121), incl. the reference's
    odd sizes (test_fused_ops.py:29-40) and stride preservation (test_fused_ops.py:37)."""
    g = gen(D)
    B, H, T = 2, 3, 7
    q = randn(g, B, T, H, D, dtype=dtype).transpose(1, 2)       # [B,H,T,D] strided
    w = (1 + 0.1 * randn(g, D)).to(dtype)
    cos, sin = tables(D, 64, 1e4)
    cos, sin = cos[10:10 + T], sin[10:10 + T]
    ref = oracle.head_norm_rope(q, w, 1e-6, cos, sin)
    got = ops().head_norm_rope(q.to(DEV), w.to(DEV), 1e-6, cos.to(DEV), sin.to(DEV))
    assert got.shape == q.shape and got.stride() == q.stride()
    assert max_abs(got, ref) <= (2e-6 if dtype == torch.float32 else tol(dtype))
    # norm only / rope only
    ref2 = oracle.head_norm_rope(q, None, 1e-6)
    got2 = ops().head_norm_rope(q.to(DEV), None, 1e-6)
    assert max_abs(got2, ref2) <= (2e-6 if dtype == torch.float32 else tol(dtype))
    ref3 = oracle.head_norm_rope(q, None, 0.0, cos, sin, norm=False)
    got3 = ops().head_norm_rope(q.to(DEV), None, 0.0, cos.to(DEV), sin.to(DEV), norm=False)
    assert max_abs(got3, ref3) <= (2e-6 if dtype == torch.float32 else tol(dtype))


def test_head_norm_rope_rows_independent():
    """A row's result does not depend on how many rows run together (bitwise;
    test_fused_ops.py:41-44)."""
    g = gen(3)
    x = randn(g, 4, 6, 9, 128, dtype=torch.bfloat16).to(DEV)
    w = (1 + 0.1 * randn(g, 128)).to(DEV)
    a = ops().head_norm_rope(x, w, 1e-6)[:1]
    b = ops().head_norm_rope(x[:1].contiguous(), w, 1e-6)
    assert torch.equal(a, b)


# ------------------------------------------------------------------ kv_append
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("D", [32, 64, 128, 256])
@pytest.mark.parametrize("mode", ["pos", "row_pos", "pos_dev"])
def test_kv_append(dtype, D, mode):
    g = gen(D + len(mode))
    B, K, T, L = 3, 2, 5, 40
    _, k, v = qkv_proj_views(g, B, T, 4, K, D, dtype)
    kw_ = (1 + 0.1 * randn(g, D)).to(dtype)
    cos, sin = tables(D, L, 1e6)
    base = [7, 7, 7] if mode != "row_pos" else [0, 13, 35]
    cache_k = torch.full((B, K, L, D), 1e4, dtype=dtype)   # poison: must survive outside the write
    cache_v = cache_k.clone()
    kc, vc = cache_k.to(DEV), cache_v.to(DEV)
    if mode == "row_pos":
        c = torch.stack([cos[b:b + T] for b in base])
        s = torch.stack([sin[b:b + T] for b in base])
        ops().kv_append(k.to(DEV), v.to(DEV), kc, vc, row_pos=torch.tensor(base, dtype=torch.int32, device=DEV),
                        k_weight=kw_.to(DEV), eps=1e-6, norm_k=True, norm_v=True, cos=c.to(DEV), sin=s.to(DEV))
    else:
        c, s = cos[7:7 + T], sin[7:7 + T]
        kwargs = {"pos": 7} if mode == "pos" else {"pos_dev": torch.tensor([7], device=DEV)}
        ops().kv_append(k.to(DEV), v.to(DEV), kc, vc, k_weight=kw_.to(DEV), eps=1e-6, norm_k=True,
                        norm_v=True, cos=c.to(DEV), sin=s.to(DEV), **kwargs)
    t = tol(dtype) if dtype != torch.float32 else 2e-6
    for b in range(B):
        p = base[b]
        cb, sb = (c[b], s[b]) if mode == "row_pos" else (c, s)
        ref_k = oracle.head_norm_rope(k[b:b + 1], kw_, 1e-6, cb, sb)
        ref_v = oracle.head_norm_rope(v[b:b + 1], None, 1e-6)
        assert max_abs(kc[b:b + 1, :, p:p + T].cpu(), ref_k) <= t
        assert max_abs(vc[b:b + 1, :, p:p + T].cpu(), ref_v) <= t
        keep = torch.ones(L, dtype=torch.bool)
        keep[p:p + T] = False
        poison = torch.tensor(1e4, dtype=dtype).item()
        assert torch.all(kc[b, :, keep.to(DEV)].float() == poison)
        assert torch.all(vc[b, :, keep.to(DEV)].float() == poison)


def test_kv_append_full_cache_rejected():
    k = torch.zeros(1, 1, 4, 64, device=DEV, dtype=torch.bfloat16)
    c = torch.zeros(1, 1, 8, 64, device=DEV, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="KV cache full"):
        ops().kv_append(k, k, c, c.clone(), pos=6)


# ------------------------------------------------------------------ split-K decode / verify
def _decode_case(seed, dtype, B, H, K, D, T, lens, window, theta=1e4, max_len=None, fuse=True, chunk=0):
    """Cache rows filled with N(0,1) up to lens[b] (the new tokens' K/V included); raw q
    normalised in the kernel (fuse) or beforehand. Returns (got [B,T,H,D], ref [B,T,H,D])."""
    g = gen(seed)
    max_len = max_len or max(lens) + 3
    kc = randn(g, B, K, max_len, D, dtype=dtype)
    vc = randn(g, B, K, max_len, D, dtype=dtype)
    q = randn(g, B, T, H, D, dtype=dtype).transpose(1, 2)
    w = (1 + 0.1 * randn(g, D)).to(dtype)
    cos_t, sin_t = tables(D, max_len, theta)
    base = [L - T for L in lens]
    c = torch.stack([cos_t[p:p + T] for p in base])
    s = torch.stack([sin_t[p:p + T] for p in base])
    qn = oracle.head_norm_rope(q, w, 1e-6, c, s)
    ref = oracle.ragged_decode(qn.float(), kc.float(), vc.float(), lens, window, scale_of(D))
    row_pos = torch.tensor(base, dtype=torch.int32, device=DEV)
    if fuse:
        got = ops().attn_decode(q.to(DEV), kc.to(DEV), vc.to(DEV), scale=scale_of(D), row_pos=row_pos,
                                max_kv_len=max(lens), window=window, q_weight=w.to(DEV), eps=1e-6,
                                norm_q=True, cos=c.to(DEV), sin=s.to(DEV), chunk=chunk)
    else:
        got = ops().attn_decode(qn.to(DEV), kc.to(DEV), vc.to(DEV), scale=scale_of(D), row_pos=row_pos,
                                max_kv_len=max(lens), window=window, chunk=chunk)
    return got.cpu(), ref.transpose(1, 2)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("D", [32, 64, 128, 256])
@pytest.mark.parametrize("HK", [(8, 4), (12, 4), (16, 8), (8, 1), (4, 4)])
def test_decode_single_token(dtype, D, HK):
    H, K = HK
    lens = [1, 17, 300, 777]
    got, ref = _decode_case(100 + D + H, dtype, 4, H, K, D, 1, lens, 0)
    assert max_abs(got, ref) <= tol(dtype)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("T", [2, 4, 5, 16])
@pytest.mark.parametrize("window", [0, 64])
def test_verify_multi_token(dtype, T, window):
    """k-token speculative verify (attention.py:192-193): causal among the new tokens."""
    got, ref = _decode_case(7 + T + window, dtype, 3, 8, 1, 256 if dtype != torch.float32 else 128,
                            T, [T, 200, 1100], window, theta=1e6)
    assert max_abs(got, ref) <= tol(dtype)


@pytest.mark.parametrize("window", [0, 5, 100])
def test_fp32_prefill_through_splitk(window):
    """Config-1 shape: fp32 causal prefill of 256 tokens on the general (split-K) path."""
    got, ref = _decode_case(11, torch.float32, 1, 8, 4, 32, 256, [256], window)
    assert max_abs(got, ref) <= 1e-4


def test_decode_prenormalised_q():
    got, ref = _decode_case(12, torch.bfloat16, 2, 16, 8, 128, 1, [4000, 4097], 0, fuse=False)
    assert max_abs(got, ref) <= 2e-2


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("H,K,D", [(8, 2, 128), (8, 1, 256), (6, 2, 64)])
def test_verify_rows_equal_single_decodes_bitwise(dtype, H, K, D):
    """A verify row (T = 5) equals decoding that token alone, bit for bit (same chunk):
    the property speculative decoding relies on (fused_ops.py:19-20). Covers the wide-group
    MFMA kernel (G = 4, 8 at hd 128/256) and the VALU kernel (G = 3, fp32)."""
    g = gen(5)
    B, T, L = 2, 5, 1500
    kc = randn(g, B, K, L + 8, D, dtype=dtype).to(DEV)
    vc = randn(g, B, K, L + 8, D, dtype=dtype).to(DEV)
    q = randn(g, B, H, T, D, dtype=dtype).to(DEV)
    sc = scale_of(D)
    for window in (0, 300):
        allv = ops().attn_decode(q, kc, vc, scale=sc, pos=L - T, window=window, chunk=256)
        for t in range(T):
            one = ops().attn_decode(q[:, :, t:t + 1], kc, vc, scale=sc, pos=L - T + t, window=window, chunk=256)
            assert torch.equal(allv[:, t:t + 1], one), (window, t)


@pytest.mark.parametrize("H,K", [(16, 8), (8, 1)])
def test_decode_pos_dev_matches_host_pos(H, K):
    """Device-held position equals the host position bit for bit at one chunk, on the VALU
    kernel (G = 2) and the wide-group MFMA kernel (G = 8)."""
    g = gen(9)
    B, D, T, L = 2, 128, 3, 900
    kc = randn(g, B, K, 1024, D, dtype=torch.bfloat16).to(DEV)
    vc = randn(g, B, K, 1024, D, dtype=torch.bfloat16).to(DEV)
    q = randn(g, B, H, T, D, dtype=torch.bfloat16).to(DEV)
    a = ops().attn_decode(q, kc, vc, scale=0.1, pos=L - T, chunk=128)
    b = ops().attn_decode(q, kc, vc, scale=0.1, pos_dev=torch.tensor([L - T], device=DEV),
                          max_kv_len=1024, chunk=128)
    assert torch.equal(a, b)


@pytest.mark.parametrize("cap", [2048, 8192])
def test_decode_pos_dev_default_chunk(cap):
    """One device-held position for every row (graph decode steps) takes the host position's
    default chunk (the uniform rule) and dense grid: 32 rows x 8 KV heads fill the CUs, so
    rows of 2,000 keys stay unsplit in a cache of their length and of four times it, where
    the per-row rule would split them. Bit for bit the host-position call, within bf16
    tolerance of the oracle, and blind to the 1e4-poisoned cache past the rows' end."""
    g = gen(41)
    B, H, K, D, L = 32, 16, 8, 128, 2000
    kc = randn(g, B, K, cap, D, dtype=torch.bfloat16)
    vc = randn(g, B, K, cap, D, dtype=torch.bfloat16)
    kc[:, :, L:] = 1e4
    vc[:, :, L:] = 1e4
    q = randn(g, B, H, 1, D, dtype=torch.bfloat16)
    assert ops().decode_chunk(torch.bfloat16, B, 1, H, K, D, cap, uniform=True) != \
        ops().decode_chunk(torch.bfloat16, B, 1, H, K, D, cap)
    kd, vd, qd = kc.to(DEV), vc.to(DEV), q.to(DEV)
    a = ops().attn_decode(qd, kd, vd, scale=scale_of(D), pos=L - 1)
    b = ops().attn_decode(qd, kd, vd, scale=scale_of(D), max_kv_len=cap,
                          pos_dev=torch.tensor([L - 1], dtype=torch.int64, device=DEV))
    assert torch.equal(a, b)
    ref = oracle.ragged_decode(q.float(), kc[:, :, :L].float(), vc[:, :, :L].float(), [L] * B, 0, scale_of(D))
    assert max_abs(b.cpu(), ref.transpose(1, 2)) <= 2e-2


@pytest.mark.parametrize("B", [8, 300])
def test_persistent_grid_equals_dense_grid_bitwise(B):
    """The persistent grid (device positions, units taken by ticket in any order) equals the
    dense grid of host positions bit for bit, with few rows and with many."""
    g = gen(21)
    H, K, D, T, L = 4, 2, 64, 1, 700
    kc = randn(g, B, K, 768, D, dtype=torch.bfloat16).to(DEV)
    vc = randn(g, B, K, 768, D, dtype=torch.bfloat16).to(DEV)
    q = randn(g, B, H, T, D, dtype=torch.bfloat16).to(DEV)
    a = ops().attn_decode(q, kc, vc, scale=0.1, pos=L - T, chunk=128)
    rp = torch.full((B,), L - T, dtype=torch.int32, device=DEV)
    b = ops().attn_decode(q, kc, vc, scale=0.1, row_pos=rp, max_kv_len=768, chunk=128)
    assert torch.equal(a, b)


@pytest.mark.parametrize("case", range(200))
def test_random_shapes_against_oracle(case):
    """Seeded random shapes over every decode/verify kernel: dtype, head dim, head group
    (G 1-8: the VALU kernel's 1-8-row blocks and the MFMA kernel from G = 4 at hd 128/256),
    T up to 8, ragged per-row lengths (the persistent grids), windows and chunks (the
    default rule, 256 and 1024 keys), against the oracle at the north-star tolerances."""
    rng = random.Random(7000 + case)
    dtype = rng.choice(DTYPES)
    D = rng.choice([32, 64, 128, 256])
    G, K = rng.choice([1, 2, 3, 4, 8]), rng.choice([1, 2, 4])
    T = rng.choice([1, 1, 2, 3, 4, 5, 8])
    lens = [rng.randint(T, 1200) for _ in range(rng.randint(1, 5))]
    window = rng.choice([0, 0, 1, 9, 100])
    chunk = rng.choice([0, 0, 256, 1024])
    print(f"case {case}: {dtype} D={D} H={G * K} K={K} T={T} lens={lens} window={window} chunk={chunk}",
          flush=True)
    got, ref = _decode_case(9000 + case, dtype, len(lens), G * K, K, D, T, lens, window, chunk=chunk)
    assert max_abs(got, ref) <= tol(dtype)


@pytest.mark.parametrize("case", range(64))
def test_random_position_modes_bitwise(case):
    """Seeded random shapes with one length for every row, given three ways at one chunk:
    the host position (dense grid), the device-held position (dense grid) and per-row
    positions (the persistent grids): bit for bit the same outputs."""
    rng = random.Random(8000 + case)
    dtype = rng.choice(DTYPES)
    D = rng.choice([64, 128, 256])
    G, K = rng.choice([1, 2, 3, 4, 8]), rng.choice([1, 2, 4])
    T = rng.choice([1, 2, 4, 5])
    B = rng.randint(1, 6)
    L = rng.randint(T, 2000)
    cap = L + rng.randint(0, 300)
    window = rng.choice([0, 0, 50])
    chunk = rng.choice([256, 1024])
    print(f"case {case}: {dtype} D={D} H={G * K} K={K} T={T} B={B} L={L} cap={cap} window={window} "
          f"chunk={chunk}", flush=True)
    g = gen(8100 + case)
    kc = randn(g, B, K, cap, D, dtype=dtype).to(DEV)
    vc = randn(g, B, K, cap, D, dtype=dtype).to(DEV)
    q = randn(g, B, G * K, T, D, dtype=dtype).to(DEV)
    kw = dict(scale=scale_of(D), window=window, chunk=chunk)
    a = ops().attn_decode(q, kc, vc, pos=L - T, **kw)
    b = ops().attn_decode(q, kc, vc, pos_dev=torch.tensor([L - T], dtype=torch.int64, device=DEV),
                          max_kv_len=cap, **kw)
    c = ops().attn_decode(q, kc, vc, row_pos=torch.full((B,), L - T, dtype=torch.int32, device=DEV),
                          max_kv_len=cap, **kw)
    assert torch.equal(a, b)
    assert torch.equal(a, c)


@pytest.mark.parametrize("B", [40, 300])
def test_decode_ragged_many_rows(B):
    """Ragged lengths over many rows of the persistent grid."""
    lens = torch.randint(1, 700, (B,), generator=torch.Generator().manual_seed(B)).tolist()
    got, ref = _decode_case(31, torch.bfloat16, B, 4, 2, 64, 1, lens, 0, chunk=128)
    assert max_abs(got, ref) <= 2e-2


@pytest.mark.parametrize("B,H,K,D,T,window", [(1000, 4, 2, 64, 1, 0), (2048, 2, 2, 32, 2, 0),
                                                (200, 16, 4, 128, 3, 0), (512, 8, 2, 128, 1, 90)])
def test_persistent_tail_order_many_rows(B, H, K, D, T, window):
    """The persistent grids hand the rows' last chunks out last, largest first, in an order
    every block derives alike (a stable counting sort by size class, in passes of 64 rows).
    Many rows, many of one class (lengths repeat): the split kernel up to its 2048-row limit
    and the MFMA kernel (G = 4) up to its 512, against the oracle."""
    rng = random.Random(B + T)
    lens = [rng.choice([T, 97, 128, 129, 256, 300, rng.randint(T, 600)]) for _ in range(B)]
    lens = [max(L, T) for L in lens]
    got, ref = _decode_case(B + 17, torch.bfloat16, B, H, K, D, T, lens, window, chunk=128)
    assert max_abs(got, ref) <= 2e-2


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_persistent_verify_row_blocks_with_early_returns(dtype):
    """Device lengths (the persistent grid), T = 4 with G = 3 (12 query rows: row blocks of
    8 and 4), window 40 and 64-key chunks. The two row blocks see different key ranges, and
    the lengths put a chunk boundary just past row block 0's last key (L = 321) and just
    before row block 1's first key (L = 553), so units return early without a block barrier:
    the path on which the block's next work ticket must not be overwritten before every wave
    has read the previous one. Equal to the oracle, and the uniform-length case equal bit
    for bit to the dense grid of the host position."""
    B, H, K, D, T = 6, 12, 4, 64, 4
    lens = [44, 321, 553, 617, 1000, 257]
    got, ref = _decode_case(77, dtype, B, H, K, D, T, lens, 40, chunk=64)
    assert max_abs(got, ref) <= tol(dtype)
    g = gen(78)
    L = 321
    kc = randn(g, B, K, 400, D, dtype=dtype).to(DEV)
    vc = randn(g, B, K, 400, D, dtype=dtype).to(DEV)
    q = randn(g, B, H, T, D, dtype=dtype).to(DEV)
    dense = ops().attn_decode(q, kc, vc, scale=0.125, pos=L - T, window=40, chunk=64)
    rp = torch.full((B,), L - T, dtype=torch.int32, device=DEV)
    for _ in range(3):
        persistent = ops().attn_decode(q, kc, vc, scale=0.125, row_pos=rp, max_kv_len=400, window=40, chunk=64)
        assert torch.equal(dense, persistent)


@pytest.mark.parametrize("T,H,K", [(1, 16, 8), (2, 8, 8), (1, 32, 8), (5, 32, 8), (4, 8, 1)])
def test_persistent_runs_equal_per_row_dense_calls(T, H, K):
    """Ragged rows on the persistent grid (64 rows, up to 47 chunks each, units taken by
    ticket in any order) equal bit for bit the same rows computed one at a time on the dense
    grid (T = 2: two query rows with different last keys in one row block). G >= 4 runs the
    MFMA verify kernel, persistent too (at T = 1 and 5 for 32 q / 8 KV heads, and the MQA
    verify shape at head dim 256)."""
    g = gen(61)
    B, chunk = 64, 128
    D = 256 if K == 1 else 128
    lens = torch.randint(T, 6000, (B,), generator=torch.Generator().manual_seed(61)).tolist()
    L = max(lens)
    kc = randn(g, B, K, L, D, dtype=torch.bfloat16).to(DEV)
    vc = randn(g, B, K, L, D, dtype=torch.bfloat16).to(DEV)
    q = randn(g, B, H, T, D, dtype=torch.bfloat16).to(DEV)
    rp = torch.tensor([n - T for n in lens], dtype=torch.int32, device=DEV)
    o = ops()
    for _ in range(2):   # the second call reuses the first one's cleared work ticket
        got = o.attn_decode(q, kc, vc, scale=0.1, row_pos=rp, max_kv_len=L, chunk=chunk)
        for b in range(B):
            want = o.attn_decode(q[b:b + 1], kc[b:b + 1], vc[b:b + 1], scale=0.1, pos=lens[b] - T, chunk=chunk)
            assert torch.equal(got[b:b + 1], want), (b, lens[b])


def test_decode_append_runs_equal_per_row_dense_calls():
    """forge_attn_decode_append on ragged rows of the persistent grid (the unit holding a
    row's last chunk also makes the new keys) equals the two calls, and each row equals its
    own dense-grid decode over the cache the append wrote, bit for bit."""
    lens = torch.randint(2, 5000, (64,), generator=torch.Generator().manual_seed(62)).tolist()
    (y1, k1, v1), (y2, k2, v2), (q, k, v, wq, wk, c, s) = _append_decode_pair(
        63, torch.bfloat16, 64, 16, 8, 128, 1, lens, 0, "row_pos", chunk=128)
    assert torch.equal(y1, y2) and torch.equal(k1, k2) and torch.equal(v1, v2)
    o = ops()
    for b, n in enumerate(lens):
        want = o.attn_decode(q[b:b + 1], k1[b:b + 1], v1[b:b + 1], scale=scale_of(128), pos=n - 1,
                             q_weight=wq, eps=1e-6, norm_q=True, cos=c[b], sin=s[b], chunk=128,
                             max_kv_len=n)
        assert torch.equal(y2[b:b + 1], want), (b, n)


# ------------------------------------------------------------------ MTP drafter attention
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("H,K,D", [(8, 2, 128), (8, 1, 256)])
@pytest.mark.parametrize("n_past,window", [(1, 0), (300, 0), (1000, 0), (200, 512), (900, 512), (512, 512)])
def test_drafter_attention(dtype, H, K, D, n_past, window):
    """The drafter's query at position n_past over the target's stored keys (mtp.py:73-92),
    host position and device position (the graph form, mtp.py:169-188)."""
    g = gen(400 + n_past + window)
    B, L = 2, 1024
    q = randn(g, B, H, 1, D, dtype=dtype)
    kc = randn(g, B, K, L, D, dtype=dtype)
    vc = randn(g, B, K, L, D, dtype=dtype)
    ref = oracle.drafter_attention(q.float(), kc.float(), vc.float(), n_past, window, 1.0 / 16)
    got = ops().attn_drafter(q.to(DEV), kc.to(DEV), vc.to(DEV), n_past=n_past, window=window, scale=1.0 / 16)
    assert max_abs(got.cpu().transpose(1, 2), ref) <= tol(dtype)
    got_dev = ops().attn_drafter(q.to(DEV), kc.to(DEV), vc.to(DEV), n_past_dev=torch.tensor([n_past], device=DEV),
                                 window=window, scale=1.0 / 16)
    assert torch.equal(got_dev, got)


def test_drafter_attention_rejects_bad_positions():
    q = torch.zeros(1, 4, 1, 64, device=DEV, dtype=torch.bfloat16)
    c = torch.zeros(1, 2, 16, 64, device=DEV, dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        ops().attn_drafter(q, c, c, n_past=0)
    with pytest.raises(ValueError):
        ops().attn_drafter(q, c, c, n_past=4, window=1)


# ------------------------------------------------------------------ MFMA prefill
def _prefill_case(seed, dtype, B, H, K, D, T, offset, window, theta=1e4):
    g = gen(seed)
    S = offset + T
    q = randn(g, B, T, H, D, dtype=dtype).transpose(1, 2)
    w = (1 + 0.1 * randn(g, D)).to(dtype)
    kc = randn(g, B, K, S + 5, D, dtype=dtype)
    vc = randn(g, B, K, S + 5, D, dtype=dtype)
    cos_t, sin_t = tables(D, S, theta)
    c, s = cos_t[offset:S], sin_t[offset:S]
    qn = oracle.head_norm_rope(q, w, 1e-6, c, s)
    ref = oracle.sdpa(qn.float(), kc[:, :, :S].float(), vc[:, :, :S].float(), offset, window, scale_of(D))
    got = ops().attn_prefill(q.to(DEV), kc.to(DEV), vc.to(DEV), scale=scale_of(D), offset=offset,
                             window=window, q_weight=w.to(DEV), eps=1e-6, norm_q=True,
                             cos=c.to(DEV), sin=s.to(DEV))
    return got.cpu(), ref.transpose(1, 2)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("D", [64, 128, 256])
@pytest.mark.parametrize("T,offset", [(128, 0), (300, 0), (200, 37), (65, 500)])
def test_prefill(dtype, D, T, offset):
    got, ref = _prefill_case(D + T + offset, dtype, 2, 4, 2, D, T, offset, 0)
    assert max_abs(got, ref) <= tol(dtype)


@pytest.mark.parametrize("case", range(48))
def test_random_prefill_shapes_against_oracle(case):
    """Seeded random prefill shapes: bf16/fp16, head dims 64/128/256, head groups 1-8,
    T 17-700 (partial query and key tiles), offsets into a filled cache, windows."""
    rng = random.Random(6000 + case)
    dtype = rng.choice([torch.bfloat16, torch.float16])
    D = rng.choice([64, 128, 256])
    G, K = rng.choice([1, 2, 3, 4, 8]), rng.choice([1, 2])
    B, T = rng.randint(1, 3), rng.randint(17, 700)
    offset = rng.choice([0, 0, rng.randint(1, 600)])
    window = rng.choice([0, 0, 1, 33, 256])
    print(f"case {case}: {dtype} D={D} H={G * K} K={K} B={B} T={T} offset={offset} window={window}", flush=True)
    got, ref = _prefill_case(6100 + case, dtype, B, G * K, K, D, T, offset, window)
    assert max_abs(got, ref) <= tol(dtype)


@pytest.mark.parametrize("window", [1, 64, 100, 1024])
def test_prefill_sliding_window(window):
    got, ref = _prefill_case(window, torch.bfloat16, 1, 8, 1, 128, 700, 40, window)
    assert max_abs(got, ref) <= 2e-2


def _doc_ids(lengths_per_row):
    """[B, T] document numbers from each row's document lengths."""
    rows = [torch.cat([torch.full((n,), d) for d, n in enumerate(ls)]) for ls in lengths_per_row]
    return torch.stack(rows)


def _doc_starts_of(doc_ids):
    """First position of each position's document (documents are contiguous runs)."""
    B, T = doc_ids.shape
    start = torch.zeros(B, T, dtype=torch.int32)
    for b in range(B):
        for t in range(1, T):
            start[b, t] = start[b, t - 1] if doc_ids[b, t] == doc_ids[b, t - 1] else t
    return start


# documents per row: a 1-token document, boundaries on and off the 64/128-key tiles, one
# document longer than a query block, and a row that is one document
DOC_LAYOUTS = [[[5, 1, 122, 64, 256, 252], [700]],
               [[128, 128, 1, 63, 380], [64] * 10 + [60]]]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("D", [64, 128, 256])
@pytest.mark.parametrize("layout", [0, 1])
@pytest.mark.parametrize("window", [0, 100])
def test_prefill_with_documents(dtype, D, layout, window):
    """forge_attn_prefill_docs: causal and within each query's document (the reference's
    same_doc mask, transformer.py:271-275 with attention.py:184-186), against the oracle's
    SDPA with that mask (K/V heads repeated, as the reference does with a document mask)."""
    g = gen(900 + D + layout + window)
    docs = _doc_ids(DOC_LAYOUTS[layout])
    B, T = docs.shape
    H, K = 4, 2
    q = randn(g, B, T, H, D, dtype=dtype).transpose(1, 2)
    w = (1 + 0.1 * randn(g, D)).to(dtype)
    kc = randn(g, B, K, T, D, dtype=dtype)
    vc = randn(g, B, K, T, D, dtype=dtype)
    c, s = tables(D, T, 1e4)
    qn = oracle.head_norm_rope(q, w, 1e-6, c, s)
    ref = oracle.sdpa(qn.float(), kc.float(), vc.float(), 0, window, scale_of(D),
                      oracle.document_mask(docs)).transpose(1, 2)
    ds = _doc_starts_of(docs).to(DEV)
    got = ops().attn_prefill(q.to(DEV), kc.to(DEV), vc.to(DEV), scale=scale_of(D), window=window,
                             q_weight=w.to(DEV), eps=1e-6, norm_q=True, cos=c.to(DEV), sin=s.to(DEV),
                             doc_start=ds).cpu()
    assert max_abs(got, ref) <= tol(dtype)


@pytest.mark.parametrize("case", range(32))
def test_random_document_prefill_against_oracle(case):
    """Seeded random document layouts (every row cut into documents of random lengths,
    single-token ones included), head dims, head groups and windows, against the oracle's
    SDPA under the reference's same_doc mask."""
    rng = random.Random(4000 + case)
    dtype = rng.choice([torch.bfloat16, torch.float16])
    D = rng.choice([64, 128, 256])
    G, K = rng.choice([1, 2, 4]), rng.choice([1, 2])
    B, T = rng.randint(1, 3), rng.randint(17, 600)
    window = rng.choice([0, 0, 50])
    layout = []
    for _ in range(B):
        cuts = sorted(rng.sample(range(1, T), rng.randint(0, min(8, T - 1))))
        layout.append([e - b for b, e in zip([0] + cuts, cuts + [T])])
    print(f"case {case}: {dtype} D={D} H={G * K} K={K} window={window} docs={layout}", flush=True)
    g = gen(4100 + case)
    docs = _doc_ids(layout)
    H = G * K
    q = randn(g, B, T, H, D, dtype=dtype).transpose(1, 2)
    w = (1 + 0.1 * randn(g, D)).to(dtype)
    kc = randn(g, B, K, T, D, dtype=dtype)
    vc = randn(g, B, K, T, D, dtype=dtype)
    c, s = tables(D, T, 1e4)
    qn = oracle.head_norm_rope(q, w, 1e-6, c, s)
    ref = oracle.sdpa(qn.float(), kc.float(), vc.float(), 0, window, scale_of(D),
                      oracle.document_mask(docs)).transpose(1, 2)
    got = ops().attn_prefill(q.to(DEV), kc.to(DEV), vc.to(DEV), scale=scale_of(D), window=window,
                             q_weight=w.to(DEV), eps=1e-6, norm_q=True, cos=c.to(DEV), sin=s.to(DEV),
                             doc_start=_doc_starts_of(docs).to(DEV)).cpu()
    assert max_abs(got, ref) <= tol(dtype)


def test_prefill_one_document_equals_plain_prefill():
    """Document starts all 0 (one document per row) change nothing, bit for bit."""
    g = gen(950)
    B, H, K, D, T = 2, 8, 2, 128, 333
    q = randn(g, B, H, T, D, dtype=torch.bfloat16).to(DEV)
    kc = randn(g, B, K, T, D, dtype=torch.bfloat16).to(DEV)
    vc = randn(g, B, K, T, D, dtype=torch.bfloat16).to(DEV)
    a = ops().attn_prefill(q, kc, vc, scale=0.1)
    b = ops().attn_prefill(q, kc, vc, scale=0.1, doc_start=torch.zeros(B, T, dtype=torch.int32, device=DEV))
    assert torch.equal(a, b)


def test_prefill_documents_rejects_bad_starts():
    q = torch.zeros(1, 2, 40, 64, dtype=torch.bfloat16, device=DEV)
    k = torch.zeros(1, 1, 40, 64, dtype=torch.bfloat16, device=DEV)
    bad = [torch.arange(40, dtype=torch.int32).flip(0)[None],       # decreasing
           torch.full((1, 40), 5, dtype=torch.int32)]                 # after the first queries
    for ds in bad:
        with pytest.raises(ValueError):
            ops().attn_prefill(q, k, k, scale=0.1, doc_start=ds.to(DEV))


def test_prefill_rejects_fp32():
    q = torch.zeros(1, 2, 4, 128, device=DEV)
    with pytest.raises(ValueError):
        ops().attn_prefill(q, q[:, :1], q[:, :1], scale=1.0)


# ------------------------------------------------------------------ decode with the cache write
def _append_decode_pair(seed, dtype, B, H, K, D, T, lens, window, where, norm_v=False, chunk=0,
                        theta=1e6, max_len=None):
    """One step twice on one cache: forge_kv_append then forge_attn_decode, and
    forge_attn_decode_append. lens[b] = keys row b holds after the step (its T new ones
    included); earlier positions hold N(0,1), later ones 1e4 poison. `where` picks the
    position source: 'pos' (host, lens equal), 'row_pos' (device, per row), 'pos_dev'."""
    g = gen(seed)
    max_len = max_len or max(lens) + 9
    qkv = randn(g, B, T, H + 2 * K, D, dtype=dtype).to(DEV)
    q = qkv[:, :, :H].transpose(1, 2)
    k = qkv[:, :, H:H + K].transpose(1, 2)
    v = qkv[:, :, H + K:].transpose(1, 2)
    wq = (1 + 0.1 * randn(g, D)).float().to(DEV)
    wk = (1 + 0.1 * randn(g, D)).float().to(DEV)
    base = [L - T for L in lens]
    cos_t, sin_t = tables(D, max_len + T, theta)
    c = torch.stack([cos_t[p:p + T] for p in base]).to(DEV)
    s = torch.stack([sin_t[p:p + T] for p in base]).to(DEV)
    kc = torch.full((B, K, max_len, D), 1e4, dtype=dtype)
    vc = torch.full((B, K, max_len, D), 1e4, dtype=dtype)
    for b, p in enumerate(base):
        kc[b, :, :p] = randn(g, K, p, D, dtype=dtype)
        vc[b, :, :p] = randn(g, K, p, D, dtype=dtype)
    kc, vc = kc.to(DEV), vc.to(DEV)
    mk = dict(max_kv_len=max_len)
    if where == "pos":
        assert len(set(base)) == 1
        pk, mk = dict(pos=base[0]), {}
        c, s = c[0], s[0]
    elif where == "row_pos":
        pk = dict(row_pos=torch.tensor(base, dtype=torch.int32, device=DEV))
    else:
        assert len(set(base)) == 1
        pk = dict(pos_dev=torch.tensor([base[0]], dtype=torch.int64, device=DEV))
        c, s = c[0], s[0]
    qa = dict(scale=scale_of(D), window=window, q_weight=wq, eps=1e-6, norm_q=True, cos=c, sin=s,
              chunk=chunk, **mk)
    o = ops()
    k1, v1 = kc.clone(), vc.clone()
    o.kv_append(k, v, k1, v1, k_weight=wk, eps=1e-6, norm_k=True, norm_v=norm_v, cos=c, sin=s, **pk)
    y1 = o.attn_decode(q, k1, v1, **pk, **qa)
    k2, v2 = kc.clone(), vc.clone()
    y2 = o.attn_decode_append(q, k, v, k2, v2, k_weight=wk, norm_k=True, norm_v=norm_v, **pk, **qa)
    torch.cuda.synchronize()
    return (y1, k1, v1), (y2, k2, v2), (q, k, v, wq, wk, c, s)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("D", [32, 64, 128, 256])
@pytest.mark.parametrize("HK", [(8, 4), (12, 4), (16, 8), (8, 1)])
def test_decode_append_equals_append_then_decode(dtype, D, HK):
    """forge_attn_decode_append == forge_kv_append + forge_attn_decode bit for bit: the
    outputs and the whole caches (the rows before, the new ones, the poisoned rest). One
    new token on ragged rows (persistent grid), through the fused kernel or, for the
    wide-group MFMA path (G = 8 at bf16/fp16 hd 128/256), the two launches."""
    H, K = HK
    a, b, _ = _append_decode_pair(D + H + K, dtype, 4, H, K, D, 1, [1, 18, 300, 777], 0, "row_pos")
    for x, y in zip(a, b):
        assert torch.equal(x, y)


@pytest.mark.parametrize("T", [2, 5, 16])
@pytest.mark.parametrize("window", [0, 40])
@pytest.mark.parametrize("where", ["pos", "row_pos", "pos_dev"])
def test_decode_append_verify_steps(T, window, where):
    """Verify steps of T new tokens (the new keys may straddle a chunk boundary: 64-key
    chunks, the new keys at 510 .. 510 + T - 1), host, per-row and device positions, and
    a values norm: equal to the two calls bit for bit. The last case is the MFMA verify
    path (MQA, hd 256: 32 query rows of one KV head in one unit up to T = 4, two launches
    beyond)."""
    lens = [510 + T] * 3 if where != "row_pos" else [T, 510 + T, 900]
    for dtype, D, (H, K) in ((torch.bfloat16, 128, (16, 8)), (torch.float32, 64, (12, 4)),
                             (torch.float16, 256, (4, 2)), (torch.bfloat16, 256, (8, 1))):
        a, b, _ = _append_decode_pair(T + window, dtype, 3, H, K, D, T, lens, window, where,
                                      norm_v=(T == 5), chunk=64 if D < 256 else 128)
        for x, y in zip(a, b):
            assert torch.equal(x, y), (dtype, D)


@pytest.mark.parametrize("case", range(64))
def test_random_decode_append_equals_two_calls(case):
    """Seeded random steps with the cache write: forge_attn_decode_append against
    forge_kv_append + forge_attn_decode, bit for bit (outputs and whole caches), over dtypes,
    head dims 32-256, head groups 1-8, T up to 8, host / per-row / device positions,
    windows, the values norm and the default or explicit chunks."""
    rng = random.Random(5000 + case)
    dtype = rng.choice(DTYPES)
    D = rng.choice([32, 64, 128, 256])
    G, K = rng.choice([1, 2, 3, 4, 8]), rng.choice([1, 2, 4])
    T = rng.choice([1, 1, 2, 3, 5, 8])
    B = rng.randint(1, 5)
    where = rng.choice(["pos", "row_pos", "pos_dev"])
    if where == "row_pos":
        lens = [rng.randint(T, 1500) for _ in range(B)]
    else:
        lens = [rng.randint(T, 1500)] * B
    window = rng.choice([0, 0, 1, 40])
    chunk = rng.choice([0, 0, 256, 1024])
    norm_v = rng.random() < 0.3
    print(f"case {case}: {dtype} D={D} H={G * K} K={K} T={T} lens={lens} {where} window={window} "
          f"chunk={chunk} norm_v={norm_v}", flush=True)
    a, b, _ = _append_decode_pair(5100 + case, dtype, B, G * K, K, D, T, lens, window, where,
                                  norm_v=norm_v, chunk=chunk)
    for x, y in zip(a, b):
        assert torch.equal(x, y)


def test_decode_append_against_the_oracle():
    """The fused step against the oracle: the keys the reference's KVCache.update would
    store after head_norm_rope (kv_cache.py:52-60, fused_ops.py:101-121), the values as
    given, and the attention output of the new token over the whole row."""
    B, H, K, D, T = 3, 16, 8, 128, 1
    lens = [40, 1000, 3000]
    _, (y, kc, vc), (q, k, v, wq, wk, c, s) = _append_decode_pair(77, torch.bfloat16, B, H, K, D, T, lens, 0,
                                                                  "row_pos")
    kn = oracle.head_norm_rope(k.cpu(), wk.cpu(), 1e-6, c.cpu(), s.cpu())
    qn = oracle.head_norm_rope(q.cpu(), wq.cpu(), 1e-6, c.cpu(), s.cpu())
    for b, L in enumerate(lens):
        assert max_abs(kc[b, :, L - 1:L], kn[b]) <= 2e-2
        assert torch.equal(vc[b, :, L - 1:L].cpu(), v[b].cpu())
        assert (kc[b, :, L:].cpu() == 1e4).all() and (vc[b, :, L:].cpu() == 1e4).all()
    ref = oracle.ragged_decode(qn.float(), kc.float().cpu(), vc.float().cpu(), lens, 0, scale_of(D))
    assert max_abs(y, ref.transpose(1, 2)) <= 2e-2


def test_decode_append_with_a_cleared_workspace_across_calls():
    """FORGE_WS_ZEROED: a workspace cleared once, reused by calls of different shapes on the
    persistent grid (per-row lengths) without the ticket-reset kernel, gives the results of
    calls that reset it, bit for bit, and is left with a zero ticket after each call."""
    o = ops()
    ws = torch.zeros(8 << 20, dtype=torch.uint8, device=DEV)
    for i, (B, H, K, D, T, lens) in enumerate([(6, 16, 8, 128, 1, [900, 40, 3000, 1, 2200, 700]),
                                               (3, 12, 4, 64, 4, [515, 2049, 64]),
                                               (6, 16, 8, 128, 1, [901, 41, 3001, 2, 2201, 701])]):
        a, b, (q, k, v, wq, wk, c, s) = _append_decode_pair(40 + i, torch.bfloat16, B, H, K, D, T, lens, 0,
                                                            "row_pos", chunk=64)
        kc, vc = a[1].clone(), a[2].clone()
        base = [L - T for L in lens]
        # rewind the rows the pair already wrote (the fused call writes them again)
        y = o.attn_decode_append(q, k, v, kc, vc, scale=scale_of(D),
                                 row_pos=torch.tensor(base, dtype=torch.int32, device=DEV),
                                 max_kv_len=kc.shape[2], q_weight=wq, k_weight=wk, eps=1e-6, norm_q=True,
                                 norm_k=True, cos=c, sin=s, chunk=64, workspace=ws, workspace_zeroed=True)
        torch.cuda.synchronize()
        assert torch.equal(y, a[0]) and torch.equal(kc, a[1]) and torch.equal(vc, a[2]), i
        assert int(ws[:4].view(torch.int32).item()) == 0, i
