"""Pins of the CPU oracle (oracle/attention_ref.py) against closed forms, the reference's
own golden lists, an independent float64 brute force and the cache invariants the
reference's tests assert. Each pin is a check_* function; the mutation tests plant a
plausible mistake in a copy of the oracle function and show the pin rejects it."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle
from oracle import attention_ref as ref

# ----------------------------------------------------------------------------- pins


def check_rope_tables(tables_fn) -> None:
    """cos/sin[p, i] = cos/sin(p * theta^(-2i/d)) for i < d/2, halves duplicated
    (rope.py:21-38). Angles are formed in fp32 as the reference does, so compare with
    the float64 cos of the float64 angle within fp32 angle rounding."""
    d, L, theta = 64, 300, 1e4
    cos, sin = tables_fn(d, L, theta)
    assert cos.shape == (L, d) and sin.shape == (L, d) and cos.dtype == torch.float32
    i = np.arange(d // 2, dtype=np.float64)
    p = np.arange(L, dtype=np.float64)[:, None]
    ang = p * theta ** (-2 * i / d)
    tol = 4e-7 * L + 1e-6   # |angle| * fp32 eps bound on the rounding of p * inv_freq
    np.testing.assert_allclose(cos[:, : d // 2].double().numpy(), np.cos(ang), atol=tol)
    np.testing.assert_allclose(sin[:, : d // 2].double().numpy(), np.sin(ang), atol=tol)
    assert torch.equal(cos[:, : d // 2], cos[:, d // 2:]) and torch.equal(sin[:, : d // 2], sin[:, d // 2:])


def check_rope_rotation(rope_fn) -> None:
    """NEOX rope = multiplying x[:d/2] + i*x[d/2:] by e^{i*angle} (rope.py:46-55)."""
    g = torch.Generator().manual_seed(0)
    d, T = 32, 9
    x = torch.randn(2, 3, T, d, generator=g)
    cos, sin = oracle.rope_tables(d, T, 1e4)
    got = rope_fn(x, cos, sin).double()
    z = torch.complex(x[..., : d // 2].double(), x[..., d // 2:].double())
    ang = torch.atan2(sin[:, : d // 2].double(), cos[:, : d // 2].double())
    w = z * torch.exp(1j * ang)
    np.testing.assert_allclose(got[..., : d // 2].numpy(), w.real.numpy(), atol=2e-6)
    np.testing.assert_allclose(got[..., d // 2:].numpy(), w.imag.numpy(), atol=2e-6)


def check_rope_relative(rope_fn) -> None:
    """<rope(q, i), rope(k, j)> depends only on i - j."""
    g = torch.Generator().manual_seed(1)
    d = 64
    q = torch.randn(1, 1, 1, d, generator=g)
    k = torch.randn(1, 1, 1, d, generator=g)
    cos, sin = oracle.rope_tables(d, 200, 1e4)

    def score(i, j):
        return float((rope_fn(q, cos[i:i + 1], sin[i:i + 1]) * rope_fn(k, cos[j:j + 1], sin[j:j + 1])).sum())

    assert abs(score(10, 3) - score(107, 100)) < 1e-4
    assert abs(score(10, 3) - score(10, 4)) > 1e-3   # and it does depend on the difference


def check_rms_norm(norm_fn) -> None:
    """y = x / sqrt(mean(x^2) + eps) * w in fp32 (norm.py:50)."""
    g = torch.Generator().manual_seed(2)
    x = torch.randn(4, 7, 48, generator=g) * 3
    w = 1 + 0.1 * torch.randn(48, generator=g)
    eps = 1e-6
    xd = x.double()
    want = xd / torch.sqrt((xd * xd).mean(-1, keepdim=True) + eps) * w.double()
    np.testing.assert_allclose(norm_fn(x, w, eps).double().numpy(), want.numpy(), atol=2e-6)
    unit = norm_fn(x, None, eps).double()
    np.testing.assert_allclose(unit.pow(2).mean(-1).numpy(), np.ones((4, 7)), atol=1e-5)


def check_head_norm_rope(fn) -> None:
    """fp32 norm + rope, ONE rounding to bf16 (fused_ops.py:16-20, 53-85): equal to the
    float64 result rounded to bf16 except for rare ties within one bf16 ulp."""
    g = torch.Generator().manual_seed(3)
    d, T = 128, 16
    x = (3 * torch.randn(2, 4, T, d, generator=g)).bfloat16()
    w = (1 + 0.3 * torch.randn(d, generator=g)).bfloat16()
    cos, sin = oracle.rope_tables(d, 64, 1e6)
    cos, sin = cos[20:20 + T], sin[20:20 + T]
    got = fn(x, w, 1e-6, cos, sin)
    assert got.dtype == torch.bfloat16
    xd = x.double()
    n = xd / torch.sqrt((xd * xd).mean(-1, keepdim=True) + 1e-6) * w.double()
    rot = torch.cat([-n[..., d // 2:], n[..., : d // 2]], -1)
    exact = n * cos.double() + rot * sin.double()
    diff = (got.double() - exact).abs()
    ulp = exact.abs().clamp_min(1e-30) * 2.0 ** -8
    assert torch.all(diff <= ulp)
    same = (got == exact.bfloat16()).double().mean().item()
    assert same > 0.99, same


def check_mask(mask_fn) -> None:
    """The reference's golden static masks (tests/test_cuda_graph.py:55-61): a query at
    position 10 over 16 keys sees [True]*11 + [False]*5; with window 4 only 7..10."""
    assert mask_fn(1, 16, 10, 0).view(-1).tolist() == [True] * 11 + [False] * 5
    assert mask_fn(1, 16, 10, 4).view(-1).nonzero().view(-1).tolist() == [7, 8, 9, 10]
    m = mask_fn(5, 12, 7, 3)
    for i in range(5):
        for j in range(12):
            assert bool(m[i, j]) == (j <= 7 + i and 7 + i - j < 3)


CASES = [  # B, H, K, D, T, offset, window
    (1, 4, 4, 16, 6, 0, 0),
    (2, 4, 2, 16, 5, 4, 0),
    (1, 8, 1, 8, 1, 9, 0),
    (1, 4, 2, 8, 7, 3, 4),
    (2, 2, 1, 8, 1, 12, 5),
    (1, 6, 3, 8, 4, 0, 2),
]


def check_attention(attn_fn) -> None:
    """attn_fn(q, k, v, offset, window, scale) against the float64 loop restatement."""
    for n, (B, H, K, D, T, off, win) in enumerate(CASES):
        g = torch.Generator().manual_seed(10 + n)
        q = torch.randn(B, H, T, D, generator=g)
        k = torch.randn(B, K, off + T, D, generator=g)
        v = torch.randn(B, K, off + T, D, generator=g)
        sc = 1 / math.sqrt(D)
        want = oracle.brute_attention(q, k, v, off, win, sc)
        got = attn_fn(q, k, v, off, win, sc).double()
        np.testing.assert_allclose(got.numpy(), want.numpy(), atol=1e-5, err_msg=str(CASES[n]))


# ----------------------------------------------------------------------------- the oracle passes
def test_rope_tables_pinned():
    check_rope_tables(oracle.rope_tables)


def test_rope_rotation_pinned():
    check_rope_rotation(oracle.apply_rope)
    check_rope_relative(oracle.apply_rope)


def test_rms_norm_pinned():
    check_rms_norm(oracle.rms_norm)


def test_head_norm_rope_pinned():
    check_head_norm_rope(oracle.head_norm_rope)


def test_head_norm_rope_is_norm_then_rope_in_fp32():
    g = torch.Generator().manual_seed(4)
    x = torch.randn(1, 2, 5, 64, generator=g)
    w = 1 + 0.1 * torch.randn(64, generator=g)
    cos, sin = oracle.rope_tables(64, 5, 1e4)
    torch.testing.assert_close(oracle.head_norm_rope(x, w, 1e-6, cos, sin),
                               oracle.apply_rope(oracle.rms_norm(x, w, 1e-6), cos, sin), atol=1e-6, rtol=0)


def test_mask_pinned():
    check_mask(oracle.attention_mask)


def test_static_cache_mask_golden():
    """StaticKVCache.attn_mask KATs (tests/test_cuda_graph.py:55-61)."""
    c = oracle.StaticKVCache([(1, 4)], 1, 32)
    c.length, c.static = 16, True
    c.pos_t.fill_(10)
    assert c.attn_mask().view(-1).tolist() == [True] * 11 + [False] * 5
    assert c.attn_mask(4).view(-1).nonzero().view(-1).tolist() == [7, 8, 9, 10]


def test_sdpa_pinned():
    check_attention(oracle.sdpa)


def test_explicit_pinned():
    check_attention(lambda q, k, v, o, w, s: oracle.explicit_attention(q, k, v, o, w, s))


def test_explicit_probs_rows_sum_to_one_and_are_causal():
    """tests/test_model.py:81-89: pattern rows sum to 1, zero upper triangle."""
    g = torch.Generator().manual_seed(5)
    q, k, v = (torch.randn(1, 4, 12, 16, generator=g) for _ in range(3))
    _, p = oracle.explicit_attention(q, k, v, 0, 0, 0.25, return_probs=True)
    torch.testing.assert_close(p.sum(-1), torch.ones(1, 4, 12))
    assert torch.all(p.triu(1) == 0)


def test_single_key_and_equal_keys_closed_forms():
    g = torch.Generator().manual_seed(6)
    q = torch.randn(1, 2, 1, 8, generator=g)
    k = torch.randn(1, 1, 1, 8, generator=g)
    v = torch.randn(1, 1, 1, 8, generator=g)
    torch.testing.assert_close(oracle.sdpa(q, k, v, 0, 0, 0.3), v.expand(1, 2, 1, 8), atol=1e-6, rtol=0)
    k = torch.randn(1, 1, 1, 8, generator=g).expand(1, 1, 10, 8)
    v = torch.randn(1, 1, 10, 8, generator=g)
    out = oracle.sdpa(q, k, v, 9, 0, 0.3)
    torch.testing.assert_close(out, v.mean(2, keepdim=True).expand(1, 2, 1, 8), atol=1e-6, rtol=0)
    out = oracle.sdpa(q, k, v, 9, 4, 0.3)   # window 4: the last 4 values
    torch.testing.assert_close(out, v[:, :, 6:].mean(2, keepdim=True).expand(1, 2, 1, 8), atol=1e-6, rtol=0)


def test_gqa_equals_repeated_heads():
    g = torch.Generator().manual_seed(7)
    q = torch.randn(2, 8, 5, 16, generator=g)
    k = torch.randn(2, 2, 9, 16, generator=g)
    v = torch.randn(2, 2, 9, 16, generator=g)
    a = oracle.sdpa(q, k, v, 4, 0, 0.25)
    b = oracle.sdpa(q, k.repeat_interleave(4, 1), v.repeat_interleave(4, 1), 4, 0, 0.25)
    torch.testing.assert_close(a, b, atol=1e-6, rtol=0)


def test_causality():
    g = torch.Generator().manual_seed(8)
    q, k, v = (torch.randn(1, 2, 10, 8, generator=g) for _ in range(3))
    a = oracle.sdpa(q, k, v, 0, 0, 0.3)
    k2, v2 = k.clone(), v.clone()
    k2[:, :, 7] += 1
    v2[:, :, 7] -= 1
    b = oracle.sdpa(q, k2, v2, 0, 0, 0.3)
    torch.testing.assert_close(a[:, :, :7], b[:, :, :7])
    assert not torch.allclose(a[:, :, 7:], b[:, :, 7:])


def _layer_inputs(seed, B=2, T=24, H=4, K=2, D=16):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, T, H, D, generator=g).transpose(1, 2)
    k = torch.randn(B, T, K, D, generator=g).transpose(1, 2)
    v = torch.randn(B, T, K, D, generator=g).transpose(1, 2)
    w = 1 + 0.1 * torch.randn(D, generator=g)
    cos, sin = oracle.rope_tables(D, 64, 1e4)
    return q, k, v, w, cos, sin


@pytest.mark.parametrize("window", [0, 5])
def test_chunked_prefill_then_decode_matches_full(window):
    """tests/test_model.py:61-69: 9 + 6 token chunks then token by token == one pass."""
    q, k, v, w, cos, sin = _layer_inputs(11)
    T = q.shape[2]
    kw = dict(scale=0.25, q_weight=w, k_weight=w, window=window)
    full = oracle.attention_forward(q, k, v, cos=cos[:T], sin=sin[:T], **kw)
    cache = oracle.KVCache([(2, 16)], 2, 48)
    parts, pos = [], 0
    for n in [9, 6] + [1] * (T - 15):
        parts.append(oracle.attention_forward(q[:, :, pos:pos + n], k[:, :, pos:pos + n], v[:, :, pos:pos + n],
                                              cos=cos[pos:pos + n], sin=sin[pos:pos + n], cache=cache, **kw))
        cache.advance(n)
        pos += n
    torch.testing.assert_close(torch.cat(parts, 2), full, atol=1e-5, rtol=1e-4)


@pytest.mark.parametrize("window", [0, 8])
def test_static_step_matches_normal_step(window):
    """tests/test_cuda_graph.py:24-52 and 81-95: a static (graph) step over a fixed-length
    view with the position mask == the normal step, for 1 and 5 tokens."""
    q, k, v, w, cos, sin = _layer_inputs(12, B=1, T=30)
    kw = dict(scale=0.25, q_weight=w, k_weight=w, window=window)
    for tps in (1, 5):
        normal = oracle.KVCache([(2, 16)], 1, 64)
        static = oracle.StaticKVCache([(2, 16)], 1, 64, tokens_per_step=tps)
        oracle.attention_forward(q[:, :, :20], k[:, :, :20], v[:, :, :20], cos=cos[:20], sin=sin[:20],
                                 cache=normal, **kw)
        oracle.attention_forward(q[:, :, :20], k[:, :, :20], v[:, :, :20], cos=cos[:20], sin=sin[:20],
                                 cache=static, **kw)
        normal.advance(20)
        static.advance(20)
        sl = slice(20, 20 + tps)
        a = oracle.attention_forward(q[:, :, sl], k[:, :, sl], v[:, :, sl], cos=cos[sl], sin=sin[sl],
                                     cache=normal, **kw)
        static.length, static.static = 32, True
        static.pos_t.fill_(20)
        b = oracle.attention_forward(q[:, :, sl], k[:, :, sl], v[:, :, sl], cos=cos[sl], sin=sin[sl],
                                     cache=static, **kw)
        torch.testing.assert_close(a, b, atol=1e-5, rtol=1e-4)


def test_ragged_decode_rows_match_single_calls():
    g = torch.Generator().manual_seed(13)
    B, H, K, D, T, L = 3, 4, 2, 16, 2, 40
    q = torch.randn(B, H, T, D, generator=g)
    kc = torch.randn(B, K, L, D, generator=g)
    vc = torch.randn(B, K, L, D, generator=g)
    lens = [5, 40, 17]
    out = oracle.ragged_decode(q, kc, vc, lens, 0, 0.25)
    for b, Lb in enumerate(lens):
        want = oracle.brute_attention(q[b:b + 1], kc[b:b + 1, :, :Lb], vc[b:b + 1, :, :Lb], Lb - T, 0, 0.25)
        np.testing.assert_allclose(out[b:b + 1].double().numpy(), want.numpy(), atol=1e-5)


def test_golden_fixtures():
    """The committed float64 fixtures (tests/golden/make_golden.py) match the oracle."""
    from golden.make_golden import load_cases

    cases = load_cases()
    assert len(cases) >= 4
    for c in cases:
        got = oracle.sdpa(torch.from_numpy(c["q"]).float(), torch.from_numpy(c["k"]).float(),
                          torch.from_numpy(c["v"]).float(), int(c["offset"]), int(c["window"]), float(c["scale"]))
        np.testing.assert_allclose(got.double().numpy(), c["out"], atol=1e-5, err_msg=str(c["name"]))


def check_drafter(fn) -> None:
    """The drafter's key set, stated independently of the slicing in mtp.py:84-86: the query
    at position n_past sees stored keys k < n_past with n_past - k < window (window 0: all),
    checked by a float64 loop."""
    g = torch.Generator().manual_seed(31)
    B, H, K, D, L = 2, 4, 2, 16, 40
    q = torch.randn(B, H, 1, D, generator=g)
    kc = torch.randn(B, K, L, D, generator=g)
    vc = torch.randn(B, K, L, D, generator=g)
    for n_past, window in [(1, 0), (7, 0), (L, 0), (5, 8), (7, 8), (8, 8), (9, 8), (L, 8), (L, 2)]:
        got = fn(q, kc, vc, n_past, window, 1.0).double()
        want = torch.zeros(B, H, 1, D, dtype=torch.float64)
        for b in range(B):
            for h in range(H):
                kh = h // (H // K)
                keys = [k for k in range(n_past) if window == 0 or n_past - k < window]
                s = torch.tensor([float((q[b, h, 0].double() * kc[b, kh, k].double()).sum()) for k in keys],
                                 dtype=torch.float64)
                w = torch.softmax(s, 0)
                want[b, h, 0] = (w[:, None] * vc[b, kh, keys].double()).sum(0)
        np.testing.assert_allclose(got.numpy(), want.numpy(), atol=1e-5, err_msg=str((n_past, window)))


def test_drafter_attention_pinned():
    check_drafter(oracle.drafter_attention)


# ----------------------------------------------------------------------------- planted mistakes
def _raises(check, fn):
    with pytest.raises(AssertionError):
        check(fn)


def check_document_attention(fn) -> None:
    """Document-masked attention fn(q, k, v, doc_ids, window, scale) -> [B,H,T,hd] against
    the float64 loops restricted to each query's document, and against each document of a
    packed row attended alone at the same positions (the reference's note on doc_ids,
    transformer.py:258-264: a masked document behaves as if it were alone)."""
    g = torch.Generator().manual_seed(21)
    B, H, K, T, D = 2, 4, 2, 19, 8
    q = torch.randn(B, H, T, D, generator=g, dtype=torch.float64)
    k = torch.randn(B, K, T, D, generator=g, dtype=torch.float64)
    v = torch.randn(B, K, T, D, generator=g, dtype=torch.float64)
    docs = torch.tensor([[0] * 5 + [1] * 1 + [2] * 9 + [3] * 4, [7] * 11 + [8] * 8])
    for window in (0, 4):
        got = fn(q, k, v, docs, window, 0.35)
        want = ref.brute_attention(q, k, v, 0, window, 0.35, doc_ids=docs)
        torch.testing.assert_close(got.double(), want, atol=1e-10, rtol=0)
    got = fn(q, k, v, docs, 0, 0.35)
    for b in range(B):
        for d in docs[b].unique():
            idx = (docs[b] == d).nonzero().view(-1)
            a, z = int(idx[0]), int(idx[-1]) + 1
            alone = ref.sdpa(q[b:b + 1, :, a:z], k[b:b + 1, :, a:z], v[b:b + 1, :, a:z], 0, 0, 0.35)
            torch.testing.assert_close(got[b:b + 1, :, a:z].double(), alone, atol=1e-10, rtol=0)


def test_document_attention_pinned():
    check_document_attention(lambda q, k, v, d, w, sc: ref.sdpa(q, k, v, 0, w, sc, ref.document_mask(d)))


def test_pins_catch_planted_mistakes():
    # RoPE: inverse frequencies over arange(0, d) instead of arange(0, d, 2)
    def bad_tables(d, L, theta):
        inv = 1.0 / theta ** (torch.arange(0, d // 2, dtype=torch.float32) / d)
        a = torch.outer(torch.arange(L, dtype=torch.float32), inv)
        a = torch.cat([a, a], -1)
        return a.cos(), a.sin()
    _raises(check_rope_tables, bad_tables)
    # RoPE: rotated the wrong way (x cos - rot(x) sin)
    _raises(check_rope_rotation, lambda x, c, s: (x.float() * c - ref.rotate_half(x.float()) * s).to(x.dtype))
    # RoPE: interleaved (adjacent-channel) pairing instead of rotate-half
    def interleaved(x, c, s):
        x1, x2 = x[..., 0::2], x[..., 1::2]
        cc, ss = c[..., : c.shape[-1] // 2], s[..., : s.shape[-1] // 2]
        return torch.stack([x1 * cc - x2 * ss, x2 * cc + x1 * ss], -1).flatten(-2)
    _raises(check_rope_rotation, interleaved)
    # RMSNorm: eps dropped / sum instead of mean
    _raises(check_rms_norm, lambda x, w, eps: (x / x.pow(2).sum(-1, keepdim=True).sqrt()) * (1 if w is None else w))
    # head norm+rope: rounding twice (the eager path) is not the fused semantics
    _raises(check_head_norm_rope, lambda x, w, eps, c, s: ref.eager_norm_rope(x, w, eps, c, s))
    # mask: off by one, and window measured the other way
    _raises(check_mask, lambda T, S, off, win: ref.attention_mask(T, S, off - 1, win))
    _raises(check_mask, lambda T, S, off, win: ref.attention_mask(T, S, off, win + 1 if win else 0))
    # attention: GQA head -> KV head map h % K instead of h // (H/K)
    def wrong_gqa(q, k, v, off, win, sc):
        idx = torch.arange(q.shape[1]) % k.shape[1]
        return ref.sdpa(q, k[:, idx], v[:, idx], off, win, sc)
    _raises(check_attention, wrong_gqa)
    # attention: scale applied twice / window ignored
    _raises(check_attention, lambda q, k, v, off, win, sc: ref.sdpa(q, k, v, off, win, sc * sc))
    _raises(check_attention, lambda q, k, v, off, win, sc: ref.sdpa(q, k, v, off, 0, sc))
    # documents: the mask shifted by one position, or the causal part dropped
    _raises(check_document_attention,
            lambda q, k, v, d, w, sc: ref.sdpa(q, k, v, 0, w, sc, ref.document_mask(torch.roll(d, 1, 1))))
    _raises(check_document_attention,
            lambda q, k, v, d, w, sc: F.scaled_dot_product_attention(
                q, k.repeat_interleave(2, 1), v.repeat_interleave(2, 1), scale=sc,
                attn_mask=ref.document_mask(d) & (ref.attention_mask(q.shape[2], q.shape[2], 0, w) | True)))
    # drafter: the query's own position counted as stored / the window one key wider
    _raises(check_drafter, lambda q, k, v, n, win, sc: ref.drafter_attention(q, k, v, min(n + 1, k.shape[2]), win, sc))
    _raises(check_drafter, lambda q, k, v, n, win, sc: ref.drafter_attention(q, k, v, n, win + 1 if win else 0, sc))


def test_downstream_argmax_check_has_teeth():
    """The GPU tests' downstream-argmax criterion (helpers.downstream_argmax): bf16 rounding
    of a correct output passes it; plausible kernel mistakes, planted here in the oracle on
    the CPU, fail it."""
    from helpers import downstream_argmax

    g = torch.Generator().manual_seed(5)
    B, H, K, T, S, D = 4, 8, 2, 16, 300, 64
    q = torch.randn(B, H, T, D, generator=g)
    k = torch.randn(B, K, S, D, generator=g)
    v = torch.randn(B, K, S, D, generator=g)
    sc = D ** -0.5
    ref = oracle.sdpa(q, k, v, S - T, 0, sc).transpose(1, 2)
    r = downstream_argmax(ref.bfloat16().float(), ref)
    assert r["mismatched"] == 0 and r["near_ties"] <= 0.1 * r["rows"], r
    planted = {
        "scale squared": oracle.sdpa(q, k, v, S - T, 0, sc * sc),
        "window off by one": oracle.sdpa(q, k, v, S - T, S - T, sc),
        "last key dropped": oracle.sdpa(q, k[:, :, :-1], v[:, :, :-1], S - T - 1, 0, sc),
        "GQA map h % K": oracle.sdpa(q, k[:, torch.arange(H) % K], v[:, torch.arange(H) % K], S - T, 0, sc),
    }
    for name, wrong in planted.items():
        r = downstream_argmax(wrong.transpose(1, 2), ref)
        assert r["mismatched"] > 0, (name, r)


def _gated_brute(qg, k, v, cos, sin, n_rot, wq, wk, eps, offset, k_past, v_past):
    """Qwen3.5 gated attention from its definition in float64 with explicit loops: per head
    h, q = first half of qg[h], gate = second half; RMSNorm (gain) then rotation of the
    pairs (i, i + n_rot/2), i < n_rot/2, by angle cos/sin; channels >= n_rot untouched;
    softmax over keys j <= offset + t with scale hd^-1/2; KV head h // (H/K); times sigmoid(gate)."""
    B, T, H, two = qg.shape
    hd, K = two // 2, k.shape[2]

    def norm_rot(x, w, t):
        x = x.double()
        x = x / math.sqrt(float((x * x).mean()) + eps) * w.double()
        out = x.clone()
        half = n_rot // 2
        for i in range(half):
            c, s = float(cos[t, i]), float(sin[t, i])
            out[i] = x[i] * c - x[i + half] * s
            out[i + half] = x[i + half] * c + x[i] * s
        return out

    y = torch.zeros(B, T, H * hd, dtype=torch.float64)
    for b in range(B):
        keys = [k_past[b, :, j].double() for j in range(offset)]
        vals = [v_past[b, :, j].double() for j in range(offset)]
        for t in range(T):
            keys.append(torch.stack([norm_rot(k[b, t, kh], wk, t) for kh in range(K)]))
            vals.append(v[b, t].double())
        for t in range(T):
            for h in range(H):
                kh = h // (H // K)
                qv = norm_rot(qg[b, t, h, :hd], wq, t)
                js = range(offset + t + 1)
                sc = [float((qv * keys[j][kh]).sum()) / math.sqrt(hd) for j in js]
                mx = max(sc)
                wts = [math.exp(x - mx) for x in sc]
                tot = sum(wts)
                acc = sum(w_ / tot * vals[j][kh] for w_, j in zip(wts, js))
                gate = qg[b, t, h, hd:].double()
                y[b, t, h * hd:(h + 1) * hd] = acc / (1 + torch.exp(-gate))
    return y


@pytest.mark.parametrize("T,offset", [(5, 0), (1, 6), (3, 4)])
def test_gated_attention_pinned_by_float64_loops(T, offset):
    g = torch.Generator().manual_seed(40 + T)
    B, H, K, hd, n_rot = 2, 4, 2, 8, 4
    qg = torch.randn(B, T, H, 2 * hd, generator=g)
    k, v = torch.randn(B, T, K, hd, generator=g), torch.randn(B, T, K, hd, generator=g)
    kp, vp = torch.randn(B, K, offset, hd, generator=g), torch.randn(B, K, offset, hd, generator=g)
    wq, wk = 1 + 0.2 * torch.randn(hd, generator=g), 1 + 0.2 * torch.randn(hd, generator=g)
    cos_t, sin_t = oracle.rope_tables(n_rot, offset + T, 1e4)
    c, s = cos_t[offset:], sin_t[offset:]
    y, kn, vn = oracle.gated_attention(qg, k, v, cos=c, sin=s, n_rot=n_rot, q_weight=wq, k_weight=wk, eps=1e-6,
                                       k_past=kp if offset else None, v_past=vp if offset else None)
    want = _gated_brute(qg, k, v, c, s, n_rot, wq, wk, 1e-6, offset, kp, vp)
    torch.testing.assert_close(y.double(), want, atol=1e-5, rtol=1e-5)
    assert kn.shape == (B, K, T, hd) and torch.equal(vn, v.transpose(1, 2))
    # plausible slips the pin catches: q and gate swapped; RoPE over every channel
    bad = oracle.gated_attention(torch.cat([qg[..., hd:], qg[..., :hd]], -1), k, v, cos=c, sin=s, n_rot=n_rot,
                                 q_weight=wq, k_weight=wk, eps=1e-6, k_past=kp if offset else None,
                                 v_past=vp if offset else None)[0]
    assert not torch.allclose(bad.double(), want, atol=1e-3)
    c8, s8 = oracle.rope_tables(hd, offset + T, 1e4)
    bad = oracle.gated_attention(qg, k, v, cos=c8[offset:], sin=s8[offset:], n_rot=hd, q_weight=wq, k_weight=wk,
                                 eps=1e-6, k_past=kp if offset else None, v_past=vp if offset else None)[0]
    assert not torch.allclose(bad.double(), want, atol=1e-3)
