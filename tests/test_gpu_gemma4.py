"""Gemma 4's full-attention layers on the kernels: head dim 512 with one KV head (reference
sleuth/forge/infer/kv_cache.py:12-13), values taken from the keys before their norm and RoPE
(v_from_k, attention.py:108), values RMS-normalised without a gain (v_norm, 115-116) and
attention scale 1.0 (attn_scale, 84). Head dim 512 runs on forge_attn_prefill's
head-dim-split MFMA kernel, on the MFMA verify/decode kernel with 8 or more query heads per
KV head, and on the split-K kernel below that (bf16/fp16).

Against the oracle on the same seeded inputs (bf16/fp16 max-abs <= 2e-2): prefill with
offsets, windows and documents; ragged decode and a 4-token verify; the fused cache write
equal to the two calls bit for bit; verify rows equal to single-token decodes bit for bit;
and a Gemma-4-shaped Attention module (16 q heads / 1 KV head of 512, v_from_k, v_norm,
scale 1.0) through prefill, decode and a 4-token verify with a rewind, against the oracle on
the module's own projections. The norm gains are ~0.2 so that scale 1.0 gives scores of
order one, as trained q/k norms do (with unit gains the scores of random 512-wide rows have
a standard deviation of 22 and every softmax is one-hot)."""

from __future__ import annotations

import pytest
import torch

import oracle
from conftest import gpu_available
from helpers import downstream_argmax, gen, max_abs, randn, tables, tol

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not gpu_available(), reason="needs a GPU")]

DEV = "cuda"
D = 512
SCALE = 1.0
POISON = 1e4


def ops():
    from sleuth_amd import ops as o

    return o


def _gain(g, dtype):
    return (0.2 + 0.02 * randn(g, D)).to(dtype)


# ------------------------------------------------------------------ prefill
def _prefill_case(seed, dtype, B, H, K, T, offset, window, doc_lens=None):
    g = gen(seed)
    S = offset + T
    q = randn(g, B, T, H, D, dtype=dtype).transpose(1, 2)
    w = _gain(g, dtype)
    kc = (0.2 * randn(g, B, K, S + 5, D)).to(dtype)
    vc = randn(g, B, K, S + 5, D, dtype=dtype)
    cos_t, sin_t = tables(D, S, 1e6)
    c, s = cos_t[offset:S], sin_t[offset:S]
    qn = oracle.head_norm_rope(q, w, 1e-6, c, s)
    same_doc, starts = None, None
    if doc_lens is not None:
        ids = torch.cat([torch.full((n,), i) for i, n in enumerate(doc_lens)])[None].expand(B, T)
        same_doc = oracle.document_mask(ids)
        starts = torch.tensor([[sum(doc_lens[:i]) for i, n in enumerate(doc_lens) for _ in range(n)]] * B,
                              dtype=torch.int32)
    ref = oracle.sdpa(qn.float(), kc[:, :, :S].float(), vc[:, :, :S].float(), offset, window, SCALE, same_doc)
    got = ops().attn_prefill(q.to(DEV), kc.to(DEV), vc.to(DEV), scale=SCALE, offset=offset, window=window,
                             q_weight=w.to(DEV), eps=1e-6, norm_q=True, cos=c.to(DEV), sin=s.to(DEV),
                             doc_start=None if starts is None else starts.to(DEV))
    return got.cpu(), ref.transpose(1, 2)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("T,offset,window", [(32, 0, 0), (100, 0, 0), (257, 0, 0), (70, 300, 0),
                                             (300, 0, 64), (45, 1000, 1024)])
def test_prefill_head_dim_512(dtype, T, offset, window):
    got, ref = _prefill_case(T + offset + window, dtype, 2, 8, 1, T, offset, window)
    err = max_abs(got, ref)
    print(f"prefill hd 512 {dtype} T={T} offset={offset} window={window}: max-abs {err:.2e}")
    assert err <= tol(dtype)


def test_prefill_head_dim_512_gqa_and_documents():
    got, ref = _prefill_case(7, torch.bfloat16, 1, 4, 2, 200, 0, 0)
    assert max_abs(got, ref) <= 2e-2
    got, ref = _prefill_case(8, torch.bfloat16, 2, 4, 1, 200, 0, 0, doc_lens=[1, 40, 33, 126])
    assert max_abs(got, ref) <= 2e-2


@pytest.mark.parametrize("H,K,window", [(3, 1, 0), (2, 2, 0), (3, 1, 48)])
def test_prefill_head_dim_512_odd_groups(H, K, window):
    """An odd number of q heads per KV head takes the kernel's one-head-per-block form (the head
    dim in four slices); an even one shares each K/V tile between two heads (the tests above)."""
    got, ref = _prefill_case(11, torch.bfloat16, 2, H, K, 150, 0, window)
    assert max_abs(got, ref) <= 2e-2


def test_prefill_head_dim_512_downstream_argmax():
    got, ref = _prefill_case(9, torch.bfloat16, 1, 16, 1, 256, 0, 0)
    r = downstream_argmax(got, ref)
    print(f"downstream argmax: {r}")
    assert r["mismatched"] == 0 and r["near_ties"] <= max(2, 0.1 * r["rows"]), r


# ------------------------------------------------------------------ decode / verify
def _decode_case(seed, dtype, H, K, T, lens, chunk=0):
    """Rows filled up to lens[b] (the new tokens' K/V included), raw q normalised and rotated
    in the kernel; per-row positions."""
    g = gen(seed)
    B, max_len = len(lens), max(lens) + 3
    kc = (0.2 * randn(g, B, K, max_len, D)).to(dtype)
    vc = randn(g, B, K, max_len, D, dtype=dtype)
    q = randn(g, B, T, H, D, dtype=dtype).transpose(1, 2)
    w = _gain(g, dtype)
    cos_t, sin_t = tables(D, max_len, 1e6)
    base = [L - T for L in lens]
    c = torch.stack([cos_t[p:p + T] for p in base])
    s = torch.stack([sin_t[p:p + T] for p in base])
    qn = oracle.head_norm_rope(q, w, 1e-6, c, s)
    ref = oracle.ragged_decode(qn.float(), kc.float(), vc.float(), lens, 0, SCALE)
    got = ops().attn_decode(q.to(DEV), kc.to(DEV), vc.to(DEV), scale=SCALE,
                            row_pos=torch.tensor(base, dtype=torch.int32, device=DEV), max_kv_len=max(lens),
                            q_weight=w.to(DEV), eps=1e-6, norm_q=True, cos=c.to(DEV), sin=s.to(DEV), chunk=chunk)
    return got.cpu(), ref.transpose(1, 2)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("H,K", [(16, 1), (8, 1), (32, 2), (8, 2), (4, 1), (1, 1)])
@pytest.mark.parametrize("T", [1, 4])
def test_decode_and_verify_head_dim_512(dtype, H, K, T):
    got, ref = _decode_case(H * 10 + K + T, dtype, H, K, T, [37, 700, 2049, 1500])
    err = max_abs(got, ref)
    print(f"decode hd 512 {dtype} H={H} K={K} T={T}: max-abs {err:.2e}")
    assert err <= tol(dtype)


@pytest.mark.parametrize("H", [16, 4])
def test_decode_head_dim_512_many_chunks(H):
    """A 5000-key row split into 40 chunks of 128 keys (the combine kernel at head dim 512),
    on the MFMA path (16 q heads per KV head) and the split-K kernel (4)."""
    got, ref = _decode_case(5, torch.bfloat16, H, 1, 1, [5000, 130], chunk=128)
    assert max_abs(got, ref) <= 2e-2


@pytest.mark.parametrize("dtype,T,window", [(torch.bfloat16, 1, 0), (torch.bfloat16, 4, 0),
                                            (torch.float16, 4, 0), (torch.bfloat16, 4, 700),
                                            (torch.float16, 1, 100)])
def test_decode_head_dim_512_host_position(dtype, T, window):
    """One position for every row (the dense grid with the uniform chunk rule: tiles staged
    through registers, the score tile split over the waves), 16 q heads per KV head, against
    the oracle; sliding windows included."""
    g = gen(21 + T + window)
    B, H, K, L = 4, 16, 1, 3000
    kc = (0.2 * randn(g, B, K, L + 5, D)).to(dtype)
    vc = randn(g, B, K, L + 5, D, dtype=dtype)
    q = randn(g, B, T, H, D, dtype=dtype).transpose(1, 2)
    ref = oracle.ragged_decode(q.float(), kc.float(), vc.float(), [L] * B, window, SCALE)
    got = ops().attn_decode(q.to(DEV), kc.to(DEV), vc.to(DEV), scale=SCALE, pos=L - T, window=window)
    assert max_abs(got.cpu(), ref.transpose(1, 2)) <= tol(dtype)


def test_verify_rows_equal_decodes_head_dim_512():
    """A 4-token verify step's rows equal the decodes of those tokens alone, bit for bit."""
    g = gen(11)
    B, H, K, L, T = 2, 16, 1, 900, 4
    kc = (0.2 * randn(g, B, K, L + 4, D)).to(torch.bfloat16).to(DEV)
    vc = randn(g, B, K, L + 4, D, dtype=torch.bfloat16).to(DEV)
    q = randn(g, B, T, H, D, dtype=torch.bfloat16).transpose(1, 2).to(DEV)
    allv = ops().attn_decode(q, kc, vc, scale=SCALE, pos=L - T, chunk=256)
    for t in range(T):
        one = ops().attn_decode(q[:, :, t:t + 1], kc, vc, scale=SCALE, pos=L - T + t, chunk=256)
        assert torch.equal(one[:, 0], allv[:, t])


@pytest.mark.parametrize("T", [1, 4])
def test_decode_head_dim_512_per_row_equals_dense(T):
    """Per-row positions (the persistent grid, tiles loaded straight into LDS) and one host
    position (the dense grid, tiles staged through registers, the score tile split over the
    waves) give the same bits at equal chunks, q norm and RoPE included."""
    g = gen(31 + T)
    B, H, K, L = 3, 16, 1, 1500
    kc = (0.2 * randn(g, B, K, L + 4, D)).to(torch.bfloat16).to(DEV)
    vc = randn(g, B, K, L + 4, D, dtype=torch.bfloat16).to(DEV)
    q = randn(g, B, T, H, D, dtype=torch.bfloat16).transpose(1, 2).to(DEV)
    w = _gain(g, torch.bfloat16).to(DEV)
    cos_t, sin_t = tables(D, L + 4, 1e6)
    c = cos_t[L - T:L].expand(B, T, D).contiguous().to(DEV)
    s = sin_t[L - T:L].expand(B, T, D).contiguous().to(DEV)
    kw = dict(scale=SCALE, q_weight=w, eps=1e-6, norm_q=True, cos=c, sin=s, chunk=256)
    dense = ops().attn_decode(q, kc, vc, pos=L - T, **kw)
    per_row = ops().attn_decode(q, kc, vc, row_pos=torch.full((B,), L - T, dtype=torch.int32, device=DEV),
                                max_kv_len=L, **kw)
    assert torch.equal(dense, per_row)


@pytest.mark.parametrize("T", [1, 4])
def test_decode_append_head_dim_512_equals_two_calls(T):
    """forge_attn_decode_append (v from the raw keys, values normalised without a gain, scale
    1.0) equals forge_kv_append + forge_attn_decode bit for bit, outputs and caches."""
    g = gen(12 + T)
    B, H, K, L = 3, 16, 1, 600
    dt = torch.bfloat16
    base = torch.tensor([L - T, 100, 333], dtype=torch.int32)
    kc = (0.2 * randn(g, B, K, L + 8, D)).to(dt)
    vc = randn(g, B, K, L + 8, D, dtype=dt)
    q = randn(g, B, T, H, D, dtype=dt).transpose(1, 2).to(DEV)
    k = randn(g, B, T, K, D, dtype=dt).transpose(1, 2).to(DEV)
    wq, wk = _gain(g, torch.float32).to(DEV), _gain(g, torch.float32).to(DEV)
    cos_t, sin_t = tables(D, L + 8, 1e6)
    c = torch.stack([cos_t[int(p):int(p) + T] for p in base]).to(DEV)
    s = torch.stack([sin_t[int(p):int(p) + T] for p in base]).to(DEV)
    kw = dict(scale=SCALE, row_pos=base.to(DEV), max_kv_len=L + 8, q_weight=wq, eps=1e-6, norm_q=True,
              cos=c, sin=s)
    kc1, vc1 = kc.to(DEV), vc.to(DEV)
    ops().kv_append(k, k, kc1, vc1, row_pos=base.to(DEV), k_weight=wk, eps=1e-6, norm_k=True, norm_v=True,
                    cos=c, sin=s)
    two = ops().attn_decode(q, kc1, vc1, **kw)
    kc2, vc2 = kc.to(DEV), vc.to(DEV)
    one = ops().attn_decode_append(q, k, k, kc2, vc2, k_weight=wk, norm_k=True, norm_v=True, **kw)
    assert torch.equal(one, two)
    assert torch.equal(kc1, kc2) and torch.equal(vc1, vc2)


# ------------------------------------------------------------------ the module
def test_gemma4_full_layer_module_on_the_kernels():
    """A Gemma-4-shaped full-attention layer (16 q heads, 1 KV head of 512, v_from_k, v_norm,
    attn_scale 1.0, QK-norm, theta 1e6) through the module and its cache: a 100-token prefill,
    two decode steps, a 4-token verify, a rewind of 2 and a 2-token step. Every call on the
    HIP path, against the oracle on the module's own raw projections (the values are the raw
    keys, normalised without a gain)."""
    import math

    from sleuth_amd.attention import Attention
    from sleuth_amd.config import ModelConfig
    from sleuth_amd.kv_cache import KVCache

    dt = torch.bfloat16
    H, K, d_model = 16, 1, 256
    cfg = ModelConfig(vocab_size=10, d_model=d_model, n_heads=H, n_kv_heads=K, head_size=D, qk_norm=True,
                      v_norm=True, attn_scale=1.0, full_v_from_k=True, rope_theta=1e6, n_layers=1,
                      norm_eps=1e-6)
    torch.manual_seed(0)
    a = Attention(cfg, 0).eval()
    assert a.v_proj is None and a.scale == 1.0
    with torch.no_grad():
        a.q_norm.weight.copy_(0.2 + 0.02 * torch.randn(D))
        a.k_norm.weight.copy_(0.2 + 0.02 * torch.randn(D))
    a = a.to(DEV, dt)
    rec = {}
    a.q_proj.register_forward_hook(lambda m, i, o: rec.__setitem__("q", o))
    a.k_proj.register_forward_hook(lambda m, i, o: rec.__setitem__("k", o))
    seen = {}
    a.tap_z.listeners.append(lambda n, t: seen.__setitem__("z", t.clone()))
    B, max_len = 2, 160
    cache = KVCache([(K, D)], B, max_len, DEV, dt)
    cache.k[0].fill_(POISON)
    cache.v[0].fill_(POISON)
    ocache = oracle.KVCache([(K, D)], B, max_len, "cpu", torch.float32)
    cos_t, sin_t = oracle.rope_tables(D, max_len, 1e6)
    qw, kw = a.q_norm.weight.detach().cpu(), a.k_norm.weight.detach().cpu()
    g = torch.Generator().manual_seed(1)
    worst = 0.0
    for T, rewind in [(100, 0), (1, 0), (1, 0), (4, 2), (2, 0)]:
        x = torch.randn(B, T, d_model, generator=g).to(dt).to(DEV)
        p0 = cache.pos
        cos, sin = cos_t[p0:p0 + T], sin_t[p0:p0 + T]
        with torch.no_grad():
            a(x, cos.to(DEV), sin.to(DEV), cache)
        assert a.last_path == ("hip-prefill" if T > 16 else "hip-decode")
        q = rec["q"].view(B, T, H, D).transpose(1, 2).cpu()
        k = rec["k"].view(B, T, K, D).transpose(1, 2).cpu()
        qn = oracle.head_norm_rope(q, qw, 1e-6, cos, sin)
        kn = oracle.head_norm_rope(k, kw, 1e-6, cos, sin)
        vn = oracle.head_norm_rope(k, None, 1e-6)           # v_from_k, then v_norm (no gain)
        ocache.k[0][:, :, p0:p0 + T] = kn.float()
        ocache.v[0][:, :, p0:p0 + T] = vn.float()
        ref = oracle.ragged_decode(qn.float(), ocache.k[0], ocache.v[0], [p0 + T] * B, 0, 1.0)
        err = max_abs(seen["z"].float().cpu(), ref.transpose(1, 2))
        worst = max(worst, err)
        assert err <= 2e-2, (T, p0, err)
        assert math.isfinite(err)
        cache.advance(T)
        ocache.advance(T)
        if rewind:   # speculative rejection: the next step overwrites the rejected keys
            cache.pos -= rewind
            ocache.pos -= rewind
    print(f"Gemma-4 full layer: max-abs {worst:.2e} over prefill, decode, verify and rewind")
