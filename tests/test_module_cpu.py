"""Host logic of the drop-in module, cache and callers on the CPU (torch path): the same
behaviour the reference's CPU tests assert (tests/test_model.py, test_cuda_graph.py,
test_speculative.py), checked against the oracle."""

from __future__ import annotations

import sys

import pytest
import torch

import oracle
from sleuth_amd.attention import Attention
from sleuth_amd.config import ModelConfig
from sleuth_amd.generate import generate, ngram_draft, speculative_generate
from host_protocol import HostKVCache, HostStaticKVCache, HostTap, host_assign_names, host_listen
from sleuth_amd.kv_cache import KVCache
from sleuth_amd.model import Transformer
from sleuth_amd.taps import Tap, assign_tap_names, listen, tap_class, tap_names

VARIANTS = [
    dict(),
    dict(n_kv_heads=2, qk_norm=True),
    dict(n_kv_heads=1),
    dict(layer_types=["sliding", "full", "sliding"], sliding_window=5, head_size=32, n_kv_heads=1,
         swa_head_size=16, swa_kv_heads=2, swa_rope_theta=100.0, full_v_from_k=True, qk_norm=True,
         v_norm=True, attn_scale=1.0),
    dict(pos_type="none"),
]


def make(**kw):
    torch.manual_seed(0)
    cfg = ModelConfig(**{"vocab_size": 300, "d_model": 64, "n_layers": 3, "n_heads": 4, "max_seq_len": 48, **kw})
    return Transformer(cfg).eval()


def test_attention_signature_and_names():
    cfg = ModelConfig(vocab_size=10, d_model=64, n_heads=4, n_kv_heads=2, qk_norm=True)
    a = Attention(cfg, 0)
    for name in ("q_proj", "k_proj", "v_proj", "o_proj", "q_norm", "k_norm", "tap_q", "tap_k",
                 "tap_pattern", "tap_z"):
        assert hasattr(a, name), name
    x = torch.randn(2, 5, 64)
    cos, sin = oracle.rope_tables(16, 5, 1e4)
    assert a(x, cos, sin).shape == (2, 5, 64)
    assert a.last_path == "torch"


@pytest.mark.parametrize("qk_norm,v_norm,window", [(True, False, 0), (True, True, 3), (False, False, 0)])
def test_module_torch_path_matches_oracle(qk_norm, v_norm, window):
    cfg = ModelConfig(vocab_size=10, d_model=64, n_heads=4, n_kv_heads=2, qk_norm=qk_norm, v_norm=v_norm,
                      layer_types=["sliding"] if window else [], sliding_window=window, n_layers=1)
    torch.manual_seed(1)
    a = Attention(cfg, 0).eval()
    if qk_norm:
        with torch.no_grad():
            a.q_norm.weight.add_(0.1 * torch.randn(16))
            a.k_norm.weight.add_(0.1 * torch.randn(16))
    x = torch.randn(2, 7, 64)
    cos, sin = oracle.rope_tables(16, 7, 1e4)
    seen = {}
    assign_tap_names(a)
    with torch.no_grad(), listen(a, {"z": lambda n, t: seen.setdefault("z", t)}):
        a(x, cos, sin)
        q = a.q_proj(x).view(2, 7, 4, 16).transpose(1, 2)
        k = a.k_proj(x).view(2, 7, 2, 16).transpose(1, 2)
        v = a.v_proj(x).view(2, 7, 2, 16).transpose(1, 2)
        want = oracle.attention_forward(q, k, v, cos=cos, sin=sin, scale=0.25, eps=cfg.norm_eps,
                                        q_weight=a.q_norm.weight if qk_norm else None,
                                        k_weight=a.k_norm.weight if qk_norm else None, qk_norm=qk_norm,
                                        v_norm=v_norm, window=window, fused_norm=False)
    torch.testing.assert_close(seen["z"], want.transpose(1, 2), atol=1e-5, rtol=1e-4)


@pytest.mark.parametrize("kw", VARIANTS)
def test_explicit_attention_matches_fused(kw):
    """tests/test_model.py:51-58"""
    m = make(**kw)
    x = torch.randint(0, 300, (2, 20))
    with torch.no_grad():
        fused = m(x).logits
        with listen(m, {"blocks.*.attn.pattern": lambda name, t: None}):
            explicit = m(x).logits
    torch.testing.assert_close(fused, explicit, atol=1e-5, rtol=1e-4)


@pytest.mark.parametrize("kw", VARIANTS)
def test_kv_cache_matches_full_forward(kw):
    """tests/test_model.py:61-69: chunked prefill + token by token == one pass."""
    m = make(**kw)
    x = torch.randint(0, 300, (2, 24))
    with torch.no_grad():
        full = m(x).logits
        cache = KVCache.for_model(m, batch=2)
        parts = [m(x[:, :9], cache=cache).logits, m(x[:, 9:15], cache=cache).logits]
        parts += [m(x[:, i:i + 1], cache=cache).logits for i in range(15, 24)]
    torch.testing.assert_close(torch.cat(parts, 1), full, atol=1e-5, rtol=1e-4)


def test_ragged_cache_rows_match_single_rows():
    """Per-row lengths: each row of a ragged batch decodes like that row alone."""
    m = make(n_kv_heads=2, qk_norm=True)
    ids = torch.randint(0, 300, (3, 20))
    lens = [4, 11, 7]
    with torch.no_grad():
        cache = KVCache.for_model(m, batch=3)
        singles = []
        for b, L in enumerate(lens):
            c1 = KVCache.for_model(m, batch=1)
            m(ids[b:b + 1, :L], cache=c1)
            singles.append((c1, m(ids[b:b + 1, L:L + 1], cache=c1).logits))
            for layer in range(m.cfg.n_layers):
                cache.k[layer][b:b + 1, :, :L] = c1.k[layer][:, :, :L]
                cache.v[layer][b:b + 1, :, :L] = c1.v[layer][:, :, :L]
        cache.set_lengths(lens)
        step = torch.stack([ids[b, L] for b, L in enumerate(lens)])[:, None]
        out = m(step, cache=cache).logits
    for b in range(3):
        torch.testing.assert_close(out[b:b + 1], singles[b][1], atol=1e-5, rtol=1e-4)
    assert cache.seq_lens_host == [5, 12, 8] and cache.seq_lens.tolist() == [5, 12, 8]


def test_cache_protocol():
    c = KVCache([(2, 8), (1, 16)], 2, 10, "cpu", torch.float32)
    assert c.k[0].shape == (2, 2, 10, 8) and c.k[1].shape == (2, 1, 10, 16) and c.pos == 0
    assert c.nbytes() == 2 * 4 * (2 * 2 * 10 * 8 + 2 * 1 * 10 * 16)
    k = torch.randn(2, 2, 3, 8)
    ka, va = c.update(0, k, k)
    assert ka.shape == (2, 2, 3, 8) and torch.equal(ka, k)
    c.advance(3)
    with pytest.raises(ValueError, match="KV cache full"):
        c.update(0, torch.randn(2, 2, 8, 8), torch.randn(2, 2, 8, 8))
    h = c.token_history(2, "cpu")
    assert h.shape == (2, 10) and torch.all(h == -1)
    c.set_lengths([2, 5])
    assert c.ragged and c.pos == 5 and c.seq_lens.tolist() == [2, 5]
    c.pos = 4                       # the speculative decoder's rewind moves every row
    assert not c.ragged and c.seq_lens_host == [4, 4]
    c.reset()
    assert c.pos == 0
    # one allocation holds every layer's K and V
    assert c.k[1].untyped_storage().data_ptr() == c.v[0].untyped_storage().data_ptr()


@pytest.mark.parametrize("cls", [KVCache, HostStaticKVCache])
def test_static_cache_masks_and_positions(cls):
    """tests/test_cuda_graph.py:55-61 golden masks, on the product cache and the host stand-in."""
    c = cls([(1, 4)], 1, 32, "cpu", torch.float32)
    c.length, c.static = 16, True
    c.pos_t.fill_(10)
    assert c.attn_mask().view(-1).tolist() == [True] * 11 + [False] * 5
    assert c.attn_mask(4).view(-1).nonzero().view(-1).tolist() == [7, 8, 9, 10]
    c2 = cls([(1, 4)], 1, 32, "cpu", torch.float32, tokens_per_step=3)
    c2.pos_t.fill_(5)
    assert c2.positions.tolist() == [5, 6, 7]
    c2.new_step()
    c2.pos_t.fill_(9)
    assert c2.positions.tolist() == [9, 10, 11]


@pytest.mark.parametrize("static_cls", [KVCache, HostStaticKVCache])
@pytest.mark.parametrize("kw", [{}, {"layer_types": ["sliding", "full", "sliding"], "sliding_window": 8}])
def test_static_decode_matches_normal_decode(kw, static_cls):
    """tests/test_cuda_graph.py:24-52 (static steps on the CPU, two view lengths), with the
    product cache and with the host's StaticKVCache protocol."""
    m = make(n_kv_heads=2, max_seq_len=96, **kw)
    ids = torch.randint(0, 300, (1, 40))
    shapes = [(m.cfg.attn_spec(i).kv_heads, m.cfg.attn_spec(i).head_dim) for i in range(m.cfg.n_layers)]
    normal = HostKVCache(shapes, 1, 96, "cpu", torch.float32)
    static = static_cls(shapes, 1, 96, "cpu", torch.float32)
    with torch.no_grad():
        a = m(ids[:, :5], cache=normal).logits[:, -1]
        b = m(ids[:, :5], cache=static).logits[:, -1]
        assert torch.allclose(a, b, atol=1e-5)
        for t in ids[0, 5:]:
            tok = t.view(1, 1)
            a = m(tok, cache=normal).logits[:, -1]
            pos = static.pos
            static.length = 16 if pos < 16 else 64
            static.pos_t.fill_(pos)
            static.static = True
            b = m(tok, cache=static).logits[:, -1]
            static.static = False
            static.pos += 1
            assert torch.allclose(a, b, atol=1e-4), pos


def test_greedy_speculative_matches_plain():
    """tests/test_speculative.py:31-54 (prompt lookup, and a drafter that is always wrong)."""
    m = make(n_kv_heads=2, layer_types=["sliding", "full", "sliding"], sliding_window=8, max_seq_len=128)
    prompt = [1, 5, 9, 13, 5, 9, 13, 5, 9, 13, 22, 5, 9]
    plain = generate(m, prompt, 40)
    spec = speculative_generate(m, prompt, 40, k=4)
    assert spec.new_ids == plain.new_ids
    bad = speculative_generate(m, prompt, 40, k=3, draft=lambda ids, k: [7] * k)
    assert bad.new_ids == plain.new_ids


def test_ngram_draft():
    d = ngram_draft(max_ngram=3)
    assert d([1, 2, 3, 4, 5, 1, 2, 3], 3) == [4, 5, 1]
    assert d([7, 8, 9, 7, 8], 2) == [9, 7]
    assert d([1, 2, 3], 4) == []


def test_taps_and_ablation():
    m = make()
    names = tap_names(m)
    for expected in ("blocks.1.attn.z", "blocks.0.attn.q", "blocks.2.attn.pattern"):
        assert expected in names
    x = torch.randint(0, 300, (1, 8))
    with torch.no_grad():
        base = m(x).logits
        with listen(m, {"blocks.*.attn.z": lambda n, t: torch.zeros_like(t)}):
            ablated = m(x).logits
        assert not torch.allclose(base, ablated)
        torch.testing.assert_close(m(x).logits, base)


def test_too_long_and_bad_configs_rejected():
    m = make()
    with pytest.raises(ValueError):
        m(torch.zeros(1, 49, dtype=torch.long))
    with pytest.raises(ValueError):
        ModelConfig(vocab_size=10, d_model=64, n_heads=4, n_kv_heads=3)
    with pytest.raises(ValueError):
        ModelConfig(vocab_size=10, d_model=64, n_heads=4, layer_types=["sliding"] * 6)


@pytest.mark.parametrize("kw", VARIANTS[:4])
def test_module_runs_on_the_hosts_cache(kw):
    """The host's KVCache (kv_cache.py:25-70, nothing more) drives the module like the
    product cache: chunked prefill + decode give the same logits as one pass."""
    m = make(**kw)
    x = torch.randint(0, 300, (2, 24))
    with torch.no_grad():
        full = m(x).logits
        host = HostKVCache.for_model(m, 2)
        parts = [m(x[:, :9], cache=host).logits]
        parts += [m(x[:, i:i + 1], cache=host).logits for i in range(9, 24)]
    torch.testing.assert_close(torch.cat(parts, 1), full, atol=1e-5, rtol=1e-4)
    assert host.pos == 24
    with pytest.raises(ValueError, match="KV cache full"):
        m.blocks[0].attn(torch.zeros(2, 30, 64), *m.rope_rows(0, 30)[m.blocks[0].kind], cache=HostKVCache.for_model(m, 2, 20))


def test_module_taps_are_the_hosts_tap_type(monkeypatch):
    """Inside Sleuth (sleuth.forge.model.taps importable) the module builds its taps from the
    host's Tap class, so the host's isinstance-based naming and listen() find
    blocks.*.attn.{q,k,pattern,z}; outside it, this package's Tap."""
    import types

    host = types.ModuleType("sleuth.forge.model.taps")
    host.Tap = HostTap
    for name in ("sleuth", "sleuth.forge", "sleuth.forge.model"):
        monkeypatch.setitem(sys.modules, name, types.ModuleType(name))
    monkeypatch.setitem(sys.modules, "sleuth.forge.model.taps", host)
    tap_class.cache_clear()
    try:
        m = make(n_kv_heads=2, qk_norm=True)
        assert isinstance(m.blocks[1].attn.tap_z, HostTap)
        host_assign_names(m)
        seen = []
        rec = lambda name, t: seen.append((name, tuple(t.shape)))  # noqa: E731
        x = torch.randint(0, 300, (1, 6))
        with torch.no_grad():
            base = m(x).logits
            with host_listen(m, {f"blocks.*.attn.{n}": rec for n in ("q", "k", "pattern", "z")}):
                m(x)
            with host_listen(m, {"blocks.2.attn.z": lambda n, t: torch.zeros_like(t)}):
                ablated = m(x).logits
        names = {n for n, _ in seen}
        assert names == {f"blocks.{i}.attn.{t}" for i in range(3) for t in ("q", "k", "pattern", "z")}
        assert ("blocks.0.attn.pattern", (1, 4, 6, 6)) in seen and ("blocks.1.attn.z", (1, 6, 4, 16)) in seen
        assert not torch.allclose(base, ablated)
        # the package's own helpers find host taps too (duck typing)
        assert "blocks.1.attn.k" in tap_names(m)
    finally:
        monkeypatch.undo()
        tap_class.cache_clear()
    assert tap_class() is Tap and isinstance(make().blocks[0].attn.tap_q, Tap)


def test_shared_layers_each_application_has_its_own_cache_slot():
    """tests/test_shared_layers.py:44-54: looped layers share Parameters, not cache slots."""
    m = make(n_layers=5, shared_layers=[0, 1, 1, 1, 4])
    b = m.blocks
    assert b[2].attn.q_proj.weight is b[1].attn.q_proj.weight is b[3].attn.q_proj.weight
    assert b[4].attn.q_proj.weight is not b[1].attn.q_proj.weight
    assert b[2].norm1.weight is not b[1].norm1.weight
    x = torch.randint(0, 300, (1, 10))
    with torch.no_grad():
        full = m(x).logits
        cache = KVCache.for_model(m, 1)
        m(x[:, :6], cache=cache)
        steps = [m(x[:, i:i + 1], cache=cache).logits for i in range(6, 10)]
    torch.testing.assert_close(torch.cat(steps, 1), full[:, 6:], atol=1e-5, rtol=1e-5)
    assert len(cache.k) == 5 and not torch.equal(cache.k[1], cache.k[2])
    for bad in ([0, 1], [0, 2, 1, 1, 1], [0, 0, 1, 1, 1]):
        with pytest.raises(ValueError):
            ModelConfig(vocab_size=10, d_model=64, n_layers=5, n_heads=4, shared_layers=bad)


def test_hip_gate_on_cpu():
    cfg = ModelConfig(vocab_size=10, d_model=64, n_heads=4)
    a = Attention(cfg, 0)
    assert a._use_hip(torch.zeros(1, 4, 1, 16), None, None) == (False, None)


def test_document_mask_on_cpu_takes_the_torch_path():
    """A document mask on CPU tensors is the reference's eager path (the kernels' document
    starts are taken from GPU masks only; their GPU test is in test_gpu_module.py)."""
    import oracle
    from sleuth_amd import attention as att

    m = oracle.document_mask(torch.tensor([[0, 0, 1, 1, 1]]))
    assert att._doc_starts(m, 1, 5) is None


def test_flex_block_mask_matches_the_bool_document_mask():
    """A FlexAttention BlockMask from doc_block_mask gives the bool same_doc mask's output
    (attention.py:142-149 against 184-186); a pattern tap, a window or a cached prefix raise
    NotImplementedError as the reference's branch does."""
    pytest.importorskip("torch.nn.attention.flex_attention")
    import warnings

    from sleuth_amd.attention import doc_block_mask

    torch.manual_seed(5)
    doc_ids = torch.tensor([[0] * 9 + [1] * 14 + [2] * 9, [0] * 20 + [1] * 12])
    B, T = doc_ids.shape
    cfg = ModelConfig(vocab_size=10, d_model=64, n_heads=4, n_kv_heads=2, qk_norm=True, n_layers=1)
    a = Attention(cfg, 0).eval()
    x = torch.randn(B, T, 64)
    cos, sin = oracle.rope_tables(16, T, 1e4)
    with warnings.catch_warnings():
        warnings.simplefilter("ignore")      # flex_attention's eager-mode notice
        bm = doc_block_mask(doc_ids)
        with torch.no_grad():
            want = a(x, cos, sin, same_doc=oracle.document_mask(doc_ids))
            got = a(x, cos, sin, same_doc=bm)
        assert a.last_path == "torch"
        torch.testing.assert_close(got, want, atol=1e-5, rtol=1e-4)
        # the mask really is block-diagonal: the first document's output ignores the rest
        x2 = x.clone()
        x2[:, 9:] = torch.randn(B, T - 9, 64)
        with torch.no_grad():
            torch.testing.assert_close(a(x2, cos, sin, same_doc=bm)[0, :9], got[0, :9], atol=1e-5, rtol=1e-4)

        assign_tap_names(a)
        with torch.no_grad(), listen(a, {"pattern": lambda n, t: t}):
            with pytest.raises(NotImplementedError):
                a(x, cos, sin, same_doc=bm)
        w = ModelConfig(vocab_size=10, d_model=64, n_heads=4, n_kv_heads=2, n_layers=1,
                        layer_types=["sliding"], sliding_window=4)
        with torch.no_grad(), pytest.raises(NotImplementedError):
            Attention(w, 0).eval()(x, cos, sin, same_doc=bm)
        cache = KVCache([(2, 16)], B, T + 8, "cpu", torch.float32)
        with torch.no_grad():
            cfg1 = ModelConfig(vocab_size=10, d_model=64, n_heads=4, n_kv_heads=2, n_layers=1)
            a1 = Attention(cfg1, 0).eval()
            a1(x[:, :4], cos[:4], sin[:4], cache=cache)
            cache.advance(4)
            with pytest.raises(NotImplementedError):
                a1(x[:, 4:], cos[4:], sin[4:], cache=cache, same_doc=bm)


@pytest.mark.parametrize("sliding,n_past", [(False, 1), (False, 40), (True, 5), (True, 40)])
def test_drafter_attention_module_torch_path(sliding, n_past):
    """The MTP drafter's attention (mtp.py:73-92) on the CPU: RMSNorm then RoPE at position
    n_past (two roundings), the target's first n_past keys (sliding: the last window-1), scale
    1.0, GQA, o_proj -- against the oracle; the device-position form (mtp.py:169-188, n_past
    as a tensor and a mask over the whole view) gives the same result."""
    from sleuth_amd.drafter import DrafterAttention

    torch.manual_seed(2)
    H, K, hd, d, L = 4, 2, 16, 32, 48
    m = DrafterAttention(d, H, hd, sliding=sliding, window=8).eval()
    with torch.no_grad():
        m.q_norm.weight.add_(0.1 * torch.randn(hd))
    h = torch.randn(2, 1, d)
    k, v = torch.randn(2, K, L, hd), torch.randn(2, K, L, hd)
    cos_t, sin_t = oracle.rope_tables(hd, L + 1, 1e4)
    c, s_ = cos_t[n_past:n_past + 1], sin_t[n_past:n_past + 1]
    with torch.no_grad():
        got = m(h, k, v, c, s_, n_past)
        got_dev = m(h, k, v, c, s_, torch.tensor([n_past]))
        q = m.q_proj(h).view(2, 1, H, hd).transpose(1, 2)
        qn = oracle.eager_norm_rope(q, m.q_norm.weight, m.eps, c, s_)
        y = oracle.drafter_attention(qn, k, v, n_past, 8 if sliding else 0)
        want = m.o_proj(y.transpose(1, 2).reshape(2, 1, H * hd))
    assert m.last_path == "torch"
    torch.testing.assert_close(got, want, atol=1e-5, rtol=1e-4)
    torch.testing.assert_close(got_dev, want, atol=1e-5, rtol=1e-4)


def test_gated_attention_torch_path_matches_oracle():
    """Qwen3.5 gated attention (qwen35.py:187-216) on the CPU, through a cache (prefill 7,
    then 2 single tokens), against oracle.gated_attention on the module's own projections."""
    from types import SimpleNamespace

    from sleuth_amd.gated import GatedAttention

    H, K, hd, n_rot, d = 4, 2, 16, 8, 32
    cfg = SimpleNamespace(n_heads=H, n_kv_heads=K, head_dim=hd, n_rot=n_rot, norm_eps=1e-6)
    torch.manual_seed(9)
    m = GatedAttention(cfg, 0)
    m.q_proj, m.k_proj = torch.nn.Linear(d, H * 2 * hd, bias=False), torch.nn.Linear(d, K * hd, bias=False)
    m.v_proj, m.o_proj = torch.nn.Linear(d, K * hd, bias=False), torch.nn.Linear(H * hd, d, bias=False)
    with torch.no_grad():
        m.q_norm.weight.add_(0.1 * torch.randn(hd))
    m.eval()
    cos_t, sin_t = oracle.rope_tables(n_rot, 16, 1e6)
    cache = KVCache([(K, hd)], 2, 16, "cpu", torch.float32)
    kp = vp = None
    with torch.no_grad():
        for T in (7, 1, 1):
            p = cache.pos
            x = torch.randn(2, T, d)
            got = m(x, cos_t[p:p + T], sin_t[p:p + T], cache)
            cache.advance(T)
            qg = m.q_proj(x).view(2, T, H, 2 * hd)
            k, v = m.k_proj(x).view(2, T, K, hd), m.v_proj(x).view(2, T, K, hd)
            y, kn, vn = oracle.gated_attention(qg, k, v, cos=cos_t[p:p + T], sin=sin_t[p:p + T], n_rot=n_rot,
                                               q_weight=m.q_norm.weight, k_weight=m.k_norm.weight, eps=1e-6,
                                               k_past=kp, v_past=vp)
            kp = kn if kp is None else torch.cat([kp, kn], 2)
            vp = vn if vp is None else torch.cat([vp, vn], 2)
            torch.testing.assert_close(got, m.o_proj(y), atol=1e-5, rtol=1e-4)
    assert m.last_path == "torch"
