"""The drop-in module on the GPU: Attention + KVCache through the HIP kernels against
the oracle on the same projections, for the BASELINE config shapes; downstream-logit
argmax; and the callers (chunked prefill, graph decoding, speculative verify, ragged
batches, taps) behaving as the reference's tests require."""

from __future__ import annotations

import math

import pytest
import torch

import oracle
from conftest import gpu_available
from helpers import max_abs

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not gpu_available(), reason="needs a GPU")]
DEV = "cuda"
POISON = 1e4


def _modules():
    from sleuth_amd.attention import Attention
    from sleuth_amd.config import ModelConfig
    from sleuth_amd.kv_cache import KVCache

    return Attention, ModelConfig, KVCache


def _run_layer(dtype, d_model, H, K, hd, theta, steps, B=1, window=0, qk_norm=True, v_norm=False,
               seed=0, lens=None, pos_start=0):
    """Runs one Attention layer through a cache for the given token counts per call and
    returns [(got_z [B,T,H,hd], ref [B,T,H,hd], path)] per call. The oracle sees the
    module's own raw projections (recorded by hooks), normalised with one rounding to
    the dtype (fused_ops semantics), and attends in fp32 over its own cache."""
    Attention, ModelConfig, KVCache = _modules()
    cfg = ModelConfig(vocab_size=10, d_model=d_model, n_heads=H, n_kv_heads=K, head_size=hd,
                      qk_norm=qk_norm, v_norm=v_norm, rope_theta=theta, n_layers=1,
                      layer_types=["sliding"] if window else [], sliding_window=window)
    torch.manual_seed(seed)
    a = Attention(cfg, 0).eval()
    if qk_norm:
        with torch.no_grad():
            a.q_norm.weight.copy_(1 + 0.1 * torch.randn(hd))
            a.k_norm.weight.copy_(1 + 0.1 * torch.randn(hd))
    a = a.to(DEV, dtype)
    rec = {}
    a.q_proj.register_forward_hook(lambda m, i, o: rec.__setitem__("q", o))
    a.k_proj.register_forward_hook(lambda m, i, o: rec.__setitem__("k", o))
    a.v_proj.register_forward_hook(lambda m, i, o: rec.__setitem__("v", o))
    seen = {}
    a.tap_z.listeners.append(lambda n, t: seen.__setitem__("z", t.clone()))
    max_len = pos_start + sum(steps) + 8 if lens is None else max(lens) + sum(steps) + 8
    cache = KVCache([(K, hd)], B, max_len, DEV, dtype)
    cache.k[0].fill_(POISON)   # every position a row has not stored: a kernel that reads
    cache.v[0].fill_(POISON)   # past its row's length gives a visibly wrong output
    ocache = oracle.KVCache([(K, hd)], B, max_len, "cpu", torch.float32)
    cos_t, sin_t = oracle.rope_tables(hd, max_len, theta)
    g = torch.Generator().manual_seed(seed + 1)
    if lens is not None:   # ragged rows, pre-filled with N(0,1) (already normalised K/V)
        for b, L in enumerate(lens):
            kv = torch.randn(2, K, L, hd, generator=g).to(dtype)
            cache.k[0][b, :, :L] = kv[0].to(DEV)
            cache.v[0][b, :, :L] = kv[1].to(DEV)
            ocache.k[0][b, :, :L] = kv[0].float()
            ocache.v[0][b, :, :L] = kv[1].float()
        cache.set_lengths(lens)
    elif pos_start:
        kv = torch.randn(2, B, K, pos_start, hd, generator=g).to(dtype)
        cache.k[0][:, :, :pos_start] = kv[0].to(DEV)
        cache.v[0][:, :, :pos_start] = kv[1].to(DEV)
        ocache.k[0][:, :, :pos_start] = kv[0].float()
        ocache.v[0][:, :, :pos_start] = kv[1].float()
        cache.pos = ocache.pos = pos_start
    qw = a.q_norm.weight.detach().cpu() if qk_norm else None
    kw = a.k_norm.weight.detach().cpu() if qk_norm else None
    results = []
    for T in steps:
        x = torch.randn(B, T, d_model, generator=g).to(dtype).to(DEV)
        if lens is None:
            p0 = [cache.pos] * B
            cos, sin = cos_t[p0[0]:p0[0] + T], sin_t[p0[0]:p0[0] + T]
        else:
            p0 = list(cache.seq_lens_host)
            cos = torch.stack([cos_t[p:p + T] for p in p0])
            sin = torch.stack([sin_t[p:p + T] for p in p0])
        with torch.no_grad():
            a(x, cos.to(DEV), sin.to(DEV), cache)
        q = rec["q"].view(B, T, H, hd).transpose(1, 2).cpu()
        k = rec["k"].view(B, T, K, hd).transpose(1, 2).cpu()
        v = rec["v"].view(B, T, K, hd).transpose(1, 2).cpu()
        qn = oracle.head_norm_rope(q, qw, cfg.norm_eps, cos, sin, norm=qk_norm)
        kn = oracle.head_norm_rope(k, kw, cfg.norm_eps, cos, sin, norm=qk_norm)
        vn = oracle.head_norm_rope(v, None, cfg.norm_eps) if v_norm else v
        for b in range(B):
            ocache.k[0][b, :, p0[b]:p0[b] + T] = kn[b].float()
            ocache.v[0][b, :, p0[b]:p0[b] + T] = vn[b].float()
        ref = oracle.ragged_decode(qn.float(), ocache.k[0], ocache.v[0], [p + T for p in p0], window,
                                   1.0 / math.sqrt(hd))
        results.append((seen["z"].float().cpu(), ref.transpose(1, 2), a.last_path))
        cache.advance(T)
    return results


def _downstream_argmax_ok(got, ref):
    """Downstream-logit argmax agreement (the north star's bf16 criterion), from helpers:
    every row whose reference top-2 margin is at least 1% of the logits' RMS must pick the
    same token; the rows below that margin are counted, and at most 10% (or 2) may be."""
    from helpers import downstream_argmax

    r = downstream_argmax(got, ref)
    print(f"downstream argmax: {r}")
    assert r["mismatched"] == 0, r
    assert r["near_ties"] <= max(2, 0.1 * r["rows"]), r
    return True


def test_config1_fp32_prefill_then_64_decode_steps():
    """C1: fp32, batch 1, 8 q / 4 kv heads, hd 32, prefill 256 then 64 decode steps,
    QK-norm (unit gain), theta 1e4: max-abs <= 1e-4 on every step."""
    res = _run_layer(torch.float32, 256, 8, 4, 32, 1e4, [256] + [1] * 64, qk_norm=True)
    for got, ref, path in res:
        assert path == "hip-decode"
        assert max_abs(got, ref) <= 1e-4


def test_config2_bf16_decode():
    """C2 shape: bf16, batch 16, 12 q / 4 kv, hd 64, cache at 2048, decode steps."""
    res = _run_layer(torch.bfloat16, 768, 12, 4, 64, 1e4, [1] * 4, B=16, pos_start=2048)
    for got, ref, path in res:
        assert path == "hip-decode" and max_abs(got, ref) <= 2e-2
        assert _downstream_argmax_ok(got, ref)


def test_config3_bf16_prefill_and_decode():
    """C3 shape: bf16, 16 q / 8 kv, hd 128, theta 1e6, gains ~N(1, 0.1): prefill of
    1024 tokens (batch 2) through the MFMA kernel, then decode steps."""
    res = _run_layer(torch.bfloat16, 1024, 16, 8, 128, 1e6, [1024, 1, 1], B=2)
    assert [r[2] for r in res] == ["hip-prefill", "hip-decode", "hip-decode"]
    for got, ref, _ in res:
        assert max_abs(got, ref) <= 2e-2
        assert _downstream_argmax_ok(got, ref)


def test_config4_ragged_decode():
    """C4 shape at reduced size: per-row lengths, one new token per row."""
    lens = [1024, 3000, 1500, 4096, 1025, 2222, 3333, 1800]
    res = _run_layer(torch.bfloat16, 1024, 16, 8, 128, 1e6, [1, 1], B=8, lens=lens)
    for got, ref, path in res:
        assert path == "hip-decode" and max_abs(got, ref) <= 2e-2
        assert _downstream_argmax_ok(got, ref)


@pytest.mark.parametrize("window", [1024, 0])
def test_config5_mtp_verify(window):
    """C5: bf16, batch 8, k=4 draft tokens verified causally over an 8192 cache, MQA 8 q /
    1 kv, hd 256, theta 1e6; sliding-window (1024) and global layers."""
    res = _run_layer(torch.bfloat16, 2048, 8, 1, 256, 1e6, [4, 4], B=8, window=window, pos_start=8192)
    for got, ref, path in res:
        assert path == "hip-decode" and max_abs(got, ref) <= 2e-2
        assert _downstream_argmax_ok(got, ref)


def test_v_norm_and_no_qk_norm():
    res = _run_layer(torch.bfloat16, 512, 8, 2, 64, 1e4, [40, 1, 3], B=2, qk_norm=False, v_norm=True)
    for got, ref, _ in res:
        assert max_abs(got, ref) <= 2e-2


# ----------------------------------------------------------------------------- callers
def _tiny(**kw):
    from sleuth_amd.config import ModelConfig
    from sleuth_amd.model import Transformer

    torch.manual_seed(0)
    cfg = dict(vocab_size=200, d_model=128, n_layers=3, n_heads=4, n_kv_heads=2, max_seq_len=160,
               qk_norm=True)
    cfg.update(kw)
    return Transformer(ModelConfig(**cfg)).eval()


def test_kv_cache_matches_full_forward_fp32():
    """tests/test_model.py:61-69 through the HIP path (fp32)."""
    from sleuth_amd.kv_cache import KVCache

    m = _tiny(layer_types=["sliding", "full", "sliding"], sliding_window=6).to(DEV)
    x = torch.randint(0, 200, (2, 40), device=DEV)
    with torch.no_grad():
        full = m(x).logits
        cache = KVCache.for_model(m, batch=2)
        parts = [m(x[:, :20], cache=cache).logits, m(x[:, 20:25], cache=cache).logits]
        parts += [m(x[:, i:i + 1], cache=cache).logits for i in range(25, 40)]
    assert m.blocks[0].attn.last_path == "hip-decode"
    assert max_abs(torch.cat(parts, 1), full) <= 1e-4


def test_bf16_kv_cache_close_to_full_forward():
    """tests/test_gpu.py:38-49 (bf16 cache vs full forward, loose)."""
    from sleuth_amd.kv_cache import KVCache

    m = _tiny().to(DEV, torch.bfloat16)
    x = torch.randint(0, 200, (1, 48), device=DEV)
    with torch.no_grad():
        full = m(x).logits.float()
        cache = KVCache.for_model(m, 1)
        parts = [m(x[:, :32], cache=cache).logits.float()]
        parts += [m(x[:, i:i + 1], cache=cache).logits.float() for i in range(32, 48)]
    assert m.blocks[1].attn.last_path == "hip-decode"
    assert (torch.cat(parts, 1) - full).abs().max().item() < 0.1


def test_graph_generation_matches_eager():
    """tests/test_cuda_graph.py:64-78: greedy tokens with HIP graphs = without, from a short
    context to the end of the cache; one graph serves every length (the kernels read the live
    length on the device) and is reused by the next call."""
    from sleuth_amd.generate import _decoders, generate

    m = _tiny(layer_types=["sliding", "full", "sliding"], sliding_window=8, max_seq_len=96).to(DEV, torch.bfloat16)
    prompt = [1, 5, 9, 13]
    eager = generate(m, prompt, 80)
    graph = generate(m, prompt, 80, cuda_graph=True)
    assert graph.new_ids == eager.new_ids
    assert graph.stats["graph_replays"] == 79
    (dec,) = _decoders[m].values()
    assert dec.recorded
    again = generate(m, prompt, 80, cuda_graph=True)
    assert again.new_ids == eager.new_ids and dec.replays == 2 * 79


@pytest.mark.parametrize("cuda_graph", [False, True])
def test_speculative_matches_plain(cuda_graph):
    """tests/test_speculative.py:31-45, 81-94: greedy speculative == plain greedy, k = 4,
    sliding + full layers, up to the end of the context."""
    from sleuth_amd.generate import generate, speculative_generate

    m = _tiny(layer_types=["sliding", "full"], n_layers=2, sliding_window=8, max_seq_len=96).to(DEV, torch.bfloat16)
    prompt = [1, 5, 9, 13, 5, 9, 13, 5, 9, 13, 22, 5, 9]
    plain = generate(m, prompt, 83)
    spec = speculative_generate(m, prompt, 83, k=4, cuda_graph=cuda_graph)
    assert spec.new_ids == plain.new_ids
    s = spec.stats["speculative"]
    assert s["forwards"] < len(spec.new_ids)


def test_taps_on_the_hip_path():
    """Listening on attn.q / attn.k keeps the HIP path (materialised q/k) and the same
    result; attn.pattern forces the torch path; zeroing attn.z ablates the heads."""
    from sleuth_amd.taps import listen

    m = _tiny(d_model=256).to(DEV, torch.bfloat16)   # head dim 64: the MFMA prefill
    x = torch.randint(0, 200, (1, 24), device=DEV)
    with torch.no_grad():
        base = m(x).logits.float()
        assert m.blocks[0].attn.last_path == "hip-prefill"
        seen = {}
        with listen(m, {"blocks.0.attn.q": lambda n, t: seen.setdefault("q", t),
                        "blocks.0.attn.k": lambda n, t: seen.setdefault("k", t)}):
            tapped = m(x).logits.float()
        assert m.blocks[0].attn.last_path == "hip-prefill"
        assert seen["q"].shape == (1, 4, 24, 64) and seen["k"].shape == (1, 2, 24, 64)
        assert (tapped - base).abs().max().item() < 2e-2
        with listen(m, {"blocks.*.attn.pattern": lambda n, t: None}):
            m(x)
        assert m.blocks[0].attn.last_path == "torch"
        with listen(m, {"blocks.*.attn.z": lambda n, t: torch.zeros_like(t)}):
            ablated = m(x).logits.float()
        assert not torch.allclose(base, ablated)


@pytest.mark.parametrize("hd", [64, 128])
def test_document_mask_on_the_hip_path(hd, monkeypatch):
    """The reference's document mask (transformer.py:271-275, from doc_ids) over a scored
    window runs forge_attn_prefill_docs when the documents are contiguous runs, and agrees
    with the module's own torch path (the reference's SDPA with _mask & same_doc); a mask
    whose document ids repeat after a gap stays on the torch path."""
    import oracle

    Attention, ModelConfig, _ = _modules()
    cfg = ModelConfig(vocab_size=10, d_model=8 * hd, n_heads=8, n_kv_heads=2, head_size=hd,
                      qk_norm=True, rope_theta=1e4, n_layers=1)
    torch.manual_seed(3)
    a = Attention(cfg, 0).eval().to(DEV, torch.bfloat16)
    B, T = 2, 300
    x = torch.randn(B, T, 8 * hd, device=DEV, dtype=torch.bfloat16)
    cos, sin = (t.to(DEV) for t in oracle.rope_tables(hd, T, 1e4))
    docs = torch.stack([torch.repeat_interleave(torch.arange(4), torch.tensor([70, 1, 129, 100])),
                        torch.repeat_interleave(torch.arange(3), torch.tensor([64, 64, 172]))]).to(DEV)
    same_doc = oracle.document_mask(docs)
    with torch.no_grad():
        got = a(x, cos, sin, same_doc=same_doc).float()
        assert a.last_path == "hip-prefill-docs"
        monkeypatch.setenv("SLEUTH_AMD_NO_HIP", "1")
        want = a(x, cos, sin, same_doc=same_doc).float()
        assert a.last_path == "torch"
        monkeypatch.delenv("SLEUTH_AMD_NO_HIP")
        assert (got - want).abs().max().item() <= 2e-2
        gapped = docs.clone()
        gapped[0, 250:] = 0                         # document 0 again, after documents 1-3
        a(x, cos, sin, same_doc=oracle.document_mask(gapped))
        assert a.last_path == "torch"
    # under inference_mode the mask is an inference tensor (no version counter): its starts
    # are read again at each call, so a mask changed in place is seen
    with torch.inference_mode():
        m_inf = oracle.document_mask(docs)
        got_inf = a(x, cos, sin, same_doc=m_inf).float()
        assert a.last_path == "hip-prefill-docs"
        assert torch.equal(got_inf, got)
        m_inf.copy_(oracle.document_mask(torch.zeros_like(docs)))   # one document per row
        one = a(x, cos, sin, same_doc=m_inf).float()
        assert a.last_path == "hip-prefill-docs"
        plain = a(x, cos, sin).float()
        assert torch.equal(one, plain)


@pytest.mark.parametrize("host_cache", [False, True])
def test_static_step_equals_normal_step_on_gpu(host_cache):
    """A static (graph-ready) step of 5 tokens == the normal path (tests/test_cuda_graph.py:81-95),
    with the product cache and with the host's StaticKVCache protocol."""
    from host_protocol import HostStaticKVCache
    from sleuth_amd.kv_cache import KVCache

    m = _tiny(layer_types=["sliding", "full", "sliding"], sliding_window=8).to(DEV)
    ids = torch.randint(0, 200, (1, 30), device=DEV)
    shapes = [(m.cfg.attn_spec(i).kv_heads, m.cfg.attn_spec(i).head_dim) for i in range(m.cfg.n_layers)]
    with torch.no_grad():
        full = m(ids).logits[0]
        st = (HostStaticKVCache if host_cache else KVCache)(shapes, 1, 96, DEV, torch.float32, tokens_per_step=5)
        m(ids[:, :20], cache=st)
        st.length, st.static = 32, True
        st.pos_t.fill_(20)
        out = m(ids[:, 20:25], cache=st).logits[0]
        st.static = False
    assert max_abs(out, full[20:25]) <= 1e-4


def test_fused_qkv_projection_matches_separate():
    """On the GPU inference path q, k and v come from one GEMM over the concatenated
    weights (the three projections of attention.py:106-108 as one call). The module's output
    matches the separate projections' (a forward hook on a projection forces those), the
    weights become views of one buffer, and an in-place weight update is picked up."""
    Attention, ModelConfig, _ = _modules()
    cfg = ModelConfig(vocab_size=10, d_model=256, n_heads=8, n_kv_heads=4, head_size=32, qk_norm=True,
                      n_layers=1)
    torch.manual_seed(0)
    a = Attention(cfg, 0).eval().to(DEV, torch.bfloat16)
    x = torch.randn(2, 5, 256, device=DEV, dtype=torch.bfloat16)
    cos, sin = oracle.rope_tables(32, 16, 1e4)
    cos, sin = cos[:5].to(DEV), sin[:5].to(DEV)

    def separate():
        h = a.q_proj.register_forward_hook(lambda m, i, o: None)
        try:
            return a(x, cos, sin)
        finally:
            h.remove()

    from sleuth_amd.attention import fused_qkv_entry

    with torch.no_grad():
        fused = a(x, cos, sin)
        assert a.q_proj.weight.data_ptr() == fused_qkv_entry(a.q_proj.weight).w.data_ptr()
        assert max_abs(fused.float().cpu(), separate().float().cpu()) <= 2e-2
        a.k_proj.weight.mul_(2.0)
        fused2 = a(x, cos, sin)
        assert max_abs(fused2.float().cpu(), separate().float().cpu()) <= 2e-2
        assert not torch.equal(fused2, fused)
    # built under inference_mode, the buffer is an ordinary tensor: plain no_grad calls and
    # in-place updates still work afterwards
    b = Attention(cfg, 0).eval().to(DEV, torch.bfloat16)
    with torch.inference_mode():
        b(x, cos, sin)
    with torch.no_grad():
        b.q_proj.weight.mul_(1.5)
        assert torch.isfinite(b(x, cos, sin)).all()


def _hip_against_cpu(mod, d_model, kv, cos_t, sin_t, seed, expect_hip, oracle_step=None):
    """Runs mod on the GPU (HIP path) and a copy of it on the CPU (the reference's eager
    path, so no reference attention runs on the GPU) over a 40-token prefill and 3 decode
    steps through a cache; returns [(gpu_out, cpu_out, oracle_out)] per call, oracle_out
    from oracle_step(T, pos) (called right after the GPU call) or None."""
    import copy

    from sleuth_amd.kv_cache import KVCache

    dtype = next(mod.parameters()).dtype
    cpu = copy.deepcopy(mod).cpu()
    outs = []
    caches = {"gpu": KVCache([kv], 2, 64, DEV, dtype), "cpu": KVCache([kv], 2, 64, "cpu", dtype)}
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        for T in (40, 1, 1, 1):
            x = torch.randn(2, T, d_model, generator=g).to(dtype)
            p = caches["gpu"].pos
            c, s_ = cos_t[p:p + T], sin_t[p:p + T]
            got = mod(x.to(DEV), c.to(DEV), s_.to(DEV), caches["gpu"]).float().cpu()
            assert mod.last_path == expect_hip(T)
            want = None if oracle_step is None else oracle_step(T, p).float()
            ref = cpu(x, c, s_, caches["cpu"]).float()
            assert cpu.last_path == "torch"
            outs.append((got, ref, want))
            for cache in caches.values():
                cache.advance(T)
    return outs


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_partial_rope_on_the_hip_path(dtype):
    """Partial RoPE (rope_dim < head dim, rope.py:46-55): norm and RoPE in torch as the
    reference's eager path, attention and the cache write in the kernels; the outputs match
    the eager path run on the CPU."""
    Attention, ModelConfig, _ = _modules()
    cfg = ModelConfig(vocab_size=10, d_model=256, n_heads=4, n_kv_heads=2, head_size=64, qk_norm=True,
                      rope_dim=32, n_layers=1)
    torch.manual_seed(1)
    a = Attention(cfg, 0).eval().to(DEV, dtype)
    cos_t, sin_t = oracle.rope_tables(32, 64, 1e4)
    prefill = "hip-prefill" if dtype != torch.float32 else "hip-decode"
    for got, ref, _ in _hip_against_cpu(a, 256, (2, 64), cos_t, sin_t, 2,
                                        lambda T: prefill if T > 16 else "hip-decode"):
        assert max_abs(got, ref) <= (1e-4 if dtype == torch.float32 else 2e-2)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_gated_attention_hip_matches_oracle(dtype):
    """Qwen3.5 gated attention (qwen35.py:187-216): q/gate split, partial RoPE, sigmoid gate.
    The module on the HIP path (cache write and attention in the kernels) over a 40-token
    prefill and 3 decode steps, against oracle.gated_attention (pinned by float64 loops) on
    the module's own projections, and the module's torch path on the CPU."""
    from types import SimpleNamespace

    from sleuth_amd.gated import GatedAttention

    H, K, hd, n_rot, d = 4, 2, 64, 32, 256
    cfg = SimpleNamespace(n_heads=H, n_kv_heads=K, head_dim=hd, n_rot=n_rot, norm_eps=1e-6)
    torch.manual_seed(3)
    m = GatedAttention(cfg, 0)
    m.q_proj = torch.nn.Linear(d, H * 2 * hd, bias=False)
    m.k_proj = torch.nn.Linear(d, K * hd, bias=False)
    m.v_proj = torch.nn.Linear(d, K * hd, bias=False)
    m.o_proj = torch.nn.Linear(H * hd, d, bias=False)
    with torch.no_grad():
        m.q_norm.weight.add_(0.1 * torch.randn(hd))
        m.k_norm.weight.add_(0.1 * torch.randn(hd))
    m = m.eval().to(DEV, dtype)
    rec = {}
    for name in ("q", "k", "v"):
        getattr(m, f"{name}_proj").register_forward_hook(lambda mod, i, o, n=name: rec.__setitem__(n, o))
    cos_t, sin_t = oracle.rope_tables(n_rot, 64, 1e6)
    tol_ = 1e-4 if dtype == torch.float32 else 2e-2
    past = {}

    def oracle_step(T, p):
        qg = rec["q"].cpu().view(2, T, H, 2 * hd)
        k = rec["k"].cpu().view(2, T, K, hd)
        v = rec["v"].cpu().view(2, T, K, hd)
        y, kn, vn = oracle.gated_attention(qg, k, v, cos=cos_t[p:p + T], sin=sin_t[p:p + T], n_rot=n_rot,
                                           q_weight=m.q_norm.weight.cpu(), k_weight=m.k_norm.weight.cpu(),
                                           eps=1e-6, k_past=past.get("k"), v_past=past.get("v"))
        past["k"] = kn if "k" not in past else torch.cat([past["k"], kn], 2)
        past["v"] = vn if "v" not in past else torch.cat([past["v"], vn], 2)
        return torch.nn.functional.linear(y.float(), m.o_proj.weight.float().cpu())

    for got, ref, want in _hip_against_cpu(m, d, (K, hd), cos_t, sin_t, 4, lambda T: "hip", oracle_step):
        assert max_abs(got, want) <= tol_
        assert max_abs(got, ref) <= tol_


# ----------------------------------------------------------------------------- host objects
def test_hip_path_on_the_hosts_caches():
    """The drop-in on the host's own cache objects (tests/host_protocol.py: exactly the
    protocol of kv_cache.py:25-138, no per-row lengths, no room check): a 40-token prefill,
    a decode step, a 5-token verify rewound as the speculative decoder does, and a
    graph-captured static step replayed at two positions -- each against the oracle."""
    from host_protocol import HostStaticKVCache

    Attention, ModelConfig, _ = _modules()
    H, K, hd, d, max_len, tps = 16, 8, 128, 1024, 128, 5
    cfg = ModelConfig(vocab_size=10, d_model=d, n_heads=H, n_kv_heads=K, head_size=hd, qk_norm=True,
                      rope_theta=1e6, n_layers=1)
    torch.manual_seed(7)
    a = Attention(cfg, 0).eval()
    with torch.no_grad():
        a.q_norm.weight.copy_(1 + 0.1 * torch.randn(hd))
        a.k_norm.weight.copy_(1 + 0.1 * torch.randn(hd))
    a = a.to(DEV, torch.bfloat16)
    rec = {}
    for name in ("q", "k", "v"):
        getattr(a, f"{name}_proj").register_forward_hook(lambda m, i, o, n=name: rec.__setitem__(n, o))
    seen = {}
    a.tap_z.listeners.append(lambda n, t: seen.__setitem__("z", t))
    cache = HostStaticKVCache([(K, hd)], 1, max_len, DEV, torch.bfloat16, tokens_per_step=tps)
    cache.k[0].fill_(POISON)
    cache.v[0].fill_(POISON)
    ocache = oracle.KVCache([(K, hd)], 1, max_len, "cpu", torch.float32)
    cos_t, sin_t = oracle.rope_tables(hd, max_len, 1e6)
    cos_d, sin_d = cos_t.to(DEV), sin_t.to(DEV)
    qw, kw = a.q_norm.weight.detach().float().cpu(), a.k_norm.weight.detach().float().cpu()
    g = torch.Generator().manual_seed(8)

    def oracle_out(p0, T):
        q = rec["q"].view(1, T, H, hd).transpose(1, 2).float().cpu()
        k = rec["k"].view(1, T, K, hd).transpose(1, 2).float().cpu()
        v = rec["v"].view(1, T, K, hd).transpose(1, 2).float().cpu()
        c, s_ = cos_t[p0:p0 + T], sin_t[p0:p0 + T]
        qn = oracle.head_norm_rope(q.bfloat16(), qw, cfg.norm_eps, c, s_).float()
        ocache.k[0][:, :, p0:p0 + T] = oracle.head_norm_rope(k.bfloat16(), kw, cfg.norm_eps, c, s_).float()
        ocache.v[0][:, :, p0:p0 + T] = v
        kk, vv = ocache.k[0][:, :, :p0 + T], ocache.v[0][:, :, :p0 + T]
        return oracle.sdpa(qn, kk, vv, p0, 0, a.scale).transpose(1, 2)

    def eager(T):
        p0 = cache.pos
        x = torch.randn(1, T, d, generator=g).to(torch.bfloat16).to(DEV)
        with torch.no_grad():
            a(x, cos_d[p0:p0 + T], sin_d[p0:p0 + T], cache)
        return seen["z"].float().cpu(), oracle_out(p0, T)

    for T, path in ((40, "hip-prefill"), (1, "hip-decode")):
        got, ref = eager(T)
        assert a.last_path == path and max_abs(got, ref) <= 2e-2, (T, max_abs(got, ref))
        cache.advance(T)
    start = cache.pos
    got, ref = eager(5)                      # verify of [pending] + 4 guesses ...
    assert a.last_path == "hip-decode" and max_abs(got, ref) <= 2e-2
    cache.advance(5)
    cache.pos = start + 2                    # ... of which the caller keeps two
    assert torch.all(cache.k[0][0, :, start + 5:] == POISON)

    # graph-captured static step: positions pos_t .. pos_t + 4 on the device
    x_buf = torch.zeros(1, tps, d, device=DEV, dtype=torch.bfloat16)

    def static_step():
        cache.new_step()
        pos = cache.positions
        return a(x_buf, cos_d.index_select(0, pos), sin_d.index_select(0, pos), cache)

    cache.static, cache.length = True, 64
    cache.pos_t.fill_(cache.pos)
    with torch.no_grad():
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            static_step()
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            static_step()
    assert a.last_path == "hip-decode"
    for _ in range(2):
        p0 = cache.pos
        x_buf.copy_(torch.randn(1, tps, d, generator=g).to(torch.bfloat16))
        cache.pos_t.fill_(p0)
        graph.replay()
        torch.cuda.synchronize()
        got, ref = seen["z"].float().cpu(), oracle_out(p0, tps)
        assert max_abs(got, ref) <= 2e-2, (p0, max_abs(got, ref))
        cache.pos = p0 + 3                   # keep three of the five
    cache.static = False


@pytest.mark.parametrize("cuda_graph", [False, True])
def test_shared_layers_on_gpu(cuda_graph):
    """Looped layers (tests/test_shared_layers.py:44-54, reference transformer.py:215-228):
    blocks 1-3 share one set of projection Parameters. The fused q/k/v buffer is built once
    per set of Parameters and never again (eager and graph-captured decoding); chunked
    decoding matches one pass; graph decoding gives the eager tokens, and both match the
    torch path's first logits."""
    from sleuth_amd.attention import _FusedQKV
    from sleuth_amd.generate import generate
    from sleuth_amd.kv_cache import KVCache

    m = _tiny(n_layers=5, shared_layers=[0, 1, 1, 1, 4], max_seq_len=64).to(DEV, torch.bfloat16)
    x = torch.randint(0, 200, (1, 24), device=DEV)
    with torch.no_grad():
        before = _FusedQKV.builds
        full = m(x).logits.float()
        assert _FusedQKV.builds - before == 3        # blocks 0, 1 (= 2 = 3) and 4
        built = _FusedQKV.builds
        cache = KVCache.for_model(m, 1)
        parts = [m(x[:, :16], cache=cache).logits.float()]
        parts += [m(x[:, i:i + 1], cache=cache).logits.float() for i in range(16, 24)]
        assert (torch.cat(parts, 1) - full).abs().max().item() < 0.1
        assert not torch.equal(cache.k[1], cache.k[2])
        out = generate(m, [3, 1, 4, 1, 5], 30, cuda_graph=cuda_graph)
        assert _FusedQKV.builds == built
        if cuda_graph:
            assert out.new_ids == generate(m, [3, 1, 4, 1, 5], 30).new_ids
        import os

        os.environ["SLEUTH_AMD_NO_HIP"] = "1"
        try:
            torch_logits = m(x).logits.float()
        finally:
            del os.environ["SLEUTH_AMD_NO_HIP"]
        assert m.blocks[0].attn.last_path == "torch"
        assert (torch_logits - full).abs().max().item() < 0.1


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("sliding", [False, True])
def test_drafter_attention_module_on_gpu(dtype, sliding):
    """The drafter's attention module (mtp.py:73-92) on the HIP path, against the oracle
    (oracle.drafter_attention after the reference's eager norm + RoPE); then its graph form
    (mtp.py:169-188): n_past held in a device tensor, the call captured once and replayed at
    two positions, each against the oracle."""
    from sleuth_amd.drafter import DrafterAttention

    torch.manual_seed(11)
    H, K, hd, d, L, window = 8, 2, 128, 512, 1200, 512
    m = DrafterAttention(d, H, hd, sliding=sliding, window=window).eval()
    with torch.no_grad():
        m.q_norm.weight.add_(0.1 * torch.randn(hd))
    m = m.to(DEV, dtype)
    g = torch.Generator().manual_seed(12)
    k = torch.randn(1, K, L, hd, generator=g).to(dtype)
    v = torch.randn(1, K, L, hd, generator=g).to(dtype)
    cos_t, sin_t = oracle.rope_tables(hd, L + 1, 1e6)
    kd, vd, cd, sd = k.to(DEV), v.to(DEV), cos_t.to(DEV), sin_t.to(DEV)
    tol_ = 1e-4 if dtype == torch.float32 else 2e-2

    def want(h, n_past):
        with torch.no_grad():
            q = torch.nn.functional.linear(h.cpu().float(), m.q_proj.weight.cpu().float())
            q = q.to(dtype).view(1, 1, H, hd).transpose(1, 2)
            qn = oracle.eager_norm_rope(q, m.q_norm.weight.cpu(), m.eps, cos_t[n_past:n_past + 1],
                                        sin_t[n_past:n_past + 1])
            y = oracle.drafter_attention(qn.float(), k.float(), v.float(), n_past, window if sliding else 0)
            return torch.nn.functional.linear(y.transpose(1, 2).reshape(1, 1, H * hd).to(dtype).float(),
                                              m.o_proj.weight.cpu().float())

    for n_past in (1, 300, 1100):
        h = torch.randn(1, 1, d, generator=g).to(dtype).to(DEV)
        with torch.no_grad():
            got = m(h, kd, vd, cd[n_past:n_past + 1], sd[n_past:n_past + 1], n_past)
        assert m.last_path == "hip"
        assert max_abs(got, want(h, n_past)) <= tol_, n_past

    h_buf = torch.zeros(1, 1, d, device=DEV, dtype=dtype)
    pos = torch.zeros(1, dtype=torch.long, device=DEV)

    def call():
        return m(h_buf, kd, vd, cd.index_select(0, pos), sd.index_select(0, pos), pos)

    with torch.no_grad():
        pos.fill_(600)
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            call()
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            out = call()
    for n_past in (700, 1190):
        h = torch.randn(1, 1, d, generator=g).to(dtype)
        h_buf.copy_(h)
        pos.fill_(n_past)
        graph.replay()
        torch.cuda.synchronize()
        assert max_abs(out, want(h_buf, n_past)) <= tol_, n_past
