"""Grouped-query attention with QK-norm, RoPE and a KV cache: the drop-in for
sleuth/forge/model/attention.py:76-206.

Same constructor (cfg, layer_idx), submodule names (q_proj/k_proj/v_proj/o_proj/q_norm/
k_norm, the loaders' contract), taps (tap_q, tap_k, tap_pattern, tap_z) and forward
signature forward(x, cos, sin, cache=None, same_doc=None) -> [B, T, d].

Paths (the reference's own dispatch, attention.py:109-153, with the HIP kernels in place
of head_norm_rope + cache.update + SDPA):
  * HIP (GPU inference: no grad, dtype fp32/bf16/fp16, head dim 32/64/128/256, and 512 in
    bf16/fp16, nobody listening on attn.pattern; a document mask only as below):
      k norm + RoPE (+ v norm), written into the cache at pos / pos_t / per-row
      lengths (with partial RoPE, norm and RoPE run in torch as the reference's eager
      code does, and the kernels take q and k as they are), then attention:
      T > 16, bf16/fp16, head dim 64-512:     forge_kv_append, then forge_attn_prefill
                        (MFMA flash) with the q norm + RoPE in its q load;
      otherwise         forge_attn_decode_append: the cache write and the split-K
                        attention (decode, verify, static steps, fp32, other head sizes)
                        in one launch, the q norm + RoPE fused into the q load.
      A boolean document mask (transformer.py:271-275) over a whole window (no cache,
      T > 16, the prefill dtypes and head dims) whose documents are contiguous runs goes
      to forge_attn_prefill_docs, which takes each query's first visible key.
    The output comes back as [B, T, H, hd], the layout o_proj reads.
  * torch (CPU, training, FlexAttention block masks and other document masks, the
    pattern tap, or SLEUTH_AMD_NO_HIP=1): the reference's eager code, unchanged in meaning;
    a BlockMask goes to flex_attention with the reference's NotImplementedError for a
    pattern tap, a window or a cached prefix (attention.py:142-149).
If a GPU tensor would take the HIP path and the library is missing or fails its
first-use self-check, forward raises: there is no silent fallback.
"""

from __future__ import annotations

import math
import os
import weakref

import torch
import torch.nn.functional as F
from torch import nn

from .config import ModelConfig
from .norm import RMSNorm
from .rope import apply_rope
from .taps import make_tap, tap_active

DECODE_MAX_T = 16
_HIP_HEAD_DIMS = (32, 64, 128, 256, 512)   # 512 (Gemma 4's full layers) in bf16/fp16 only
_HIP_DTYPES = (torch.float32, torch.bfloat16, torch.float16)


def hip_shape_ok(dtype: torch.dtype, head_dim: int) -> bool:
    """The kernels take this dtype and head dim (a 512-wide key row must be 2-byte elements:
    the split-K kernel holds one row in a wave's 16-byte lanes)."""
    return dtype in _HIP_DTYPES and head_dim in _HIP_HEAD_DIMS and not (head_dim == 512 and dtype == torch.float32)
_checked: dict[tuple, bool] = {}


def hip_disabled() -> bool:
    return os.environ.get("SLEUTH_AMD_NO_HIP") == "1"


_FLEX_LIMITS = ("FlexAttention document masks are for training: no attention taps, sliding windows "
                "or KV cache")


def doc_block_mask(doc_ids: torch.Tensor):
    """[B, T] document numbers -> a FlexAttention BlockMask that is causal and within one
    document (the reference's doc_block_mask, attention.py:54-64): built once per batch and
    shared by every layer; the torch path passes it to flex_attention."""
    from torch.nn.attention.flex_attention import create_block_mask

    B, T = doc_ids.shape

    def mask_mod(b, h, qi, ki):
        return (ki <= qi) & (doc_ids[b, ki] == doc_ids[b, qi])

    return create_block_mask(mask_mod, B, None, T, T, device=doc_ids.device)


def causal_mask(T: int, S: int, offset: int, window: int, device) -> torch.Tensor:
    """[T, S] bool, True = may attend: query t sits at position offset + t, key s at s; keys
    after the query are hidden, and with a window those window or more positions before it
    (attention.py:160-169)."""
    qpos = torch.arange(T, device=device)[:, None] + offset
    kpos = torch.arange(S, device=device)[None, :]
    mask = kpos <= qpos
    if window:
        mask &= qpos - kpos < window
    return mask


def _is_block_mask(m) -> bool:
    """A FlexAttention BlockMask (anything but a tensor) in place of the bool same_doc mask."""
    return m is not None and not isinstance(m, torch.Tensor)


_DOC_STARTS: dict = {}   # the last mask's doc starts: one mask serves every layer of a pass


def _doc_starts(same_doc, B: int, T: int) -> torch.Tensor | None:
    """The reference's document mask (transformer.py:271-275: [B or 1, 1, T, T] bool, True
    where query and key are in one document) as each query's first visible key, [B, T]
    int32, for forge_attn_prefill_docs. None where it is not such a mask, or where a query's
    visible keys (mask and causal) are not one run ending at the query itself, i.e. its
    document is not a contiguous run of positions."""
    m = same_doc
    if not (isinstance(m, torch.Tensor) and m.dtype == torch.bool and m.is_cuda and m.dim() == 4
            and m.shape[1] == 1 and tuple(m.shape[2:]) == (T, T) and m.shape[0] in (1, B)):
        return None
    # inference tensors keep no version counter, so a mask made under inference_mode is
    # read again at every layer rather than trusted unchanged
    cached = not m.is_inference()
    hit = _DOC_STARTS.get("last") if cached else None
    if hit is not None and hit[0]() is m and hit[1] == (m._version, B):
        return hit[2]
    vis = m[:, 0] & torch.ones(T, T, dtype=torch.bool, device=m.device).tril()
    start = vis.to(torch.int32).argmax(-1)                  # the first visible key
    pos = torch.arange(T, device=m.device)
    run = (vis.sum(-1) == pos - start + 1).all() & vis.diagonal(dim1=-2, dim2=-1).all()
    run &= (start[:, 1:] >= start[:, :-1]).all()
    res = start.to(torch.int32).expand(B, T).contiguous() if bool(run) else None
    if cached:
        _DOC_STARTS["last"] = (weakref.ref(m), (m._version, B), res)
    return res


def _hip_ready(device: torch.device, dtype: torch.dtype) -> None:
    """First use per (device, dtype): the library must load and pass its self-check."""
    key = (device.type, device.index, dtype)
    if key not in _checked:
        from .selfcheck import self_check

        self_check(device, dtype)   # raises on failure
        _checked[key] = True


class _FusedQKV:
    """The concatenated q/k/v projection weights of one set of projection Parameters."""

    builds = 0   # buffers built so far in this process (tests check that tied layers share one)

    def __init__(self, owner, ids, state, w, b):
        self.owner = weakref.ref(owner)
        self.ids, self.state, self.w, self.b = ids, state, w, b


# keyed by id() of the q_proj weight Parameter (tensors compare elementwise, so they cannot be
# dict keys by value): one buffer per set of Parameters, whichever modules hold them; the
# entry is dropped when that Parameter is collected
_FUSED_QKV: dict[int, _FusedQKV] = {}


def fused_qkv_entry(weight: torch.Tensor) -> "_FusedQKV | None":
    e = _FUSED_QKV.get(id(weight))
    return e if e is not None and e.owner() is weight else None


class Attention(nn.Module):
    def __init__(self, cfg: ModelConfig, layer_idx: int):
        super().__init__()
        spec = cfg.attn_spec(layer_idx)
        self.layer_idx = layer_idx
        self.kind = spec.kind
        self.n_heads, self.n_kv, self.hd = cfg.n_heads, spec.kv_heads, spec.head_dim
        self.window = spec.window
        self.scale = cfg.attn_scale or 1.0 / math.sqrt(self.hd)
        self.eps = cfg.norm_eps
        self.use_rope = cfg.pos_type == "rope"
        self.partial_rope = bool(cfg.rope_dim) and cfg.rope_dim < self.hd
        qkv_bias = cfg.bias or cfg.qkv_bias
        self.q_proj = nn.Linear(cfg.d_model, self.n_heads * self.hd, bias=qkv_bias)
        self.k_proj = nn.Linear(cfg.d_model, self.n_kv * self.hd, bias=qkv_bias)
        self.v_proj = None if spec.v_from_k else nn.Linear(cfg.d_model, self.n_kv * self.hd, bias=qkv_bias)
        self.o_proj = nn.Linear(self.n_heads * self.hd, cfg.d_model, bias=cfg.bias)
        self.q_norm = RMSNorm(self.hd, cfg.norm_eps) if cfg.qk_norm else None
        self.k_norm = RMSNorm(self.hd, cfg.norm_eps) if cfg.qk_norm else None
        self.v_norm = cfg.v_norm
        # the host's Tap type when running inside Sleuth, so its analyzer finds these
        self.tap_q = make_tap()
        self.tap_k = make_tap()
        self.tap_pattern = make_tap()
        self.tap_z = make_tap()
        self.last_path = ""   # "hip-decode" | "hip-prefill" | "torch" (for tests and stats)

    # ------------------------------------------------------------------ projections
    def _qkv_fused(self, x: torch.Tensor) -> torch.Tensor | None:
        """q_proj, k_proj and v_proj (attention.py:106-108) as one GEMM during GPU inference.

        The weights are concatenated once into a [(H + 2K)·hd, d] buffer and the projections'
        weights (and biases) become views of it, so no second copy is kept. The buffer
        belongs to the Parameters, not to this module: modules that share their projection
        Parameters (tied / looped layers, reference transformer.py:215-228) find the same
        buffer and never rebuild it for each other. It is rebuilt when a weight is replaced,
        moved or modified in place (its storage, dtype or version changes), but never while
        a graph is being captured (the captured GEMM would read a buffer a later rebuild
        frees): then the separate projections run. Returns None where they run: on the
        CPU, with autograd, and whenever a projection is not a plain nn.Linear or has hooks
        (adapters, quantised layers and forward hooks see the same calls as in the reference)."""
        if not x.is_cuda or torch.is_grad_enabled() or hip_disabled():
            return None
        mods = [self.q_proj, self.k_proj] + ([self.v_proj] if self.v_proj is not None else [])
        if any(type(m) is not nn.Linear or m._forward_hooks or m._forward_pre_hooks for m in mods):
            return None
        if nn.modules.module._global_forward_hooks or nn.modules.module._global_forward_pre_hooks:
            return None
        params = tuple(t for m in mods for t in (m.weight, m.bias) if t is not None)
        ids = tuple(id(t) for t in params)
        state = tuple((t.data_ptr(), t._version, t.dtype, t.device) for t in params)
        entry = fused_qkv_entry(mods[0].weight)
        if entry is not None and entry.ids == ids and entry.state == state:
            return F.linear(x, entry.w, entry.b)
        if entry is not None and entry.ids != ids:
            return None   # the q weight is tied to another module with different k/v: no fusion
        if torch.cuda.is_current_stream_capturing():
            return None
        if any(m.weight.dtype != x.dtype or m.weight.device != x.device for m in mods):
            return None
        if len({m.bias is None for m in mods}) > 1:
            return None
        with torch.inference_mode(False):  # ordinary tensors, also under inference_mode
            w = torch.cat([m.weight.detach() for m in mods], 0)
            b = torch.cat([m.bias.detach() for m in mods], 0) if mods[0].bias is not None else None
            off = 0
            for m in mods:
                n = m.weight.shape[0]
                m.weight.data = w[off:off + n]
                if b is not None:
                    m.bias.data = b[off:off + n]
                off += n
        state = tuple((t.data_ptr(), t._version, t.dtype, t.device) for t in params)
        key = id(mods[0].weight)
        if key not in _FUSED_QKV:
            weakref.finalize(mods[0].weight, _FUSED_QKV.pop, key, None)
        _FUSED_QKV[key] = _FusedQKV(mods[0].weight, ids, state, w, b)
        _FusedQKV.builds += 1
        return F.linear(x, w, b)

    # ------------------------------------------------------------------ dispatch
    def _use_hip(self, q: torch.Tensor, cache, same_doc) -> tuple[bool, torch.Tensor | None]:
        """(take the HIP path, the document starts of a document mask or None)"""
        if not q.is_cuda or hip_disabled():
            return False, None
        if torch.is_grad_enabled() and q.requires_grad:
            return False, None
        if tap_active(self.tap_pattern):
            return False, None
        if not hip_shape_ok(q.dtype, self.hd):
            return False, None
        if cache is not None and cache.k[self.layer_idx].dtype != q.dtype:
            return False, None   # the reference's SDPA needs q and the cache in one dtype too
        docs = None
        if same_doc is not None:
            from . import ops

            if cache is not None or q.shape[2] <= DECODE_MAX_T or not ops.prefill_supported(q) or \
                    torch.cuda.is_current_stream_capturing():
                return False, None
            docs = _doc_starts(same_doc, q.shape[0], q.shape[2])
            if docs is None:
                return False, None
        _hip_ready(q.device, q.dtype)
        return True, docs

    def forward(self, x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, cache=None,
                same_doc=None) -> torch.Tensor:
        B, T, _ = x.shape
        H, K, hd = self.n_heads, self.n_kv, self.hd
        y = self._qkv_fused(x)
        if y is not None:  # one GEMM; q, k, v are strided views of its rows
            q = y[..., :H * hd].view(B, T, H, hd).transpose(1, 2)
            k = y[..., H * hd:(H + K) * hd].view(B, T, K, hd).transpose(1, 2)
            v = k if self.v_proj is None else y[..., (H + K) * hd:].view(B, T, K, hd).transpose(1, 2)
        else:
            q = self.q_proj(x).view(B, T, H, hd).transpose(1, 2)  # [B, H, T, hd]
            k = self.k_proj(x).view(B, T, K, hd).transpose(1, 2)  # [B, K, T, hd]
            v = k if self.v_proj is None else self.v_proj(x).view(B, T, K, hd).transpose(1, 2)
        hip, docs = self._use_hip(q, cache, same_doc)
        if hip:
            y = self._forward_hip(q, k, v, cos, sin, cache, docs)
        else:
            y = self._forward_torch(q, k, v, cos, sin, cache, same_doc).transpose(1, 2)
            self.last_path = "torch"
        y = self.tap_z(y)                # [B, T, H, hd] per-head outputs
        return self.o_proj(y.reshape(B, T, self.n_heads * self.hd))

    # ------------------------------------------------------------------ HIP path
    def _forward_hip(self, q, k, v, cos, sin, cache, docs=None) -> torch.Tensor:
        from . import ops

        B, H, T, hd = q.shape
        qn, kn = self.q_norm is not None, self.k_norm is not None
        rc, rs = (cos, sin) if self.use_rope else (None, None)
        if rc is not None and rc.dtype != torch.float32:
            rc, rs = rc.float(), rs.float()
        qw = self.q_norm.weight_f32() if qn else None
        kw = self.k_norm.weight_f32() if kn else None
        if self.partial_rope:
            # RoPE over the first rope_dim channels only: the reference keeps this off its fused
            # kernel (attention.py:109) and runs RMSNorm then apply_rope, each rounded to the
            # dtype (attention.py:120-126, rope.py:46-55); so does this path, and the kernels
            # take q and k as they are.
            if qn:
                q, k = self.q_norm(q), self.k_norm(k)
            if self.use_rope:
                c, s_ = (cos[:, None], sin[:, None]) if cos.dim() == 3 else (cos, sin)
                q, k = apply_rope(q, c, s_), apply_rope(k, c, s_)
            q, k = self.tap_q(q), self.tap_k(k)
            q_args = dict(norm_q=False, cos=None, sin=None)
            k_args = dict(norm_k=False, cos=None, sin=None)
        elif tap_active(self.tap_q) or tap_active(self.tap_k):
            # Listeners see (and may replace) q and k after RoPE: materialise them.
            if qn or rc is not None:
                q = ops.head_norm_rope(q, qw, self.eps if qn else 0.0, rc, rs, qn)
                k = ops.head_norm_rope(k, kw, self.eps if kn else 0.0, rc, rs, kn)
            q, k = self.tap_q(q), self.tap_k(k)
            q_args = dict(norm_q=False, cos=None, sin=None)
            k_args = dict(norm_k=False, cos=None, sin=None)
        else:
            q_args = dict(q_weight=qw, eps=self.eps, norm_q=qn, cos=rc, sin=rs)
            k_args = dict(k_weight=kw, eps=self.eps, norm_k=kn, cos=rc, sin=rs)
        norm_v = bool(self.v_norm)
        if q.stride(-1) != 1:
            q = q.contiguous()

        if cache is None:
            kc = torch.empty(B, self.n_kv, T, hd, device=q.device, dtype=q.dtype)
            vc = torch.empty_like(kc)
            pos_kw, max_kv, offset, chunk = dict(pos=0), T, 0, 0
        else:
            kc, vc = cache.k[self.layer_idx], cache.v[self.layer_idx]
            if getattr(cache, "static", False):
                # StaticKVCache (kv_cache.py:73-138): positions pos_t + arange(T) on the device
                pos_kw, max_kv, offset = dict(pos_dev=cache.positions), min(cache.length, cache.max_len), None
            else:
                # the reference's KVCache has one host `pos`; per-row lengths (`ragged`,
                # `seq_lens`) are this package's extension and read only where present
                rows = getattr(cache, "seq_lens", None) if getattr(cache, "ragged", False) else None
                top = max(cache.seq_lens_host) if rows is not None else cache.pos
                if top + T > cache.max_len:   # KVCache.update's check (kv_cache.py:56-57)
                    raise ValueError(f"KV cache full ({cache.max_len} tokens)")
                if rows is not None:
                    pos_kw, max_kv, offset = dict(row_pos=rows), top + T, None
                else:
                    pos_kw, max_kv, offset = dict(pos=cache.pos), cache.pos + T, cache.pos
            # from the cache's capacity and T = 1: every step of this layer, decode or verify,
            # splits its rows at the same keys
            chunk = ops.decode_chunk(q.dtype, B, 1, H, self.n_kv, hd, cache.max_len, self.window,
                                     uniform="row_pos" not in pos_kw)

        if T > DECODE_MAX_T and offset is not None and ops.prefill_supported(q) and \
                (q_args["cos"] is None or q_args["cos"].dim() == 2):
            ops.kv_append(k, v, kc, vc, norm_v=norm_v, **pos_kw, **k_args)
            self.last_path = "hip-prefill" if docs is None else "hip-prefill-docs"
            return ops.attn_prefill(q, kc, vc, scale=self.scale, offset=offset, window=self.window,
                                    doc_start=docs, check_doc_start=False, **q_args)
        if docs is not None:
            raise RuntimeError("a document mask needs the prefill path (no cache, T > 16)")
        # the cache write and the attention in one call (one launch where the shape allows);
        # q and k share the RoPE tables and the eps (both come from this module's config)
        self.last_path = "hip-decode"
        return ops.attn_decode_append(q, k, v, kc, vc, scale=self.scale, max_kv_len=max_kv, window=self.window,
                                      chunk=chunk, norm_v=norm_v, k_weight=k_args.get("k_weight"),
                                      norm_k=k_args["norm_k"], **pos_kw, **q_args)

    # ------------------------------------------------------------------ torch path
    def _forward_torch(self, q, k, v, cos, sin, cache, same_doc) -> torch.Tensor:
        """The reference's eager path (attention.py:120-153), returns [B, H, T, hd]."""
        if self.q_norm is not None:
            q, k = self.q_norm(q), self.k_norm(k)
        if self.v_norm:
            v = F.rms_norm(v.float(), (self.hd,), None, self.eps).to(v.dtype)
        if self.use_rope:
            q, k = apply_rope(q, cos, sin), apply_rope(k, cos, sin)
        q, k = self.tap_q(q), self.tap_k(k)
        if cache is not None and getattr(cache, "ragged", False) and not getattr(cache, "static", False):
            if _is_block_mask(same_doc):
                raise NotImplementedError(_FLEX_LIMITS)
            return self._ragged_torch(q, k, v, cache, same_doc)
        if cache is not None:
            k, v = cache.update(self.layer_idx, k, v)
        S = k.shape[2]
        offset = S - q.shape[2]
        if getattr(cache, "static", False) and not tap_active(self.tap_pattern):
            kwargs = {"enable_gqa": True} if self.n_kv != self.n_heads else {}
            return F.scaled_dot_product_attention(q, k, v, attn_mask=cache.attn_mask(self.window),
                                                  scale=self.scale, **kwargs)
        if _is_block_mask(same_doc):
            # FlexAttention document mask (doc_block_mask, attention.py:54-64): the reference
            # hands it to flex_attention and allows no pattern tap, window or cached prefix
            # (attention.py:142-149)
            if tap_active(self.tap_pattern) or self.window or offset:
                raise NotImplementedError(_FLEX_LIMITS)
            from torch.nn.attention.flex_attention import flex_attention

            return flex_attention(q, k, v, block_mask=same_doc, scale=self.scale,
                                  enable_gqa=self.n_kv != self.n_heads)
        if tap_active(self.tap_pattern):
            return self._explicit(q, k, v, offset, same_doc)
        return self._fused(q, k, v, offset, same_doc)

    def _ragged_torch(self, q, k, v, cache, same_doc):
        """Per-row torch attention for a cache with per-row lengths."""
        T = q.shape[2]
        lens = list(cache.seq_lens_host)
        cache.update(self.layer_idx, k, v)
        out = []
        for b, L in enumerate(lens):
            kb = cache.k[self.layer_idx][b:b + 1, :, :L + T]
            vb = cache.v[self.layer_idx][b:b + 1, :, :L + T]
            fn = self._explicit if tap_active(self.tap_pattern) else self._fused
            out.append(fn(q[b:b + 1], kb, vb, L, same_doc))
        return torch.cat(out, 0)

    def _mask(self, T: int, S: int, offset: int, device) -> torch.Tensor:
        """[T, S] bool, True = may attend (attention.py:160-169)."""
        return causal_mask(T, S, offset, self.window, device)

    def _fused(self, q, k, v, offset, same_doc=None):
        T, S = q.shape[2], k.shape[2]
        kwargs = {"scale": self.scale}
        if self.n_kv != self.n_heads:
            if same_doc is None:
                kwargs["enable_gqa"] = True
            else:
                k = k.repeat_interleave(self.n_heads // self.n_kv, dim=1)
                v = v.repeat_interleave(self.n_heads // self.n_kv, dim=1)
        windowed = self.window and S > self.window
        if same_doc is not None:
            mask = self._mask(T, S, offset, q.device) & same_doc
            return F.scaled_dot_product_attention(q, k, v, attn_mask=mask, **kwargs)
        if offset == 0 and not windowed:
            return F.scaled_dot_product_attention(q, k, v, is_causal=True, **kwargs)
        if T == 1 and not windowed:
            return F.scaled_dot_product_attention(q, k, v, **kwargs)
        mask = self._mask(T, S, offset, q.device)
        return F.scaled_dot_product_attention(q, k, v, attn_mask=mask, **kwargs)

    def _explicit(self, q, k, v, offset, same_doc=None):
        T, S = q.shape[2], k.shape[2]
        rep = self.n_heads // self.n_kv
        k = k.repeat_interleave(rep, dim=1)
        v = v.repeat_interleave(rep, dim=1)
        scores = (q.float() @ k.float().transpose(-2, -1)) * self.scale
        mask = self._mask(T, S, offset, q.device)
        if same_doc is not None:
            mask = mask & same_doc
        scores = scores.masked_fill(~mask, float("-inf"))
        probs = self.tap_pattern(scores.softmax(dim=-1))
        return (probs @ v.float()).to(q.dtype)
