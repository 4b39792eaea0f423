"""CPU restatement of Sleuth FORGE's attention hot path (torch on the CPU).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg, never by the product. Each function cites the reference code it
restates (paths relative to the reference's repository root, sleuth/forge/...).

Parity pins (tests/test_oracle.py), chosen so that a plausible slip fails one of them:
  rope_tables / apply_rope   closed form cos(p * theta^(-2i/d)) in float64; the rotation
                             equals multiplication by e^{i angle} of x[:d/2] + i x[d/2:];
                             scores depend only on the position difference
  rms_norm / head_norm_rope  closed form in float64; unit RMS; one rounding
  attention_mask             the reference's own golden lists (tests/test_cuda_graph.py:59,61)
  sdpa / explicit_attention  float64 brute force with explicit loops and the GQA map
                             kv = h // (H/K) (brute_attention); single-key and equal-key
                             closed forms; causality
  document_mask / sdpa with  the loops restricted to the query's document; a packed window
    same_doc                 equals each document attended alone
  gated_attention            float64 loops from the definition (partial RoPE on the first
                             n_rot channels, q | gate split per head, sigmoid gate, causal
                             at an offset), tests/test_oracle.py
  KVCache / StaticKVCache    chunked prefill + decode == full forward
                             (tests/test_model.py:61-69), static step == normal step
                             (tests/test_cuda_graph.py:24-52, 81-95)
Every function here has at least one such check; none is "parity unpinned".
"""

from __future__ import annotations

import math

import torch
import torch.nn.functional as F


# ----------------------------------------------------------------------------- RoPE
def rope_tables(head_dim: int, max_len: int, theta: float,
                freq_factors: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """cos/sin [max_len, head_dim] in float32 (rope.py:21-38): inv_freq =
    1 / theta^(arange(0, d, 2)/d), angles = outer(pos, inv_freq), halves duplicated."""
    inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim))
    if freq_factors is not None:
        if freq_factors.numel() != head_dim // 2:
            raise ValueError(f"{freq_factors.numel()} RoPE frequency factors for head_dim {head_dim}")
        inv_freq = inv_freq / freq_factors.float().cpu()
    pos = torch.arange(max_len, dtype=torch.float32)
    angles = torch.outer(pos, inv_freq)
    angles = torch.cat([angles, angles], dim=-1)
    return angles.cos(), angles.sin()


def rotate_half(x: torch.Tensor) -> torch.Tensor:
    """(a, b) -> (-b, a) on the two halves of the last dim (rope.py:41-43)."""
    x1, x2 = x.chunk(2, dim=-1)
    return torch.cat([-x2, x1], dim=-1)


def apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """x·cos + rotate_half(x)·sin in fp32, rounded to x.dtype (rope.py:46-55); partial
    RoPE when the tables are narrower than x (rope.py:52-54)."""
    rd = cos.shape[-1]
    if rd < x.shape[-1]:
        return torch.cat([apply_rope(x[..., :rd], cos, sin), x[..., rd:]], dim=-1)
    return (x.float() * cos + rotate_half(x.float()) * sin).to(x.dtype)


# ----------------------------------------------------------------------------- norms
def rms_norm(x: torch.Tensor, weight: torch.Tensor | None, eps: float) -> torch.Tensor:
    """RMSNorm.forward (norm.py:50): F.rms_norm in fp32 (gain in fp32), cast back."""
    w = None if weight is None else weight.float()
    return F.rms_norm(x.float(), (x.shape[-1],), w, eps).to(x.dtype)


def head_norm_rope(x: torch.Tensor, weight: torch.Tensor | None = None, eps: float = 1e-6,
                   cos: torch.Tensor | None = None, sin: torch.Tensor | None = None,
                   norm: bool = True) -> torch.Tensor:
    """fused_ops.head_norm_rope / _head_kernel (fused_ops.py:53-85, 101-121): per-head
    RMSNorm (optional gain) then NEOX RoPE, all in fp32, ONE rounding to x.dtype.
    cos/sin: [T, D] or [B, T, D] (per-row positions) -- broadcast over heads."""
    y = x.float()
    if norm:
        w = None if weight is None else weight.float()
        y = F.rms_norm(y, (y.shape[-1],), w, eps)
    if cos is not None:
        c, s = cos.float(), sin.float()
        if c.dim() == 3:  # [B, T, D] -> [B, 1, T, D]
            c, s = c[:, None], s[:, None]
        y = y * c + rotate_half(y) * s
    return y.to(x.dtype)


def eager_norm_rope(x, weight, eps, cos, sin, norm=True, rope=True):
    """The eager GPU/CPU path of Attention.forward (attention.py:120-126): RMSNorm rounds
    to x.dtype, then RoPE rounds again (two roundings)."""
    if norm:
        x = rms_norm(x, weight, eps)
    if rope:
        x = apply_rope(x, cos, sin)
    return x


# ----------------------------------------------------------------------------- masks
def attention_mask(T: int, S: int, offset: int, window: int = 0) -> torch.Tensor:
    """Attention._mask (attention.py:160-169): [T, S] bool, True = may attend; query i is
    at position offset + i and sees keys kpos <= qpos, and qpos - kpos < window."""
    qpos = torch.arange(T)[:, None] + offset
    kpos = torch.arange(S)[None, :]
    mask = kpos <= qpos
    if window:
        mask &= qpos - kpos < window
    return mask


def document_mask(doc_ids: torch.Tensor) -> torch.Tensor:
    """Transformer.forward's document mask (transformer.py:271-275): doc_ids [B, T] ->
    same_doc [B, 1, T, T] bool, True where query and key belong to one document."""
    return (doc_ids[:, :, None] == doc_ids[:, None, :])[:, None]


# ----------------------------------------------------------------------------- attention
def sdpa(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, offset: int, window: int,
         scale: float, same_doc: torch.Tensor | None = None) -> torch.Tensor:
    """Attention._fused (attention.py:171-193) with enable_gqa: q [B,H,T,hd], k/v
    [B,K,S,hd] -> [B,H,T,hd]. Same dispatch: with a document mask same_doc [B,1,T,S],
    K/V heads repeated and _mask & same_doc (attention.py:177-186); else is_causal when
    offset == 0 and not windowed, no mask when T == 1 and not windowed, else the boolean
    _mask."""
    T, S = q.shape[2], k.shape[2]
    kw = {"scale": scale}
    if same_doc is not None:
        rep = q.shape[1] // k.shape[1]
        k, v = k.repeat_interleave(rep, dim=1), v.repeat_interleave(rep, dim=1)
        mask = attention_mask(T, S, offset, window).to(q.device) & same_doc
        return F.scaled_dot_product_attention(q, k, v, attn_mask=mask, **kw)
    if k.shape[1] != q.shape[1]:
        kw["enable_gqa"] = True
    windowed = bool(window) and S > window
    if offset == 0 and not windowed:
        return F.scaled_dot_product_attention(q, k, v, is_causal=True, **kw)
    if T == 1 and not windowed:
        return F.scaled_dot_product_attention(q, k, v, **kw)
    mask = attention_mask(T, S, offset, window).to(q.device)
    return F.scaled_dot_product_attention(q, k, v, attn_mask=mask, **kw)


def explicit_attention(q, k, v, offset: int, window: int, scale: float,
                       return_probs: bool = False):
    """Attention._explicit (attention.py:195-206): fp32 scores, repeat_interleave GQA,
    masked softmax, probs @ v, cast back."""
    T, S = q.shape[2], k.shape[2]
    rep = q.shape[1] // k.shape[1]
    kk = k.repeat_interleave(rep, dim=1)
    vv = v.repeat_interleave(rep, dim=1)
    scores = (q.float() @ kk.float().transpose(-2, -1)) * scale
    mask = attention_mask(T, S, offset, window).to(q.device)
    scores = scores.masked_fill(~mask, float("-inf"))
    probs = scores.softmax(dim=-1)
    out = (probs @ vv.float()).to(q.dtype)
    return (out, probs) if return_probs else out


def brute_attention(q, k, v, offset: int, window: int, scale: float,
                    doc_ids: torch.Tensor | None = None) -> torch.Tensor:
    """Independent float64 restatement with explicit loops (small inputs only): for each
    batch row b, head h (KV head h // (H/K)) and query i at position offset + i, a
    softmax over the keys j with j <= pos and pos - j < window (and, with doc_ids [B, S]
    of the key positions, doc_ids[b, j] == doc_ids[b, pos]). Returns float64."""
    B, H, T, D = q.shape
    K, S = k.shape[1], k.shape[2]
    G = H // K
    qd, kd, vd = q.double(), k.double(), v.double()
    out = torch.zeros(B, H, T, D, dtype=torch.float64)
    for b in range(B):
        for h in range(H):
            kvh = h // G
            for i in range(T):
                pos = offset + i
                js = [j for j in range(S) if j <= pos and (not window or pos - j < window)
                      and (doc_ids is None or int(doc_ids[b, j]) == int(doc_ids[b, pos]))]
                s = [float((qd[b, h, i] * kd[b, kvh, j]).sum()) * scale for j in js]
                mx = max(s)
                w = [math.exp(x - mx) for x in s]
                tot = sum(w)
                acc = torch.zeros(D, dtype=torch.float64)
                for wj, j in zip(w, js):
                    acc += (wj / tot) * vd[b, kvh, j]
                out[b, h, i] = acc
    return out


def ragged_decode(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                  kv_lens: list[int], window: int, scale: float) -> torch.Tensor:
    """Per-row decode/verify for a batch whose rows hold different numbers of keys: row
    b's T queries are its last T positions (kv_lens[b] - T ..) and attend over the
    row's own prefix with the reference's mask (one SDPA per row, attention.py:171-193).
    q [B,H,T,hd], caches [B,K,max_len,hd] -> [B,H,T,hd]."""
    B, H, T, D = q.shape
    out = torch.empty_like(q)
    for b in range(B):
        L = int(kv_lens[b])
        out[b:b + 1] = sdpa(q[b:b + 1], k_cache[b:b + 1, :, :L], v_cache[b:b + 1, :, :L],
                            L - T, window, scale)
    return out


def drafter_attention(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                      n_past: int, window: int, scale: float = 1.0) -> torch.Tensor:
    """The MTP drafter's attention onto the target's cache (infer/mtp.py:73-92,
    AssistantLayer.forward with mask=None): the first n_past cached keys, and for a
    sliding layer with n_past > window - 1 only the last window - 1 of them (mtp.py:84-86),
    then SDPA with scale 1.0 and GQA (mtp.py:87-88). q [B,H,1,hd] -> [B,H,1,hd]."""
    k, v = k_cache[:, :, :n_past], v_cache[:, :, :n_past]
    if window and n_past > window - 1:
        k, v = k[:, :, n_past - (window - 1):], v[:, :, n_past - (window - 1):]
    kw = {"scale": scale}
    if k.shape[1] != q.shape[1]:
        kw["enable_gqa"] = True
    return F.scaled_dot_product_attention(q, k.to(q.dtype), v.to(q.dtype), **kw)


# ----------------------------------------------------------------------------- caches
class KVCache:
    """kv_cache.py:25-70: per-layer k/v [B, K, max_len, hd] zeros, one shared `pos`;
    update() slice-assigns at pos and returns the views [:, :, :pos+T]."""

    def __init__(self, shapes, batch, max_len, device="cpu", dtype=torch.float32):
        self.k = [torch.zeros(batch, kv, max_len, hd, device=device, dtype=dtype) for kv, hd in shapes]
        self.v = [torch.zeros_like(k) for k in self.k]
        self.max_len = max_len
        self.pos = 0
        self.static = False

    def update(self, layer, k_new, v_new):
        T = k_new.shape[2]
        end = self.pos + T
        if end > self.max_len:
            raise ValueError(f"KV cache full ({self.max_len} tokens)")
        self.k[layer][:, :, self.pos:end] = k_new.to(self.k[layer].dtype)
        self.v[layer][:, :, self.pos:end] = v_new.to(self.v[layer].dtype)
        return self.k[layer][:, :, :end], self.v[layer][:, :, :end]

    def advance(self, n):
        self.pos += n


class StaticKVCache(KVCache):
    """kv_cache.py:73-138: positions = pos_t + arange(tokens_per_step), index_copy_ at
    them, fixed [:, :, :length] views and the [1,1,T,length] bool mask."""

    def __init__(self, shapes, batch, max_len, device="cpu", dtype=torch.float32, tokens_per_step=1):
        super().__init__(shapes, batch, max_len, device, dtype)
        self.length = max_len
        self.pos_t = torch.zeros(1, dtype=torch.long, device=device)
        self.tokens_per_step = tokens_per_step

    @property
    def positions(self):
        return self.pos_t + torch.arange(self.tokens_per_step, device=self.pos_t.device)

    def update(self, layer, k_new, v_new):
        if not self.static:
            return super().update(layer, k_new, v_new)
        pos = self.positions
        self.k[layer].index_copy_(2, pos, k_new.to(self.k[layer].dtype))
        self.v[layer].index_copy_(2, pos, v_new.to(self.v[layer].dtype))
        return self.k[layer][:, :, :self.length], self.v[layer][:, :, :self.length]

    def attn_mask(self, window=0):
        kpos = torch.arange(self.length, device=self.pos_t.device)[None, :]
        qpos = self.positions[:, None]
        mask = kpos <= qpos
        if window:
            mask = mask & (qpos - kpos < window)
        return mask[None, None]

    def advance(self, n):
        if not self.static:
            super().advance(n)


# ----------------------------------------------------------------------------- one layer
def attention_forward(q, k, v, *, cos, sin, scale, eps=1e-6, q_weight=None, k_weight=None,
                      qk_norm=True, v_norm=False, use_rope=True, window=0, cache=None, layer=0,
                      fused_norm=True, same_doc=None):
    """Attention.forward after the projections (attention.py:109-153): q [B,H,T,hd],
    k/v [B,K,T,hd] raw projections -> y [B,H,T,hd]. fused_norm=True follows the GPU
    inference path (head_norm_rope, one rounding, attention.py:109-119), False the eager
    path (attention.py:120-126). The cache (KVCache / StaticKVCache above) is updated."""
    if fused_norm:
        if v_norm:
            v = head_norm_rope(v, None, eps)
        if qk_norm or use_rope:
            rc, rs = (cos, sin) if use_rope else (None, None)
            q = head_norm_rope(q, q_weight if qk_norm else None, eps if qk_norm else 0.0, rc, rs, qk_norm)
            k = head_norm_rope(k, k_weight if qk_norm else None, eps if qk_norm else 0.0, rc, rs, qk_norm)
    else:
        if qk_norm:
            q, k = rms_norm(q, q_weight, eps), rms_norm(k, k_weight, eps)
        if v_norm:
            v = F.rms_norm(v.float(), (v.shape[-1],), None, eps).to(v.dtype)
        if use_rope:
            q, k = apply_rope(q, cos, sin), apply_rope(k, cos, sin)
    if cache is not None:
        k, v = cache.update(layer, k, v)
    S, T = k.shape[2], q.shape[2]
    if getattr(cache, "static", False):
        kw = {"enable_gqa": True} if k.shape[1] != q.shape[1] else {}
        return F.scaled_dot_product_attention(q, k, v, attn_mask=cache.attn_mask(window), scale=scale, **kw)
    return sdpa(q, k, v, S - T, window, scale, same_doc)


# ----------------------------------------------------------------------------- gated attention
def gated_attention(qg, k, v, *, cos, sin, n_rot, q_weight, k_weight, eps, k_past=None, v_past=None):
    """Qwen3.5 gated attention after the projections (formats/qwen35.py:194-214).
    qg [B,T,H,2hd]: each head's q_proj output as [q | gate]; k, v [B,T,K,hd] raw projections;
    k_past/v_past [B,K,offset,hd]: keys and values already stored (normalised and rotated).
    q and k: RMSNorm with gain (rounded to the dtype), NEOX RoPE on the first n_rot channels
    (rounded); causal SDPA of the T queries at positions offset.. over past + new keys (no
    mask for one token), GQA. Returns (y * sigmoid(gate) [B,T,H*hd], new keys, new values),
    the new keys/values [B,K,T,hd] as the cache stores them."""
    B, T, H, two_hd = qg.shape
    hd = two_hd // 2
    q, gate = qg[..., :hd], qg[..., hd:]
    q = rms_norm(q, q_weight, eps).transpose(1, 2)
    kn = rms_norm(k, k_weight, eps).transpose(1, 2)
    vn = v.transpose(1, 2)
    q, kn = apply_rope(q, cos[..., :n_rot], sin[..., :n_rot]), apply_rope(kn, cos[..., :n_rot], sin[..., :n_rot])
    kk = kn if k_past is None else torch.cat([k_past.to(kn.dtype), kn], 2)
    vv = vn if v_past is None else torch.cat([v_past.to(vn.dtype), vn], 2)
    offset = kk.shape[2] - T
    mask = None if T == 1 else attention_mask(T, kk.shape[2], offset).to(q.device)
    kw = {"enable_gqa": True} if kk.shape[1] != H else {}
    y = F.scaled_dot_product_attention(q, kk, vv, attn_mask=mask, **kw)
    y = y.transpose(1, 2).reshape(B, T, H * hd)
    return y * torch.sigmoid(gate.reshape(B, T, -1)), kn, vn
