"""Torch-tensor front ends of the HIP kernels (C ABI in include/forge_attn.h).

These functions only check shapes on the host, pick pointers/strides and launch on
torch's current stream. They never compute anything themselves: if the library is not
built they raise (sleuth_amd._lib.ForgeError).

Layouts (reference names): q [B,H,T,D] (any strides, last dim contiguous: the transposed
q_proj view, attention.py:106), k/v [B,K,T,D], caches [B,K,max_len,D] (kv_cache.py:31),
outputs [B,T,H,D] (attention.py:155).
"""

from __future__ import annotations

import torch

from . import _lib
from ._lib import BF16, F16, F32, NORM_QK, NORM_V, ROPE, WS_ZEROED, check, lib

_DTYPES = {torch.float32: F32, torch.bfloat16: BF16, torch.float16: F16}


def dtype_code(t: torch.Tensor) -> int:
    try:
        return _DTYPES[t.dtype]
    except KeyError:
        raise TypeError(f"unsupported dtype {t.dtype} (float32, bfloat16, float16)") from None


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _need_device(*ts: torch.Tensor | None) -> torch.device:
    dev = None
    for t in ts:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise ValueError("forge kernels need tensors on the GPU")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError("all tensors must be on the same GPU")
    assert dev is not None
    return dev


def _last_dim_contiguous(t: torch.Tensor, name: str) -> None:
    if t.stride(-1) != 1:
        raise ValueError(f"{name}: the last dimension must be contiguous")


def _weight(w: torch.Tensor | None, D: int) -> torch.Tensor | None:
    if w is None:
        return None
    if w.numel() != D:
        raise ValueError(f"norm gain has {w.numel()} values for head dim {D}")
    w = w.detach()
    if w.dtype == torch.float32 and w.is_contiguous():
        return w
    return w.to(torch.float32).contiguous()


def _rope_tables(cos, sin, B: int, T: int, D: int):
    """cos/sin [T, D] (shared positions) or [B, T, D] (per row) fp32 -> (cos, sin, s_b, s_t)."""
    if cos is None and sin is None:
        return None, None, 0, 0
    if cos is None or sin is None:
        raise ValueError("cos and sin must both be given")
    if cos.shape != sin.shape or cos.shape[-1] != D or cos.shape[-2] != T or cos.dim() not in (2, 3):
        raise ValueError(f"cos/sin must be [T, D] or [B, T, D] with T={T}, D={D}; got {tuple(cos.shape)}")
    if cos.dim() == 3 and cos.shape[0] not in (1, B):
        raise ValueError("per-row cos/sin need batch size B")
    cos = cos.to(torch.float32)
    sin = sin.to(torch.float32)
    if cos.stride(-1) != 1:
        cos = cos.contiguous()
    if sin.stride() != cos.stride():
        sin = sin.contiguous()
        cos = cos.contiguous()
    s_b = cos.stride(0) if cos.dim() == 3 and cos.shape[0] == B and B > 1 else 0
    return cos, sin, s_b, cos.stride(-2)


def _positions(pos, pos_dev, row_pos, B: int, device):
    """(row_pos int32 [B] | None, pos_dev int64 [1] | None, pos0 int)."""
    if row_pos is not None:
        if row_pos.dtype != torch.int32 or row_pos.numel() != B or row_pos.device != device:
            raise ValueError("row_pos must be an int32 [B] tensor on the GPU")
        return row_pos.contiguous(), None, 0
    if pos_dev is not None:
        if pos_dev.dtype != torch.int64 or pos_dev.device != device:
            raise ValueError("pos_dev must be an int64 tensor on the GPU")
        return None, pos_dev, 0
    return None, None, int(pos or 0)


def head_norm_rope(x: torch.Tensor, weight: torch.Tensor | None = None, eps: float = 1e-6,
                   cos: torch.Tensor | None = None, sin: torch.Tensor | None = None,
                   norm: bool = True) -> torch.Tensor:
    """fused_ops.head_norm_rope (fused_ops.py:101-121): x [B,H,T,D] -> per-head RMSNorm
    (gain `weight`, if norm) then NEOX RoPE (if cos/sin), one rounding; same layout as x."""
    B, H, T, D = x.shape
    dev = _need_device(x, cos, sin)
    if x.stride(-1) != 1:
        x = x.contiguous()
    y = torch.empty_like(x)
    c, s, s_b, s_t = _rope_tables(cos, sin, B, T, D)
    w = _weight(weight, D)
    st = lib().forge_head_norm_rope(dtype_code(x), _ptr(x), _ptr(y), B, H, T, D,
                                    x.stride(0), x.stride(1), x.stride(2),
                                    y.stride(0), y.stride(1), y.stride(2),
                                    _ptr(w), float(eps), int(bool(norm)),
                                    _ptr(c), _ptr(s), s_b, s_t, _stream(dev))
    check(st, "forge_head_norm_rope")
    return y


def kv_append(k: torch.Tensor, v: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, *,
              pos: int | None = None, pos_dev: torch.Tensor | None = None,
              row_pos: torch.Tensor | None = None, k_weight: torch.Tensor | None = None,
              eps: float = 1e-6, norm_k: bool = False, norm_v: bool = False,
              cos: torch.Tensor | None = None, sin: torch.Tensor | None = None) -> None:
    """Normalise/rotate the new k (and v_norm v) and write them into the cache at
    base_b + t (KVCache.update, kv_cache.py:52-60; StaticKVCache.update 107-114)."""
    B, K, T, D = k.shape
    if v.shape != k.shape:
        raise ValueError(f"k {tuple(k.shape)} and v {tuple(v.shape)} differ")
    if k_cache.shape != v_cache.shape or k_cache.dim() != 4 or k_cache.shape[0] != B or \
            k_cache.shape[1] != K or k_cache.shape[3] != D:
        raise ValueError(f"cache {tuple(k_cache.shape)} does not fit new k {tuple(k.shape)}")
    if k_cache.stride() != v_cache.stride():
        raise ValueError("k and v caches must have the same strides")
    if k.dtype != k_cache.dtype or v.dtype != k_cache.dtype:
        k, v = k.to(k_cache.dtype), v.to(k_cache.dtype)
    dev = _need_device(k, v, k_cache, v_cache, cos, sin)
    for t, n in ((k, "k"), (v, "v"), (k_cache, "k_cache")):
        _last_dim_contiguous(t, n)
    rp, pd, p0 = _positions(pos, pos_dev, row_pos, B, dev)
    c, s, s_b, s_t = _rope_tables(cos, sin, B, T, D)
    flags = (NORM_QK if norm_k else 0) | (ROPE if c is not None else 0) | (NORM_V if norm_v else 0)
    w = _weight(k_weight, D) if norm_k else None
    st = lib().forge_kv_append(dtype_code(k_cache), B, T, K, D,
                               _ptr(k), k.stride(0), k.stride(1), k.stride(2),
                               _ptr(v), v.stride(0), v.stride(1), v.stride(2),
                               _ptr(k_cache), _ptr(v_cache), k_cache.stride(0), k_cache.stride(1),
                               k_cache.stride(2), k_cache.shape[2], _ptr(rp), _ptr(pd), p0,
                               _ptr(w), float(eps), flags, _ptr(c), _ptr(s), s_b, s_t, _stream(dev))
    check(st, "forge_kv_append")


DECODE_CHUNK_MAX_T = 16  # the longest verify step the chunk span allows for (as the C default)


def decode_chunk(dtype: torch.dtype, B: int, T: int, H: int, K: int, D: int, max_kv_len: int,
                 window: int = 0, uniform: bool = False) -> int:
    """Default split-K chunk. T does not enter (decode and verify of a model share chunk
    boundaries, so verify rows equal single-token decodes bit for bit); with a sliding window
    it is sized for the keys a row can see, window + 16, not the cache length. `uniform`:
    every row of the calls starts at one position (`pos`, or `pos_dev` on the device), so
    rows have one length and the chunk only spreads the work over the CUs
    (forge_attn_decode_chunk_uniform)."""
    span = int(max_kv_len)
    if window > 0 and window + DECODE_CHUNK_MAX_T < span:
        span = window + DECODE_CHUNK_MAX_T
    fn = lib().forge_attn_decode_chunk_uniform if uniform else lib().forge_attn_decode_chunk
    return fn(_DTYPES[dtype], B, T, H, K, D, span)


def decode_workspace_bytes(dtype: torch.dtype, B: int, T: int, H: int, K: int, D: int,
                           max_kv_len: int, chunk: int = 0) -> int:
    return lib().forge_attn_decode_workspace_bytes(_DTYPES[dtype], B, T, H, K, D, int(max_kv_len), int(chunk))


def _decode_args(q, k_cache, v_cache, scale, pos, pos_dev, row_pos, max_kv_len, window, q_weight,
                 eps, norm_q, cos, sin, chunk, out, workspace):
    """Host checks of a decode call; returns (C arguments up to `out`'s strides, out,
    device, max_kv_len, chunk)."""
    B, H, T, D = q.shape
    Bc, K, max_len, Dc = k_cache.shape
    if Bc != B or Dc != D or v_cache.shape != k_cache.shape or H % K:
        raise ValueError(f"q {tuple(q.shape)} does not fit cache {tuple(k_cache.shape)}")
    if k_cache.stride() != v_cache.stride():
        raise ValueError("k and v caches must have the same strides")
    if q.dtype != k_cache.dtype:
        raise ValueError(f"q is {q.dtype} but the cache is {k_cache.dtype}")
    dev = _need_device(q, k_cache, v_cache, cos, sin, out, workspace)
    _last_dim_contiguous(q, "q")
    _last_dim_contiguous(k_cache, "k_cache")
    rp, pd, p0 = _positions(pos, pos_dev, row_pos, B, dev)
    if max_kv_len is None:
        max_kv_len = p0 + T if (rp is None and pd is None) else max_len
    max_kv_len = max(1, min(int(max_kv_len), max_len))
    c, s, s_b, s_t = _rope_tables(cos, sin, B, T, D)
    flags = (NORM_QK if norm_q else 0) | (ROPE if c is not None else 0)
    w = _weight(q_weight, D) if norm_q else None
    if out is None:
        out = torch.empty(B, T, H, D, dtype=q.dtype, device=dev)
    elif out.shape != (B, T, H, D) or out.dtype != q.dtype:
        raise ValueError(f"out must be [B,T,H,D] = {(B, T, H, D)} {q.dtype}")
    if chunk <= 0:  # from the cache's capacity, not this call's length: stable across steps
        chunk = decode_chunk(q.dtype, B, T, H, K, D, max_len, window, uniform=rp is None)
    args = (dtype_code(q), B, T, H, K, D, _ptr(q), q.stride(0), q.stride(1), q.stride(2),
            _ptr(w), float(eps), flags, _ptr(c), _ptr(s), s_b, s_t,
            _ptr(k_cache), _ptr(v_cache), k_cache.stride(0), k_cache.stride(1),
            k_cache.stride(2), max_len, _ptr(rp), _ptr(pd), p0, max_kv_len,
            int(window), float(scale), int(chunk),
            _ptr(out), out.stride(0), out.stride(1), out.stride(2))
    return args, out, dev, max_kv_len, chunk


def attn_decode(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, *, scale: float,
                pos: int | None = None, pos_dev: torch.Tensor | None = None,
                row_pos: torch.Tensor | None = None, max_kv_len: int | None = None,
                window: int = 0, q_weight: torch.Tensor | None = None, eps: float = 1e-6,
                norm_q: bool = False, cos: torch.Tensor | None = None,
                sin: torch.Tensor | None = None, chunk: int = 0, out: torch.Tensor | None = None,
                workspace: torch.Tensor | None = None) -> torch.Tensor:
    """Split-K attention of the T new queries q [B,H,T,D] against the cache, whose rows
    hold base_b + T valid keys (the new ones included). Returns [B,T,H,D]."""
    args, out, dev, max_kv_len, chunk = _decode_args(q, k_cache, v_cache, scale, pos, pos_dev, row_pos,
                                                     max_kv_len, window, q_weight, eps, norm_q, cos, sin,
                                                     chunk, out, workspace)
    B, H, T, D = q.shape
    need = lib().forge_attn_decode_workspace_bytes(args[0], B, T, H, k_cache.shape[1], D, max_kv_len, chunk)
    if need and (workspace is None or workspace.numel() * workspace.element_size() < need):
        workspace = torch.empty(need, dtype=torch.uint8, device=dev)
    ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    st = lib().forge_attn_decode(*args, _ptr(workspace), ws_bytes, _stream(dev))
    check(st, "forge_attn_decode")
    return out


_STREAM_WS: dict = {}
_STREAM_WS_MAX = 16   # streams whose workspace is kept (the oldest is dropped beyond that)


def _stream_workspace(dev: torch.device, need: int) -> torch.Tensor:
    """A split-K workspace per (device, stream), cleared when it is made: every call leaves
    its work ticket zero, so calls ordered on that stream may skip the ticket reset. Grown
    (a new cleared buffer) when a call needs more. Dropping a buffer is safe while its calls
    are in flight: torch's allocator reuses the memory only in that stream's order."""
    key = (dev.index, torch.cuda.current_stream(dev).cuda_stream)
    ws = _STREAM_WS.pop(key, None)
    if ws is None or ws.numel() < need:
        ws = torch.zeros(max(need, 1 << 20), dtype=torch.uint8, device=dev)
    _STREAM_WS[key] = ws   # most recently used last
    while len(_STREAM_WS) > _STREAM_WS_MAX:
        _STREAM_WS.pop(next(iter(_STREAM_WS)))
    return ws


def attn_decode_append(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, k_cache: torch.Tensor,
                       v_cache: torch.Tensor, *, scale: float, pos: int | None = None,
                       pos_dev: torch.Tensor | None = None, row_pos: torch.Tensor | None = None,
                       max_kv_len: int | None = None, window: int = 0,
                       q_weight: torch.Tensor | None = None, k_weight: torch.Tensor | None = None,
                       eps: float = 1e-6, norm_q: bool = False, norm_k: bool = False,
                       norm_v: bool = False, cos: torch.Tensor | None = None,
                       sin: torch.Tensor | None = None, chunk: int = 0, out: torch.Tensor | None = None,
                       workspace: torch.Tensor | None = None, workspace_zeroed: bool = False) -> torch.Tensor:
    """kv_append(k, v, ...) then attn_decode(q, ...), as one forge_attn_decode_append call:
    the new keys (norm_k with k_weight, RoPE) and values (norm_v) go into the cache at
    base_b + t and the T queries attend over it, the new keys included. Returns [B,T,H,D].
    Without a workspace (and outside graph capture) the call uses this module's zeroed
    workspace for the current stream (FORGE_WS_ZEROED: no ticket-reset kernel);
    workspace_zeroed=True makes the same promise for a workspace the caller cleared once."""
    B, K, T, D = k.shape
    if v.shape != k.shape or q.shape[0] != B or q.shape[2] != T or q.shape[3] != D:
        raise ValueError(f"q {tuple(q.shape)}, k {tuple(k.shape)} and v {tuple(v.shape)} do not fit")
    if k_cache.shape[1] != K:
        raise ValueError(f"cache {tuple(k_cache.shape)} does not fit new k {tuple(k.shape)}")
    if k.dtype != k_cache.dtype:
        k = k.to(k_cache.dtype)
    if v.dtype != k_cache.dtype:
        v = v.to(k_cache.dtype)
    _need_device(k, v)
    _last_dim_contiguous(k, "k")
    _last_dim_contiguous(v, "v")
    args, out, dev, max_kv_len, chunk = _decode_args(q, k_cache, v_cache, scale, pos, pos_dev, row_pos,
                                                     max_kv_len, window, q_weight, eps, norm_q, cos, sin,
                                                     chunk, out, workspace)
    c = args[13]
    kv_flags = (NORM_QK if norm_k else 0) | (ROPE if c is not None else 0) | (NORM_V if norm_v else 0)
    kw = _weight(k_weight, D) if norm_k else None
    need = lib().forge_attn_decode_workspace_bytes(args[0], B, T, q.shape[1], K, D, max_kv_len, chunk)
    zeroed = bool(workspace_zeroed)
    if need and workspace is None and not torch.cuda.is_current_stream_capturing():
        workspace, zeroed = _stream_workspace(dev, need), True
    if need and (workspace is None or workspace.numel() * workspace.element_size() < need):
        workspace, zeroed = torch.empty(need, dtype=torch.uint8, device=dev), False
    ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    st = lib().forge_attn_decode_append(*args[:13], _ptr(k), k.stride(0), k.stride(1), k.stride(2),
                                        _ptr(v), v.stride(0), v.stride(1), v.stride(2), _ptr(kw), kv_flags,
                                        *args[13:], _ptr(workspace), ws_bytes, WS_ZEROED if zeroed else 0,
                                        _stream(dev))
    check(st, "forge_attn_decode_append")
    return out


def attn_decode_noalloc(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, *, scale: float,
                        out: torch.Tensor, pos: int | None = None, pos_dev: torch.Tensor | None = None,
                        row_pos: torch.Tensor | None = None, max_kv_len: int | None = None,
                        window: int = 0, q_weight: torch.Tensor | None = None, eps: float = 1e-6,
                        norm_q: bool = False, cos: torch.Tensor | None = None,
                        sin: torch.Tensor | None = None, chunk: int = 0) -> torch.Tensor:
    """attn_decode through forge_attn_decode_noalloc: the split-K partials live in the
    library's own device array (at most NOALLOC_SCRATCH_BYTES), so the call allocates
    nothing on the device; `out` must be given. Calls that may overlap on one GPU race on
    that array."""
    args, out, dev, _, _ = _decode_args(q, k_cache, v_cache, scale, pos, pos_dev, row_pos, max_kv_len,
                                        window, q_weight, eps, norm_q, cos, sin, chunk, out, None)
    check(lib().forge_attn_decode_noalloc(*args, _stream(dev)), "forge_attn_decode_noalloc")
    return out


def attn_drafter(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, *,
                 n_past: int | None = None, n_past_dev: torch.Tensor | None = None,
                 window: int = 0, scale: float = 1.0, **kw) -> torch.Tensor:
    """The MTP drafter's attention onto the target's cache (sleuth/forge/infer/mtp.py:73-92,
    and its graph form with the position on the device, mtp.py:169-188): one query per
    row, at position n_past, over the n_past keys the target has stored (positions
    0 .. n_past-1); with a sliding window only keys k with n_past - k < window (llama.cpp's
    rule, mtp.py:84-86). Scale 1.0 by default. This is forge_attn_decode with the query
    placed at n_past - 1 (so it sees keys up to n_past - 1) and the window narrowed by
    one. q [B,H,1,D] (normalised and rotated by the drafter, or raw with norm_q/cos/sin
    as for attn_decode); returns [B,1,H,D]."""
    if q.shape[2] != 1:
        raise ValueError("the drafter attends with one query per row")
    if window < 0 or window == 1:
        raise ValueError("window must be 0 (global) or at least 2")
    w = window - 1 if window else 0
    if n_past_dev is not None:
        if n_past is not None:
            raise ValueError("give n_past or n_past_dev, not both")
        return attn_decode(q, k_cache, v_cache, scale=scale, pos_dev=n_past_dev.to(torch.int64) - 1,
                           window=w, **kw)
    if n_past is None or int(n_past) < 1:
        raise ValueError("n_past must be at least 1: the drafter needs keys the target stored")
    return attn_decode(q, k_cache, v_cache, scale=scale, pos=int(n_past) - 1, window=w, **kw)


PREFILL_HEAD_DIMS = (64, 128, 256, 512)


def prefill_supported(q: torch.Tensor) -> bool:
    return q.dtype in (torch.bfloat16, torch.float16) and q.shape[-1] in PREFILL_HEAD_DIMS


def attn_prefill(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *, scale: float, offset: int = 0,
                 window: int = 0, q_weight: torch.Tensor | None = None, eps: float = 1e-6,
                 norm_q: bool = False, cos: torch.Tensor | None = None,
                 sin: torch.Tensor | None = None, out: torch.Tensor | None = None,
                 doc_start: torch.Tensor | None = None, check_doc_start: bool = True) -> torch.Tensor:
    """Causal flash attention on MFMA: queries at positions offset..offset+T-1 over keys
    0..offset+T-1 of k/v [B,K,>=offset+T,D]. Returns [B,T,H,D].

    doc_start: [B, T] int32, the position of the first token of each query's document (the
    reference's document mask, transformer.py:271-275): query t also sees no key before it.
    It must be non-decreasing along T and at most the query's own position: checked here
    (two host synchronisations) unless check_doc_start is False, for a caller that built
    it so (the module's own starts, taken from the mask), or under graph capture."""
    B, H, T, D = q.shape
    Bk, K, S, Dk = k.shape
    if Bk != B or Dk != D or v.shape != k.shape or H % K:
        raise ValueError(f"q {tuple(q.shape)} does not fit k/v {tuple(k.shape)}")
    if S < offset + T:
        raise ValueError(f"k/v hold {S} positions, need offset + T = {offset + T}")
    if k.stride() != v.stride():
        raise ValueError("k and v must have the same strides")
    if not prefill_supported(q) or k.dtype != q.dtype:
        raise ValueError(f"MFMA prefill takes bf16/fp16 with head dim in {PREFILL_HEAD_DIMS}")
    dev = _need_device(q, k, v, cos, sin, out)
    _last_dim_contiguous(q, "q")
    _last_dim_contiguous(k, "k")
    c, s, s_b, s_t = _rope_tables(cos, sin, B, T, D)
    if s_b:
        raise ValueError("prefill takes [T, D] cos/sin shared by the batch")
    flags = (NORM_QK if norm_q else 0) | (ROPE if c is not None else 0)
    w = _weight(q_weight, D) if norm_q else None
    if out is None:
        out = torch.empty(B, T, H, D, dtype=q.dtype, device=dev)
    elif out.shape != (B, T, H, D) or out.dtype != q.dtype:
        raise ValueError(f"out must be [B,T,H,D] = {(B, T, H, D)} {q.dtype}")
    if doc_start is None:
        st = lib().forge_attn_prefill(dtype_code(q), B, T, H, K, D, _ptr(q), q.stride(0), q.stride(1),
                                      q.stride(2), _ptr(w), float(eps), flags, _ptr(c), _ptr(s), s_t,
                                      _ptr(k), _ptr(v), k.stride(0), k.stride(1), k.stride(2),
                                      int(offset), int(window), float(scale),
                                      _ptr(out), out.stride(0), out.stride(1), out.stride(2), _stream(dev))
        check(st, "forge_attn_prefill")
        return out
    if doc_start.dtype != torch.int32 or doc_start.shape != (B, T) or doc_start.device != dev:
        raise ValueError(f"doc_start must be int32 [B, T] = {(B, T)} on {dev}")
    if doc_start.stride(1) != 1:
        raise ValueError("doc_start: the last dimension must be contiguous")
    if check_doc_start and not torch.cuda.is_current_stream_capturing():
        pos = offset + torch.arange(T, device=dev, dtype=torch.int32)
        if bool(((doc_start < 0) | (doc_start > pos)).any()) or \
                bool((doc_start[:, 1:] < doc_start[:, :-1]).any()):
            raise ValueError("doc_start must be non-decreasing and in [0, the query's position]")
    st = lib().forge_attn_prefill_docs(dtype_code(q), B, T, H, K, D, _ptr(q), q.stride(0), q.stride(1),
                                       q.stride(2), _ptr(w), float(eps), flags, _ptr(c), _ptr(s), s_t,
                                       _ptr(k), _ptr(v), k.stride(0), k.stride(1), k.stride(2),
                                       int(offset), int(window), float(scale), _ptr(doc_start),
                                       doc_start.stride(0), _ptr(out), out.stride(0), out.stride(1),
                                       out.stride(2), _stream(dev))
    check(st, "forge_attn_prefill_docs")
    return out


__all__ = ["head_norm_rope", "kv_append", "attn_decode", "attn_decode_append", "attn_decode_noalloc", "attn_prefill", "decode_chunk",
           "decode_workspace_bytes", "attn_drafter", "prefill_supported", "dtype_code", "_lib"]
