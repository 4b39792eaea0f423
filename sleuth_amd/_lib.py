"""ctypes binding of libforge_attn.so (include/forge_attn.h).

The library is built in-tree (python -m sleuth_amd.csrc.build, or __graft_entry__.build())
into sleuth_amd/_lib/. Loading it never falls back to anything: if the file is missing
or its ABI version differs, `lib()` raises.
"""

from __future__ import annotations

import ctypes as C
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "_lib" / "libforge_attn.so"
ABI_VERSION = 3

F32, BF16, F16 = 0, 1, 2
NOALLOC_SCRATCH_BYTES = 48 * 1024 * 1024   # FORGE_NOALLOC_SCRATCH_BYTES
NORM_QK, ROPE, NORM_V = 1, 2, 4
WS_ZEROED = 1                              # FORGE_WS_ZEROED

_p = C.c_void_p
_i = C.c_int
_i64 = C.c_int64
_f = C.c_float

# name -> (restype, argtypes); every exported symbol of include/forge_attn.h
SIGNATURES: dict[str, tuple] = {
    "forge_abi_version": (_i, []),
    "forge_last_error": (C.c_char_p, []),
    "forge_head_norm_rope": (_i, [
        _i, _p, _p, _i, _i, _i, _i,          # dtype, x, y, B, H, T, D
        _i64, _i64, _i64, _i64, _i64, _i64,  # x strides, y strides
        _p, _f, _i,                          # weight, eps, norm
        _p, _p, _i64, _i64,                  # cos, sin, s_cos_b, s_cos_t
        _p]),                                # stream
    "forge_kv_append": (_i, [
        _i, _i, _i, _i, _i,                  # dtype, B, T, K, D
        _p, _i64, _i64, _i64,                # k + strides
        _p, _i64, _i64, _i64,                # v + strides
        _p, _p, _i64, _i64, _i64, _i64,      # k_dst, v_dst, sdb, sdh, sds, dst_len
        _p, _p, _i64,                        # row_pos, pos_dev, pos0
        _p, _f, _i,                          # k_weight, eps, flags
        _p, _p, _i64, _i64,                  # cos, sin, s_cos_b, s_cos_t
        _p]),
    "forge_attn_decode": (_i, [
        _i, _i, _i, _i, _i, _i,              # dtype, B, T, H, K, D
        _p, _i64, _i64, _i64,                # q + strides
        _p, _f, _i,                          # q_weight, eps, flags
        _p, _p, _i64, _i64,                  # cos, sin, s_cos_b, s_cos_t
        _p, _p, _i64, _i64, _i64, _i64,      # k_cache, v_cache, skb, skh, sks, max_len
        _p, _p, _i64, _i64,                  # row_pos, pos_dev, pos0, max_kv_len
        _i, _f, _i,                          # window, scale, chunk
        _p, _i64, _i64, _i64,                # out + strides (b, t, h)
        _p, C.c_size_t,                      # workspace, bytes
        _p]),
    "forge_attn_decode_append": (_i, [
        _i, _i, _i, _i, _i, _i,              # dtype, B, T, H, K, D
        _p, _i64, _i64, _i64,                # q + strides
        _p, _f, _i,                          # q_weight, eps, flags
        _p, _i64, _i64, _i64,                # new k + strides
        _p, _i64, _i64, _i64,                # new v + strides
        _p, _i,                              # k_weight, kv_flags
        _p, _p, _i64, _i64,                  # cos, sin, s_cos_b, s_cos_t
        _p, _p, _i64, _i64, _i64, _i64,      # k_cache, v_cache, skb, skh, sks, max_len
        _p, _p, _i64, _i64,                  # row_pos, pos_dev, pos0, max_kv_len
        _i, _f, _i,                          # window, scale, chunk
        _p, _i64, _i64, _i64,                # out + strides (b, t, h)
        _p, C.c_size_t, _i,                  # workspace, bytes, ws_flags
        _p]),
    "forge_attn_decode_noalloc": (_i, [
        _i, _i, _i, _i, _i, _i,              # dtype, B, T, H, K, D
        _p, _i64, _i64, _i64,                # q + strides
        _p, _f, _i,                          # q_weight, eps, flags
        _p, _p, _i64, _i64,                  # cos, sin, s_cos_b, s_cos_t
        _p, _p, _i64, _i64, _i64, _i64,      # k_cache, v_cache, skb, skh, sks, max_len
        _p, _p, _i64, _i64,                  # row_pos, pos_dev, pos0, max_kv_len
        _i, _f, _i,                          # window, scale, chunk
        _p, _i64, _i64, _i64,                # out + strides (b, t, h)
        _p]),                                # stream
    "forge_attn_decode_chunk": (_i, [_i, _i, _i, _i, _i, _i, _i64]),
    "forge_attn_decode_chunk_uniform": (_i, [_i, _i, _i, _i, _i, _i, _i64]),
    "forge_attn_decode_workspace_bytes": (C.c_size_t, [_i, _i, _i, _i, _i, _i, _i64, _i]),
    "forge_attn_prefill": (_i, [
        _i, _i, _i, _i, _i, _i,              # dtype, B, T, H, K, D
        _p, _i64, _i64, _i64,                # q + strides
        _p, _f, _i,                          # q_weight, eps, flags
        _p, _p, _i64,                        # cos, sin, s_cos_t
        _p, _p, _i64, _i64, _i64,            # k, v, skb, skh, sks
        _i64, _i, _f,                        # offset, window, scale
        _p, _i64, _i64, _i64,                # out + strides (b, t, h)
        _p]),
    "forge_attn_prefill_docs": (_i, [
        _i, _i, _i, _i, _i, _i,              # dtype, B, T, H, K, D
        _p, _i64, _i64, _i64,                # q + strides
        _p, _f, _i,                          # q_weight, eps, flags
        _p, _p, _i64,                        # cos, sin, s_cos_t
        _p, _p, _i64, _i64, _i64,            # k, v, skb, skh, sks
        _i64, _i, _f,                        # offset, window, scale
        _p, _i64,                            # doc_start, its row stride
        _p, _i64, _i64, _i64,                # out + strides (b, t, h)
        _p]),
}

_lock = threading.Lock()
_lib: C.CDLL | None = None


class ForgeError(RuntimeError):
    """A libforge_attn call was rejected (status < 0) or its launch failed (status > 0)."""


def lib() -> C.CDLL:
    """The loaded library (loaded once). Raises if it was not built or does not match."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise ForgeError(f"{LIB_PATH} is missing: build it with `python -m sleuth_amd.csrc.build` "
                                 "(or __graft_entry__.build())")
            import torch  # noqa: F401  load torch's HIP runtime first so the library shares it

            handle = C.CDLL(str(LIB_PATH), mode=C.RTLD_GLOBAL)
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(handle, name)
                fn.restype = res
                fn.argtypes = args
            v = handle.forge_abi_version()
            if v != ABI_VERSION:
                raise ForgeError(f"libforge_attn ABI version {v}, expected {ABI_VERSION}: rebuild it")
            _lib = handle
    return _lib


def check(status: int, what: str) -> None:
    if status != 0:
        msg = lib().forge_last_error().decode(errors="replace")
        raise ForgeError(f"{what}: status {status}: {msg}")
