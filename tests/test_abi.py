"""The C ABI library without a GPU: it loads, exports every function include/forge_attn.h
declares (and ctypes knows each signature), its pure host functions work, and bad
arguments are rejected before anything is launched."""

from __future__ import annotations

import ctypes as C
import re
from pathlib import Path

import pytest
import torch

from sleuth_amd import _lib, ops

HEADER = Path(__file__).resolve().parents[1] / "include" / "forge_attn.h"


def declared() -> set[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return set(re.findall(r"\b(forge_\w+)\s*\(", text))


def test_library_loads_with_abi_version():
    lib = _lib.lib()
    assert lib.forge_abi_version() == _lib.ABI_VERSION == 3
    assert lib.forge_last_error() == b""


def test_every_declared_symbol_is_exported_and_bound():
    names = declared()
    assert {"forge_abi_version", "forge_last_error", "forge_head_norm_rope", "forge_kv_append",
            "forge_attn_decode", "forge_attn_decode_append", "forge_attn_decode_chunk",
            "forge_attn_decode_chunk_uniform", "forge_attn_decode_workspace_bytes",
            "forge_attn_prefill", "forge_attn_prefill_docs"} <= names
    raw = C.CDLL(str(_lib.LIB_PATH))
    for n in names:
        assert hasattr(raw, n), n
    assert names == set(_lib.SIGNATURES), names ^ set(_lib.SIGNATURES)


def test_host_only_functions():
    lib = _lib.lib()
    # C4: the auto chunk is a multiple of the keys per iteration (64 for hd 128 bf16)
    ch = lib.forge_attn_decode_chunk(_lib.BF16, 64, 1, 16, 8, 128, 32768)
    assert ch >= 64 and ch % 64 == 0
    ws = lib.forge_attn_decode_workspace_bytes(_lib.BF16, 64, 1, 16, 8, 128, 32768, ch)
    chunks = -(-32768 // ch)
    assert ws >= 64 * 16 * chunks * (128 * 4 + 8)
    assert lib.forge_attn_decode_workspace_bytes(_lib.BF16, 1, 1, 8, 4, 64, 50, 64) == 0  # one chunk
    assert lib.forge_attn_decode_chunk(_lib.BF16, 1, 1, 8, 3, 64, 100) == 0              # H % K != 0
    # the MFMA path (G >= 4) for per-row positions: 1024-key chunks on the persistent grid
    # (up to 512 rows), 512 on the dense grid beyond it
    assert lib.forge_attn_decode_chunk(_lib.BF16, 64, 1, 32, 8, 128, 32768) == 1024
    assert lib.forge_attn_decode_chunk(_lib.BF16, 600, 1, 32, 8, 128, 32768) == 512
    # the cap is max(1024, 16 block iterations): 2048 keys at head dim 32 in bf16/fp16 (128
    # keys per iteration), 1024 at head dim 64 and above and in fp32
    assert lib.forge_attn_decode_chunk(_lib.BF16, 64, 1, 16, 8, 32, 32768) == 2048
    assert lib.forge_attn_decode_chunk(_lib.F16, 64, 1, 16, 8, 32, 32768) == 2048
    assert lib.forge_attn_decode_chunk(_lib.BF16, 64, 1, 16, 8, 64, 32768) == 1024
    assert lib.forge_attn_decode_chunk(_lib.F32, 64, 1, 16, 8, 32, 32768) == 1024


def test_uniform_chunk_rule():
    """One host position for every row: chunks sized so the CUs get equal work, no split when
    the (row, KV head) pairs fill them (this container has no GPU: 256 CUs assumed, as on
    MI355X)."""
    lib = _lib.lib()
    ch = lambda B, H, K, D, L, dt=_lib.BF16: lib.forge_attn_decode_chunk_uniform(dt, B, 1, H, K, D, L)
    assert ch(32, 16, 8, 128, 8192) == 8192      # C3 decode: 256 pairs, one unit per CU
    assert ch(64, 16, 8, 128, 4096) == 4096      # 512 pairs: two per CU, still no split
    assert ch(48, 16, 8, 128, 8192) == 4096      # 384 pairs: 768 units = 3 per CU
    assert ch(24, 16, 8, 128, 8192) == 1024      # 192 pairs: the rule's 2048, at most 1024 below 256 pairs
    assert ch(16, 12, 4, 64, 32768) == 1024      # C2's pairs at a large capacity: rows stay split
    assert ch(16, 12, 4, 64, 2049) == 576        # C2: 64 pairs x 4 chunks = 256 units
    assert ch(1, 8, 4, 64, 50) == 64             # one short row: one chunk of one iteration
    for B, H, K, D, L in [(32, 16, 8, 128, 8192), (16, 12, 4, 64, 2049), (3, 8, 2, 32, 777),
                          (100, 8, 8, 256, 70000)]:
        c = ch(B, H, K, D, L)
        kpi = (256 // (D // 8)) * 2
        assert c % kpi == 0 and c >= min(4 * kpi, -(-L // kpi) * kpi)
    # the MFMA verify shapes (G >= 4, hd 128/256, bf16/fp16): one round of block slots
    assert ch(8, 8, 1, 256, 8196) == 288 == lib.forge_attn_decode_chunk(_lib.BF16, 8, 1, 8, 1, 256, 8196)
    assert ch(32, 32, 8, 128, 8192) == 4096      # 256 pairs, 512 slots: two chunks per row
    assert ch(8, 8, 1, 256, 131072) == 512       # split rows of a large capacity: at most 512 keys
    assert ch(1, 8, 3, 64, 100) == 0             # H % K != 0


def _decode_args(**over):
    a = dict(dtype=_lib.BF16, B=1, T=1, H=8, K=4, D=128, q=16, sqb=1024, sqh=128, sqt=128, qw=None,
             eps=1e-6, flags=0, cos=None, sin=None, csb=0, cst=0, k=16, v=16, skb=512 * 128 * 4,
             skh=512 * 128, sks=128, max_len=512, row_pos=None, pos_dev=None, pos0=10, max_kv_len=0,
             window=0, scale=0.1, chunk=0, out=16, sob=1024, sot=1024, soh=128, ws=None, ws_bytes=0,
             stream=None)
    a.update(over)
    return list(a.values())


@pytest.mark.parametrize("over,msg", [
    (dict(D=48), "head dim"),
    (dict(H=6, K=4), "multiple"),
    (dict(pos0=512), "KV cache full"),
    (dict(q=None), "null"),
    (dict(flags=_lib.ROPE), "cos and sin"),
    (dict(dtype=7), "dtype"),
    (dict(chunk=100), "chunk"),
    (dict(q=18), "aligned"),
    (dict(pos0=100, max_len=512, chunk=64, ws=None), "workspace"),
])
def test_decode_rejects_bad_arguments(over, msg):
    lib = _lib.lib()
    st = lib.forge_attn_decode(*_decode_args(**over))
    assert st < 0
    assert msg in lib.forge_last_error().decode()


def test_prefill_rejects_bad_arguments():
    lib = _lib.lib()
    base = [_lib.BF16, 1, 64, 8, 4, 128, 16, 8192, 128, 1024, None, 1e-6, 0, None, None, 0,
            16, 16, 8192, 1024, 128, 0, 0, 0.1, 16, 8192, 1024, 128, None]
    for idx, val, msg in ((0, _lib.F32, "bf16 or fp16"), (5, 96, "head dim"), (21, -1, "offset"),
                          (6, 24, "aligned"), (8, 100, "multiples")):
        args = list(base)
        args[idx] = val
        assert lib.forge_attn_prefill(*args) < 0
        assert msg in lib.forge_last_error().decode()


def test_kv_append_rejects_overflow_and_odd_dims():
    lib = _lib.lib()
    args = [_lib.BF16, 1, 4, 2, 64, 16, 512, 64, 64, 16, 512, 64, 64, 16, 16, 1024, 512, 64, 8,
            None, None, 6, None, 1e-6, 0, None, None, 0, 0, None]
    assert lib.forge_kv_append(*args) < 0 and "KV cache full" in lib.forge_last_error().decode()
    args[4] = 63
    assert lib.forge_kv_append(*args) < 0 and "even" in lib.forge_last_error().decode()


def test_ops_refuse_cpu_tensors():
    q = torch.zeros(1, 2, 1, 64)
    with pytest.raises(ValueError, match="GPU"):
        ops.attn_decode(q, torch.zeros(1, 1, 8, 64), torch.zeros(1, 1, 8, 64), scale=1.0, pos=0)
    with pytest.raises(ValueError, match="GPU"):
        ops.head_norm_rope(q)


def test_ops_shape_checks_before_any_launch():
    q = torch.zeros(1, 3, 1, 64)
    with pytest.raises(ValueError):
        ops.attn_decode(q, torch.zeros(1, 2, 8, 64), torch.zeros(1, 2, 8, 64), scale=1.0)
    with pytest.raises(ValueError):
        ops.kv_append(torch.zeros(1, 1, 2, 64), torch.zeros(1, 1, 3, 64), torch.zeros(1, 1, 8, 64),
                      torch.zeros(1, 1, 8, 64))
