"""Writes tests/golden/attn_cases.npz: small attention cases whose expected outputs come
from the float64 loop restatement (oracle.brute_attention), independent of torch SDPA.

Run from the repository root:  python -m tests.golden.make_golden
The cases follow the BASELINE configs at reduced size: C1 (fp32, 8q/4kv, hd 32, causal
prefill then decode), C2 (12q/4kv, hd 64 decode), C3/C4 (16q/8kv, hd 128, decode at a
long offset), C5 (MQA 8q/1kv, hd 256, k=4 verify, sliding window and global).
"""

from __future__ import annotations

import math
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
FIXTURE = HERE / "attn_cases.npz"

# name, B, H, K, D, T, offset, window, seed
CASES = [
    ("c1_prefill", 1, 8, 4, 32, 24, 0, 0, 1),
    ("c1_decode", 1, 8, 4, 32, 1, 40, 0, 2),
    ("c2_decode", 2, 12, 4, 64, 1, 40, 0, 3),
    ("c3_chunked_prefill", 1, 16, 8, 128, 6, 9, 0, 4),
    ("c4_decode", 1, 16, 8, 128, 1, 20, 0, 5),
    ("c5_verify_window", 1, 8, 1, 256, 4, 30, 16, 6),
    ("c5_verify_global", 1, 8, 1, 256, 4, 30, 0, 7),
]


def build() -> dict:
    import torch

    sys.path.insert(0, str(HERE.parents[1]))
    import oracle

    out = {}
    for name, B, H, K, D, T, off, win, seed in CASES:
        g = torch.Generator().manual_seed(seed)
        # inputs are stored as float16; the expected output is computed from those values
        q = torch.randn(B, H, T, D, generator=g).half().float()
        k = torch.randn(B, K, off + T, D, generator=g).half().float()
        v = torch.randn(B, K, off + T, D, generator=g).half().float()
        sc = 1.0 / math.sqrt(D)
        o = oracle.brute_attention(q, k, v, off, win, sc)
        for key, val in (("q", q), ("k", k), ("v", v)):
            out[f"{name}.{key}"] = val.numpy().astype(np.float16)
        out[f"{name}.out"] = o.numpy().astype(np.float32)
        out[f"{name}.meta"] = np.array([off, win, sc], dtype=np.float64)
    return out


def load_cases() -> list[dict]:
    data = np.load(FIXTURE, allow_pickle=False)
    cases = []
    for name, *_ in CASES:
        off, win, sc = data[f"{name}.meta"]
        cases.append({"name": name, "q": data[f"{name}.q"].astype(np.float32),
                      "k": data[f"{name}.k"].astype(np.float32), "v": data[f"{name}.v"].astype(np.float32),
                      "out": data[f"{name}.out"].astype(np.float64), "offset": int(off), "window": int(win), "scale": float(sc)})
    return cases


if __name__ == "__main__":
    np.savez_compressed(FIXTURE, **build())
    print(f"wrote {FIXTURE} ({FIXTURE.stat().st_size} bytes)")
