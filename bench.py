"""Benchmark of the FORGE attention hot path on one MI355X.

Headline (BASELINE.json metric): decode attention of config C4 -- batch 64, Qwen3-0.6B
heads (16 q / 8 kv, head dim 128, bf16), per-row KV lengths uniform in [1024, 32768]
from a seed, one new token per row. A step is one layer's attention for the batch, as
the module runs it: one forge_attn_decode_append call, in which the new K/V are
normalised/rotated and written into the cache and the split-K attention (q norm + RoPE
fused into its q load) attends over it. `value` is the step's algorithmic HBM bytes /
step time (GB/s); tokens/s = 64 / (28 layers x step).
Beside it: C3 causal prefill (4 x 4096 tokens, bf16) in TFLOP/s, each dominant kernel's
roofline fraction, and the oracle (torch SDPA on the CPU) timed on a bounded sample.

Usage: python bench.py [--gpus 1] [--steps 20] [--warmup 5] [--no-cpu] [--no-extra]
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

import torch

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0        # MI355X HBM3E, GB/s
BF16_PEAK_TFLOPS = 2500.0    # MI355X dense bf16 MFMA, TFLOP/s
N_LAYERS = 28                # Qwen3-0.6B: tokens/s counts 28 layers per token
WARM_S = 0.1                 # untimed back-to-back calls before each headline timing
METRIC = "decode attn HBM GB/s + tokens/s (bs64, 32k ctx); prefill bf16 TFLOPS at 4k"


# ----------------------------------------------------------------------------- inputs
def c4_lengths(seed: int = 0, B: int = 64, lo: int = 1024, hi: int = 32768) -> list[int]:
    g = torch.Generator().manual_seed(seed)
    return torch.randint(lo, hi + 1, (B,), generator=g).tolist()


class DecodeWorkload:
    """One layer of a ragged decode batch: caches [B, K, max_len, D] filled with N(0,1)
    up to each row's length, raw q/k/v of the new token, norm gains, RoPE rows."""

    def __init__(self, lens, H, K, D, theta, dtype, dev, seed=0, T=1, window=0, n_layers=1):
        self.lens, self.B, self.H, self.K, self.D, self.T = lens, len(lens), H, K, D, T
        self.window, self.dtype, self.dev = window, dtype, dev
        self.max_len = max(lens)
        g = torch.Generator(device=dev).manual_seed(seed)
        shape = (self.B, K, self.max_len, D)
        self.k_caches = [torch.randn(shape, generator=g, device=dev, dtype=dtype) for _ in range(n_layers)]
        self.v_caches = [torch.randn(shape, generator=g, device=dev, dtype=dtype) for _ in range(n_layers)]
        B = self.B
        self.q = torch.randn(B, T, H, D, generator=g, device=dev, dtype=dtype).transpose(1, 2)
        self.k = torch.randn(B, T, K, D, generator=g, device=dev, dtype=dtype).transpose(1, 2)
        self.v = torch.randn(B, T, K, D, generator=g, device=dev, dtype=dtype).transpose(1, 2)
        # norm gains: bf16 parameters, held in fp32 by the caller (converted once, like the module)
        self.wq = (1 + 0.1 * torch.randn(D, generator=g, device=dev)).to(dtype).float()
        self.wk = (1 + 0.1 * torch.randn(D, generator=g, device=dev)).to(dtype).float()
        from sleuth_amd.rope import rope_tables  # the tables the model's buffers hold

        cos, sin = rope_tables(D, self.max_len + T, theta)
        base = torch.tensor([L - T for L in lens])
        idx = base[:, None] + torch.arange(T)[None, :]
        self.cos = cos[idx].to(dev)
        self.sin = sin[idx].to(dev)
        self.row_pos = base.to(torch.int32).to(dev)
        # rows of one length use the host position, as the module does with a plain KVCache
        self.pos = int(base[0]) if len(set(lens)) == 1 else None
        self.scale = 1.0 / math.sqrt(D)
        self.out = torch.empty(B, T, H, D, device=dev, dtype=dtype)
        from sleuth_amd import ops

        self.chunk = ops.decode_chunk(dtype, B, T, H, K, D, self.max_len, window, uniform=self.pos is not None)
        nbytes = ops.decode_workspace_bytes(dtype, B, T, H, K, D, self.max_len, self.chunk)
        # cleared once: each call leaves the persistent grid's work ticket zero, as the
        # module's per-stream workspace does (no ticket-reset kernel per step)
        self.ws = torch.zeros(max(nbytes, 1), dtype=torch.uint8, device=dev)
        self.layer = 0

    def append(self, layer=None):
        from sleuth_amd import ops

        i = self.layer if layer is None else layer
        where = dict(pos=self.pos) if self.pos is not None else dict(row_pos=self.row_pos)
        cos, sin = (self.cos[0], self.sin[0]) if self.pos is not None else (self.cos, self.sin)
        ops.kv_append(self.k, self.v, self.k_caches[i], self.v_caches[i], **where,
                      k_weight=self.wk, eps=1e-6, norm_k=True, cos=cos, sin=sin)

    def attend(self, layer=None):
        from sleuth_amd import ops

        i = self.layer if layer is None else layer
        where = dict(pos=self.pos) if self.pos is not None else dict(row_pos=self.row_pos)
        cos, sin = (self.cos[0], self.sin[0]) if self.pos is not None else (self.cos, self.sin)
        return ops.attn_decode(self.q, self.k_caches[i], self.v_caches[i], scale=self.scale, **where,
                               max_kv_len=self.max_len, window=self.window,
                               q_weight=self.wq, eps=1e-6, norm_q=True, cos=cos, sin=sin,
                               chunk=self.chunk, out=self.out, workspace=self.ws)

    def step(self):
        """The module's decode step: the new tokens' keys and values go into the cache and the
        queries attend over it, in one forge_attn_decode_append call."""
        from sleuth_amd import ops

        i = self.layer
        where = dict(pos=self.pos) if self.pos is not None else dict(row_pos=self.row_pos)
        cos, sin = (self.cos[0], self.sin[0]) if self.pos is not None else (self.cos, self.sin)
        ops.attn_decode_append(self.q, self.k, self.v, self.k_caches[i], self.v_caches[i], scale=self.scale,
                               **where, max_kv_len=self.max_len, window=self.window, q_weight=self.wq,
                               k_weight=self.wk, eps=1e-6, norm_q=True, norm_k=True, cos=cos, sin=sin,
                               chunk=self.chunk, out=self.out, workspace=self.ws, workspace_zeroed=True)
        self.layer = (self.layer + 1) % len(self.k_caches)

    def step_two_pass(self):
        """The same step as two calls: forge_kv_append, then forge_attn_decode."""
        self.append()
        self.attend()
        self.layer = (self.layer + 1) % len(self.k_caches)

    def visible(self, L):
        return min(L, self.window + self.T - 1) if self.window else L

    def kv_bytes(self) -> int:
        s = torch.finfo(self.dtype).bits // 8
        return sum(2 * self.K * self.visible(L) * self.D * s for L in self.lens)

    def step_bytes(self) -> int:
        """Algorithmic bytes of one step: K/V of the positions each row reads, q read,
        o written, new K/V written."""
        s = torch.finfo(self.dtype).bits // 8
        B, H, K, D, T = self.B, self.H, self.K, self.D, self.T
        return self.kv_bytes() + 2 * B * H * T * D * s + 2 * B * K * T * D * s

    def attend_bytes(self) -> int:
        """Algorithmic bytes of the attention call: K/V reads + q read + o write."""
        s = torch.finfo(self.dtype).bits // 8
        return self.kv_bytes() + 2 * self.B * self.H * self.T * self.D * s


class PrefillWorkload:
    """C3 prefill: B x T causal, raw q/k/v, gains N(1, 0.1), RoPE theta 1e6."""

    def __init__(self, B, T, H, K, D, theta, dtype, dev, seed=1):
        self.B, self.T, self.H, self.K, self.D = B, T, H, K, D
        g = torch.Generator(device=dev).manual_seed(seed)
        self.q = torch.randn(B, T, H, D, generator=g, device=dev, dtype=dtype).transpose(1, 2)
        self.k = torch.randn(B, T, K, D, generator=g, device=dev, dtype=dtype).transpose(1, 2)
        self.v = torch.randn(B, T, K, D, generator=g, device=dev, dtype=dtype).transpose(1, 2)
        self.wq = (1 + 0.1 * torch.randn(D, generator=g, device=dev)).to(dtype).float()
        self.wk = (1 + 0.1 * torch.randn(D, generator=g, device=dev)).to(dtype).float()
        from sleuth_amd.rope import rope_tables

        cos, sin = rope_tables(D, T, theta)
        self.cos, self.sin = cos.to(dev), sin.to(dev)
        self.kc = torch.zeros(B, K, T, D, device=dev, dtype=dtype)
        self.vc = torch.zeros_like(self.kc)
        self.out = torch.empty(B, T, H, D, device=dev, dtype=dtype)
        self.scale = 1.0 / math.sqrt(D)

    def append(self):
        from sleuth_amd import ops

        ops.kv_append(self.k, self.v, self.kc, self.vc, pos=0, k_weight=self.wk, eps=1e-6, norm_k=True,
                      cos=self.cos, sin=self.sin)

    def attend(self):
        from sleuth_amd import ops

        return ops.attn_prefill(self.q, self.kc, self.vc, scale=self.scale, offset=0, q_weight=self.wq,
                                eps=1e-6, norm_q=True, cos=self.cos, sin=self.sin, out=self.out)

    def step(self):
        self.append()
        self.attend()

    def flops(self) -> float:
        """4 * hd * sum over (b, h, query) of the keys it sees (causal: T(T+1)/2)."""
        return 4.0 * self.D * self.B * self.H * self.T * (self.T + 1) / 2

    def flops_full_s(self) -> float:
        """The reference's attention FLOP convention (flops.py:84-89, forward third of its
        12*H*hd*S training term): 4 * H * hd * S per token with S = T, no causal halving."""
        return 4.0 * self.D * self.H * self.T * self.B * self.T


# ----------------------------------------------------------------------------- timing
def time_loop(fn, steps: int, warmup: int) -> float:
    """Seconds per call of fn, with HIP events on torch's current stream (the stream
    every kernel of this package is launched on)."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        fn()
    stop.record()
    torch.cuda.synchronize()
    return start.elapsed_time(stop) / 1e3 / steps


def warm(fn, seconds: float = WARM_S) -> int:
    """Runs fn back to back for about `seconds` of GPU time before a timing: the GPU only
    reaches its steady clock after some tens of milliseconds of load (C3 prefill on MI355X:
    about 355 us per call in the first 20 calls, 290 us from about the 60th on; the C4
    attention call: 642 us over its first 20 calls, 615 us over the next 20).
    Returns the number of calls made."""
    calls = 0
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        for _ in range(8):
            fn()
        calls += 8
        torch.cuda.synchronize()
    return calls


def time_graph(fn, n: int, replays: int, warmup: int) -> float:
    """Seconds per call of fn(0) .. fn(n - 1) captured once in a HIP graph and replayed:
    the GPU time of a call without the host's launch cost (the reference decodes under
    CUDA graphs, cuda_graph.py:96-108). fn must not allocate."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(max(warmup, 1)):
            for i in range(n):
                fn(i)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(n):
            fn(i)
    g.replay()
    torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(replays):
        g.replay()
    stop.record()
    torch.cuda.synchronize()
    return start.elapsed_time(stop) / 1e3 / (replays * n)


def read_traffic(name: str):
    """HBM bytes per launch of a kernel, measured with rocprofv3 --pmc (FETCH_SIZE and
    WRITE_SIZE, scaled by a copy kernel of known size) and recorded in the text summary
    profiles/<name>.txt as a line `hbm_bytes_per_launch: N`; None if not measured."""
    p = ROOT / "profiles" / f"{name}.txt"
    if not p.exists():
        return None
    for line in p.read_text().splitlines():
        if line.startswith("hbm_bytes_per_launch:"):
            try:
                return int(float(line.split(":", 1)[1]))
            except ValueError:
                return None
    return None


# ----------------------------------------------------------------------------- CPU baseline
CPU_WARMUP, CPU_RUNS = 3, 10   # 3 warm-up runs, then the median of >= 10


def cpu_info() -> dict:
    """The host CPU as the baseline reports it: model strings, logical and physical cores,
    the affinity mask and the cgroup CPU quota."""
    info = {"model": "unknown", "logical": os.cpu_count(), "affinity": len(os.sched_getaffinity(0))}
    try:
        cores, fields = set(), {}
        phys = core = None
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            key, _, val = (x.strip() for x in line.partition(":"))
            if key == "physical id":
                phys = val
            elif key == "core id":
                core = val
            elif key in ("model name", "cpu family", "model", "stepping", "vendor_id") and key not in fields:
                fields[key] = val
            elif not key and phys is not None:
                cores.add((phys, core))
                phys = core = None
        if phys is not None:
            cores.add((phys, core))
        info["model"] = fields.get("model name", "unknown")
        info["cpuid"] = {k: fields[k] for k in ("vendor_id", "cpu family", "model", "stepping") if k in fields}
        info["physical_cores"] = len(cores) or None
    except OSError:
        pass
    try:
        import subprocess

        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            key, _, val = (x.strip() for x in line.partition(":"))
            if key in ("Model name", "Core(s) per socket", "Socket(s)", "Thread(s) per core"):
                info[f"lscpu {key}"] = val
    except (OSError, subprocess.SubprocessError):
        pass
    try:
        quota, period = Path("/sys/fs/cgroup/cpu.max").read_text().split()
        info["cgroup_cpus"] = None if quota == "max" else round(int(quota) / int(period), 2)
    except (OSError, ValueError):
        pass
    return info


def _median_runs(fn) -> tuple[float, float, int]:
    """CPU_WARMUP untimed calls, then CPU_RUNS timed ones: (median s, min s, runs)."""
    for _ in range(CPU_WARMUP):
        fn()
    ts = []
    for _ in range(CPU_RUNS):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    ts.sort()
    return ts[len(ts) // 2] if len(ts) % 2 else 0.5 * (ts[len(ts) // 2 - 1] + ts[len(ts) // 2]), ts[0], len(ts)


def cpu_baseline_decode(wl: "DecodeWorkload", fp32_rows: int = 8) -> dict:
    """The oracle's eager CPU path (torch SDPA on the host: attention.py:171-193 with the
    one-rounding q norm + RoPE, one SDPA per ragged row over its prefix) over the whole C4
    batch for one layer, in bf16; the same in fp32 over the first `fp32_rows` rows (the fp32
    copy of the whole batch would need 17 GB of host memory). GB/s of algorithmic bytes."""
    import oracle

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    q = oracle.head_norm_rope(wl.q.cpu(), wl.wq.cpu(), 1e-6, wl.cos.cpu(), wl.sin.cpu())
    kc, vc = wl.k_caches[0].cpu(), wl.v_caches[0].cpu()
    s = torch.finfo(wl.dtype).bits // 8

    def row_bytes(rows):
        return sum(2 * wl.K * wl.visible(wl.lens[b]) * wl.D * s + 2 * wl.H * wl.T * wl.D * s for b in rows)

    def run(rows, qq, kk, vv):
        for b in rows:
            L = wl.lens[b]
            oracle.ragged_decode(qq[b:b + 1], kk[b:b + 1, :, :L], vv[b:b + 1, :, :L], [L], wl.window, wl.scale)

    every = range(wl.B)
    med, best, n = _median_runs(lambda: run(every, q, kc, vc))
    few = range(min(fp32_rows, wl.B))
    L32 = max(wl.lens[b] for b in few)
    k32, v32 = kc[:len(few), :, :L32].float(), vc[:len(few), :, :L32].float()
    med32, best32, _ = _median_runs(lambda: run(few, q.float(), k32, v32))
    return {"value": round(row_bytes(every) / med / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"the whole C4 batch for one layer ({sum(wl.lens)} cached tokens, 64 rows), bf16 torch SDPA "
                      f"on the host CPU, one call per row; median of {n} runs after {CPU_WARMUP} warm-ups",
            "value_best": round(row_bytes(every) / best / 1e9, 3),
            "value_fp32": round(row_bytes(few) / med32 / 1e9, 3),
            "value_fp32_sample": f"rows 0..{len(few) - 1} in fp32, median of {n} runs",
            "cpu": cpu_info()}


def cpu_baseline_prefill(B, T, H, K, D) -> dict:
    """torch SDPA (is_causal, enable_gqa) on the host at the full C3 shape (4 x 4096) in
    bf16, and in fp32; TFLOP/s of the causal count."""
    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    g = torch.Generator().manual_seed(2)
    q = torch.randn(B, H, T, D, generator=g).bfloat16()
    k = torch.randn(B, K, T, D, generator=g).bfloat16()
    v = torch.randn(B, K, T, D, generator=g).bfloat16()
    sdpa = torch.nn.functional.scaled_dot_product_attention
    fl = 4.0 * D * B * H * T * (T + 1) / 2
    med, best, n = _median_runs(lambda: sdpa(q, k, v, is_causal=True, enable_gqa=True, scale=D ** -0.5))
    q, k, v = q.float(), k.float(), v.float()
    med32, _, _ = _median_runs(lambda: sdpa(q, k, v, is_causal=True, enable_gqa=True, scale=D ** -0.5))
    return {"value": round(fl / med / 1e12, 4), "unit": "TFLOP/s", "cores": threads, "kind": "port",
            "sample": f"the whole C3 prefill ({B} x {T} causal), bf16 torch SDPA on the host CPU, median of {n} "
                      f"runs after {CPU_WARMUP} warm-ups",
            "value_best": round(fl / best / 1e12, 4), "value_fp32": round(fl / med32 / 1e12, 4)}


# ----------------------------------------------------------------------------- main
# ----------------------------------------------------------------------------- output check
CHECK_TOL = 2e-2   # bf16 max-abs bound (north star)


def _norm_rope_fp32(x, w, cos, sin, eps=1e-6):
    """RMSNorm with gain w, then NEOX RoPE, in fp32 with one rounding to x's dtype: the
    arithmetic of the fused q/k load (reference fused_ops.py:53-85), as plain torch."""
    xf = x.float()
    y = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps) * w
    h = y.shape[-1] // 2
    return (y * cos + torch.cat([-y[..., h:], y[..., :h]], -1) * sin).to(x.dtype)


def check_decode(wl: "DecodeWorkload") -> float:
    """The last step's own output against fp32 torch attention on the GPU, for the longest
    and the shortest row, over the cache the step wrote (the new key at L - 1 must be the
    normalised, rotated one). Returns the max-abs error; raises if it exceeds CHECK_TOL."""
    assert wl.T == 1
    G = wl.H // wl.K
    i = (wl.layer - 1) % len(wl.k_caches)
    kc, vc = wl.k_caches[i], wl.v_caches[i]
    worst = 0.0
    for b in (max(range(wl.B), key=lambda r: wl.lens[r]), min(range(wl.B), key=lambda r: wl.lens[r])):
        L = wl.lens[b]
        c, s_ = wl.cos[b, 0], wl.sin[b, 0]
        kn = _norm_rope_fp32(wl.k[b, :, 0], wl.wk, c, s_).float()
        err_k = (kc[b, :, L - 1].float() - kn).abs().max().item()
        if not err_k <= CHECK_TOL * (1 + kn.abs().max().item()):
            raise RuntimeError(f"bench check: row {b}: the new key in the cache is off by {err_k:.3e}")
        qn = _norm_rope_fp32(wl.q[b, :, 0], wl.wq, c, s_).float().view(wl.K, G, wl.D)
        k, v = kc[b, :, :L].float(), vc[b, :, :L].float()
        p = (torch.matmul(qn, k.transpose(1, 2).contiguous()) * wl.scale).softmax(-1)
        y = torch.matmul(p, v).reshape(wl.H, wl.D)
        worst = max(worst, (wl.out[b, 0].float() - y).abs().max().item())
    if not worst <= CHECK_TOL:
        raise RuntimeError(f"bench check: decode output off by {worst:.3e} (bound {CHECK_TOL})")
    return worst


def check_prefill(pf: "PrefillWorkload", b: int = 0) -> float:
    """The last prefill's own output for batch row b (its first 64 and last 128 queries,
    every head) against fp32 causal attention in torch on the GPU over the cache the append
    wrote. Returns the max-abs error; raises if it exceeds CHECK_TOL."""
    G = pf.H // pf.K
    idx = torch.cat([torch.arange(64), torch.arange(pf.T - 128, pf.T)]).to(pf.out.device)
    qn = _norm_rope_fp32(pf.q[b][:, idx], pf.wq, pf.cos[idx], pf.sin[idx]).float()     # [H, n, D]
    k = pf.kc[b].float().repeat_interleave(G, 0)                                        # [H, T, D]
    v = pf.vc[b].float().repeat_interleave(G, 0)
    s = torch.matmul(qn, k.transpose(1, 2).contiguous()) * pf.scale                     # [H, n, T]
    s = s.masked_fill(torch.arange(pf.T, device=s.device)[None, None, :] > idx[None, :, None], float("-inf"))
    y = torch.matmul(s.softmax(-1), v)                                                  # [H, n, D]
    worst = (pf.out[b][idx].float() - y.transpose(0, 1)).abs().max().item()
    if not worst <= CHECK_TOL:
        raise RuntimeError(f"bench check: prefill output off by {worst:.3e} (bound {CHECK_TOL})")
    return worst


def mean_step_bytes(wl: "DecodeWorkload", lo: int = 1024, hi: int = 32768) -> float:
    """Algorithmic bytes of a step whose rows have the mean length of U[lo, hi]."""
    s = torch.finfo(wl.dtype).bits // 8
    return wl.step_bytes() + 2 * wl.K * wl.D * s * (wl.B * (lo + hi) / 2 - sum(wl.lens))


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-extra", action="store_true", help="skip the reported configs C2, C3-decode, C5")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--config", default="", help="with --only extra: run only the configs whose name contains this")
    ap.add_argument("--only", choices=["decode", "prefill", "prefill512", "copy", "gemm", "sdpa", "qkv", "extra"],
                    help="time one workload (for rocprofv3 runs); copy = a 1 GiB torch copy, the "
                         "known-size kernel that calibrates the HBM byte counters; gemm = a bf16 "
                         "library GEMM, the practical MFMA rate beside the vendor peak; sdpa = torch's "
                         "SDPA (the reference's GPU attention call) on the C3 shapes; qkv = the "
                         "module's q/k/v projections, separate against fused")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: the attention hot path runs on a single MI355X here "
              "(multi-GPU sharding is design-only). Run with --gpus 1.", file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    dt = torch.bfloat16

    if args.only:
        return run_only(args, dev)

    # ---- C4 ragged decode (headline)
    lens = c4_lengths(args.seed)
    wl = DecodeWorkload(lens, 16, 8, 128, 1e6, dt, dev, seed=args.seed)
    wl.append()  # write the new tokens once so the rows are complete before timing
    torch.cuda.synchronize()
    print(f"[bench] C4 decode: B=64, sum L = {sum(lens)}, chunk {wl.chunk}", file=sys.stderr, flush=True)
    warm(wl.step)
    t_step = time_loop(wl.step, args.steps, args.warmup)
    t_attn = time_loop(wl.attend, args.steps, args.warmup)
    t_two = time_loop(wl.step_two_pass, args.steps, args.warmup)
    step_gbs = wl.step_bytes() / t_step / 1e9
    attn_gbs = wl.attend_bytes() / t_attn / 1e9
    tok_s = wl.B / (N_LAYERS * t_step)
    print(f"[bench] C4 step {t_step * 1e6:.1f} us ({step_gbs:.0f} GB/s), attention call "
          f"{t_attn * 1e6:.1f} us ({attn_gbs:.0f} GB/s), two-call step {t_two * 1e6:.1f} us",
          file=sys.stderr, flush=True)
    wl.step()   # the timed call once more; its output is checked below
    torch.cuda.synchronize()
    err_decode = check_decode(wl)

    # ---- C3 prefill
    pf = PrefillWorkload(4, 4096, 16, 8, 128, 1e6, dt, dev)
    pf.append()
    warm(pf.step)
    t_pstep = time_loop(pf.step, max(3, args.steps // 2), max(1, args.warmup // 2))
    t_pattn = time_loop(pf.attend, max(3, args.steps // 2), max(1, args.warmup // 2))
    p_tflops = pf.flops() / t_pattn / 1e12
    p_step_tflops = pf.flops() / t_pstep / 1e12
    print(f"[bench] C3 prefill step {t_pstep * 1e6:.1f} us ({p_step_tflops:.0f} TFLOP/s), attention kernel "
          f"{t_pattn * 1e6:.1f} us ({p_tflops:.0f} TFLOP/s)", file=sys.stderr, flush=True)
    torch.cuda.synchronize()
    err_prefill = check_prefill(pf)
    print(f"[bench] outputs checked against fp32 torch: decode max-abs {err_decode:.2e} (longest and "
          f"shortest rows), prefill max-abs {err_prefill:.2e}", file=sys.stderr, flush=True)
    p_flops, p_flops_full = pf.flops(), pf.flops_full_s()
    del pf
    torch.cuda.empty_cache()
    # Gemma 4's full-attention layer shape: 1 x 4096 causal, 16 q / 1 KV head of 512 (reported)
    pg = PrefillWorkload(1, 4096, 16, 1, 512, 1e6, dt, dev)
    pg.append()
    warm(pg.attend)
    t_g4 = time_loop(pg.attend, max(3, args.steps // 2), max(1, args.warmup // 2))
    g4_prefill = {"config": "1 x 4096 causal, 16 q / 1 kv heads, head dim 512, bf16, QK-norm, RoPE theta 1e6",
                  "us": round(t_g4 * 1e6, 2), "TFLOPs": round(pg.flops() / t_g4 / 1e12, 1),
                  "frac": round(pg.flops() / t_g4 / 1e12 / BF16_PEAK_TFLOPS, 4),
                  "kernel": "forge::prefill_wide_kernel<bf16, 2>", "traffic": read_traffic("prefill_g4full_traffic")}
    print(f"[bench] Gemma-4 full-layer prefill (hd 512): {g4_prefill}", file=sys.stderr, flush=True)
    del pg
    torch.cuda.empty_cache()
    gemm = gemm_tflops(dev)
    print(f"[bench] bf16 8192^3 library GEMM {gemm:.0f} TFLOP/s", file=sys.stderr, flush=True)
    sdpa = sdpa_reference(dev)
    print(f"[bench] torch SDPA on the same GPU: {sdpa}", file=sys.stderr, flush=True)

    line = {
        "metric": METRIC,
        "value": round(step_gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(t_step * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "C4 ragged decode, one layer per step: batch 64, 16 q / 8 kv heads, head dim 128, "
                               "bf16, KV lengths U[1024, 32768] (seed 0), 1 new token per row, QK-norm, "
                               "RoPE theta 1e6",
                   "global_batch": wl.B, "kv_tokens": sum(lens), "chunk": wl.chunk,
                   "parallelism": "single GPU"},
        "decode_tokens_per_s": round(tok_s, 1),
        # this seed's draw has sum L = 948,477 keys, 12% below the distribution's mean of
        # 1,081,344; tokens/s at the same GB/s for a batch of the mean size
        "decode_tokens_per_s_at_mean_lengths": round(tok_s * wl.step_bytes() / mean_step_bytes(wl), 1),
        # the timed calls' own outputs against fp32 torch attention on the GPU (max-abs)
        "output_check": {"decode_max_abs": err_decode, "prefill_max_abs": err_prefill, "bound": CHECK_TOL},
        "decode_attention_call_us": round(t_attn * 1e6, 2),
        # the same step as forge_kv_append + forge_attn_decode (two launches, and the
        # persistent grid's ticket reset and the combine), for comparison
        "decode_step_two_calls_us": round(t_two * 1e6, 2),
        "prefill_tflops": round(p_tflops, 1),
        # the reference's convention (sleuth/forge/model/flops.py:84-89): 4*H*hd*S FLOPs per
        # token forward with S the full 4096, i.e. twice the causal count above; for
        # comparison only (the roofline fraction uses the causal count)
        "prefill_tflops_full_s_convention": round(p_tflops * p_flops_full / p_flops, 1),
        "prefill_step_ms": round(t_pstep * 1e3, 4),
        # the whole prefill step (forge_kv_append of the 4 x 4096 keys and values, then the
        # attention kernel) against the same causal FLOP count
        "prefill_step_tflops": round(p_step_tflops, 1),
        "warm_s": WARM_S,
        "prefill_config": "C3: 4 x 4096 causal, 16 q / 8 kv heads, head dim 128, bf16, QK-norm, RoPE theta 1e6",
        # the reference's own GPU attention call (torch SDPA, flash / memory-efficient backends)
        # on the same GPU and the C3 shapes, attention only
        "torch_sdpa_same_gpu": sdpa,
        # the step's one call: splitk_kernel (the new keys/values made and written inside)
        # + combine_kernel, launched by forge_attn_decode_append
        "roofline": {"bound": "hbm",
                     "kernel": "forge::splitk_kernel + combine_kernel (one forge_attn_decode_append call)",
                     "achieved": round(step_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(step_gbs / HBM_PEAK_GBS, 4),
                     "traffic": read_traffic("decode_c4_traffic"),
                     "algorithmic_bytes": wl.step_bytes()},
        # the attention alone (forge_attn_decode over the cache the step wrote)
        "decode_attention_call_GBs": round(attn_gbs, 1),
        "roofline_prefill": {"bound": "mfma", "kernel": "forge::prefill_kernel<bf16,128>",
                             "achieved": round(p_tflops, 1), "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                             "frac": round(p_tflops / BF16_PEAK_TFLOPS, 4),
                             "traffic": read_traffic("prefill_c3_traffic"), "flops": p_flops,
                             "library_gemm_tflops": round(gemm, 1),
                             "frac_of_library_gemm": round(p_tflops / gemm, 4)},
        "prefill_gemma4_full_hd512": g4_prefill,
    }
    if not args.no_cpu:
        print("[bench] CPU baseline (decode sample) ...", file=sys.stderr, flush=True)
        line["cpu_baseline"] = cpu_baseline_decode(wl)
        print("[bench] CPU baseline (prefill sample) ...", file=sys.stderr, flush=True)
        line["cpu_baseline_prefill"] = cpu_baseline_prefill(4, 4096, 16, 8, 128)
    else:
        line["cpu_baseline"] = None
    if not args.no_extra:
        line["configs"] = extra_configs(dev, args)
    print(json.dumps(line), flush=True)
    return 0


def gemm_tflops(dev, n: int = 8192, steps: int = 20, warmup: int = 5) -> float:
    """bf16 n x n x n torch.matmul (hipBLASLt on ROCm), in TFLOP/s: what a tuned library GEMM
    reaches on this GPU, reported beside the 2.5 PFLOP/s vendor figure the roofline uses."""
    g = torch.Generator(device=dev).manual_seed(0)
    a = torch.randn(n, n, device=dev, dtype=torch.bfloat16, generator=g)
    b = torch.randn(n, n, device=dev, dtype=torch.bfloat16, generator=g)
    c = torch.empty(n, n, device=dev, dtype=torch.bfloat16)
    warm(lambda: torch.matmul(a, b, out=c))
    t = time_loop(lambda: torch.matmul(a, b, out=c), steps, warmup)
    return 2.0 * n ** 3 / t / 1e12


def sdpa_reference(dev, steps: int = 10, warmup: int = 3) -> dict:
    """torch's scaled_dot_product_attention, the call the reference makes on the GPU
    (attention.py:187-191), on the C3 shapes, timed like the kernels here. Only the flash and
    memory-efficient backends are allowed (no math fallback); K/V heads are repeated to H
    (attention.py:181-182) so that no GQA path is involved. Attention only: the reference's
    norm, RoPE and cache update are not in the timing."""
    import torch.nn.functional as F
    from torch.nn.attention import SDPBackend, sdpa_kernel

    g = torch.Generator(device=dev).manual_seed(3)
    bf = torch.bfloat16
    out = {}
    backends = [SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]
    # C3 prefill: 4 x 4096 causal, 16 heads (8 KV heads repeated), head dim 128
    B, T, H, D = 4, 4096, 16, 128
    q = torch.randn(B, H, T, D, device=dev, dtype=bf, generator=g)
    k = torch.randn(B, H // 2, T, D, device=dev, dtype=bf, generator=g).repeat_interleave(2, 1)
    v = torch.randn(B, H // 2, T, D, device=dev, dtype=bf, generator=g).repeat_interleave(2, 1)
    fn = lambda: F.scaled_dot_product_attention(q, k, v, is_causal=True, scale=D ** -0.5)
    try:
        with sdpa_kernel(backends):
            warm(fn)
            t = time_loop(fn, steps, warmup)
        flops = 4 * D * H * B * (T * (T + 1) / 2)
        out["C3_prefill"] = {"us": round(t * 1e6, 2), "TFLOPs": round(flops / t / 1e12, 1)}
    except RuntimeError as e:
        out["C3_prefill"] = {"error": str(e)[:200]}
    del q, k, v
    # C3 decode: 32 rows at 8192 keys, one query each
    B, S = 32, 8192
    q = torch.randn(B, H, 1, D, device=dev, dtype=bf, generator=g)
    k = torch.randn(B, H // 2, S, D, device=dev, dtype=bf, generator=g).repeat_interleave(2, 1)
    v = torch.randn(B, H // 2, S, D, device=dev, dtype=bf, generator=g).repeat_interleave(2, 1)
    fn = lambda: F.scaled_dot_product_attention(q, k, v, scale=D ** -0.5)
    try:
        with sdpa_kernel(backends):
            t = time_loop(fn, steps * 2, warmup)
        kv_bytes = 2 * B * (H // 2) * S * D * 2  # the distinct K/V bytes a GQA kernel reads
        out["C3_decode"] = {"us": round(t * 1e6, 2), "GBs_of_distinct_kv": round(kv_bytes / t / 1e9, 1)}
    except RuntimeError as e:
        out["C3_decode"] = {"error": str(e)[:200]}
    del q, k, v
    # C4 ragged decode as the reference's eager path would run it: one SDPA per batch row over
    # that row's keys (its cache holds one position for the batch, kv_cache.py:34)
    lens = c4_lengths(0)
    B, S = len(lens), max(lens)
    q = torch.randn(B, H, 1, D, device=dev, dtype=bf, generator=g)
    k = torch.randn(B, H // 2, S, D, device=dev, dtype=bf, generator=g).repeat_interleave(2, 1)
    v = torch.randn(B, H // 2, S, D, device=dev, dtype=bf, generator=g).repeat_interleave(2, 1)
    rows = [(q[i:i + 1], k[i:i + 1, :, :L], v[i:i + 1, :, :L]) for i, L in enumerate(lens)]
    fn = lambda: [F.scaled_dot_product_attention(a, b_, c, scale=D ** -0.5) for a, b_, c in rows]
    try:
        with sdpa_kernel(backends):
            t = time_loop(fn, steps, warmup)
        kv_bytes = sum(2 * (H // 2) * L * D * 2 for L in lens)
        out["C4_decode_per_row"] = {"us": round(t * 1e6, 2), "GBs_of_distinct_kv": round(kv_bytes / t / 1e9, 1)}
    except RuntimeError as e:
        out["C4_decode_per_row"] = {"error": str(e)[:200]}
    return out


def qkv_projection(dev, steps: int = 50, warmup: int = 10) -> dict:
    """The attention module's q/k/v projections on the Qwen3-0.6B shapes (d_model 1024,
    16 q / 8 kv heads of 128): three nn.Linear calls (the reference, attention.py:106-108)
    against the module's one GEMM over the concatenated weights."""
    from sleuth_amd.attention import Attention
    from sleuth_amd.config import ModelConfig

    cfg = ModelConfig(d_model=1024, n_heads=16, head_size=128, n_kv_heads=8, qk_norm=True,
                      rope_theta=1e6, max_seq_len=8192)
    att = Attention(cfg, 0).to(dev).to(torch.bfloat16).eval()
    out = {}
    with torch.no_grad():
        for B, T in ((64, 1), (4, 4096)):
            x = torch.randn(B, T, cfg.d_model, device=dev, dtype=torch.bfloat16)
            sep = lambda: (att.q_proj(x), att.k_proj(x), att.v_proj(x))
            fus = lambda: att._qkv_fused(x)
            ts, tf = time_loop(sep, steps, warmup), time_loop(fus, steps, warmup)
            out[f"B{B}_T{T}"] = {"separate_us": round(ts * 1e6, 1), "fused_us": round(tf * 1e6, 1)}
    return out


def run_only(args, dev) -> int:
    """One workload's step loop and nothing else, for rocprofv3 runs."""
    if args.only == "decode":
        wl = DecodeWorkload(c4_lengths(args.seed), 16, 8, 128, 1e6, torch.bfloat16, dev, seed=args.seed)
        wl.append()
        warm(wl.step)
        t = time_loop(wl.step, args.steps, args.warmup)
        print(json.dumps({"workload": "C4 decode step", "us": round(t * 1e6, 2),
                          "GBs": round(wl.step_bytes() / t / 1e9, 1)}), flush=True)
    elif args.only == "prefill":
        pf = PrefillWorkload(4, 4096, 16, 8, 128, 1e6, torch.bfloat16, dev)
        warm(pf.step)
        t = time_loop(pf.step, args.steps, args.warmup)
        ta = time_loop(pf.attend, args.steps, args.warmup)
        print(json.dumps({"workload": "C3 prefill step", "us": round(t * 1e6, 2), "attention_us": round(ta * 1e6, 2),
                          "attention_tflops": round(pf.flops() / ta / 1e12, 1)}), flush=True)
    elif args.only == "prefill512":
        pf = PrefillWorkload(1, 4096, 16, 1, 512, 1e6, torch.bfloat16, dev)
        pf.append()
        warm(pf.attend)
        ta = time_loop(pf.attend, args.steps, args.warmup)
        print(json.dumps({"workload": "Gemma-4 full-layer prefill, 1 x 4096, 16 q / 1 kv heads, hd 512",
                          "attention_us": round(ta * 1e6, 2), "attention_tflops": round(pf.flops() / ta / 1e12, 1)}),
              flush=True)
    elif args.only == "extra":
        print(json.dumps(extra_configs(dev, args)), flush=True)
    elif args.only == "sdpa":
        print(json.dumps({"workload": "torch SDPA on the C3 shapes and C4 row by row", **sdpa_reference(dev)}), flush=True)
    elif args.only == "qkv":
        print(json.dumps({"workload": "q/k/v projections, Qwen3-0.6B shapes", **qkv_projection(dev)}), flush=True)
    elif args.only == "gemm":
        print(json.dumps({"workload": "bf16 8192^3 torch.matmul", "TFLOPs": round(gemm_tflops(dev), 1)}),
              flush=True)
    else:
        n = 1 << 30
        src = torch.empty(n, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        t = time_loop(lambda: dst.copy_(src), args.steps, args.warmup)
        print(json.dumps({"workload": "copy 1 GiB", "bytes_read": n, "bytes_written": n, "us": round(t * 1e6, 2),
                          "GBs": round(2 * n / t / 1e9, 1)}), flush=True)
    return 0


EXTRA_CONFIGS = {
    "C2_decode_b16_12q4kv_hd64_S2048": dict(lens=[2049] * 16, H=12, K=4, D=64, theta=1e4, n_layers=12),
    "C3_decode_b32_16q8kv_hd128_S8192": dict(lens=[8192] * 32, H=16, K=8, D=128, theta=1e6, n_layers=1),
    "C5_verify_b8_T4_8q1kv_hd256_global": dict(lens=[8196] * 8, H=8, K=1, D=256, theta=1e6, T=4, n_layers=12),
    "C5_verify_b8_T4_8q1kv_hd256_window1024": dict(lens=[8196] * 8, H=8, K=1, D=256, theta=1e6, T=4,
                                                   window=1024, n_layers=12),
    # Gemma 4's full-attention layer shape (1 KV head of 512, kv_cache.py:12-13): decode and a
    # 4-token verify (not a BASELINE config; reported beside them)
    "G4full_decode_b16_16q1kv_hd512_S8192": dict(lens=[8192] * 16, H=16, K=1, D=512, theta=1e6, n_layers=2),
    "G4full_verify_b16_T4_16q1kv_hd512_S8192": dict(lens=[8192] * 16, H=16, K=1, D=512, theta=1e6, T=4,
                                                    n_layers=2),
}
# the rocprofv3 traffic summary of each (profiles/<name>.txt)
EXTRA_TRAFFIC = {
    "C2_decode_b16_12q4kv_hd64_S2048": "decode_c2_traffic",
    "C3_decode_b32_16q8kv_hd128_S8192": "decode_c3_traffic",
    "C5_verify_b8_T4_8q1kv_hd256_global": "verify_c5_global_traffic",
    "C5_verify_b8_T4_8q1kv_hd256_window1024": "verify_c5_window1024_traffic",
    "G4full_decode_b16_16q1kv_hd512_S8192": "decode_g4full_traffic",
    "G4full_verify_b16_T4_16q1kv_hd512_S8192": "verify_g4full_traffic",
}


def extra_configs(dev, args) -> dict:
    """Configs C2, C3-decode and C5, and Gemma 4's full-attention layer shape (reported;
    BASELINE sets no target for them). Small
    working sets rotate through several layer caches so the ~256 MB MALL does not serve
    them. The roofline uses the attention call replayed from a HIP graph (how decode steps
    run, and without the host's per-call launch cost, which exceeds these calls' GPU time);
    the eager step (append + attention) and eager attention call are reported beside it."""
    out = {}
    dt = torch.bfloat16
    for name, kw in EXTRA_CONFIGS.items():
        if args.config and args.config not in name:
            continue
        kw = dict(kw)
        lens = kw.pop("lens")
        wl = DecodeWorkload(lens, dtype=dt, dev=dev, **kw)
        for i in range(len(wl.k_caches)):
            wl.append(i)
        torch.cuda.synchronize()
        t = time_loop(wl.step, args.steps * 4, args.warmup)
        t2 = time_loop(wl.step_two_pass, args.steps * 4, args.warmup)
        ta = time_loop(lambda: (wl.attend(), setattr(wl, "layer", (wl.layer + 1) % len(wl.k_caches))),
                       args.steps * 4, args.warmup)
        tg = time_graph(lambda i: wl.attend(i), len(wl.k_caches), args.steps, args.warmup)
        gbs = wl.attend_bytes() / tg / 1e9
        out[name] = {"step_us": round(t * 1e6, 2), "step_GBs": round(wl.step_bytes() / t / 1e9, 1),
                     "step_two_calls_us": round(t2 * 1e6, 2), "attention_call_us": round(ta * 1e6, 2),
                     "attention_graph_us": round(tg * 1e6, 2), "chunk": wl.chunk,
                     "layer_caches_rotated": len(wl.k_caches),
                     "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                                  "frac": round(gbs / HBM_PEAK_GBS, 4), "algorithmic_bytes": wl.attend_bytes(),
                                  "traffic": read_traffic(EXTRA_TRAFFIC[name])}}
        print(f"[bench] {name}: {out[name]}", file=sys.stderr, flush=True)
        del wl
        torch.cuda.empty_cache()
    return out


if __name__ == "__main__":
    sys.exit(main())
