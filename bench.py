"""Benchmark of the FORGE attention hot path on one MI355X.

Headline (BASELINE.json metric): decode attention of config C4 -- batch 64, Qwen3-0.6B
heads (16 q / 8 kv, head dim 128, bf16), per-row KV lengths uniform in [1024, 32768]
from a seed, one new token per row. A step is one layer's attention for the batch:
the new K/V are normalised/rotated and appended to the cache (forge_kv_append), then
split-K attention with the q norm + RoPE fused (forge_attn_decode). `value` is the
step's algorithmic HBM bytes / step time (GB/s); tokens/s = 64 / (28 layers x step).
Beside it: C3 causal prefill (4 x 4096 tokens, bf16) in TFLOP/s, each dominant kernel's
roofline fraction, and the oracle (torch SDPA on the CPU) timed on a bounded sample.

Usage: python bench.py [--gpus 1] [--steps 20] [--warmup 5] [--no-cpu] [--extra]
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
PREFILL_WARM_S = 0.1         # untimed back-to-back calls before an MFMA-bound timing
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

        self.chunk = ops.decode_chunk(dtype, B, T, H, K, D, self.max_len, window)
        nbytes = ops.decode_workspace_bytes(dtype, B, T, H, K, D, self.max_len, self.chunk)
        self.ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev)
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


def warm(fn, seconds: float = PREFILL_WARM_S) -> int:
    """Runs fn back to back for about `seconds` of GPU time before a timing: an MFMA-heavy
    kernel only reaches its steady clock after some tens of milliseconds of load (C3 prefill
    on MI355X: about 355 us per call in the first 20 calls, 290 us from about the 60th on).
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
def cpu_info() -> dict:
    model = "unknown"
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"model": model, "logical": os.cpu_count(), "affinity": len(os.sched_getaffinity(0))}


def cpu_baseline_decode(wl: DecodeWorkload, budget_s: float = 15.0) -> dict:
    """The oracle's eager CPU path (torch SDPA on the host, bf16, one SDPA per row over
    its prefix, attention.py:171-193) on the first rows of the same batch: add rows
    until about budget_s of CPU work, then report GB/s of algorithmic bytes."""
    import oracle

    threads = min(16, len(os.sched_getaffinity(0)))
    torch.set_num_threads(threads)
    B, H, K, D = wl.B, wl.H, wl.K, wl.D
    q = oracle.head_norm_rope(wl.q.cpu(), wl.wq.cpu(), 1e-6, wl.cos.cpu(), wl.sin.cpu())
    layer = wl.k_caches[0], wl.v_caches[0]
    rows, total_b, total_t = 0, 0, 0.0
    s = torch.finfo(wl.dtype).bits // 8
    for b in range(B):
        L = wl.lens[b]
        kc = layer[0][b:b + 1, :, :L].cpu()
        vc = layer[1][b:b + 1, :, :L].cpu()
        oracle.ragged_decode(q[b:b + 1], kc, vc, [L], wl.window, wl.scale)  # warm
        t0 = time.perf_counter()
        reps = 3
        for _ in range(reps):
            oracle.ragged_decode(q[b:b + 1], kc, vc, [L], wl.window, wl.scale)
        dt = (time.perf_counter() - t0) / reps
        rows += 1
        total_t += dt
        total_b += 2 * K * wl.visible(L) * D * s + 2 * H * wl.T * D * s
        if total_t * (reps + 1) > budget_s:
            break
    # the same rows in fp32 (same algorithmic bytes), one run each after a warm-up
    t32 = 0.0
    for b in range(rows):
        L = wl.lens[b]
        kc = layer[0][b:b + 1, :, :L].float().cpu()
        vc = layer[1][b:b + 1, :, :L].float().cpu()
        q32 = q[b:b + 1].float()
        oracle.ragged_decode(q32, kc, vc, [L], wl.window, wl.scale)
        t0 = time.perf_counter()
        oracle.ragged_decode(q32, kc, vc, [L], wl.window, wl.scale)
        t32 += time.perf_counter() - t0
    return {"value": round(total_b / total_t / 1e9, 3), "unit": "GB/s", "cores": threads,
            "kind": "port",
            "sample": f"rows 0..{rows - 1} of the C4 batch ({sum(wl.lens[:rows])} cached tokens), one layer, "
                      f"bf16 torch SDPA on the host CPU, median-free mean of 3 runs per row",
            "value_fp32": round(total_b / t32 / 1e9, 3),
            "cpu": cpu_info()}


def cpu_baseline_prefill(B, T, H, K, D, budget_s: float = 10.0) -> dict:
    """torch SDPA (is_causal, enable_gqa) on the host in bf16 at the C3 shape, one
    batch row (the sample), TFLOP/s."""
    threads = min(16, len(os.sched_getaffinity(0)))
    torch.set_num_threads(threads)
    g = torch.Generator().manual_seed(2)
    q = torch.randn(1, H, T, D, generator=g).bfloat16()
    k = torch.randn(1, K, T, D, generator=g).bfloat16()
    v = torch.randn(1, K, T, D, generator=g).bfloat16()
    f = lambda: torch.nn.functional.scaled_dot_product_attention(q, k, v, is_causal=True,  # noqa: E731
                                                                  enable_gqa=True, scale=D ** -0.5)
    f()
    t0 = time.perf_counter()
    n = 0
    while time.perf_counter() - t0 < budget_s / 2 or n < 2:
        f()
        n += 1
    dt = (time.perf_counter() - t0) / n
    fl = 4.0 * D * H * T * (T + 1) / 2
    q, k, v = q.float(), k.float(), v.float()  # the same in fp32
    f()
    t0 = time.perf_counter()
    n32 = 0
    while time.perf_counter() - t0 < budget_s / 4 or n32 < 2:
        f()
        n32 += 1
    dt32 = (time.perf_counter() - t0) / n32
    return {"value": round(fl / dt / 1e12, 4), "unit": "TFLOP/s", "cores": threads, "kind": "port",
            "sample": f"1 of the {B} batch rows ({T} tokens causal), bf16 torch SDPA, mean of {n} runs",
            "value_fp32": round(fl / dt32 / 1e12, 4)}


# ----------------------------------------------------------------------------- main
def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--extra", action="store_true", help="also print lines for configs C2, C3-decode, C5")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--config", default="", help="with --only extra: run only the configs whose name contains this")
    ap.add_argument("--only", choices=["decode", "prefill", "copy", "gemm", "sdpa", "qkv", "extra"],
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
    t_step = time_loop(wl.step, args.steps, args.warmup)
    t_attn = time_loop(wl.attend, args.steps, args.warmup)
    step_gbs = wl.step_bytes() / t_step / 1e9
    attn_gbs = wl.attend_bytes() / t_attn / 1e9
    tok_s = wl.B / (N_LAYERS * t_step)
    print(f"[bench] C4 step {t_step * 1e6:.1f} us ({step_gbs:.0f} GB/s), attention call "
          f"{t_attn * 1e6:.1f} us ({attn_gbs:.0f} GB/s)", file=sys.stderr, flush=True)

    # ---- C3 prefill
    pf = PrefillWorkload(4, 4096, 16, 8, 128, 1e6, dt, dev)
    pf.append()
    warm(pf.step)
    t_pstep = time_loop(pf.step, max(3, args.steps // 2), max(1, args.warmup // 2))
    t_pattn = time_loop(pf.attend, max(3, args.steps // 2), max(1, args.warmup // 2))
    p_tflops = pf.flops() / t_pattn / 1e12
    print(f"[bench] C3 prefill step {t_pstep * 1e6:.1f} us, attention kernel {t_pattn * 1e6:.1f} us "
          f"({p_tflops:.0f} TFLOP/s)", file=sys.stderr, flush=True)
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
        "decode_attention_call_us": round(t_attn * 1e6, 2),
        "prefill_tflops": round(p_tflops, 1),
        # the reference's convention (sleuth/forge/model/flops.py:84-89): 4*H*hd*S FLOPs per
        # token forward with S the full 4096, i.e. twice the causal count above; for
        # comparison only (the roofline fraction uses the causal count)
        "prefill_tflops_full_s_convention": round(p_tflops * pf.flops_full_s() / pf.flops(), 1),
        "prefill_step_ms": round(t_pstep * 1e3, 4),
        "prefill_warm_s": PREFILL_WARM_S,
        "prefill_config": "C3: 4 x 4096 causal, 16 q / 8 kv heads, head dim 128, bf16, QK-norm, RoPE theta 1e6",
        # the reference's own GPU attention call (torch SDPA, flash / memory-efficient backends)
        # on the same GPU and the C3 shapes, attention only
        "torch_sdpa_same_gpu": sdpa,
        "roofline": {"bound": "hbm", "kernel": "forge::splitk_kernel + combine_kernel (one forge_attn_decode call)",
                     "achieved": round(attn_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(attn_gbs / HBM_PEAK_GBS, 4),
                     "traffic": read_traffic("decode_c4_traffic"),
                     "algorithmic_bytes": wl.attend_bytes()},
        "roofline_prefill": {"bound": "mfma", "kernel": "forge::prefill_kernel<bf16,128>",
                             "achieved": round(p_tflops, 1), "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                             "frac": round(p_tflops / BF16_PEAK_TFLOPS, 4),
                             "traffic": read_traffic("prefill_c3_traffic"), "flops": pf.flops(),
                             "library_gemm_tflops": round(gemm, 1),
                             "frac_of_library_gemm": round(p_tflops / gemm, 4)},
    }
    if not args.no_cpu:
        print("[bench] CPU baseline (decode sample) ...", file=sys.stderr, flush=True)
        line["cpu_baseline"] = cpu_baseline_decode(wl)
        print("[bench] CPU baseline (prefill sample) ...", file=sys.stderr, flush=True)
        line["cpu_baseline_prefill"] = cpu_baseline_prefill(4, 4096, 16, 8, 128)
    else:
        line["cpu_baseline"] = None
    if args.extra:
        line["extra"] = extra_configs(dev, args)
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
        t = time_loop(wl.step, args.steps, args.warmup)
        print(json.dumps({"workload": "C4 decode step", "us": round(t * 1e6, 2),
                          "GBs": round(wl.step_bytes() / t / 1e9, 1)}), flush=True)
    elif args.only == "prefill":
        pf = PrefillWorkload(4, 4096, 16, 8, 128, 1e6, torch.bfloat16, dev)
        warm(pf.step)
        t = time_loop(pf.step, args.steps, args.warmup)
        print(json.dumps({"workload": "C3 prefill step", "us": round(t * 1e6, 2)}), flush=True)
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


def extra_configs(dev, args) -> dict:
    """Configs C2, C3-decode and C5 (reported, no targets). Small working sets rotate
    through several layer caches so the ~256 MB MALL does not serve them."""
    out = {}
    dt = torch.bfloat16
    for name, kw in {
        "C2_decode_b16_12q4kv_hd64_S2048": dict(lens=[2049] * 16, H=12, K=4, D=64, theta=1e4, n_layers=12),
        "C3_decode_b32_16q8kv_hd128_S8192": dict(lens=[8192] * 32, H=16, K=8, D=128, theta=1e6, n_layers=1),
        "C5_verify_b8_T4_8q1kv_hd256_global": dict(lens=[8196] * 8, H=8, K=1, D=256, theta=1e6, T=4, n_layers=12),
        "C5_verify_b8_T4_8q1kv_hd256_window1024": dict(lens=[8196] * 8, H=8, K=1, D=256, theta=1e6, T=4,
                                                       window=1024, n_layers=12),
    }.items():
        if args.config and args.config not in name:
            continue
        lens = kw.pop("lens")
        wl = DecodeWorkload(lens, dtype=dt, dev=dev, **kw)
        for i in range(len(wl.k_caches)):
            wl.append(i)
        torch.cuda.synchronize()
        t = time_loop(wl.step, args.steps * 4, args.warmup)
        ta = time_loop(lambda: (wl.attend(), setattr(wl, "layer", (wl.layer + 1) % len(wl.k_caches))),
                       args.steps * 4, args.warmup)
        tg = time_graph(lambda i: wl.attend(i), len(wl.k_caches), args.steps, args.warmup)
        out[name] = {"step_us": round(t * 1e6, 2), "step_GBs": round(wl.step_bytes() / t / 1e9, 1),
                     "attention_call_us": round(ta * 1e6, 2),
                     "attention_GBs": round(wl.attend_bytes() / ta / 1e9, 1),
                     "attention_graph_us": round(tg * 1e6, 2),
                     "attention_graph_GBs": round(wl.attend_bytes() / tg / 1e9, 1), "chunk": wl.chunk}
        print(f"[bench] {name}: {out[name]}", file=sys.stderr, flush=True)
        del wl
        torch.cuda.empty_cache()
    return out


if __name__ == "__main__":
    sys.exit(main())
