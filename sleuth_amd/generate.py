"""The callers the attention path has to serve: plain decoding, speculative
draft-then-verify, and graph-captured static decoding.

generate()             sleuth/forge/infer/generate.py:49-136 (prefill, then one token
                       per step through the cache; greedy or temperature sampling)
speculative_generate() sleuth/forge/infer/speculative.py:83-277 (verify = one forward of
                       [pending] + k guesses at offset cache.pos; keep() rewinds pos)
GraphDecoder           sleuth/forge/infer/cuda_graph.py:33-144 (StaticKVCache, one HIP
                       graph per length bucket 64, 128, ..., max_len; verify() runs
                       tokens_per_step tokens)
Greedy output is what the tests compare; sampling policies beyond temperature are out
of scope (they act after attention).
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Callable

import torch

from .kv_cache import KVCache, StaticKVCache


@dataclass
class GenerationResult:
    prompt_ids: list[int]
    new_ids: list[int]
    stop_reason: str
    stats: dict = field(default_factory=dict)


def _choose(logits: torch.Tensor, temperature: float, gen) -> torch.Tensor:
    if temperature <= 0:
        return logits.argmax(-1)
    probs = (logits.float() / temperature).softmax(-1)
    return torch.multinomial(probs, 1, generator=gen).view(-1)


@torch.no_grad()
def generate(model, prompt_ids: list[int], max_new_tokens: int = 32, temperature: float = 0.0,
             stop_ids: set[int] | None = None, seed: int | None = None, cuda_graph: bool = False,
             cache_dtype: torch.dtype | None = None) -> GenerationResult:
    if not prompt_ids:
        raise ValueError("prompt must contain at least one token")
    p = next(model.parameters())
    dev, max_len = p.device, model.cfg.max_seq_len
    stop_ids = stop_ids or set()
    gen = torch.Generator(device=dev)
    gen.manual_seed(0 if seed is None else seed)
    dtype = cache_dtype or p.dtype
    decoder = None
    if cuda_graph:
        decoder = decoder_for(model, max_len, dtype=dtype)
        cache = decoder.cache
    else:
        cache = KVCache.for_model(model, 1, max_len, dtype)
    model.eval()
    logits = model(torch.tensor([prompt_ids], device=dev), cache=cache).logits[:, -1]
    new, reason = [], "max_new_tokens"
    for _ in range(max_new_tokens):
        nxt = _choose(logits, temperature, gen)
        tok = int(nxt.item())
        new.append(tok)
        if tok in stop_ids:
            reason = "stop_token"
            break
        if cache.pos >= max_len:
            reason = "context_full"
            break
        if decoder is not None:
            logits = decoder.step(nxt.view(1))
        else:
            logits = model(nxt.view(1, 1), cache=cache).logits[:, -1]
    stats = {"kv_cache_mb": round(cache.nbytes() / 1e6, 2)}
    if decoder is not None:
        stats["graphs"] = sorted(decoder.graphs)
    return GenerationResult(list(prompt_ids), new, reason, stats)


def ngram_draft(max_ngram: int = 3) -> Callable[[list[int], int], list[int]]:
    """Prompt-lookup drafter: the tokens that followed the latest earlier occurrence of
    the longest suffix n-gram (n <= max_ngram)."""
    def draft(ids: list[int], k: int) -> list[int]:
        for n in range(min(max_ngram, len(ids) - 1), 0, -1):
            tail = ids[-n:]
            for start in range(len(ids) - n - 1, -1, -1):
                if ids[start:start + n] == tail:
                    return ids[start + n:start + n + k]
        return []
    return draft


@torch.no_grad()
def speculative_generate(model, prompt_ids: list[int], max_new_tokens: int = 32, k: int = 4,
                         draft: Callable[[list[int], int], list[int]] | None = None,
                         cuda_graph: bool = False, cache_dtype: torch.dtype | None = None) -> GenerationResult:
    """Greedy draft-then-verify: each round runs [pending] + guesses in one forward at
    offset cache.pos (T = 1 + k), keeps the longest agreeing prefix and rewinds pos."""
    draft = draft or ngram_draft()
    p = next(model.parameters())
    dev, max_len = p.device, model.cfg.max_seq_len
    dtype = cache_dtype or p.dtype
    decoder = decoder_for(model, max_len, dtype=dtype, tokens_per_step=k + 1) if cuda_graph else None
    cache = decoder.cache if decoder is not None else KVCache.for_model(model, 1, max_len, dtype)
    model.eval()
    logits = model(torch.tensor([prompt_ids], device=dev), cache=cache).logits[0, -1]
    ids, new = list(prompt_ids), []
    stats = {"forwards": 0, "drafted": 0, "accepted": 0}
    tok = int(logits.argmax())
    ids.append(tok)
    new.append(tok)
    while len(new) < max_new_tokens:
        pending = new[-1]
        room = min(k, max_new_tokens - len(new), max_len - cache.pos - 1)
        if room < 0:
            break
        guess = draft(ids, room)[:room] if room > 0 else []
        start = cache.pos
        if decoder is not None and start + k + 1 <= max_len:
            padded = [pending] + guess + [pending] * (k - len(guess))
            out = decoder.verify(torch.tensor(padded, device=dev))
        else:
            out = model(torch.tensor([[pending] + guess], device=dev), cache=cache).logits[0]
            cache.pos = start
        stats["forwards"] += 1
        stats["drafted"] += len(guess)
        choice = out[: len(guess) + 1].argmax(-1).tolist()
        n_ok = 0
        while n_ok < len(guess) and choice[n_ok] == guess[n_ok]:
            n_ok += 1
        stats["accepted"] += n_ok
        accepted = guess[:n_ok] + [choice[n_ok]]
        cache.pos = start + 1 + n_ok          # keep(): the pending token + accepted guesses
        for t in accepted:
            if len(new) >= max_new_tokens:
                break
            ids.append(t)
            new.append(t)
    res = GenerationResult(list(prompt_ids), new, "max_new_tokens", {"speculative": stats})
    if decoder is not None:
        res.stats["graphs"] = sorted(decoder.graphs)
    return res


# ----------------------------------------------------------------------------- graphs
def _buckets(max_len: int, smallest: int = 64) -> list[int]:
    out, b = [], smallest
    while b < max_len:
        out.append(b)
        b *= 2
    return out + [max_len]


def decoder_for(model, max_len: int, dtype: torch.dtype, tokens_per_step: int = 1) -> "GraphDecoder":
    decs = model.__dict__.setdefault("_graph_decoders", {})
    key = (max_len, tokens_per_step, dtype)
    if key not in decs:
        decs[key] = GraphDecoder(model, max_len, dtype, tokens_per_step)
    decs[key].cache.reset()
    return decs[key]


class GraphDecoder:
    """Static-shape decode/verify steps replayed as HIP graphs (torch.cuda.CUDAGraph is
    hipGraph on ROCm), one per length bucket. The position lives in cache.pos_t, the
    attention kernels read it on the device, and they read only the live keys
    (pos_t + T) instead of the whole bucket."""

    def __init__(self, model, max_len: int, dtype: torch.dtype, tokens_per_step: int = 1):
        p = next(model.parameters())
        if p.device.type != "cuda":
            raise ValueError("graph decoding needs a model on the GPU")
        self.model, self.device, self.max_len, self.T = model, p.device, max_len, tokens_per_step
        shapes = [(model.cfg.attn_spec(i).kv_heads, model.cfg.attn_spec(i).head_dim)
                  for i in range(model.cfg.n_layers)]
        self.cache = StaticKVCache(shapes, 1, max_len, self.device, dtype, tokens_per_step)
        self.token = torch.zeros(1, self.T, dtype=torch.long, device=self.device)
        self.graphs: dict[int, tuple[torch.cuda.CUDAGraph, torch.Tensor]] = {}
        self.pool = torch.cuda.graph_pool_handle()
        self.buckets = _buckets(max_len)

    def _forward(self):
        return self.model(self.token, cache=self.cache).logits[0]

    def _record(self, length: int):
        self.cache.length = length
        side = torch.cuda.Stream(self.device)
        side.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(side):
            for _ in range(2):
                self._forward()
        torch.cuda.current_stream(self.device).wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, pool=self.pool):
            out = self._forward()
        self.graphs[length] = (graph, out)

    @torch.no_grad()
    def _run(self, tokens: torch.Tensor) -> torch.Tensor:
        pos = self.cache.pos
        if pos + self.T > self.max_len:
            raise ValueError(f"KV cache full ({self.max_len} tokens)")
        length = next(b for b in self.buckets if b >= pos + self.T)
        self.token.copy_(tokens.view(1, self.T))
        self.cache.pos_t.fill_(pos)
        self.cache.static = True
        try:
            if length not in self.graphs:
                self._record(length)
            self.cache.length = length
            graph, out = self.graphs[length]
            graph.replay()
        finally:
            self.cache.static = False
        return out

    def step(self, token: torch.Tensor) -> torch.Tensor:
        if self.T != 1:
            raise ValueError("step() is for one token at a time; use verify()")
        out = self._run(token)
        self.cache.pos += 1
        return out

    def verify(self, tokens: torch.Tensor) -> torch.Tensor:
        return self._run(tokens)

