"""The callers the attention path has to serve: plain decoding, speculative
draft-then-verify, and graph-replayed decode steps.

generate()             the decode loop of sleuth/forge/infer/generate.py:49-136: the prompt's
                       prefill, then one token per step through the cache (greedy or
                       temperature sampling)
speculative_generate() greedy draft-then-verify as in speculative.py:83-277: [pending] + k
                       guesses in one forward at offset cache.pos, the agreeing prefix kept by
                       moving pos back (the rewind the reference's keep() does)
GraphDecoder           decode/verify steps replayed from a HIP graph (the role of
                       cuda_graph.py:67-144), built for kernels that read the live length on
                       the device: the attention reads only the keys below pos_t + T, whatever
                       the graph was recorded at, so ONE graph per step size serves every
                       context length -- no length buckets, no re-recording as the context
                       grows, no masked reads of a bucket's unused tail.
Sampling policies beyond temperature act after attention and are out of scope.
"""

from __future__ import annotations

import weakref
from dataclasses import dataclass, field
from typing import Callable

import torch

from .kv_cache import KVCache


@dataclass
class GenerationResult:
    prompt_ids: list[int]
    new_ids: list[int]
    stop_reason: str
    stats: dict = field(default_factory=dict)


def _pick(logits: torch.Tensor, temperature: float, gen: torch.Generator) -> torch.Tensor:
    """Next token id(s) [n] from logits [n, vocab]: argmax, or a draw at `temperature`."""
    if temperature > 0:
        return torch.multinomial((logits.float() / temperature).softmax(-1), 1, generator=gen).view(-1)
    return logits.argmax(-1)


class GraphDecoder:
    """Batch-1 decode (`step`) or verify (`verify`) steps of `tokens_per_step` tokens,
    recorded into one HIP graph (torch.cuda.CUDAGraph is hipGraph on ROCm) on first use and
    replayed afterwards. The position lives in cache.pos_t on the device; the host copies the
    new token ids and the position into the graph's input buffers before each replay.
    Use `cache` for the prompt's prefill (an ordinary eager forward)."""

    def __init__(self, model, max_len: int, dtype: torch.dtype, tokens_per_step: int = 1):
        p = next(model.parameters())
        if p.device.type != "cuda":
            raise ValueError("graph decoding needs a model on the GPU")
        self.model, self.T = model, tokens_per_step
        self.cache = KVCache.for_model(model, 1, max_len, dtype, tokens_per_step)
        self._ids = torch.zeros(1, tokens_per_step, dtype=torch.long, device=p.device)
        self._graph: torch.cuda.CUDAGraph | None = None
        self._logits: torch.Tensor | None = None
        self.replays = 0

    @property
    def recorded(self) -> bool:
        return self._graph is not None

    def _pass(self) -> torch.Tensor:
        return self.model(self._ids, cache=self.cache).logits[0]

    def _record(self) -> None:
        # one eager pass first (on a side stream, as graph capture wants): first-use
        # self-checks, library workspaces and the fused projection weights are set up
        # outside the capture; it writes the same K/V the real step writes
        side = torch.cuda.Stream(self._ids.device)
        side.wait_stream(torch.cuda.current_stream(self._ids.device))
        with torch.cuda.stream(side):
            self._pass()
        torch.cuda.current_stream(self._ids.device).wait_stream(side)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            self._logits = self._pass()
        self._graph = g

    @torch.no_grad()
    def _launch(self, tokens: torch.Tensor) -> torch.Tensor:
        c = self.cache
        if c.pos + self.T > c.max_len:
            raise ValueError(f"KV cache full ({c.max_len} tokens)")
        self._ids.copy_(tokens.view(1, self.T))
        c.pos_t.fill_(c.pos)
        c.static = True
        try:
            if self._graph is None:
                self._record()
            self._graph.replay()
        finally:
            c.static = False
        self.replays += 1
        return self._logits

    def step(self, token: torch.Tensor) -> torch.Tensor:
        """Logits [1, vocab] of `token` at position cache.pos; the cache moves on by one.
        The result is the graph's output buffer: read it before the next replay."""
        if self.T != 1:
            raise ValueError("step() is for one token at a time; use verify()")
        logits = self._launch(token)
        self.cache.pos += 1
        return logits

    def verify(self, tokens: torch.Tensor) -> torch.Tensor:
        """Logits [T, vocab] of T tokens at positions cache.pos, ...; cache.pos stays (the
        caller sets it to what it keeps)."""
        return self._launch(tokens)


_decoders: "weakref.WeakKeyDictionary[torch.nn.Module, dict]" = weakref.WeakKeyDictionary()


def decoder_for(model, max_len: int, dtype: torch.dtype, tokens_per_step: int = 1) -> GraphDecoder:
    """The model's graph decoder for this context and step size, kept across calls (the
    graph is recorded once per model); its cache is rewound for the new prompt."""
    per_model = _decoders.setdefault(model, {})
    dec = per_model.get((max_len, tokens_per_step, dtype))
    if dec is None:
        dec = per_model[(max_len, tokens_per_step, dtype)] = GraphDecoder(model, max_len, dtype, tokens_per_step)
    dec.cache.reset()
    return dec


@torch.no_grad()
def generate(model, prompt_ids: list[int], max_new_tokens: int = 32, temperature: float = 0.0,
             stop_ids: set[int] | None = None, seed: int | None = None, cuda_graph: bool = False,
             cache_dtype: torch.dtype | None = None) -> GenerationResult:
    if not prompt_ids:
        raise ValueError("prompt must contain at least one token")
    p = next(model.parameters())
    max_len = model.cfg.max_seq_len
    gen = torch.Generator(device=p.device).manual_seed(seed or 0)
    dec = decoder_for(model, max_len, cache_dtype or p.dtype) if cuda_graph else None
    cache = dec.cache if dec is not None else KVCache.for_model(model, 1, max_len, cache_dtype or p.dtype)
    model.eval()
    logits = model(torch.tensor([prompt_ids], device=p.device), cache=cache).logits[:, -1]
    new: list[int] = []
    reason = "max_new_tokens"
    while max_new_tokens > 0:
        tok = _pick(logits, temperature, gen)
        new.append(int(tok.item()))
        if stop_ids and new[-1] in stop_ids:
            reason = "stop_token"
            break
        if len(new) == max_new_tokens:
            break
        if cache.pos >= max_len:
            reason = "context_full"
            break
        logits = dec.step(tok.view(1)) if dec is not None else model(tok.view(1, 1), cache=cache).logits[:, -1]
    stats = {"kv_cache_mb": round(cache.nbytes() / 1e6, 2)}
    if dec is not None:
        stats["graph_replays"] = dec.replays
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
    max_len = model.cfg.max_seq_len
    dtype = cache_dtype or p.dtype
    dec = decoder_for(model, max_len, dtype, tokens_per_step=k + 1) if cuda_graph else None
    cache = dec.cache if dec is not None else KVCache.for_model(model, 1, max_len, dtype)
    model.eval()
    logits = model(torch.tensor([prompt_ids], device=p.device), cache=cache).logits[0, -1]
    ids = list(prompt_ids) + [int(logits.argmax())]
    new = ids[len(prompt_ids):]
    stats = {"forwards": 0, "drafted": 0, "accepted": 0}
    while len(new) < max_new_tokens:
        room = min(k, max_new_tokens - len(new), max_len - cache.pos - 1)
        if room < 0:
            break
        guess = draft(ids, room)[:room] if room > 0 else []
        start = cache.pos
        if dec is not None and start + k + 1 <= max_len:
            row = [new[-1]] + guess + [new[-1]] * (k - len(guess))   # fixed T: pad the guesses
            out = dec.verify(torch.tensor(row, device=p.device))
        else:
            out = model(torch.tensor([[new[-1]] + guess], device=p.device), cache=cache).logits[0]
        choice = out[:len(guess) + 1].argmax(-1).tolist()
        n_ok = next((i for i, (c, g) in enumerate(zip(choice, guess)) if c != g), len(guess))
        stats["forwards"] += 1
        stats["drafted"] += len(guess)
        stats["accepted"] += n_ok
        cache.pos = start + 1 + n_ok          # keep the pending token and the accepted guesses
        for t in (guess[:n_ok] + [choice[n_ok]])[:max_new_tokens - len(new)]:
            ids.append(t)
            new.append(t)
    res = GenerationResult(list(prompt_ids), new, "max_new_tokens", {"speculative": stats})
    if dec is not None:
        res.stats["graph_replays"] = dec.replays
    return res
