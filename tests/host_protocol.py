"""Stand-ins for the host (Sleuth) objects the drop-in module must work with, written for
these tests from the reference's protocol:

  HostKVCache        exactly the members of sleuth/forge/infer/kv_cache.py:25-70 (k, v,
                     max_len, pos, token_history, for_model, update, advance, reset, nbytes)
                     and nothing more: no per-row lengths, no room check of its own
  HostStaticKVCache  exactly the members added by kv_cache.py:73-138 (static, length, pos_t,
                     tokens_per_step, positions, update, attn_mask, new_step, advance)
  HostTap, host_assign_names, host_listen
                     a separate Tap class with isinstance-based discovery, as the host's
                     analyzer does it (sleuth/forge/model/taps.py:47-102)

They let the tests show that the HIP attention runs on the host's own objects.
"""

from __future__ import annotations

import fnmatch
from contextlib import contextmanager

import torch
from torch import nn


class HostKVCache:
    def __init__(self, shapes, batch, max_len, device, dtype):
        self.k = [torch.zeros(batch, kv, max_len, hd, device=device, dtype=dtype) for kv, hd in shapes]
        self.v = [torch.zeros_like(t) for t in self.k]
        self.max_len = max_len
        self.pos = 0
        self._tokens = None

    def token_history(self, batch, device):
        if self._tokens is None:
            self._tokens = torch.full((batch, self.max_len), -1, dtype=torch.long, device=device)
        return self._tokens

    @classmethod
    def for_model(cls, model, batch, max_len=None, dtype=None):
        cfg, p = model.cfg, next(model.parameters())
        shapes = [(cfg.attn_spec(i).kv_heads, cfg.attn_spec(i).head_dim) for i in range(cfg.n_layers)]
        return cls(shapes, batch, max_len or cfg.max_seq_len, p.device, dtype or p.dtype)

    def update(self, layer, k_new, v_new):
        end = self.pos + k_new.shape[2]
        if end > self.max_len:
            raise ValueError(f"KV cache full ({self.max_len} tokens)")
        self.k[layer][:, :, self.pos:end] = k_new.to(self.k[layer].dtype)
        self.v[layer][:, :, self.pos:end] = v_new.to(self.v[layer].dtype)
        return self.k[layer][:, :, :end], self.v[layer][:, :, :end]

    def advance(self, n):
        self.pos += n

    def reset(self):
        self.pos = 0

    def nbytes(self):
        return sum(2 * t.numel() * t.element_size() for t in self.k)


class HostStaticKVCache(HostKVCache):
    """The static (graph) members only; the step's positions and masks are made on first
    use after new_step() and kept until the next one."""

    def __init__(self, shapes, batch, max_len, device, dtype, tokens_per_step=1):
        super().__init__(shapes, batch, max_len, device, dtype)
        self.static = False
        self.length = max_len
        self.pos_t = torch.zeros(1, dtype=torch.long, device=device)
        self.tokens_per_step = tokens_per_step
        self.new_step()

    def new_step(self, positions=None):
        self._step = {"positions": positions}

    @property
    def positions(self):
        if self._step["positions"] is None:
            self._step["positions"] = self.pos_t + torch.arange(self.tokens_per_step, device=self.pos_t.device)
        return self._step["positions"]

    def update(self, layer, k_new, v_new):
        if not self.static:
            return super().update(layer, k_new, v_new)
        for cache, new in ((self.k[layer], k_new), (self.v[layer], v_new)):
            cache.index_copy_(2, self.positions, new.to(cache.dtype))
        return self.k[layer][:, :, :self.length], self.v[layer][:, :, :self.length]

    def attn_mask(self, window=0):
        if window not in self._step:
            q = self.positions[:, None]
            k = torch.arange(self.length, device=q.device)[None, :]
            ok = k <= q
            if window:
                ok &= q - k < window
            self._step[window] = ok[None, None]
        return self._step[window]

    def advance(self, n):
        if not self.static:
            super().advance(n)


class HostTap(nn.Module):
    def __init__(self):
        super().__init__()
        self.name = "<unnamed>"
        self.listeners = []

    @property
    def active(self):
        return bool(self.listeners)

    def forward(self, x):
        for fn in self.listeners:
            out = fn(self.name, x)
            if out is not None:
                x = out
        return x


def host_assign_names(model):
    for path, m in model.named_modules():
        if isinstance(m, HostTap):
            *head, leaf = path.split(".")
            m.name = ".".join(head + [leaf[4:] if leaf.startswith("tap_") else leaf])


@contextmanager
def host_listen(model, listeners):
    attached = []
    try:
        for pattern, fn in listeners.items():
            hits = [m for m in model.modules() if isinstance(m, HostTap) and fnmatch.fnmatchcase(m.name, pattern)]
            if not hits:
                raise KeyError(f"no tap matches {pattern!r}")
            for t in hits:
                t.listeners.append(fn)
                attached.append((t, fn))
        yield
    finally:
        for t, fn in attached:
            t.listeners.remove(fn)
