"""Key/value caches with the reference's layout and protocol.

KVCache (sleuth/forge/infer/kv_cache.py:25-70): per-layer k[layer], v[layer] =
zeros(B, K, max_len, hd), one shared `pos`, update()/advance()/reset()/nbytes()/
token_history()/for_model(). StaticKVCache (kv_cache.py:73-138): the CUDA-graph variant
with the position in a device tensor `pos_t`, `length` (the bucket the graph was
recorded for), `positions`, attn_mask(window) and new_step().

The HIP attention writes the new K/V straight into these tensors (forge_kv_append)
and reads them in place, so code that looks at cache.k[layer][:, :, :n] (MTP drafters,
the analyzer) sees the same data as with the reference.

Extension for ragged batches: set_lengths([L_0, .., L_B-1]) gives each row its own
length (`seq_lens`, int32 [B] on the device, with a host mirror); token t of row b
then goes to position seq_lens[b] + t and advance(n) moves every row. Without it,
`pos` keeps the reference's meaning.
"""

from __future__ import annotations

import torch


class KVCache:
    def __init__(self, shapes: list[tuple[int, int]], batch: int, max_len: int,
                 device: torch.device | str, dtype: torch.dtype):
        """shapes: (n_kv_heads, head_dim) for each layer."""
        self.k = [torch.zeros(batch, kv, max_len, hd, device=device, dtype=dtype) for kv, hd in shapes]
        self.v = [torch.zeros_like(k) for k in self.k]
        self.max_len = max_len
        self.batch = batch
        self.pos = 0
        self._tokens: torch.Tensor | None = None
        self.seq_lens: torch.Tensor | None = None
        self.seq_lens_host: list[int] | None = None

    def token_history(self, batch: int, device) -> torch.Tensor:
        """[batch, max_len] token ids by position (-1 = none yet), made on first use."""
        if self._tokens is None:
            self._tokens = torch.full((batch, self.max_len), -1, dtype=torch.long, device=device)
        return self._tokens

    @classmethod
    def for_model(cls, model, batch: int, max_len: int | None = None,
                  dtype: torch.dtype | None = None) -> "KVCache":
        cfg = model.cfg
        p = next(model.parameters())
        shapes = [(cfg.attn_spec(i).kv_heads, cfg.attn_spec(i).head_dim) for i in range(cfg.n_layers)]
        return cls(shapes, batch, max_len or cfg.max_seq_len, p.device, dtype or p.dtype)

    # ------------------------------------------------------------------ ragged rows
    def set_lengths(self, lengths: list[int]) -> None:
        """Per-row lengths (tokens already stored in each row)."""
        if len(lengths) != self.batch:
            raise ValueError(f"{len(lengths)} lengths for batch {self.batch}")
        if any(L < 0 or L > self.max_len for L in lengths):
            raise ValueError(f"lengths must be in [0, {self.max_len}]")
        self.seq_lens_host = [int(L) for L in lengths]
        self.seq_lens = torch.tensor(self.seq_lens_host, dtype=torch.int32, device=self.k[0].device)
        self.pos = max(self.seq_lens_host)

    @property
    def ragged(self) -> bool:
        return self.seq_lens is not None

    # ------------------------------------------------------------------ reference protocol
    def update(self, layer: int, k_new: torch.Tensor, v_new: torch.Tensor):
        """Store this step's K/V for `layer`; return all K/V so far: [B, K, pos+T, hd]."""
        T = k_new.shape[2]
        if self.ragged:
            for b, L in enumerate(self.seq_lens_host):
                if L + T > self.max_len:
                    raise ValueError(f"KV cache full ({self.max_len} tokens)")
                self.k[layer][b, :, L:L + T] = k_new[b].to(self.k[layer].dtype)
                self.v[layer][b, :, L:L + T] = v_new[b].to(self.v[layer].dtype)
            end = self.pos + T
            return self.k[layer][:, :, :end], self.v[layer][:, :, :end]
        end = self.pos + T
        if end > self.max_len:
            raise ValueError(f"KV cache full ({self.max_len} tokens)")
        self.k[layer][:, :, self.pos:end] = k_new.to(self.k[layer].dtype)
        self.v[layer][:, :, self.pos:end] = v_new.to(self.v[layer].dtype)
        return self.k[layer][:, :, :end], self.v[layer][:, :, :end]

    def check_room(self, T: int) -> None:
        """Raise like update() does when T more tokens do not fit (kv_cache.py:56-57)."""
        top = max(self.seq_lens_host) if self.ragged else self.pos
        if top + T > self.max_len:
            raise ValueError(f"KV cache full ({self.max_len} tokens)")

    def advance(self, n: int) -> None:
        """Called by the model once all layers have stored the new tokens."""
        if self.ragged:
            self.seq_lens_host = [L + n for L in self.seq_lens_host]
            self.seq_lens += n
            self.pos = max(self.seq_lens_host)
        else:
            self.pos += n

    def reset(self) -> None:
        self.pos = 0
        self.seq_lens = self.seq_lens_host = None

    def nbytes(self) -> int:
        return sum(2 * k.numel() * k.element_size() for k in self.k)


class StaticKVCache(KVCache):
    """A KVCache that one-token (or tokens_per_step) decode steps can use inside a HIP
    graph: the position lives in `pos_t` (int64 [1] on the device); outside `static`
    mode (the prompt's prefill) it behaves like KVCache."""

    def __init__(self, shapes, batch, max_len, device, dtype, tokens_per_step: int = 1):
        super().__init__(shapes, batch, max_len, device, dtype)
        self.static = False
        self.length = max_len
        self.pos_t = torch.zeros(1, dtype=torch.long, device=device)
        self._kpos = torch.arange(max_len, device=device)
        self.tokens_per_step = tokens_per_step
        self._qoff = torch.arange(tokens_per_step, device=device)
        self._masks: dict[int, torch.Tensor] = {}
        self._pos: torch.Tensor | None = None

    @property
    def positions(self) -> torch.Tensor:
        """[tokens_per_step] positions of this static step's tokens (pos_t, pos_t+1, ..)."""
        if self._pos is None:
            self._pos = self.pos_t + self._qoff
        return self._pos

    def update(self, layer, k_new, v_new):
        if not self.static:
            return super().update(layer, k_new, v_new)
        pos = self.positions
        self.k[layer].index_copy_(2, pos, k_new.to(self.k[layer].dtype))
        self.v[layer].index_copy_(2, pos, v_new.to(self.v[layer].dtype))
        return self.k[layer][:, :, :self.length], self.v[layer][:, :, :self.length]

    def attn_mask(self, window: int = 0) -> torch.Tensor:
        """[1, 1, T, length] bool, True = may attend (built once per pass per window)."""
        if window not in self._masks:
            kpos = self._kpos[:self.length][None, :]
            qpos = self.positions[:, None]
            mask = kpos <= qpos
            if window:
                mask = mask & (qpos - kpos < window)
            self._masks[window] = mask[None, None]
        return self._masks[window]

    def new_step(self, positions: torch.Tensor | None = None) -> None:
        """Start of a forward pass: positions may have moved (or are given explicitly)."""
        self._masks, self._pos = {}, positions

    def advance(self, n):
        if not self.static:  # in static mode the caller moves pos and pos_t
            super().advance(n)
