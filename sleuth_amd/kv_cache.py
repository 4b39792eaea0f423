"""KV cache with per-row lengths, laid out for the HIP attention kernels.

The attention module runs on any object with the reference's cache protocol
(sleuth/forge/infer/kv_cache.py:25-138) -- the host's own KVCache and StaticKVCache
included. This class is the cache of this package's callers (generate(), the graph
decoder, the benchmark); it speaks the same protocol and adds what the kernels can use:

  storage    every layer's K and V are views [B, K, max_len, hd] of ONE device allocation
             (the arena), so a whole model's cache is a single block of HBM;
  row lengths  each batch row has its own length (`set_lengths`, `seq_lens` int32 [B] on
             the device with a host mirror `seq_lens_host`); `pos` is the longest row, and
             setting it sets every row (what the speculative decoder's rewind does);
  static mode  (graph replays) the position is the device scalar `pos_t`; `positions`
             (pos_t + 0 .. tokens_per_step-1) is computed into a fixed buffer, so a
             captured graph recomputes it on every replay.

Protocol members: k, v, pos, max_len, update, advance, reset, nbytes, token_history,
for_model; static, pos_t, length, tokens_per_step, positions, attn_mask, new_step.
"""

from __future__ import annotations

import torch


class KVCache:
    def __init__(self, shapes: list[tuple[int, int]], batch: int, max_len: int,
                 device: torch.device | str, dtype: torch.dtype, tokens_per_step: int = 1):
        """shapes: (n_kv_heads, head_dim) of each layer."""
        if batch < 1 or max_len < 1 or tokens_per_step < 1:
            raise ValueError("batch, max_len and tokens_per_step must be positive")
        dev = torch.device(device)
        sizes = [batch * kv * max_len * hd for kv, hd in shapes]
        half = sum(sizes)
        self._arena = torch.zeros(2 * half, device=dev, dtype=dtype)   # [all K | all V]
        self.k, self.v, off = [], [], 0
        for (kv, hd), n in zip(shapes, sizes):
            self.k.append(self._arena[off:off + n].view(batch, kv, max_len, hd))
            self.v.append(self._arena[half + off:half + off + n].view(batch, kv, max_len, hd))
            off += n
        self.max_len, self.batch, self.device = max_len, batch, dev
        self._rows = [0] * batch
        self._rows_dev: torch.Tensor | None = None   # device mirror, made when rows differ
        self._history: torch.Tensor | None = None
        # static (graph) mode
        self.static = False
        self.length = max_len
        self.tokens_per_step = tokens_per_step
        self.pos_t = torch.zeros(1, dtype=torch.long, device=dev)
        self._steps = torch.arange(tokens_per_step, device=dev)
        self._pos_buf = torch.zeros(tokens_per_step, dtype=torch.long, device=dev)
        self._pass_pos: torch.Tensor | None = None
        self._pass_masks: dict[int, torch.Tensor] = {}

    @classmethod
    def for_model(cls, model, batch: int, max_len: int | None = None, dtype: torch.dtype | None = None,
                  tokens_per_step: int = 1) -> "KVCache":
        cfg = model.cfg
        p = next(model.parameters())
        specs = [cfg.attn_spec(i) for i in range(cfg.n_layers)]
        return cls([(s.kv_heads, s.head_dim) for s in specs], batch, max_len or cfg.max_seq_len,
                   p.device, dtype or p.dtype, tokens_per_step)

    # ------------------------------------------------------------------ lengths
    @property
    def pos(self) -> int:
        return max(self._rows)

    @pos.setter
    def pos(self, value: int) -> None:
        self._rows = [int(value)] * self.batch
        self._rows_dev = None

    def set_lengths(self, lengths: list[int]) -> None:
        """Give each row its own length (tokens already stored in it)."""
        rows = [int(n) for n in lengths]
        if len(rows) != self.batch:
            raise ValueError(f"{len(rows)} lengths for batch {self.batch}")
        if min(rows) < 0 or max(rows) > self.max_len:
            raise ValueError(f"lengths must be in [0, {self.max_len}]")
        self._rows = rows
        self._rows_dev = None

    @property
    def ragged(self) -> bool:
        return min(self._rows) != max(self._rows)

    @property
    def seq_lens_host(self) -> list[int]:
        return list(self._rows)

    @property
    def seq_lens(self) -> torch.Tensor:
        """int32 [B] row lengths on the device (what forge_kv_append / forge_attn_decode
        read as row_pos)."""
        if self._rows_dev is None:
            self._rows_dev = torch.tensor(self._rows, dtype=torch.int32).to(self.device)
        return self._rows_dev

    def _room_for(self, T: int) -> None:
        if self.pos + T > self.max_len:
            raise ValueError(f"KV cache full ({self.max_len} tokens)")

    # ------------------------------------------------------------------ protocol
    def update(self, layer: int, k_new: torch.Tensor, v_new: torch.Tensor):
        """Torch-path write of this step's K/V [B, K, T, hd]; returns the K/V views the
        step attends over: [:, :, :pos+T] (static mode: [:, :, :length])."""
        kc, vc = self.k[layer], self.v[layer]
        B, _, T, _ = k_new.shape
        if self.static:
            where = self.positions
            kc.index_copy_(2, where, k_new.to(kc.dtype))
            vc.index_copy_(2, where, v_new.to(vc.dtype))
            return kc[:, :, :self.length], vc[:, :, :self.length]
        self._room_for(T)
        # one scatter for all rows: row b's token t goes to position rows[b] + t
        cols = torch.tensor(self._rows, device=kc.device)[:, None] + torch.arange(T, device=kc.device)
        rows = torch.arange(B, device=kc.device)[:, None].expand(B, T)
        kc[rows, :, cols] = k_new.transpose(1, 2).to(kc.dtype)
        vc[rows, :, cols] = v_new.transpose(1, 2).to(vc.dtype)
        top = self.pos + T
        return kc[:, :, :top], vc[:, :, :top]

    def advance(self, n: int) -> None:
        """All layers have stored n more tokens per row. In static mode the caller owns
        the position (pos and pos_t), so nothing moves here."""
        if self.static:
            return
        self._rows = [r + n for r in self._rows]
        if self._rows_dev is not None:
            self._rows_dev.add_(n)

    def reset(self) -> None:
        self.pos = 0
        self.static = False

    def nbytes(self) -> int:
        return self._arena.numel() * self._arena.element_size()

    def token_history(self, batch: int, device) -> torch.Tensor:
        """[batch, max_len] token ids by position, -1 where none yet (made on first use)."""
        if self._history is None:
            self._history = torch.full((batch, self.max_len), -1, dtype=torch.long, device=device)
        return self._history

    # ------------------------------------------------------------------ static mode
    @property
    def positions(self) -> torch.Tensor:
        """int64 [tokens_per_step]: this pass's token positions, pos_t + 0, 1, ..."""
        if self._pass_pos is None:
            torch.add(self.pos_t, self._steps, out=self._pos_buf)
            self._pass_pos = self._pos_buf
        return self._pass_pos

    def new_step(self, positions: torch.Tensor | None = None) -> None:
        """Start of a forward pass: positions are recomputed from pos_t (or taken as given)."""
        self._pass_pos = positions
        self._pass_masks = {}

    def attn_mask(self, window: int = 0) -> torch.Tensor:
        """[1, 1, T, length] bool, True where a query may see a key; one per window per pass."""
        mask = self._pass_masks.get(window)
        if mask is None:
            gap = self.positions[:, None] - torch.arange(self.length, device=self.device)[None, :]
            mask = gap >= 0
            if window:
                mask &= gap < window
            mask = self._pass_masks[window] = mask[None, None]
        return mask
