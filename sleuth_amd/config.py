"""Attention hyperparameters (the attention fields of the reference's ModelConfig).

Mirrors sleuth/forge/model/config.py: ModelConfig fields used by attention (24-63),
the per-layer AttnSpec (180-187) and attn_spec(i) (142-147), with the same validation
of head counts, head sizes and layer kinds (96-137). 0 means "use the default" for
head_size / n_kv_heads, as in the reference.
"""

from __future__ import annotations

from dataclasses import dataclass, field


@dataclass(frozen=True)
class AttnSpec:
    kind: str        # "full" | "sliding"
    head_dim: int
    kv_heads: int
    rope_theta: float
    window: int      # 0 = sees the whole context
    v_from_k: bool   # no v_proj: values come from the keys


@dataclass
class ModelConfig:
    vocab_size: int = 0
    d_model: int = 384
    n_layers: int = 6
    n_heads: int = 6
    head_size: int = 0
    n_kv_heads: int = 0
    norm_eps: float = 1e-5
    pos_type: str = "rope"        # "rope" | "none" | "learned"
    rope_theta: float = 10000.0
    rope_dim: int = 0             # 0 = rotate every channel
    max_seq_len: int = 1024
    qk_norm: bool = False
    bias: bool = False
    qkv_bias: bool = False
    v_norm: bool = False
    attn_scale: float = 0.0       # 0 = 1/sqrt(head_dim)
    layer_types: list[str] = field(default_factory=list)
    sliding_window: int = 0
    swa_head_size: int = 0
    swa_kv_heads: int = 0
    swa_rope_theta: float = 0.0
    full_v_from_k: bool = False
    # layer i reuses layer shared_layers[i]'s Linear Parameters (config.py's looped layers,
    # tied in transformer.py:215-228); empty = every layer has its own
    shared_layers: list[int] = field(default_factory=list)
    # harness-only (the tiny decoder in sleuth_amd.model): MLP width, tied embeddings
    ffn_hidden: int = 0
    tie_embeddings: bool = True
    init_std: float = 0.02

    def __post_init__(self):
        if not self.head_size and self.d_model % self.n_heads:
            raise ValueError(f"d_model ({self.d_model}) must be divisible by n_heads ({self.n_heads})")
        if self.kv_heads <= 0 or self.n_heads % self.kv_heads:
            raise ValueError(f"n_heads ({self.n_heads}) must be a multiple of n_kv_heads ({self.kv_heads})")
        if self.layer_types and len(self.layer_types) != self.n_layers:
            raise ValueError(f"layer_types has {len(self.layer_types)} entries for {self.n_layers} layers")
        if any(t not in ("full", "sliding") for t in self.layer_types):
            raise ValueError(f"layer_types entries must be 'full' or 'sliding', got {sorted(set(self.layer_types))}")
        if "sliding" in self.layer_types and self.sliding_window <= 0:
            raise ValueError("sliding layers need sliding_window > 0")
        if self.shared_layers:
            src = self.shared_layers
            if len(src) != self.n_layers:
                raise ValueError(f"shared_layers has {len(src)} entries for {self.n_layers} layers")
            for i, j in enumerate(src):
                if not 0 <= j <= i or src[j] != j:
                    raise ValueError(f"layer {i} cannot share layer {j}'s weights: the source must be "
                                     "an earlier (or the same) layer that is not shared itself")
        if self.pos_type not in ("rope", "none", "learned"):
            raise ValueError(f"pos_type must be one of ('rope', 'none', 'learned'), got {self.pos_type!r}")
        for spec in {self.attn_spec(i) for i in range(self.n_layers)}:
            if spec.kv_heads <= 0 or self.n_heads % spec.kv_heads:
                raise ValueError(f"n_heads ({self.n_heads}) must be a multiple of the KV heads ({spec.kv_heads})")
            if spec.head_dim % 2 and self.pos_type == "rope":
                raise ValueError("RoPE needs an even head_dim")
            if self.rope_dim and (self.rope_dim % 2 or self.rope_dim > spec.head_dim):
                raise ValueError(f"rope_dim ({self.rope_dim}) must be even and at most the head size")

    def layer_type(self, i: int) -> str:
        return self.layer_types[i] if self.layer_types else "full"

    def attn_spec(self, i: int) -> AttnSpec:
        """The attention shape of layer i: sliding layers take the swa_* overrides."""
        if self.layer_type(i) == "sliding":
            return AttnSpec("sliding", self.swa_head_size or self.head_dim, self.swa_kv_heads or self.kv_heads,
                            self.swa_rope_theta or self.rope_theta, self.sliding_window, False)
        return AttnSpec("full", self.head_dim, self.kv_heads, self.rope_theta, 0, self.full_v_from_k)

    @property
    def head_dim(self) -> int:
        return self.head_size or self.d_model // self.n_heads

    @property
    def kv_heads(self) -> int:
        return self.n_kv_heads or self.n_heads

    @property
    def hidden(self) -> int:
        return self.ffn_hidden or ((int(8 * self.d_model / 3) + 63) // 64 * 64)
