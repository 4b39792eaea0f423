"""Attention hyperparameters (the attention fields of the reference's ModelConfig).

The fields follow sleuth/forge/model/config.py's ModelConfig (24-63), so the module also
accepts the reference's own config object; AttnSpec and attn_spec(i) give each layer's
shape as config.py:142-147,180-187 define it (sliding layers take the swa_* overrides).
0 means "use the default" for head_size / n_kv_heads, as in the reference. The checks
below only reject what this package's module and harness cannot build.
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
        """Rejects the shapes the attention module and the harness cannot build."""
        n = self.n_layers
        kinds = self.layer_types or ["full"] * n
        bad = [
            (not self.head_size and self.d_model % self.n_heads, "d_model is not a multiple of n_heads"),
            (len(kinds) != n, "layer_types needs one entry per layer"),
            (not set(kinds) <= {"full", "sliding"}, "layer_types entries are 'full' or 'sliding'"),
            ("sliding" in kinds and self.sliding_window <= 0, "sliding layers need sliding_window > 0"),
            (self.pos_type not in ("rope", "none", "learned"), "pos_type is 'rope', 'none' or 'learned'"),
            (bool(self.shared_layers) and len(self.shared_layers) != n, "shared_layers needs one entry per layer"),
        ]
        if not bad[1][0]:
            specs = [self.attn_spec(i) for i in range(n)]
            for s in specs:
                bad += [(s.kv_heads <= 0 or self.n_heads % s.kv_heads, "n_heads is not a multiple of the KV heads"),
                        (self.pos_type == "rope" and s.head_dim % 2, "RoPE needs an even head size"),
                        (self.rope_dim % 2 or self.rope_dim > s.head_dim, "rope_dim must be even and fit the head")]
            # a shared layer points at an earlier (or the same) layer that owns its weights
            bad += [(not (0 <= j <= i and self.shared_layers[j] == j), f"layer {i} cannot share layer {j}")
                    for i, j in enumerate(self.shared_layers) if len(self.shared_layers) == n]
        for failed, why in bad:
            if failed:
                raise ValueError(f"bad attention config: {why}")

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
