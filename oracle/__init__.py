"""CPU oracle for the FORGE attention hot path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this
package, and only as the checker (or, in bench.py, as the timed CPU baseline). The
product (sleuth_amd) never calls it: its kernels run on the GPU or raise.
"""

from .attention_ref import (  # noqa: F401
    KVCache,
    StaticKVCache,
    apply_rope,
    attention_forward,
    attention_mask,
    brute_attention,
    document_mask,
    eager_norm_rope,
    drafter_attention,
    explicit_attention,
    gated_attention,
    head_norm_rope,
    ragged_decode,
    rms_norm,
    rope_tables,
    rotate_half,
    sdpa,
)
