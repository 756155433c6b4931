"""RoPE on MI355X (drop-in for kernels/rope/forge_rope_v3.py)."""
from .forge_rope_v3 import (  # noqa: F401
    ForgeRoPEv3,
    ForgeRoPEPositionsFunction,
    ForgeRoPEv3Function,
    apply_rope,
    get_autotune_cache_for,
    rope_cos_sin,
)
