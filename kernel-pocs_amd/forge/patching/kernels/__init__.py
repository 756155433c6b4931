"""Registry of the patch adapters (reference
forge/forge/patching/kernels/__init__.py:11-33): kernel name -> factory
`maker(module, config) -> forward`.  A factory raises ForgeSkipPatch when its
kernel does not apply to the module it is offered.

"embedding" is declared but not wired: this build has no embedding kernel
(the reference's lives outside the hot path), so it is registered as a stub
that a patch loop skips unless it is asked for by name.
"""
from __future__ import annotations

from typing import Callable, Dict

from .basic import make_geglu_forward, make_not_implemented, make_rmsnorm_forward, make_swiglu_forward
from .common import ForgeSkipPatch
from .fused_linear_ce import make_fused_linear_ce_forward
from .lora import make_lora_mlp_forward, make_lora_qkv_forward

FORWARD_MAKERS: Dict[str, Callable] = {
    "embedding": make_not_implemented("embedding", "no embedding kernel in this build"),
    "rmsnorm": make_rmsnorm_forward,
    "swiglu": make_swiglu_forward,
    "fused_linear_ce": make_fused_linear_ce_forward,
    "lora_mlp": make_lora_mlp_forward,
    "lora_qkv": make_lora_qkv_forward,
    "geglu": make_geglu_forward,
}

__all__ = ["FORWARD_MAKERS", "ForgeSkipPatch"]
