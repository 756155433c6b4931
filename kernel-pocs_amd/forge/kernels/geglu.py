"""GeGLU re-export (reference forge/forge/kernels/geglu.py)."""
from kernels.geglu import (
    ForgeGEGLUFunction,
    ForgePackedGEGLUFunction,
    geglu,
    geglu_backward,
    geglu_forward,
    geglu_packed,
    geglu_packed_backward,
    geglu_packed_forward,
    torch_geglu_packed_reference,
    torch_geglu_reference,
)

__all__ = [
    "ForgeGEGLUFunction",
    "ForgePackedGEGLUFunction",
    "geglu",
    "geglu_backward",
    "geglu_forward",
    "geglu_packed",
    "geglu_packed_backward",
    "geglu_packed_forward",
    "torch_geglu_packed_reference",
    "torch_geglu_reference",
]
