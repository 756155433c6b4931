"""SwiGLU re-export (reference forge/forge/kernels/swiglu.py:7-31)."""
from kernels.swiglu import (
    ForgePackedSwiGLUFunction,
    ForgeSwiGLUFunction,
    swiglu,
    swiglu_backward,
    swiglu_forward,
    swiglu_packed,
    swiglu_packed_backward,
    swiglu_packed_forward,
    torch_swiglu_packed_reference,
    torch_swiglu_reference,
)

__all__ = [
    "ForgePackedSwiGLUFunction",
    "ForgeSwiGLUFunction",
    "swiglu",
    "swiglu_backward",
    "swiglu_forward",
    "swiglu_packed",
    "swiglu_packed_backward",
    "swiglu_packed_forward",
    "torch_swiglu_packed_reference",
    "torch_swiglu_reference",
]
