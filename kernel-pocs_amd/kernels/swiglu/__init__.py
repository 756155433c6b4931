from .swiglu import ForgeSwiGLUFunction
from .swiglu import ForgePackedSwiGLUFunction
from .swiglu import swiglu
from .swiglu import swiglu_backward
from .swiglu import swiglu_forward
from .swiglu import swiglu_packed
from .swiglu import swiglu_packed_backward
from .swiglu import swiglu_packed_forward
from .swiglu import torch_swiglu_packed_reference
from .swiglu import torch_swiglu_reference

__all__ = [
    "ForgeSwiGLUFunction",
    "ForgePackedSwiGLUFunction",
    "swiglu",
    "swiglu_backward",
    "swiglu_forward",
    "swiglu_packed",
    "swiglu_packed_backward",
    "swiglu_packed_forward",
    "torch_swiglu_packed_reference",
    "torch_swiglu_reference",
]
