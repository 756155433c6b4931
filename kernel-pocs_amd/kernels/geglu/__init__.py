from .geglu import ForgeGEGLUFunction
from .geglu import ForgePackedGEGLUFunction
from .geglu import geglu
from .geglu import geglu_backward
from .geglu import geglu_forward
from .geglu import geglu_mlp
from .geglu import geglu_packed
from .geglu import geglu_packed_backward
from .geglu import geglu_packed_forward
from .geglu import pack_geglu_gate_up_bias
from .geglu import pack_geglu_gate_up_weight
from .geglu import torch_geglu_mlp_reference
from .geglu import torch_geglu_packed_reference
from .geglu import torch_geglu_reference

__all__ = [
    "ForgeGEGLUFunction",
    "ForgePackedGEGLUFunction",
    "geglu",
    "geglu_backward",
    "geglu_forward",
    "geglu_mlp",
    "geglu_packed",
    "geglu_packed_backward",
    "geglu_packed_forward",
    "pack_geglu_gate_up_bias",
    "pack_geglu_gate_up_weight",
    "torch_geglu_mlp_reference",
    "torch_geglu_packed_reference",
    "torch_geglu_reference",
]
