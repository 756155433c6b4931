from .cross_entropy_kernel_v2 import CrossEntropyOutput
from .cross_entropy_kernel_v2 import ForgeCrossEntropyFunction
from .cross_entropy_kernel_v2 import ForgeCrossEntropyLoss
from .cross_entropy_kernel_v2 import cross_entropy_backward
from .cross_entropy_kernel_v2 import cross_entropy_forward
from .cross_entropy_kernel_v2 import forge_cross_entropy
from .fused_linear_cross_entropy import ForgeFusedLinearCrossEntropyFunction
from .fused_linear_cross_entropy import ForgeFusedLinearCrossEntropyLoss
from .fused_linear_cross_entropy import forge_fused_linear_cross_entropy
from .fused_linear_cross_entropy import fused_linear_cross_entropy_backward
from .fused_linear_cross_entropy import fused_linear_cross_entropy_forward

__all__ = [
    "CrossEntropyOutput",
    "ForgeCrossEntropyFunction",
    "ForgeCrossEntropyLoss",
    "ForgeFusedLinearCrossEntropyFunction",
    "ForgeFusedLinearCrossEntropyLoss",
    "cross_entropy_backward",
    "cross_entropy_forward",
    "forge_cross_entropy",
    "forge_fused_linear_cross_entropy",
    "fused_linear_cross_entropy_backward",
    "fused_linear_cross_entropy_forward",
]
