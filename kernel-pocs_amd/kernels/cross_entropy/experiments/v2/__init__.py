from .cross_entropy_kernel_v2 import CrossEntropyOutput
from .cross_entropy_kernel_v2 import ForgeCrossEntropyFunction
from .cross_entropy_kernel_v2 import ForgeCrossEntropyLoss
from .cross_entropy_kernel_v2 import cross_entropy_backward
from .cross_entropy_kernel_v2 import cross_entropy_forward
from .cross_entropy_kernel_v2 import forge_cross_entropy

__all__ = [
    "CrossEntropyOutput",
    "ForgeCrossEntropyFunction",
    "ForgeCrossEntropyLoss",
    "cross_entropy_backward",
    "cross_entropy_forward",
    "forge_cross_entropy",
]
