"""Cross-entropy re-export (reference forge/forge/kernels/cross_entropy.py:8-27)."""
from kernels.cross_entropy.experiments.v2 import (
    CrossEntropyOutput,
    ForgeCrossEntropyFunction,
    ForgeCrossEntropyLoss,
    ForgeFusedLinearCrossEntropyFunction,
    ForgeFusedLinearCrossEntropyLoss,
    forge_cross_entropy,
    forge_fused_linear_cross_entropy,
    fused_linear_cross_entropy_backward,
    fused_linear_cross_entropy_forward,
)

__all__ = [
    "CrossEntropyOutput",
    "ForgeCrossEntropyFunction",
    "ForgeCrossEntropyLoss",
    "ForgeFusedLinearCrossEntropyFunction",
    "ForgeFusedLinearCrossEntropyLoss",
    "forge_cross_entropy",
    "forge_fused_linear_cross_entropy",
    "fused_linear_cross_entropy_backward",
    "fused_linear_cross_entropy_forward",
]
