"""Cross-entropy re-export (reference forge/forge/kernels/cross_entropy.py:8-27)."""
from kernels.cross_entropy.experiments.v2 import (
    CrossEntropyOutput,
    ForgeCrossEntropyFunction,
    ForgeCrossEntropyLoss,
    forge_cross_entropy,
)

__all__ = [
    "CrossEntropyOutput",
    "ForgeCrossEntropyFunction",
    "ForgeCrossEntropyLoss",
    "forge_cross_entropy",
]
