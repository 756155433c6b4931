"""Forge cross entropy v1 on MI355X (drop-in for
kernels/cross_entropy/experiments/v1 of Forge-researchlab/kernel-POCs)."""
from .cross_entropy_kernel_v1 import forge_cross_entropy

__all__ = ["forge_cross_entropy"]
