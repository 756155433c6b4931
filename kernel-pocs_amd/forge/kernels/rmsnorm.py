"""RMSNorm re-export (reference forge/forge/kernels/rmsnorm.py)."""
from kernels.rmsnorm import (
    ForgeRMSNormFunction,
    apply_rmsnorm,
    rmsnorm,
    rmsnorm_backward,
    rmsnorm_forward,
    torch_rmsnorm_reference,
)

__all__ = [
    "ForgeRMSNormFunction",
    "apply_rmsnorm",
    "rmsnorm",
    "rmsnorm_backward",
    "rmsnorm_forward",
    "torch_rmsnorm_reference",
]
