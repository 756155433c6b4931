"""Forge RMSNorm on MI355X (kernels/rmsnorm/__init__.py of the reference):
the versioned entry points v1-v4, `apply_rmsnorm` = v4 (the shipping
kernel), and the legacy unversioned names aliased to v1.  All versions run
on csrc/rmsnorm.hip."""
from .forge_rmsnorm_v1 import (
    ForgeRMSNormv1Function,
    rmsnorm_v1,
    rmsnorm_v1_backward,
    rmsnorm_v1_forward,
    torch_rmsnorm_reference,
)
from .forge_rmsnorm_v2 import ForgeRMSNormv2, ForgeRMSNormv2Function, apply_rmsnorm_v2, torch_rmsnorm_reference_v2
from .forge_rmsnorm_v3 import ForgeRMSNormv3, ForgeRMSNormv3Function, apply_rmsnorm_v3
from .forge_rmsnorm_v4 import ForgeRMSNormv4, ForgeRMSNormv4Function, apply_rmsnorm_v4, torch_rmsnorm_reference_v4

apply_rmsnorm = apply_rmsnorm_v4

ForgeRMSNormFunction = ForgeRMSNormv1Function
rmsnorm = rmsnorm_v1
rmsnorm_forward = rmsnorm_v1_forward
rmsnorm_backward = rmsnorm_v1_backward

__all__ = [
    "ForgeRMSNormv1Function",
    "rmsnorm_v1", "rmsnorm_v1_forward", "rmsnorm_v1_backward",
    "torch_rmsnorm_reference",
    "apply_rmsnorm",
    "ForgeRMSNormFunction", "rmsnorm", "rmsnorm_forward", "rmsnorm_backward",
    "ForgeRMSNormv2Function", "ForgeRMSNormv2", "apply_rmsnorm_v2", "torch_rmsnorm_reference_v2",
    "ForgeRMSNormv3Function", "ForgeRMSNormv3", "apply_rmsnorm_v3",
    "ForgeRMSNormv4Function", "ForgeRMSNormv4", "apply_rmsnorm_v4", "torch_rmsnorm_reference_v4",
]
