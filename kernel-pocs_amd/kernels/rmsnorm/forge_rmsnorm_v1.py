"""ForgeRMSNorm v1 on MI355X (kernels/rmsnorm/forge_rmsnorm_v1.py of the
reference, the legacy unversioned API): y = (x rsqrt(mean(x^2) + eps)).to(dtype)
* weight with the promoted output dtype, no offset, and v1's roundings in
backward (dy * weight and the dw terms rounded to x's dtype).  Runs on the
same kernels as v4 (csrc/rmsnorm.hip, variant 1)."""
from __future__ import annotations

import torch

from . import _engine as E
from ._engine import MAX_BLOCK_SIZE, _check_inputs  # noqa: F401

BACKWARD_ROWS_PER_PROGRAM = 16


def torch_rmsnorm_reference(x, weight, eps=1e-6):
    """forge_rmsnorm_v1.py:109-113."""
    x_fp32 = x.float()
    variance = x_fp32.pow(2).mean(dim=-1, keepdim=True)
    normed = x_fp32 * torch.rsqrt(variance + eps)
    return normed.to(dtype=x.dtype) * weight


def rmsnorm_v1_forward(x, weight, eps=1e-6):
    """forge_rmsnorm_v1.py:147-172 -> (y, x_2d, weight_1d, rstd)."""
    _check_inputs(x, weight)
    if not x.is_cuda:
        raise RuntimeError("rmsnorm_forward requires CUDA; use rmsnorm() for the CPU fallback")
    out_dtype = torch.result_type(x, weight)
    return E.forward(x, weight, eps, 0.0, E._CASTING_LLAMA, out_dtype=out_dtype, what="RMSNorm")


def rmsnorm_v1_backward(dy, x_2d, weight, rstd):
    """forge_rmsnorm_v1.py:175-206 -> (dx, dweight)."""
    return E.backward(dy, x_2d, weight, rstd, 0.0, 1, in_place=False)


class ForgeRMSNormv1Function(torch.autograd.Function):
    """forge_rmsnorm_v1.py:209-220."""

    @staticmethod
    def forward(ctx, x, weight, eps=1e-6):
        y, x_2d, weight_1d, rstd = rmsnorm_v1_forward(x, weight, eps)
        ctx.save_for_backward(x_2d, weight_1d, rstd)
        return y

    @staticmethod
    def backward(ctx, dy):
        x_2d, weight, rstd = ctx.saved_tensors
        dx, dweight = rmsnorm_v1_backward(dy, x_2d, weight, rstd)
        return dx, dweight, None


def rmsnorm_v1(x, weight, eps=1e-6):
    """forge_rmsnorm_v1.py:223-227."""
    _check_inputs(x, weight)
    if not x.is_cuda:
        return torch_rmsnorm_reference(x, weight, eps)
    return ForgeRMSNormv1Function.apply(x, weight, eps)
