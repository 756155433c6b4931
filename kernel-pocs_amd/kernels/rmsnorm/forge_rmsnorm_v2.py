"""ForgeRMSNorm v2 on MI355X (kernels/rmsnorm/forge_rmsnorm_v2.py of the
reference): offset, the llama / gemma / none casting modes, fp32 (fp64 for
fp64 input) accumulation and a fresh dX in backward.  Runs on the same
kernels as v4 (csrc/rmsnorm.hip)."""
from __future__ import annotations

import torch

from . import _engine as E
from ._engine import (  # noqa: F401  (reference module-level names)
    MAX_BLOCK_SIZE,
    _CASTING_GEMMA,
    _CASTING_LLAMA,
    _CASTING_MODE_BY_NAME,
    _CASTING_NONE,
    _check_inputs,
    _resolve_casting_mode,
)


def torch_rmsnorm_reference_v2(x, weight, eps=1e-6, offset=0.0, casting_mode="llama"):
    """forge_rmsnorm_v2.py:248-276: the PyTorch formula (HF LlamaRMSNorm for
    offset 0, Gemma2RMSNorm for offset 1); CPU path of apply_rmsnorm_v*."""
    mode = _resolve_casting_mode(casting_mode)
    input_dtype = x.dtype
    x_fp32 = x.float()
    variance = x_fp32.pow(2).mean(dim=-1, keepdim=True)
    rstd = torch.rsqrt(variance + eps)
    if mode == _CASTING_LLAMA:
        normed = (x_fp32 * rstd).to(input_dtype)
        return normed * (weight + offset)
    if mode == _CASTING_GEMMA:
        return ((x_fp32 * rstd) * (weight.float() + offset)).to(input_dtype)
    rstd_native = rstd.to(input_dtype)
    return (x * rstd_native) * (weight + offset)


def rmsnorm_v2_forward(x, weight, eps=1e-6, offset=0.0, casting_mode="llama"):
    """forge_rmsnorm_v2.py:283-324 -> (y, x_2d, weight_1d, rstd, mode)."""
    _check_inputs(x, weight)
    if not x.is_cuda:
        raise RuntimeError("rmsnorm_v2_forward requires CUDA")
    mode = _resolve_casting_mode(casting_mode)
    y, x_2d, w, rstd = E.forward(x, weight, eps, offset, mode, what="RMSNorm v2")
    return y, x_2d, w, rstd, mode


def rmsnorm_v2_backward(dy, x_2d, weight, rstd, offset=0.0, casting_mode_int=_CASTING_LLAMA):
    """forge_rmsnorm_v2.py:327-374 -> (dx, dw)."""
    return E.backward(dy, x_2d, weight, rstd, offset, 0, in_place=False)


class ForgeRMSNormv2Function(torch.autograd.Function):
    """forward(ctx, x, weight, eps=1e-6, offset=0.0, casting_mode="llama");
    backward returns (dx, dw, None, None, None)."""

    @staticmethod
    def forward(ctx, x, weight, eps=1e-6, offset=0.0, casting_mode="llama"):
        y, x_2d, weight_1d, rstd, mode = rmsnorm_v2_forward(x, weight, eps, offset, casting_mode)
        ctx.save_for_backward(x_2d, weight_1d, rstd)
        ctx.eps = eps
        ctx.offset = float(offset)
        ctx.casting_mode_int = mode
        return y

    @staticmethod
    def backward(ctx, dy):
        x_2d, weight_1d, rstd = ctx.saved_tensors
        dx, dw = rmsnorm_v2_backward(dy, x_2d, weight_1d, rstd, ctx.offset, ctx.casting_mode_int)
        return dx, dw, None, None, None


class ForgeRMSNormv2(torch.nn.Module):
    """forge_rmsnorm_v2.py:422-475."""

    def __init__(self, hidden_size, eps=1e-6, offset=0.0, casting_mode="llama", weight_init="ones", dtype=None,
                 device=None):
        super().__init__()
        if weight_init not in ("ones", "zeros"):
            raise ValueError(f"weight_init must be 'ones' or 'zeros', got {weight_init!r}")
        self.variance_epsilon = float(eps)
        self.eps = self.variance_epsilon
        self.offset = float(offset)
        self.casting_mode = casting_mode
        init_fn = torch.ones if weight_init == "ones" else torch.zeros
        self.weight = torch.nn.Parameter(init_fn(hidden_size, dtype=dtype, device=device))

    def forward(self, x):
        return apply_rmsnorm_v2(x, self.weight, eps=self.variance_epsilon, offset=self.offset,
                                casting_mode=self.casting_mode)

    def extra_repr(self):
        return (f"hidden_size={self.weight.numel()}, eps={self.variance_epsilon}, offset={self.offset}, "
                f"casting_mode={self.casting_mode!r}")


def apply_rmsnorm_v2(x, weight, eps=1e-6, offset=0.0, casting_mode="llama"):
    """forge_rmsnorm_v2.py:478-504."""
    _check_inputs(x, weight)
    if not x.is_cuda:
        return torch_rmsnorm_reference_v2(x, weight, eps, offset, casting_mode)
    return ForgeRMSNormv2Function.apply(x, weight, eps, offset, casting_mode)


__all__ = [
    "apply_rmsnorm_v2",
    "ForgeRMSNormv2",
    "ForgeRMSNormv2Function",
    "torch_rmsnorm_reference_v2",
    "rmsnorm_v2_forward",
    "rmsnorm_v2_backward",
]
