"""ForgeRMSNorm v4 on MI355X: v3 semantics plus the in-place dY -> dX
backward (kernels/rmsnorm/forge_rmsnorm_v4.py of the reference).

Same public names, signatures, checks, saved tensors and in-place contract;
the Triton kernels are replaced by `forge_rmsnorm_fwd` / `forge_rmsnorm_bwd`
(csrc/rmsnorm.hip), whose weight gradient is deterministic (fixed-order
reduction of per-workgroup partials instead of the reference's
`dw_partial.sum(0)`).  `in_place=True` (default) writes dx over dy's storage,
which is unsafe where dy feeds another backward node (Gemma2's residual-paired
RMSNorm): pass False there, as the reference documents.
"""
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
from .forge_rmsnorm_v2 import torch_rmsnorm_reference_v2 as torch_rmsnorm_reference_v4


def rmsnorm_v4_forward(x, weight, eps=1e-6, offset=0.0, casting_mode="llama"):
    """forge_rmsnorm_v4.py:242-270 -> (y, x_2d, weight_1d, rstd, mode)."""
    _check_inputs(x, weight)
    if not x.is_cuda:
        raise RuntimeError("rmsnorm_v4_forward requires CUDA")
    mode = _resolve_casting_mode(casting_mode)
    y, x_2d, w, rstd = E.forward(x, weight, eps, offset, mode, what="RMSNorm v4")
    return y, x_2d, w, rstd, mode


def rmsnorm_v4_backward(dy, x_2d, weight, rstd, offset=0.0, casting_mode_int=_CASTING_LLAMA, in_place=True):
    """forge_rmsnorm_v4.py:273-336 -> (dx, dw); dx over dy's storage when in_place."""
    return E.backward(dy, x_2d, weight, rstd, offset, 0, in_place)


class ForgeRMSNormv4Function(torch.autograd.Function):
    """forward(ctx, x, weight, eps, offset=0.0, casting_mode="llama", in_place=True);
    backward returns (dx, dw, None, None, None, None)."""

    @staticmethod
    def forward(ctx, x, weight, eps=1e-6, offset=0.0, casting_mode="llama", in_place=True):
        y, x_2d, weight_1d, rstd, mode = rmsnorm_v4_forward(x, weight, eps, offset, casting_mode)
        ctx.save_for_backward(x_2d, weight_1d, rstd)
        ctx.eps = eps
        ctx.offset = float(offset)
        ctx.casting_mode_int = mode
        ctx.in_place = bool(in_place)
        return y

    @staticmethod
    def backward(ctx, dy):
        x_2d, weight_1d, rstd = ctx.saved_tensors
        dx, dw = rmsnorm_v4_backward(dy, x_2d, weight_1d, rstd, offset=ctx.offset,
                                     casting_mode_int=ctx.casting_mode_int, in_place=ctx.in_place)
        return dx, dw, None, None, None, None


class ForgeRMSNormv4(torch.nn.Module):
    """forge_rmsnorm_v4.py:382-422."""

    def __init__(self, hidden_size, eps=1e-6, offset=0.0, casting_mode="llama", in_place=True, weight_init="ones",
                 dtype=None, device=None):
        super().__init__()
        if weight_init not in ("ones", "zeros"):
            raise ValueError(f"weight_init must be 'ones' or 'zeros', got {weight_init!r}")
        self.variance_epsilon = float(eps)
        self.eps = self.variance_epsilon
        self.offset = float(offset)
        self.casting_mode = casting_mode
        self.in_place = bool(in_place)
        init_fn = torch.ones if weight_init == "ones" else torch.zeros
        self.weight = torch.nn.Parameter(init_fn(hidden_size, dtype=dtype, device=device))

    def forward(self, x):
        return apply_rmsnorm_v4(x, self.weight, eps=self.variance_epsilon, offset=self.offset,
                                casting_mode=self.casting_mode, in_place=self.in_place)

    def extra_repr(self):
        return (f"hidden_size={self.weight.numel()}, eps={self.variance_epsilon}, offset={self.offset}, "
                f"casting_mode={self.casting_mode!r}, in_place={self.in_place}")


def apply_rmsnorm_v4(x, weight, eps=1e-6, offset=0.0, casting_mode="llama", in_place=True):
    """forge_rmsnorm_v4.py:425-455: the HIP path on a GPU, the PyTorch
    reference for CPU tensors."""
    _check_inputs(x, weight)
    if not x.is_cuda:
        return torch_rmsnorm_reference_v4(x, weight, eps, offset, casting_mode)
    return ForgeRMSNormv4Function.apply(x, weight, eps, offset, casting_mode, in_place)


__all__ = [
    "apply_rmsnorm_v4",
    "ForgeRMSNormv4",
    "ForgeRMSNormv4Function",
    "torch_rmsnorm_reference_v4",
    "rmsnorm_v4_forward",
    "rmsnorm_v4_backward",
]
