"""ForgeRMSNorm v3 on MI355X (kernels/rmsnorm/forge_rmsnorm_v3.py of the
reference: v2 plus Triton autotuning).  There is no autotuner here: the HIP
kernels pick their vector width and register residency from the shape, so
v3 is v2's contract under v3's names."""
from __future__ import annotations

import torch

from . import _engine as E
from ._engine import _CASTING_LLAMA, _check_inputs, _resolve_casting_mode  # noqa: F401
from .forge_rmsnorm_v2 import torch_rmsnorm_reference_v2 as torch_rmsnorm_reference_v3


def rmsnorm_v3_forward(x, weight, eps=1e-6, offset=0.0, casting_mode="llama"):
    """-> (y, x_2d, weight_1d, rstd, mode)."""
    _check_inputs(x, weight)
    if not x.is_cuda:
        raise RuntimeError("rmsnorm_v3_forward requires CUDA")
    mode = _resolve_casting_mode(casting_mode)
    y, x_2d, w, rstd = E.forward(x, weight, eps, offset, mode, what="RMSNorm v3")
    return y, x_2d, w, rstd, mode


def rmsnorm_v3_backward(dy, x_2d, weight, rstd, offset=0.0, casting_mode_int=_CASTING_LLAMA):
    """-> (dx, dw)."""
    return E.backward(dy, x_2d, weight, rstd, offset, 0, in_place=False)


class ForgeRMSNormv3Function(torch.autograd.Function):
    """forge_rmsnorm_v3.py:296-314."""

    @staticmethod
    def forward(ctx, x, weight, eps=1e-6, offset=0.0, casting_mode="llama"):
        y, x_2d, weight_1d, rstd, mode = rmsnorm_v3_forward(x, weight, eps, offset, casting_mode)
        ctx.save_for_backward(x_2d, weight_1d, rstd)
        ctx.offset = float(offset)
        ctx.casting_mode_int = mode
        return y

    @staticmethod
    def backward(ctx, dy):
        x_2d, weight_1d, rstd = ctx.saved_tensors
        dx, dw = rmsnorm_v3_backward(dy, x_2d, weight_1d, rstd, ctx.offset, ctx.casting_mode_int)
        return dx, dw, None, None, None


class ForgeRMSNormv3(torch.nn.Module):
    """forge_rmsnorm_v3.py:317-344."""

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
        return apply_rmsnorm_v3(x, self.weight, eps=self.variance_epsilon, offset=self.offset,
                                casting_mode=self.casting_mode)

    def extra_repr(self):
        return (f"hidden_size={self.weight.numel()}, eps={self.variance_epsilon}, offset={self.offset}, "
                f"casting_mode={self.casting_mode!r}")


def apply_rmsnorm_v3(x, weight, eps=1e-6, offset=0.0, casting_mode="llama"):
    """forge_rmsnorm_v3.py:347-356."""
    _check_inputs(x, weight)
    if not x.is_cuda:
        return torch_rmsnorm_reference_v3(x, weight, eps, offset, casting_mode)
    return ForgeRMSNormv3Function.apply(x, weight, eps, offset, casting_mode)


__all__ = ["apply_rmsnorm_v3", "ForgeRMSNormv3", "ForgeRMSNormv3Function", "torch_rmsnorm_reference_v3",
           "rmsnorm_v3_forward", "rmsnorm_v3_backward"]
