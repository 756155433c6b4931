"""Host side shared by the RMSNorm versions: argument checks, casting modes
and the launches of `forge_rmsnorm_fwd` / `forge_rmsnorm_bwd`
(libforge_hip.so, csrc/rmsnorm.hip).

Every version runs on the same kernels; they differ only in their
reference's contract (v1: offset-free llama forward with the promoted output
dtype and its own roundings in backward; v2/v3: fresh dX; v4: optional
in-place dY -> dX)."""
from __future__ import annotations

import torch

from forge_hip import _lib as L

MAX_BLOCK_SIZE = 131072

_CASTING_LLAMA = 0
_CASTING_GEMMA = 1
_CASTING_NONE = 2
_CASTING_MODE_BY_NAME = {"llama": _CASTING_LLAMA, "gemma": _CASTING_GEMMA, "none": _CASTING_NONE}


def _resolve_casting_mode(casting_mode) -> int:
    """forge_rmsnorm_v4.py:187-200."""
    if isinstance(casting_mode, int):
        if casting_mode not in (_CASTING_LLAMA, _CASTING_GEMMA, _CASTING_NONE):
            raise ValueError(f"Invalid casting_mode int: {casting_mode}")
        return casting_mode
    if isinstance(casting_mode, str):
        try:
            return _CASTING_MODE_BY_NAME[casting_mode]
        except KeyError as exc:
            raise ValueError(
                f"Invalid casting_mode {casting_mode!r}; expected one of {sorted(_CASTING_MODE_BY_NAME)}"
            ) from exc
    raise TypeError(f"casting_mode must be int or str, got {type(casting_mode).__name__}")


def _check_inputs(x: torch.Tensor, weight: torch.Tensor) -> None:
    """forge_rmsnorm_v4.py:219-233 (same checks in v1-v3)."""
    if x.dim() < 1:
        raise ValueError("x must have at least one dimension")
    if weight.dim() != 1:
        raise ValueError("weight must be a 1D tensor")
    if x.shape[-1] != weight.numel():
        raise ValueError(f"x.shape[-1] ({x.shape[-1]}) must equal weight.numel() ({weight.numel()})")
    if x.device != weight.device:
        raise ValueError("x and weight must be on the same device")
    if not x.is_floating_point() or not weight.is_floating_point():
        raise TypeError("x and weight must be floating point tensors")


def _block_size(n_cols: int, what: str = "RMSNorm v4") -> int:
    """The reference's row-size limit (forge_rmsnorm_v4.py:203-210), kept for
    API parity: the HIP kernels themselves have no row limit."""
    block = 1 << max(0, (n_cols - 1).bit_length())
    if block > MAX_BLOCK_SIZE:
        raise RuntimeError(
            f"{what}: hidden size {n_cols} requires block size {block} which exceeds MAX_BLOCK_SIZE={MAX_BLOCK_SIZE}."
        )
    return block


def acc_dtype(dtype: torch.dtype) -> torch.dtype:
    return torch.float64 if dtype == torch.float64 else torch.float32


def forward(x, weight, eps, offset, mode, out_dtype=None, what="RMSNorm v4"):
    """-> (y [x.shape], x_2d, weight_1d, rstd)."""
    L.require_gpu(x, weight)
    n_cols = x.shape[-1]
    _block_size(n_cols, what)
    x_2d = x.contiguous().view(-1, n_cols)
    w = weight.contiguous()
    rows = x_2d.shape[0]
    y = torch.empty(x_2d.shape, device=x.device, dtype=out_dtype or x.dtype)
    rstd = torch.empty((rows,), device=x.device, dtype=acc_dtype(x.dtype))
    if rows and n_cols:
        L.check(L.forge_rmsnorm_fwd(L.dtype_code(x.dtype), L.dtype_code(w.dtype), L.dtype_code(y.dtype),
                                    x_2d.data_ptr(), n_cols, w.data_ptr(), y.data_ptr(), n_cols, rstd.data_ptr(),
                                    rows, n_cols, float(eps), float(offset), int(mode), L.stream_of(x_2d)),
                "forge_rmsnorm_fwd")
    return y.view(x.shape), x_2d, w, rstd


def backward(dy, x_2d, weight, rstd, offset, variant, in_place, need_dw=True):
    """-> (dx [dy.shape], dw or None).  in_place: dx is written over dy's
    (contiguous) storage."""
    shape = dy.shape
    n_cols = shape[-1]
    dy_2d = dy.contiguous().view(-1, n_cols)
    if dy_2d.dtype != x_2d.dtype:  # e.g. v1's promoted fp32 output: the kernels take dy in x's dtype
        dy_2d = dy_2d.to(x_2d.dtype)
    rows = dy_2d.shape[0]
    dx = dy_2d if in_place else torch.empty_like(x_2d)
    dw = torch.empty(n_cols, device=x_2d.device, dtype=weight.dtype) if need_dw else None
    if rows and n_cols:
        ws = L.forge_rmsnorm_bwd_workspace(L.dtype_code(x_2d.dtype), rows, n_cols) if need_dw else 0
        work = torch.empty(ws, device=x_2d.device, dtype=torch.uint8) if need_dw else None
        L.check(L.forge_rmsnorm_bwd(L.dtype_code(x_2d.dtype), L.dtype_code(weight.dtype), dy_2d.data_ptr(), n_cols,
                                    x_2d.data_ptr(), n_cols, weight.data_ptr(), rstd.data_ptr(), dx.data_ptr(),
                                    n_cols, L.ptr(dw), L.ptr(work), rows, n_cols, float(offset), int(variant),
                                    L.stream_of(dy_2d)),
                "forge_rmsnorm_bwd")
    elif need_dw:
        dw.zero_()
    return dx.view(shape), dw
