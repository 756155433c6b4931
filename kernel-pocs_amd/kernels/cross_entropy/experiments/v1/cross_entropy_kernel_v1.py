"""Forge cross entropy v1 on MI355X.

Drop-in for kernels/cross_entropy/experiments/v1/cross_entropy_kernel_v1.py
of Forge-researchlab/kernel-POCs: `ForgeCrossEntropyFunction` (forward(ctx,
logits, target, ignore_index, reduction, label_smoothing), saves the
dlogits buffer, 5-tuple backward) and `forge_cross_entropy` with the same
arguments, ValueErrors, F.cross_entropy compatibility path and semantics:

  * hard-label CE with ignore_index, reduction mean / sum / none and label
    smoothing; no class weights, z-loss, softcap, accuracy or predictions
    (a `weight` sends the call to F.cross_entropy, as in the reference);
  * targets are validated on the host before the launch: IndexError
    "Target {t} is out of bounds. Expected < V" / "... Expected >= 0" (:252-267);
  * per-row losses are stored in the logits dtype (mean rows already divided
    by n_non_ignore) and summed with torch.sum (:292, :316);
  * `mean` with every target ignored returns NaN (0 / 0, :309-315), with
    zero gradients; v2 returns 0 there;
  * dlogits are written over the logits when they require grad; the
    backward multiplies by a per-row grad_output out of place ('none') or
    scales in place (scalar, skipped when it equals 1).

The row kernel is the v2 engine (`forge_ce_fwd`, csrc/cross_entropy.hip) run
without weights, z-loss, softcap or extra outputs, whose formulas reduce to
v1's for these features; target statistics come from
`forge_ce_target_stats`.
"""
from __future__ import annotations

from typing import Optional

import torch
import torch.nn.functional as F

from forge_hip import _lib as L


def _is_hip_path_supported(logits: torch.Tensor, target: torch.Tensor, weight: Optional[torch.Tensor],
                           reduction: str) -> bool:
    """The reference's `_is_triton_path_supported` (:200-218)."""
    return (
        logits.is_cuda
        and target.is_cuda
        and logits.ndim == 2
        and target.ndim == 1
        and target.numel() == logits.shape[0]
        and weight is None
        and reduction in {"mean", "sum", "none"}
        and logits.dtype in {torch.float16, torch.bfloat16, torch.float32}
    )


def _target_stats(target: torch.Tensor, ignore_index: int, vocab_size: int):
    """(n_non_ignore, min, max) of the masked targets from one device
    reduction (the reference's `_target_stats_triton`, :231-249) read by the
    host; returns the device stats buffer too."""
    stats = torch.empty(4, dtype=torch.int64, device=target.device)
    L.check(L.forge_ce_target_stats(target.data_ptr(), target.stride(-1), target.numel(), int(ignore_index),
                                    int(vocab_size), stats.data_ptr(), L.stream_of(target)),
            "forge_ce_target_stats")
    n, tmin, tmax, _ = stats.tolist()
    return int(n), int(tmin), int(tmax), stats


def _validate_targets(target: torch.Tensor, ignore_index: int, vocab_size: int):
    """The reference's `_validate_targets` (:252-267)."""
    n_non_ignore, min_target, max_target, stats = _target_stats(target, ignore_index, vocab_size)
    if n_non_ignore == 0:
        return 0, stats
    if max_target >= vocab_size:
        raise IndexError(f"Target {max_target} is out of bounds. Expected < {vocab_size}")
    if min_target < 0:
        raise IndexError(f"Target {min_target} is out of bounds. Expected >= 0")
    return n_non_ignore, stats


def _forward_hip(logits: torch.Tensor, target: torch.Tensor, ignore_index: int, reduction: str,
                 label_smoothing: float):
    """The reference's `_forward_triton` (:270-316)."""
    bt, vocab_size = logits.shape
    if target.dtype != torch.int64:
        target = target.to(torch.int64)
    if logits.stride(-1) != 1:
        logits = logits.contiguous()
    if target.stride(-1) != 1:
        target = target.contiguous()
    n_non_ignore, stats = _validate_targets(target, ignore_index, vocab_size)

    loss_rows = torch.empty(bt, dtype=torch.float32, device=logits.device)
    flags = L.CE_HAS_GRADIENTS if logits.requires_grad else 0
    if reduction == "mean":
        flags |= L.CE_REDUCTION_MEAN
    if bt > 0:
        L.check(
            L.forge_ce_fwd(L.dtype_code(logits.dtype), logits.data_ptr(), logits.stride(0), bt, vocab_size,
                           target.data_ptr(), target.stride(0), None, loss_rows.data_ptr(), None, None, None,
                           int(ignore_index), float(n_non_ignore), 0.0, 0.0, 0.0, float(label_smoothing), 0.0,
                           flags, stats.data_ptr(), L.stream_of(logits)),
            "forge_ce_fwd",
        )
    # the reference's loss_1d holds each row in the logits dtype
    loss_1d = loss_rows.to(logits.dtype)
    saved = logits if logits.requires_grad else None
    if reduction == "none":
        return loss_1d, saved
    if reduction == "mean" and n_non_ignore == 0:
        # every target ignored: 0 / 0 = NaN, as PyTorch returns (:309-315)
        return torch.sum(loss_1d) / n_non_ignore, saved
    return torch.sum(loss_1d), saved


def _scale_saved_gradient(saved_grad: torch.Tensor, grad_output: torch.Tensor) -> torch.Tensor:
    """The reference's `_scale_saved_gradient` (:319-333).  The scalar case
    runs `forge_ce_scale`, which skips the multiply on the device when
    grad_output == 1 (the reference compares on the host)."""
    if grad_output.ndim > 0:
        return saved_grad * grad_output.unsqueeze(1)
    g = grad_output.detach()
    if g.dtype not in (torch.float32, torch.bfloat16, torch.float16):
        g = g.to(torch.float32)
    g = g.reshape(1).contiguous()
    bt, vocab_size = saved_grad.shape
    L.check(L.forge_ce_scale(L.dtype_code(saved_grad.dtype), saved_grad.data_ptr(), saved_grad.stride(0), bt,
                             vocab_size, g.data_ptr(), L.dtype_code(g.dtype), L.stream_of(saved_grad)),
            "forge_ce_scale")
    return saved_grad


class ForgeCrossEntropyFunction(torch.autograd.Function):
    """cross_entropy_kernel_v1.py:336-361."""

    @staticmethod
    def forward(ctx, logits: torch.Tensor, target: torch.Tensor, ignore_index: int, reduction: str,
                label_smoothing: float) -> torch.Tensor:
        loss, saved_grad = _forward_hip(logits, target, ignore_index, reduction, label_smoothing)
        if saved_grad is not None:
            ctx.save_for_backward(saved_grad.detach())
        else:
            ctx.save_for_backward()
        return loss

    @staticmethod
    def backward(ctx, grad_output: torch.Tensor):
        saved = ctx.saved_tensors
        grad_logits = _scale_saved_gradient(saved[0], grad_output) if saved else None
        return grad_logits, None, None, None, None


def forge_cross_entropy(
    logits: torch.Tensor,
    target: torch.Tensor,
    weight: Optional[torch.Tensor] = None,
    ignore_index: int = -100,
    reduction: str = "mean",
    label_smoothing: float = 0.0,
) -> torch.Tensor:
    """cross_entropy_kernel_v1.py:364-389."""
    if reduction not in {"mean", "sum", "none"}:
        raise ValueError(f"reduction must be one of 'mean', 'sum', or 'none'. Got: {reduction}")
    if not 0.0 <= label_smoothing <= 1.0:
        raise ValueError(f"label_smoothing must be between 0.0 and 1.0. Got: {label_smoothing}")

    if not _is_hip_path_supported(logits, target, weight, reduction):
        return F.cross_entropy(
            logits,
            target,
            weight=weight,
            ignore_index=ignore_index,
            reduction=reduction,
            label_smoothing=label_smoothing,
        )

    return ForgeCrossEntropyFunction.apply(logits, target, ignore_index, reduction, label_smoothing)


__all__ = ["ForgeCrossEntropyFunction", "forge_cross_entropy"]
