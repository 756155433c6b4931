"""Forge cross entropy v2 on MI355X.

Drop-in for kernels/cross_entropy/experiments/v2/cross_entropy_kernel_v2.py of
Forge-researchlab/kernel-POCs: same public API (`CrossEntropyOutput`,
`ForgeCrossEntropyFunction`, `forge_cross_entropy`, `ForgeCrossEntropyLoss`,
`cross_entropy_forward`, `cross_entropy_backward`) and the same execution
contract: the forward computes the loss and, when the logits require grad,
writes dloss/dlogits over the logits buffer, which is what backward returns.
Features: class weights, ignore_index, label smoothing, z-loss, softcap,
token accuracy, predicted tokens, mean/sum/none reductions.

Device work: `forge_ce_fwd` (row kernel), `forge_sum_f32` (loss reduction)
and `forge_ce_scale` (grad_output != 1) in libforge_hip.so
(csrc/cross_entropy.hip).

Numerics: per-row losses are kept in fp32 and summed in fp32, then cast to the
logits dtype once (the reference rounds every row to the logits dtype before
`torch.sum`, :373 and :451); the returned dtype is the same.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import torch

from forge_hip import _lib as L


@dataclass(frozen=True)
class CrossEntropyOutput:
    """cross_entropy_kernel_v2.py:41-46."""

    loss: torch.Tensor
    z_loss: Optional[torch.Tensor] = None
    token_accuracy: Optional[torch.Tensor] = None
    predicted_tokens: Optional[torch.Tensor] = None


def _target_stats(target: torch.Tensor, ignore_index: int):
    """n_non_ignore and the masked target range in one host sync (the
    reference takes them with .item() and two asserts, :382-387)."""
    mask = target != ignore_index
    masked = target * mask
    n, tmax, tmin = torch.stack([mask.sum(), masked.max(), masked.min()]).tolist()
    return mask, int(n), int(tmax), int(tmin)


def _cross_entropy_forward_impl(
    _input,
    target,
    weight,
    ignore_index,
    lse_square_scale,
    label_smoothing,
    reduction,
    softcap,
    return_z_loss,
    return_token_accuracy=False,
    return_predicted_tokens=False,
):
    """Returns (loss_fp32, z_loss_fp32, token_accuracy, predicted_tokens, _input)
    before the final cast of loss / z_loss to the logits dtype."""
    assert isinstance(return_z_loss, bool), f"return_z_loss must be True or False. Got: {return_z_loss}"
    assert isinstance(return_token_accuracy, bool), (
        f"return_token_accuracy must be True or False. Got: {return_token_accuracy}"
    )
    assert isinstance(return_predicted_tokens, bool), (
        f"return_predicted_tokens must be True or False. Got: {return_predicted_tokens}"
    )
    L.require_gpu(_input, target)
    BT, V = _input.shape
    dev = _input.device

    loss_1d = torch.empty(BT, dtype=torch.float32, device=dev)
    z_loss_1d = torch.empty(BT, dtype=torch.float32, device=dev) if return_z_loss else None
    token_accuracy_1d = torch.empty(BT, dtype=torch.float32, device=dev) if return_token_accuracy else None
    predicted_tokens_1d = torch.empty(BT, dtype=torch.int64, device=dev) if return_predicted_tokens else None

    if BT > 0:
        target_mask, n_non_ignore, tmax, tmin = _target_stats(target, ignore_index)
        assert tmax < V, f"Target {tmax} is out of bounds. Expected < {V}"
        assert tmin >= 0, f"Target {tmin} is out of bounds. Expected >= 0"
    else:
        target_mask, n_non_ignore = target != ignore_index, 0
    sum_non_ignore_weight = float(n_non_ignore)
    weight_sum = 0.0
    if weight is not None:
        assert weight.shape[0] == V, f"If given, weight has to be a Tensor of size V. Got: {weight.shape}"
        assert torch.is_floating_point(weight), (
            f"If given, weight has to be a Tensor of floating point dtype. Got: {weight.dtype}"
        )
        sum_non_ignore_weight = torch.gather(weight, dim=0, index=target.masked_select(target_mask)).sum().item()
        weight_sum = weight.sum().item()
        weight = weight.to(torch.float32).contiguous()

    if _input.stride(-1) != 1:
        _input = _input.contiguous()
    if target.stride(-1) != 1:
        target = target.contiguous()

    flags = 0
    if _input.requires_grad:
        flags |= L.CE_HAS_GRADIENTS
    if weight is not None:
        flags |= L.CE_HAS_WEIGHT
    if softcap is not None:
        flags |= L.CE_HAS_SOFTCAP
    if return_z_loss:
        flags |= L.CE_RETURN_Z_LOSS
    if return_token_accuracy:
        flags |= L.CE_RETURN_ACCURACY
    if return_predicted_tokens:
        flags |= L.CE_RETURN_PREDICTED
    if reduction == "mean":
        flags |= L.CE_REDUCTION_MEAN

    if BT > 0:
        L.check(
            L.forge_ce_fwd(
                L.dtype_code(_input.dtype), _input.data_ptr(), _input.stride(-2), BT, V,
                target.data_ptr(), target.stride(-1), L.ptr(weight),
                loss_1d.data_ptr(), L.ptr(z_loss_1d), L.ptr(token_accuracy_1d), L.ptr(predicted_tokens_1d),
                int(ignore_index), float(n_non_ignore), float(sum_non_ignore_weight), float(weight_sum),
                float(lse_square_scale), float(label_smoothing), float(softcap or 0.0), flags,
                L.stream_of(_input),
            ),
            "forge_ce_fwd",
        )

    if reduction == "none":
        loss = loss_1d
        z_loss = z_loss_1d if return_z_loss else None
        token_accuracy = token_accuracy_1d if return_token_accuracy else None
    else:
        loss = _sum_f32(loss_1d)
        z_loss = _sum_f32(z_loss_1d) if return_z_loss else None
        token_accuracy = torch.sum(token_accuracy_1d) / n_non_ignore if return_token_accuracy else None
    predicted_tokens = predicted_tokens_1d if return_predicted_tokens else None
    return loss, z_loss, token_accuracy, predicted_tokens, _input


def _sum_f32(x: torch.Tensor) -> torch.Tensor:
    out = torch.empty((), dtype=torch.float32, device=x.device)
    L.check(L.forge_sum_f32(x.data_ptr(), x.numel(), out.data_ptr(), L.stream_of(x)), "forge_sum_f32")
    return out


def cross_entropy_forward(
    _input,
    target,
    weight,
    ignore_index,
    lse_square_scale,
    label_smoothing,
    reduction,
    softcap,
    return_z_loss,
    return_token_accuracy=False,
    return_predicted_tokens=False,
):
    """cross_entropy_kernel_v2.py:346-458 -> (loss, z_loss, token_accuracy,
    predicted_tokens, _input); with _input.requires_grad the logits now hold
    dloss/dlogits."""
    loss, z_loss, acc, pred, _input = _cross_entropy_forward_impl(
        _input, target, weight, ignore_index, lse_square_scale, label_smoothing, reduction, softcap,
        return_z_loss, return_token_accuracy, return_predicted_tokens,
    )
    loss = loss.to(_input.dtype)
    if z_loss is not None:
        z_loss = z_loss.to(_input.dtype)
    return loss, z_loss, acc, pred, _input


def cross_entropy_backward(_input, grad_output):
    """cross_entropy_kernel_v2.py:461-485."""
    # If cross entropy is the last layer, grad_output is 1.0: nothing to do.
    if torch.equal(grad_output, torch.tensor(1.0, device=grad_output.device)):
        pass
    elif grad_output.ndim > 0:
        _input = _input * grad_output.unsqueeze(dim=1)
    else:
        BT, V = _input.shape
        g = grad_output.detach().to(torch.float32).reshape(1).contiguous()
        L.check(
            L.forge_ce_scale(L.dtype_code(_input.dtype), _input.data_ptr(), _input.stride(-2), BT, V,
                             g.data_ptr(), L.stream_of(_input)),
            "forge_ce_scale",
        )
    return _input


class ForgeCrossEntropyFunction(torch.autograd.Function):
    """cross_entropy_kernel_v2.py:488-590."""

    @staticmethod
    def forward(
        ctx,
        _input: torch.Tensor,
        target: torch.Tensor,
        weight: Optional[torch.FloatTensor],
        ignore_index: int = -100,
        lse_square_scale: float = 0.0,
        label_smoothing: float = 0.0,
        reduction: str = "mean",
        softcap: Optional[float] = None,
        return_z_loss: bool = False,
        return_token_accuracy: bool = False,
        return_predicted_tokens: bool = False,
    ):
        input_requires_grad = _input.requires_grad
        loss, z_loss, token_accuracy, predicted_tokens, _input = cross_entropy_forward(
            _input, target, weight, ignore_index, lse_square_scale, label_smoothing, reduction,
            softcap, return_z_loss, return_token_accuracy, return_predicted_tokens,
        )
        if input_requires_grad:
            ctx.save_for_backward(_input.detach())
        ctx.return_z_loss = return_z_loss
        ctx.return_token_accuracy = return_token_accuracy
        ctx.return_predicted_tokens = return_predicted_tokens
        return loss, z_loss, token_accuracy, predicted_tokens

    @staticmethod
    def backward(ctx, grad_output, grad_output2, grad_output3, grad_output4):
        (_input,) = ctx.saved_tensors
        _input = cross_entropy_backward(_input, grad_output)
        return (_input, None, None, None, None, None, None, None, None, None, None)


def forge_cross_entropy(
    _input: torch.Tensor,
    target: torch.Tensor,
    weight: Optional[torch.FloatTensor] = None,
    ignore_index: int = -100,
    lse_square_scale: float = 0.0,
    label_smoothing: float = 0.0,
    reduction: str = "mean",
    softcap: Optional[float] = None,
    return_z_loss: bool = False,
    return_token_accuracy: bool = False,
    return_predicted_tokens: bool = False,
):
    """cross_entropy_kernel_v2.py:593-629."""
    loss, z_loss, token_accuracy, predicted_tokens = ForgeCrossEntropyFunction.apply(
        _input, target, weight, ignore_index, lse_square_scale, label_smoothing, reduction, softcap,
        return_z_loss, return_token_accuracy, return_predicted_tokens,
    )
    if not return_z_loss and not return_token_accuracy and not return_predicted_tokens:
        return loss
    return CrossEntropyOutput(
        loss=loss, z_loss=z_loss, token_accuracy=token_accuracy, predicted_tokens=predicted_tokens
    )


class ForgeCrossEntropyLoss(torch.nn.Module):
    """cross_entropy_kernel_v2.py:632-678."""

    def __init__(
        self,
        weight: Optional[torch.FloatTensor] = None,
        ignore_index: int = -100,
        lse_square_scale: float = 0.0,
        label_smoothing: float = 0.0,
        reduction: str = "mean",
        softcap: Optional[float] = None,
        return_z_loss: bool = False,
        return_token_accuracy: bool = False,
        return_predicted_tokens: bool = False,
    ):
        super().__init__()
        assert (label_smoothing >= 0) and (label_smoothing <= 1), (
            f"label_smoothing must be between 0.0 and 1.0. Got: {label_smoothing}"
        )
        assert reduction in {"mean", "sum", "none"}, (
            f"reduction must be one of 'mean', 'sum', or 'none'. Got: {reduction}"
        )
        assert softcap is None or softcap > 0, f"softcap must greater than 0.0 or None. Got: {softcap}"
        self.weight = weight
        self.ignore_index = ignore_index
        self.lse_square_scale = lse_square_scale
        self.label_smoothing = label_smoothing
        self.reduction = reduction
        self.softcap = softcap
        self.return_z_loss = return_z_loss
        self.return_token_accuracy = return_token_accuracy
        self.return_predicted_tokens = return_predicted_tokens

    def forward(self, _input: torch.Tensor, target: torch.Tensor):
        return forge_cross_entropy(
            _input, target, weight=self.weight, ignore_index=self.ignore_index,
            lse_square_scale=self.lse_square_scale, label_smoothing=self.label_smoothing,
            reduction=self.reduction, softcap=self.softcap, return_z_loss=self.return_z_loss,
            return_token_accuracy=self.return_token_accuracy,
            return_predicted_tokens=self.return_predicted_tokens,
        )
