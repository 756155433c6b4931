"""Forge cross entropy v2 on MI355X.

Drop-in for kernels/cross_entropy/experiments/v2/cross_entropy_kernel_v2.py of
Forge-researchlab/kernel-POCs: same public API (`CrossEntropyOutput`,
`ForgeCrossEntropyFunction`, `forge_cross_entropy`, `ForgeCrossEntropyLoss`,
`cross_entropy_forward`, `cross_entropy_backward`) and the same execution
contract: the forward computes the loss and, when the logits require grad,
writes dloss/dlogits over the logits buffer, which is what backward returns.
Features: class weights, ignore_index, label smoothing, z-loss, softcap,
token accuracy, predicted tokens, mean/sum/none reductions.

Device work (libforge_hip.so, csrc/cross_entropy.hip): without class
weights the forward is ONE launch, `forge_ce_fwd_reduce`: it computes the
target statistics (count and range), the per-row losses, dlogits in place and
the reduced loss (fixed-order sum, cast to the logits dtype); the host reads
the statistics for the reference's bounds asserts with `forge_ce_stats_wait`
as soon as the launch has them (the launch copies them to pinned host memory
itself; no event or copy sits between kernels).  With class weights the host
needs the validated count before the launch, as the reference does:
`forge_ce_target_stats`, the host check, `forge_ce_fwd`, `forge_sum_f32`.
The backward is `forge_ce_scale` (a no-op on the device when grad_output is
1).

Numerics: per-row losses are kept in fp32 and summed in fp32, then cast to the
logits dtype once (the reference rounds every row to the logits dtype before
`torch.sum`, :373 and :451); the returned dtype is the same.
"""
from __future__ import annotations

import ctypes
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


def _target_stats_launch(target: torch.Tensor, ignore_index: int, n_cols: int):
    """Queues forge_ce_target_stats and an event after it; returns (device
    stats, event).  The reference reads the same values with `.item()`
    (:374-387) before launching."""
    stats = torch.empty(4, dtype=torch.int64, device=target.device)
    L.check(
        L.forge_ce_target_stats(target.data_ptr(), target.stride(-1), target.numel(), int(ignore_index), int(n_cols),
                                stats.data_ptr(), L.stream_of(target)),
        "forge_ce_target_stats",
    )
    ready = torch.cuda.Event()
    ready.record(torch.cuda.current_stream(target.device))
    return stats, ready



def _target_stats_to_host(stats: torch.Tensor, ready):
    """Copies the 4 statistics to pinned host memory on a side stream that
    waits only for the statistics kernel (`ready`), not for the row kernel
    queued after it; returns (host stats, done event)."""
    side = _side_stream(stats.device)
    side.wait_event(ready)
    host = torch.empty(4, dtype=torch.int64, pin_memory=True)
    with torch.cuda.stream(side):
        host.copy_(stats, non_blocking=True)
        done = torch.cuda.Event()
        done.record(side)
    stats.record_stream(side)
    return host, done


def _target_stats_async(target: torch.Tensor, ignore_index: int, n_cols: int):
    """Statistics kernel and its host copy together -> (stats, host, event)
    (used where the host needs the values before the next launch)."""
    stats, ready = _target_stats_launch(target, ignore_index, n_cols)
    host, done = _target_stats_to_host(stats, ready)
    return stats, host, done


_SIDE_STREAMS = {}


def _side_stream(device) -> "torch.cuda.Stream":
    """One default-priority side stream per device for the stats copy."""
    key = torch.device(device).index
    s = _SIDE_STREAMS.get(key)
    if s is None:
        s = _SIDE_STREAMS[key] = torch.cuda.Stream(device=device)
    return s


def _check_targets(host: torch.Tensor, ev, n_cols: int) -> int:
    """The reference's bounds asserts (:382-387) on the masked target range;
    returns n_non_ignore."""
    ev.synchronize()
    n, tmin, tmax, _ = host.tolist()
    assert tmax < n_cols, f"Target {tmax} is out of bounds. Expected < {n_cols}"
    assert tmin >= 0, f"Target {tmin} is out of bounds. Expected >= 0"
    return int(n)


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
    out_dtype=None,
):
    """Returns (loss, z_loss, token_accuracy, predicted_tokens, _input); loss
    and z_loss are fp32 unless out_dtype is given (then a reduced loss is
    already cast to it, by the launch that sums it)."""
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

    if target.dtype != torch.int64:
        target = target.to(torch.int64)
    if target.stride(-1) != 1:
        target = target.contiguous()
    if _input.stride(-1) != 1:
        _input = _input.contiguous()

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
    reduce = reduction != "none"
    st = L.stream_of(_input)
    n_non_ignore = 0
    loss = z_loss = None

    if BT > 0 and weight is None:
        # one launch: target statistics, row losses, dlogits and the reduced
        # loss; the host reads the statistics (for the bounds asserts) as soon
        # as the launch has them, while the rest of it runs
        cast = None if out_dtype in (None, torch.float32) else out_dtype
        if reduce:
            loss = torch.empty((), dtype=torch.float32, device=dev)
            loss_c = torch.empty((), dtype=cast, device=dev) if cast is not None else None
            if return_z_loss:
                z_loss = torch.empty((), dtype=torch.float32, device=dev)
                z_c = torch.empty((), dtype=cast, device=dev) if cast is not None else None
        ticket = ctypes.c_uint64()
        L.check(
            L.forge_ce_fwd_reduce(
                L.dtype_code(_input.dtype), _input.data_ptr(), _input.stride(-2), BT, V,
                target.data_ptr(), target.stride(-1),
                loss_1d.data_ptr(), L.ptr(z_loss_1d), L.ptr(token_accuracy_1d), L.ptr(predicted_tokens_1d),
                int(ignore_index), float(lse_square_scale), float(label_smoothing), float(softcap or 0.0), flags,
                L.ptr(loss), L.ptr(z_loss), L.ptr(loss_c) if reduce else None,
                L.ptr(z_c) if reduce and return_z_loss else None,
                L.dtype_code(cast) if cast is not None else L.DTYPE_F32, ctypes.byref(ticket), st,
            ),
            "forge_ce_fwd_reduce",
        )
        n_non_ignore = _wait_targets(ticket.value, V, st)
        if reduce and cast is not None:
            loss = loss_c
            z_loss = z_c if return_z_loss else None
    elif BT > 0:
        # class weights: the weighted sums need validated targets first, as in
        # the reference
        stats, ready = _target_stats_launch(target, ignore_index, V)
        stats_host, stats_ev = _target_stats_to_host(stats, ready)
        n_non_ignore = _check_targets(stats_host, stats_ev, V)
        assert weight.shape[0] == V, f"If given, weight has to be a Tensor of size V. Got: {weight.shape}"
        assert torch.is_floating_point(weight), (
            f"If given, weight has to be a Tensor of floating point dtype. Got: {weight.dtype}"
        )
        target_mask = target != ignore_index
        sum_non_ignore_weight = torch.gather(weight, dim=0, index=target.masked_select(target_mask)).sum().item()
        weight_sum = weight.sum().item()
        weight = weight.to(torch.float32).contiguous()
        L.check(
            L.forge_ce_fwd(
                L.dtype_code(_input.dtype), _input.data_ptr(), _input.stride(-2), BT, V,
                target.data_ptr(), target.stride(-1), L.ptr(weight),
                loss_1d.data_ptr(), L.ptr(z_loss_1d), L.ptr(token_accuracy_1d), L.ptr(predicted_tokens_1d),
                int(ignore_index), float(n_non_ignore), float(sum_non_ignore_weight), float(weight_sum),
                float(lse_square_scale), float(label_smoothing), float(softcap or 0.0), flags,
                stats.data_ptr(), st,
            ),
            "forge_ce_fwd",
        )
    elif weight is not None:
        assert weight.shape[0] == V, f"If given, weight has to be a Tensor of size V. Got: {weight.shape}"
        assert torch.is_floating_point(weight), (
            f"If given, weight has to be a Tensor of floating point dtype. Got: {weight.dtype}"
        )

    if not reduce:
        loss = loss_1d
        z_loss = z_loss_1d if return_z_loss else None
        token_accuracy = token_accuracy_1d if return_token_accuracy else None
    else:
        if loss is None:  # weighted path, or no rows
            loss = _sum_f32(loss_1d, out_dtype)
            z_loss = _sum_f32(z_loss_1d, out_dtype) if return_z_loss else None
        token_accuracy = torch.sum(token_accuracy_1d) / n_non_ignore if return_token_accuracy else None
    predicted_tokens = predicted_tokens_1d if return_predicted_tokens else None
    return loss, z_loss, token_accuracy, predicted_tokens, _input


def _wait_targets(ticket: int, n_cols: int, stream) -> int:
    """The reference's bounds asserts (:382-387) on the statistics the
    forge_ce_fwd_reduce launch of `ticket` computed; returns n_non_ignore."""
    host = (ctypes.c_int64 * 4)()
    L.check(L.forge_ce_stats_wait(ticket, host, stream), "forge_ce_stats_wait")
    n, tmin, tmax, _ = host
    assert tmax < n_cols, f"Target {tmax} is out of bounds. Expected < {n_cols}"
    assert tmin >= 0, f"Target {tmin} is out of bounds. Expected >= 0"
    return int(n)


def _sum_f32(x: torch.Tensor, out_dtype=None) -> torch.Tensor:
    """fp32 sum of x (one deterministic workgroup); with out_dtype, the sum
    rounded to that dtype, from the same kernel."""
    out = torch.empty((), dtype=torch.float32, device=x.device)
    cast = None if out_dtype in (None, torch.float32) else torch.empty((), dtype=out_dtype, device=x.device)
    L.check(L.forge_sum_f32(x.data_ptr(), x.numel(), out.data_ptr(), L.ptr(cast),
                            L.dtype_code(out_dtype) if cast is not None else L.DTYPE_F32, L.stream_of(x)),
            "forge_sum_f32")
    return out if cast is None else cast


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
        return_z_loss, return_token_accuracy, return_predicted_tokens, out_dtype=_input.dtype,
    )
    loss = loss.to(_input.dtype)  # reduced losses already are (no-op); 'none' rows are cast here
    if z_loss is not None:
        z_loss = z_loss.to(_input.dtype)
    return loss, z_loss, acc, pred, _input


def cross_entropy_backward(_input, grad_output):
    """cross_entropy_kernel_v2.py:461-485."""
    # If cross entropy is the last layer, grad_output is 1.0: nothing to do.
    # For a scalar grad_output forge_ce_scale makes that test on the device
    # (a no-op kernel when it is 1.0), so the host does not wait on the GPU.
    if grad_output.ndim > 0:
        _input = _input * grad_output.unsqueeze(dim=1)
    else:
        BT, V = _input.shape
        g = grad_output.detach()
        if g.dtype not in (torch.float32, torch.bfloat16, torch.float16):
            g = g.to(torch.float32)
        g = g.reshape(1).contiguous()
        L.check(
            L.forge_ce_scale(L.dtype_code(_input.dtype), _input.data_ptr(), _input.stride(-2), BT, V,
                             g.data_ptr(), L.dtype_code(g.dtype), L.stream_of(_input)),
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
