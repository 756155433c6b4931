"""Fused linear + cross-entropy oracle (test infrastructure only; see
oracle/__init__.py).

Restates `fused_linear_cross_entropy_forward` / `_backward`
(kernels/cross_entropy/experiments/v2/fused_linear_cross_entropy.py:31-280)
on the CPU:
  * logits = X W^T (+ b) (:142-144);
  * the v2 CE row semantics on the logits (`ce_reference`), with the mean
    over the batch's non-ignored rows (one global n_non_ignore, :87);
  * optional token scaling (:146-160, 196-205): every row's loss, z-loss and
    dlogits times the detached softmax probability of its target
    (softcapped logits; 0 for ignored rows);
  * dX = dlogits W, dW = dlogits^T X, db = colsum(dlogits) (:207-219), for
    grad_output = 1 (the backward multiplies all three by a scalar
    grad_output, :248-280).
Chunking over tokens changes only summation order, so the oracle works on the
whole batch at once.
"""
from __future__ import annotations

import torch

from .cross_entropy import ce_reference


def fused_linear_ce(X, W, target, bias=None, ce_weight=None, ignore_index=-100, lse_square_scale=0.0,
                    label_smoothing=0.0, reduction="mean", softcap=None, use_token_scaling=False,
                    compute_dtype=torch.float64):
    """Returns a dict: loss, z_loss, token_accuracy, predicted, dX, dW, db
    (db None without bias), all in compute_dtype except predicted (int64)."""
    cd = compute_dtype
    x = X.detach().cpu().to(cd)
    w = W.detach().cpu().to(cd)
    t = target.detach().cpu().to(torch.int64)
    logits = x @ w.t()
    if bias is not None:
        logits = logits + bias.detach().cpu().to(cd)
    loss, z, loss_row, acc, pred, dlogits = ce_reference(
        logits, t, weight=ce_weight, ignore_index=ignore_index, lse_square_scale=lse_square_scale,
        label_smoothing=label_smoothing, reduction=reduction, softcap=softcap, compute_dtype=cd)
    valid = t != ignore_index
    if use_token_scaling:
        xs = softcap * torch.tanh(logits / softcap) if softcap is not None else logits
        p = torch.softmax(xs, dim=-1).gather(1, torch.where(valid, t, 0).unsqueeze(1)).squeeze(1)
        s = torch.where(valid, p, torch.zeros_like(p))
        lse = torch.logsumexp(xs, dim=-1)
        z_row = lse_square_scale * lse * lse
        if reduction == "mean":
            z_row = z_row / valid.sum().clamp_min(1)
        z_row = torch.where(valid, z_row, torch.zeros_like(z_row))
        loss_row = loss_row * s
        z_row = z_row * s
        dlogits = dlogits * s.unsqueeze(1)
        loss = loss_row if reduction == "none" else loss_row.sum()
        z = z_row if reduction == "none" else z_row.sum()
    dX = dlogits @ w
    dW = dlogits.t() @ x
    db = dlogits.sum(0) if bias is not None else None
    return {"loss": loss, "z_loss": z, "token_accuracy": acc, "predicted": pred, "dX": dX, "dW": dW, "db": db}


def flops(bt: int, h: int, v: int) -> int:
    """Algorithmic FLOPs of one forward + backward: the logits GEMM and the
    dX and dW GEMMs, 2 BT H V each."""
    return 3 * 2 * bt * h * v
