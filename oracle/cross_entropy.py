"""Cross-entropy oracle (test infrastructure only; see oracle/__init__.py).

Restates the forward/backward semantics of the reference's v2 CE kernel
(kernels/cross_entropy/experiments/v2/cross_entropy_kernel_v2.py:65-458) in
fp32 (or fp64) PyTorch on the CPU:
  * ignored rows (target == ignore_index): loss 0, gradient 0, accuracy 0,
    predicted -1 (:139-151);
  * loss = lse - x_y with class weights, label smoothing, z-loss and softcap
    as in :298-330 and the test reference
    kernels/cross_entropy/tests/test_cross_entropy.py:263-301;
  * mean divides by n_non_ignore (or the sum of the targets' weights);
  * dlogits by autograd of that loss.
`ce_reference` is written from the formulas, not from F.cross_entropy, so the
pinning test can compare it against F.cross_entropy independently.
"""
from __future__ import annotations

import torch


def ce_reference(logits, target, weight=None, ignore_index=-100, lse_square_scale=0.0,
                 label_smoothing=0.0, reduction="mean", softcap=None, compute_dtype=torch.float32):
    """Returns (loss, z_loss, per_row_loss, token_accuracy, predicted, dlogits)
    all in compute_dtype (dlogits for grad_output = 1)."""
    x = logits.detach().cpu().to(compute_dtype).requires_grad_(True)
    t = target.detach().cpu()
    BT, V = x.shape
    valid = t != ignore_index
    t_safe = torch.where(valid, t, torch.zeros_like(t))
    xs = softcap * torch.tanh(x / softcap) if softcap is not None else x
    lse = torch.logsumexp(xs, dim=-1)
    x_y = xs.gather(1, t_safe.unsqueeze(1)).squeeze(1)
    nll = lse - x_y
    eps = label_smoothing / V
    if weight is not None:
        w = weight.detach().cpu().to(compute_dtype)
        w_y = w[t_safe]
        nll = w_y * nll
        smooth = -(eps * xs * w).sum(-1) + eps * lse * w.sum()
        denom = (w_y * valid).sum()
    else:
        smooth = -(eps * xs).sum(-1) + label_smoothing * lse
        denom = valid.sum().to(compute_dtype)
    loss_row = nll * (1 - label_smoothing) + smooth if label_smoothing > 0 else nll
    z_row = lse_square_scale * lse * lse
    n = valid.sum().to(compute_dtype)
    if reduction == "mean":
        # no valid row: every row is masked below; a unit divisor keeps the
        # masked branch finite so the gradient is 0, not NaN (v2 semantics)
        loss_row = loss_row / (denom if n > 0 else torch.ones_like(denom))
        z_row = z_row / n.clamp_min(1)
    loss_row = torch.where(valid, loss_row + z_row, torch.zeros_like(loss_row))
    z_row = torch.where(valid, z_row, torch.zeros_like(z_row))
    if reduction == "none":
        loss, z = loss_row, z_row
    else:
        loss, z = loss_row.sum(), z_row.sum()
    # the z-loss term only feeds the logging output, its gradient flows through loss
    (loss if loss.dim() == 0 else loss.sum()).backward()
    pred = torch.where(valid, xs.detach().argmax(-1), torch.full_like(t, -1))
    acc_row = ((pred == t) & valid).to(torch.float32)
    acc = acc_row if reduction == "none" else acc_row.sum() / valid.sum()
    return loss.detach(), z.detach(), loss_row.detach(), acc, pred, x.grad


def ce_bytes(n_cols: int, n_valid: int, n_ignored: int, elem_size: int = 2) -> int:
    """Algorithmic HBM bytes of one forward(+in-place gradient) call: valid
    rows read and write the row, ignored rows only write zeros, plus the
    int64 labels."""
    return n_cols * elem_size * (2 * n_valid + n_ignored) + 8 * (n_valid + n_ignored)
