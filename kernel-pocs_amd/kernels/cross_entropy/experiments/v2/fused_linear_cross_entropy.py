"""Forge fused linear + cross entropy v2 on MI355X.

Drop-in for kernels/cross_entropy/experiments/v2/fused_linear_cross_entropy.py
of Forge-researchlab/kernel-POCs: same public API
(`fused_linear_cross_entropy_forward/backward`,
`ForgeFusedLinearCrossEntropyFunction`, `forge_fused_linear_cross_entropy`,
`ForgeFusedLinearCrossEntropyLoss`), argument checks and messages, and the
same execution contract: the forward computes the loss and, when the hidden
states require grad, the gradients for input, weight and bias, which the
backward returns (scaled by grad_output).  `F.cross_entropy(F.linear(x, W, b),
target)` without materialising the whole [BT, V] logits at once.

Per token chunk (all device work in libforge_hip.so):
  1. logits = X_c W^T (+ b)
       bf16 with H % 8 == 0: the MFMA GEMM (4-wave engine); the bias is one
       more 8-wide K segment ([X_c | 1] [W | b]^T), so it is added to the fp32
       accumulator.  Otherwise forge_gemm_generic (fp32 accumulation, any
       dtype / shape).
  2. optional token scaling: forge_ce_target_prob (before the CE kernel
     overwrites the logits), then forge_row_scale of the loss rows and dlogits
  3. forge_ce_fwd on the chunk, in place, with the target statistics of the
     whole batch (the mean divides by the global non-ignored count)
  4. dX_c = dlogits W (MFMA on a cached, row-padded W^T, or generic),
     dW += dlogits^T X_c (fp32, beta accumulation over chunks; on the MFMA
     path both operands are first transposed by forge_transpose_2b so the
     product is K-contiguous for the 4-wave GEMM; a batch that is one chunk
     writes bf16 dW straight from the fp32 accumulators, one rounding),
     db += colsum(dlogits) (generic GEMM with a ones row)
Chunks are sized to ~2 GiB of logits (MI355X has 288 GB of HBM): the
reference's ~V/H-fold split (256-token chunks at the Llama-3 shape) would
re-read and re-write the fp32 weight gradient 32 times.  Chunking changes
only the fp32 summation order of dW and db.  Every product is the
library's own GEMM (the reference's three torch matmuls per chunk,
kernels/cross_entropy/experiments/v2/fused_linear_cross_entropy.py:142,
212-214).
"""
from __future__ import annotations

from typing import Optional

import torch

from forge_hip import _lib as L
from kernels._lora_ops import COL, ROW, frozen_t, gemm, ld

from .cross_entropy_kernel_v2 import CrossEntropyOutput, _check_targets, _sum_f32, _target_stats_async

__all__ = [
    "ForgeFusedLinearCrossEntropyFunction",
    "ForgeFusedLinearCrossEntropyLoss",
    "fused_linear_cross_entropy_forward",
    "fused_linear_cross_entropy_backward",
    "forge_fused_linear_cross_entropy",
]

_LOGITS_CHUNK_BYTES = 1 << 31


def _chunk_rows(bt: int, row_bytes: int) -> int:
    n = max(1, _LOGITS_CHUNK_BYTES // max(1, row_bytes))
    if n >= bt:
        return bt
    return max(256, (n // 256) * 256)


def _fast_path(x: torch.Tensor, weight: torch.Tensor) -> bool:
    """bf16 operands whose rows the MFMA GEMM reads in 16-byte chunks."""
    h = x.shape[1]
    return (x.dtype == torch.bfloat16 and weight.dtype == torch.bfloat16 and h % 8 == 0
            and x.data_ptr() % 16 == 0 and weight.data_ptr() % 16 == 0)


def _generic(M, N, K, dtype, a, a_sm, a_sk, b, b_sk, b_sn, c, ldc, c_dtype, beta=0.0, bias=None):
    L.check(L.forge_gemm_generic(M, N, K, L.dtype_code(dtype), a.data_ptr(), a_sm, a_sk, b.data_ptr(), b_sk, b_sn,
                                 c.data_ptr(), ldc, L.dtype_code(c_dtype), 1.0, float(beta), L.ptr(bias),
                                 L.GEMM_ACT_NONE, L.stream_of(c)),
            "forge_gemm_generic")


def _cast_into(src_f32: torch.Tensor, out: torch.Tensor) -> torch.Tensor:
    """out[...] = src (fp32 [rows, cols] with unit last stride) rounded once."""
    rows, cols = out.shape
    L.check(L.forge_splitk_reduce(src_f32.data_ptr(), 0, 1, rows, cols, src_f32.stride(0), out.data_ptr(),
                                  out.stride(0), L.dtype_code(out.dtype), 1.0, L.stream_of(out)),
            "forge_splitk_reduce")
    return out


def fused_linear_cross_entropy_forward(
    _input: torch.Tensor,
    weight: torch.Tensor,
    target: torch.Tensor,
    ce_weight: Optional[torch.Tensor] = None,
    bias: Optional[torch.Tensor] = None,
    ignore_index: int = -100,
    lse_square_scale: float = 0.0,
    label_smoothing: float = 0.0,
    reduction: str = "mean",
    softcap: Optional[float] = None,
    return_z_loss: bool = False,
    accum_dtype: Optional[torch.dtype] = None,
    use_token_scaling: bool = False,
    return_token_accuracy: bool = False,
    return_predicted_tokens: bool = False,
):
    """fused_linear_cross_entropy.py:31-245 -> (loss, z_loss, token_accuracy,
    predicted_tokens, grad_input, grad_weight, grad_bias)."""
    assert isinstance(return_z_loss, bool), f"return_z_loss must be True or False. Got: {return_z_loss}"
    assert isinstance(return_token_accuracy, bool), (
        f"return_token_accuracy must be True or False. Got: {return_token_accuracy}"
    )
    assert isinstance(return_predicted_tokens, bool), (
        f"return_predicted_tokens must be True or False. Got: {return_predicted_tokens}"
    )

    if _input.ndim != 2:
        raise ValueError(f"_input must be 2D (B*T, H); got shape={tuple(_input.shape)}")
    if weight.ndim != 2:
        raise ValueError(f"weight must be 2D (V, H); got shape={tuple(weight.shape)}")
    if target.ndim != 1:
        raise ValueError(f"target must be 1D (B*T,); got shape={tuple(target.shape)}")

    BT, H = _input.shape
    V, weight_h = weight.shape
    if weight_h != H:
        raise ValueError(f"weight.shape[1] must match _input.shape[1]; got {weight_h} != {H}")
    if target.shape[0] != BT:
        raise ValueError(f"target length must match _input rows; got {target.shape[0]} != {BT}")
    if bias is not None and bias.shape != (V,):
        raise ValueError(f"bias must have shape ({V},); got {tuple(bias.shape)}")
    L.require_gpu(_input, weight, target)
    if weight.dtype != _input.dtype or (bias is not None and bias.dtype != _input.dtype):
        raise TypeError(f"_input, weight and bias must share a dtype; got {_input.dtype}, {weight.dtype}"
                        + (f", {bias.dtype}" if bias is not None else ""))
    if _input.dtype not in (torch.float32, torch.bfloat16, torch.float16):
        raise TypeError(f"unsupported dtype {_input.dtype}")

    dev = _input.device
    dtype = _input.dtype
    input_requires_grad = _input.requires_grad

    if target.dtype != torch.int64:
        target = target.to(torch.int64)
    target = target.contiguous()
    n_non_ignore = 0
    stats = None
    if BT > 0:
        stats, stats_host, stats_ev = _target_stats_async(target, ignore_index, V)
        n_non_ignore = _check_targets(stats_host, stats_ev, V)

    sum_non_ignore_weight = n_non_ignore
    weight_sum = 0.0
    if ce_weight is not None:
        assert ce_weight.shape[0] == V, f"If given, ce_weight has to be a Tensor of size V. Got: {ce_weight.shape}"
        assert torch.is_floating_point(ce_weight), (
            f"If given, ce_weight has to be a Tensor of floating point dtype. Got: {ce_weight.dtype}"
        )
        target_mask = target != ignore_index
        sum_non_ignore_weight = torch.gather(ce_weight, dim=0, index=target.masked_select(target_mask)).sum().item()
        weight_sum = ce_weight.sum().item()
        ce_weight = ce_weight.to(torch.float32).contiguous()

    x = _input.detach()
    if x.stride(-1) != 1 or (BT > 1 and x.stride(0) % 8 != 0) or x.data_ptr() % 16 != 0:
        x = x.contiguous()
    w = weight.detach()
    if w.stride(-1) != 1 or (V > 1 and w.stride(0) % 8 != 0) or w.data_ptr() % 16 != 0:
        w = w.contiguous()
    b = bias.detach().contiguous() if bias is not None else None

    fast = _fast_path(x, w)
    v_pad = -(-V // 8) * 8 if fast else V
    chunk = _chunk_rows(BT, v_pad * _input.element_size()) if BT > 0 else 0

    grad_input = (torch.empty_like(_input, memory_format=torch.contiguous_format) if input_requires_grad
                  else torch.zeros_like(_input))
    want_w = input_requires_grad and weight.requires_grad
    want_b = input_requires_grad and bias is not None
    # one bf16 chunk (the common case at 2 GiB of logits): dW is one GEMM
    # with bf16 output (fp32 accumulation inside, one rounding), so no fp32
    # accumulator and no final cast
    dw_direct = (want_w and fast and chunk >= BT and chunk % 8 == 0 and v_pad == V
                 and dtype == torch.bfloat16 and weight.dtype == torch.bfloat16)
    gw_out = torch.empty(V, H, dtype=weight.dtype, device=dev) if dw_direct else None
    gw32 = torch.empty(v_pad, H, dtype=torch.float32, device=dev) if want_w and not dw_direct else None
    gb32 = torch.empty(1, V, dtype=torch.float32, device=dev) if want_b else None

    loss_1d = torch.zeros(BT, dtype=torch.float32, device=dev)
    z_loss_1d = torch.zeros(BT, dtype=torch.float32, device=dev) if return_z_loss else None
    token_accuracy_1d = torch.zeros(BT, dtype=torch.float32, device=dev) if return_token_accuracy else None
    predicted_tokens_1d = (torch.full((BT,), -1, dtype=torch.int64, device=dev) if return_predicted_tokens
                           else None)

    flags = L.CE_HAS_GRADIENTS if input_requires_grad else 0
    if ce_weight is not None:
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
        # one logits buffer for every chunk; pad columns (fast path, V % 8 != 0)
        # stay zero, so the dX GEMM may read K = v_pad
        mk = torch.zeros if v_pad != V else torch.empty
        logits_buf = mk(chunk, v_pad, dtype=dtype, device=dev)
        if fast:
            # W^T with a row pitch padded to 8, cached on the weight itself
            # (kept while the weight is unchanged, e.g. a frozen lm_head)
            wt = frozen_t(weight if w.data_ptr() == weight.data_ptr() else w, 8) if input_requires_grad else None
            if b is not None:  # [X | e0] [W | b e0]^T: the bias as one more K segment
                ones8 = torch.zeros(chunk, 8, dtype=dtype, device=dev)
                ones8[:, 0] = 1
                bias8 = torch.zeros(V, 8, dtype=dtype, device=dev)
                bias8[:, 0] = b
        # dW = dlogits^T X_c reduces over tokens; with both operands
        # transposed (one HBM pass each) it is a K-contiguous product for the
        # 4-wave GEMM instead of a transposing token-major GEMM
        dw_nt = fast and want_w and chunk % 8 == 0
        if dw_nt:
            dlT_buf = torch.empty(v_pad, chunk, dtype=dtype, device=dev)
            xT_buf = torch.empty(H, chunk, dtype=dtype, device=dev)
        ones_row = torch.ones(1, chunk, dtype=dtype, device=dev) if want_b else None
        prob = torch.empty(chunk, dtype=torch.float32, device=dev) if use_token_scaling else None
        st = L.stream_of(x)

        for c0 in range(0, BT, chunk):
            n = min(chunk, BT - c0)
            x_c = x[c0:c0 + n]
            t_c = target[c0:c0 + n]
            logits = logits_buf[:n]

            if fast:
                segs = [(x_c, ld(x_c), w, ld(w), H)]
                if b is not None:
                    segs.append((ones8[:n], 8, bias8, 8, 8))
                gemm(n, V, segs, ROW, COL, out=logits[:, :V])
            else:
                _generic(n, V, H, dtype, x_c, x_c.stride(0), 1, w, 1, w.stride(0), logits, v_pad, dtype, bias=b)

            if use_token_scaling:
                L.check(L.forge_ce_target_prob(L.dtype_code(dtype), logits.data_ptr(), v_pad, n, V, t_c.data_ptr(), 1,
                                               int(ignore_index), float(softcap or 0.0), prob.data_ptr(), st),
                        "forge_ce_target_prob")

            L.check(
                L.forge_ce_fwd(
                    L.dtype_code(dtype), logits.data_ptr(), v_pad, n, V, t_c.data_ptr(), 1, L.ptr(ce_weight),
                    loss_1d[c0:].data_ptr(), L.ptr(z_loss_1d[c0:] if return_z_loss else None),
                    L.ptr(token_accuracy_1d[c0:] if return_token_accuracy else None),
                    L.ptr(predicted_tokens_1d[c0:] if return_predicted_tokens else None),
                    int(ignore_index), float(n_non_ignore), float(sum_non_ignore_weight), float(weight_sum),
                    float(lse_square_scale), float(label_smoothing), float(softcap or 0.0), flags,
                    stats.data_ptr(), st,
                ),
                "forge_ce_fwd",
            )

            if use_token_scaling:
                L.check(L.forge_row_scale(L.DTYPE_F32, loss_1d[c0:].data_ptr(), 1, n, 1, prob.data_ptr(), st),
                        "forge_row_scale")
                if return_z_loss:
                    L.check(L.forge_row_scale(L.DTYPE_F32, z_loss_1d[c0:].data_ptr(), 1, n, 1, prob.data_ptr(), st),
                            "forge_row_scale")
                if input_requires_grad:
                    L.check(L.forge_row_scale(L.dtype_code(dtype), logits.data_ptr(), v_pad, n, V, prob.data_ptr(),
                                              st), "forge_row_scale")

            if not input_requires_grad:
                continue
            beta = 0.0 if c0 == 0 else 1.0
            gi = grad_input[c0:c0 + n]
            if fast:
                gemm(n, H, [(logits, v_pad, wt, v_pad, v_pad)], ROW, COL, out=gi)
                if dw_nt and n % 8 == 0:
                    L.check(L.forge_transpose_2b(logits.data_ptr(), v_pad, n, v_pad, dlT_buf.data_ptr(), chunk, st),
                            "forge_transpose_2b")
                    L.check(L.forge_transpose_2b(x_c.data_ptr(), ld(x_c), n, H, xT_buf.data_ptr(), chunk, st),
                            "forge_transpose_2b")
                    if dw_direct:
                        gemm(V, H, [(dlT_buf, chunk, xT_buf, chunk, n)], ROW, COL, out=gw_out)
                    else:
                        gemm(v_pad, H, [(dlT_buf, chunk, xT_buf, chunk, n)], ROW, COL, out=gw32, beta=beta,
                             out_dtype=torch.float32)
                elif want_w:
                    gemm(v_pad, H, [(logits, v_pad, x_c, ld(x_c), n)], COL, ROW, out=gw32, beta=beta,
                         out_dtype=torch.float32)
            else:
                _generic(n, H, V, dtype, logits, v_pad, 1, w, w.stride(0), 1, gi, gi.stride(0), dtype)
                if want_w:
                    _generic(V, H, n, dtype, logits, 1, v_pad, x_c, x_c.stride(0), 1, gw32, H, torch.float32,
                             beta=beta)
            if want_b:  # db = 1^T dlogits
                _generic(1, V, n, dtype, ones_row, 0, 1, logits, v_pad, 1, gb32, V, torch.float32, beta=beta)

    if reduction == "none":
        loss = loss_1d
        z_loss = z_loss_1d.to(dtype) if return_z_loss else None
        token_accuracy = token_accuracy_1d if return_token_accuracy else None
    else:
        loss = _sum_f32(loss_1d)
        z_loss = _sum_f32(z_loss_1d, dtype) if return_z_loss else None
        token_accuracy = torch.sum(token_accuracy_1d) / n_non_ignore if return_token_accuracy else None
    predicted_tokens = predicted_tokens_1d if return_predicted_tokens else None

    grad_weight = gw_out if dw_direct else (
        _cast_into(gw32, torch.empty(V, H, dtype=weight.dtype, device=dev)) if want_w else None)
    grad_bias = _cast_into(gb32, torch.empty(1, V, dtype=bias.dtype, device=dev)).view(V) if want_b else None
    return loss, z_loss, token_accuracy, predicted_tokens, grad_input, grad_weight, grad_bias


def fused_linear_cross_entropy_backward(
    grad_output: torch.Tensor,
    grad_input: Optional[torch.Tensor],
    grad_weight: Optional[torch.Tensor],
    grad_bias: Optional[torch.Tensor],
):
    """fused_linear_cross_entropy.py:248-280: the forward's gradients times a
    scalar grad_output (a no-op on the device when it is 1)."""
    if grad_output.ndim > 0:
        raise NotImplementedError("Forge fused linear CE backward supports scalar losses only; use mean/sum reduction.")
    g = grad_output.detach()
    if g.dtype not in (torch.float32, torch.bfloat16, torch.float16):
        g = g.to(torch.float32)
    g = g.reshape(1).contiguous()
    for t in (grad_input, grad_weight, grad_bias):
        if t is None or t.numel() == 0:
            continue
        t2 = t.view(1, -1) if t.dim() == 1 else t
        L.check(L.forge_ce_scale(L.dtype_code(t2.dtype), t2.data_ptr(), t2.stride(0), t2.shape[0], t2.shape[1],
                                 g.data_ptr(), L.dtype_code(g.dtype), L.stream_of(t2)),
                "forge_ce_scale")
    return grad_input, grad_weight, grad_bias


class ForgeFusedLinearCrossEntropyFunction(torch.autograd.Function):
    """fused_linear_cross_entropy.py:283-371."""

    @staticmethod
    def forward(
        ctx,
        _input: torch.Tensor,
        weight: torch.Tensor,
        target: torch.Tensor,
        bias: Optional[torch.Tensor] = None,
        ce_weight: Optional[torch.Tensor] = None,
        ignore_index: int = -100,
        lse_square_scale: float = 0.0,
        label_smoothing: float = 0.0,
        reduction: str = "mean",
        softcap: Optional[float] = None,
        return_z_loss: bool = False,
        accum_dtype: Optional[torch.dtype] = None,
        use_token_scaling: bool = False,
        return_token_accuracy: bool = False,
        return_predicted_tokens: bool = False,
    ):
        loss, z_loss, token_accuracy, predicted_tokens, grad_input, grad_weight, grad_bias = (
            fused_linear_cross_entropy_forward(
                _input=_input,
                weight=weight,
                target=target,
                ce_weight=ce_weight,
                bias=bias,
                ignore_index=ignore_index,
                lse_square_scale=lse_square_scale,
                label_smoothing=label_smoothing,
                reduction=reduction,
                softcap=softcap,
                return_z_loss=return_z_loss,
                accum_dtype=accum_dtype,
                use_token_scaling=use_token_scaling,
                return_token_accuracy=return_token_accuracy,
                return_predicted_tokens=return_predicted_tokens,
            )
        )
        saved = []
        ctx.has_grad_input = grad_input is not None
        ctx.has_grad_weight = grad_weight is not None
        ctx.has_grad_bias = grad_bias is not None
        if ctx.has_grad_input:
            saved.append(grad_input.detach())
        if ctx.has_grad_weight:
            saved.append(grad_weight.detach())
        if ctx.has_grad_bias:
            saved.append(grad_bias.detach())
        ctx.save_for_backward(*saved)
        ctx.return_z_loss = return_z_loss
        ctx.return_token_accuracy = return_token_accuracy
        ctx.return_predicted_tokens = return_predicted_tokens
        return loss, z_loss, token_accuracy, predicted_tokens

    @staticmethod
    def backward(ctx, grad_output, grad_output2, grad_output3, grad_output4):
        saved = iter(ctx.saved_tensors)
        grad_input = next(saved) if ctx.has_grad_input else None
        grad_weight = next(saved) if ctx.has_grad_weight else None
        grad_bias = next(saved) if ctx.has_grad_bias else None
        grad_input, grad_weight, grad_bias = fused_linear_cross_entropy_backward(
            grad_output, grad_input, grad_weight, grad_bias
        )
        return (grad_input, grad_weight, None, grad_bias) + (None,) * 11


def forge_fused_linear_cross_entropy(
    _input: torch.Tensor,
    weight: torch.Tensor,
    target: torch.Tensor,
    bias: Optional[torch.Tensor] = None,
    ce_weight: Optional[torch.Tensor] = None,
    ignore_index: int = -100,
    lse_square_scale: float = 0.0,
    label_smoothing: float = 0.0,
    reduction: str = "mean",
    softcap: Optional[float] = None,
    return_z_loss: bool = False,
    accum_dtype: Optional[torch.dtype] = None,
    use_token_scaling: bool = False,
    return_token_accuracy: bool = False,
    return_predicted_tokens: bool = False,
):
    """fused_linear_cross_entropy.py:374-419: a bare loss unless an extra
    output is requested, then a CrossEntropyOutput."""
    loss, z_loss, token_accuracy, predicted_tokens = ForgeFusedLinearCrossEntropyFunction.apply(
        _input, weight, target, bias, ce_weight, ignore_index, lse_square_scale, label_smoothing, reduction,
        softcap, return_z_loss, accum_dtype, use_token_scaling, return_token_accuracy, return_predicted_tokens,
    )
    if not return_z_loss and not return_token_accuracy and not return_predicted_tokens:
        return loss
    return CrossEntropyOutput(loss=loss, z_loss=z_loss, token_accuracy=token_accuracy,
                              predicted_tokens=predicted_tokens)


class ForgeFusedLinearCrossEntropyLoss(torch.nn.Module):
    """fused_linear_cross_entropy.py:422-472 (Liger's call order:
    loss(weight, input, target, bias))."""

    def __init__(
        self,
        ce_weight: Optional[torch.FloatTensor] = None,
        ignore_index: int = -100,
        lse_square_scale: float = 0.0,
        label_smoothing: float = 0.0,
        reduction: str = "mean",
        softcap: Optional[float] = None,
        return_z_loss: bool = False,
        accum_dtype: Optional[torch.dtype] = None,
        use_token_scaling: bool = False,
        return_token_accuracy: bool = False,
        return_predicted_tokens: bool = False,
    ):
        super().__init__()
        assert (label_smoothing >= 0) and (label_smoothing <= 1), (
            f"label_smoothing must be between 0.0 and 1.0. Got: {label_smoothing}"
        )
        assert reduction in {"mean", "sum", "none"}, (
            f"Forge fused linear CE supports reduction='mean', 'sum', or 'none'. Got: {reduction}"
        )
        assert softcap is None or softcap > 0, f"softcap must greater than 0.0 or None. Got: {softcap}"
        self.ce_weight = ce_weight
        self.ignore_index = ignore_index
        self.lse_square_scale = lse_square_scale
        self.label_smoothing = label_smoothing
        self.reduction = reduction
        self.softcap = softcap
        self.return_z_loss = return_z_loss
        self.accum_dtype = accum_dtype
        self.use_token_scaling = use_token_scaling
        self.return_token_accuracy = return_token_accuracy
        self.return_predicted_tokens = return_predicted_tokens

    def forward(self, weight: torch.Tensor, _input: torch.Tensor, target: torch.Tensor,
                bias: Optional[torch.Tensor] = None):
        return forge_fused_linear_cross_entropy(
            _input, weight, target, bias=bias, ce_weight=self.ce_weight, ignore_index=self.ignore_index,
            lse_square_scale=self.lse_square_scale, label_smoothing=self.label_smoothing, reduction=self.reduction,
            softcap=self.softcap, return_z_loss=self.return_z_loss, accum_dtype=self.accum_dtype,
            use_token_scaling=self.use_token_scaling, return_token_accuracy=self.return_token_accuracy,
            return_predicted_tokens=self.return_predicted_tokens,
        )
