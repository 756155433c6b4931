"""`F.linear` on the library's GEMMs, with autograd: y = x W^T + b.

bf16 with in/out features that are multiples of 8: the MFMA GEMMs
(csrc/gemm.hip; forward on the LDS-DMA engine with the bias as one more K
segment, backward dX = dY W and dW = dY^T X on the register-path engine).
Every other shape or dtype: forge_gemm_generic (fp32 accumulation, exact to
fp32 rounding).  db = colsum(dY) is a generic GEMM with a ones row.  Used by
the composite entry points (`geglu_mlp`) that the reference builds from
`F.linear`.
"""
from __future__ import annotations

from typing import Optional

import torch

from forge_hip import _lib as L
from kernels._lora_ops import COL, ROW, gemm, ld


def _mfma_ok(*ts: torch.Tensor) -> bool:
    return all(t.dtype == torch.bfloat16 and t.stride(-1) == 1 and t.data_ptr() % 16 == 0
               and (t.dim() < 2 or t.shape[0] <= 1 or t.stride(0) % 8 == 0) for t in ts)


def _generic(M, N, K, a, a_sm, a_sk, b, b_sk, b_sn, c, ldc, bias=None):
    L.check(L.forge_gemm_generic(M, N, K, L.dtype_code(a.dtype), a.data_ptr(), a_sm, a_sk, b.data_ptr(), b_sk,
                                 b_sn, c.data_ptr(), ldc, L.dtype_code(c.dtype), 1.0, 0.0, L.ptr(bias),
                                 L.GEMM_ACT_NONE, L.stream_of(c)), "forge_gemm_generic")


def linear_forward(x2: torch.Tensor, w: torch.Tensor, b: Optional[torch.Tensor]) -> torch.Tensor:
    M, K = x2.shape
    N = w.shape[0]
    out = torch.empty(M, N, dtype=x2.dtype, device=x2.device)
    if M == 0 or N == 0:
        return out
    if K % 8 == 0 and _mfma_ok(x2, w) and (b is None or b.dtype == torch.bfloat16):
        segs = [(x2, ld(x2), w, ld(w), K)]
        if b is not None:  # [x | e0] [W | b e0]^T
            ones8 = torch.zeros(M, 8, dtype=x2.dtype, device=x2.device)
            ones8[:, 0] = 1
            b8 = torch.zeros(N, 8, dtype=x2.dtype, device=x2.device)
            b8[:, 0] = b
            segs.append((ones8, 8, b8, 8, 8))
        return gemm(M, N, segs, ROW, COL, out=out)
    _generic(M, N, K, x2, x2.stride(0), 1, w, 1, w.stride(0), out, N, bias=b)
    return out


class ForgeLinearFunction(torch.autograd.Function):
    """y = x W^T + b for x [..., in], W [out, in], b [out] (optional)."""

    @staticmethod
    def forward(ctx, x, weight, bias=None):
        L.require_gpu(x, weight)
        x2 = x.reshape(-1, x.shape[-1])
        if x2.stride(-1) != 1 or (x2.shape[0] > 1 and x2.stride(0) % 8 != 0) or x2.data_ptr() % 16 != 0:
            x2 = x2.contiguous()
        w = weight if weight.stride(-1) == 1 else weight.contiguous()
        b = bias.contiguous() if bias is not None else None
        out = linear_forward(x2, w, b)
        ctx.save_for_backward(x2, w)
        ctx.has_bias = bias is not None
        ctx.x_shape = x.shape
        return out.view(*x.shape[:-1], w.shape[0])

    @staticmethod
    def backward(ctx, dy):
        x2, w = ctx.saved_tensors
        M, K = x2.shape
        N = w.shape[0]
        dy2 = dy.reshape(-1, N).contiguous()
        dx = dw = db = None
        mfma = _mfma_ok(x2, w, dy2) and K % 8 == 0 and N % 8 == 0
        if ctx.needs_input_grad[0]:
            dx = torch.empty(M, K, dtype=x2.dtype, device=x2.device)
            if mfma:  # dY [M][N] @ W [N][K]
                gemm(M, K, [(dy2, ld(dy2), w, ld(w), N)], ROW, ROW, out=dx)
            else:
                _generic(M, K, N, dy2, dy2.stride(0), 1, w, w.stride(0), 1, dx, K)
            dx = dx.view(ctx.x_shape)
        if ctx.needs_input_grad[1]:
            dw = torch.empty(N, K, dtype=w.dtype, device=w.device)
            if mfma:  # dY^T [N][M] @ X [M][K]
                gemm(N, K, [(dy2, ld(dy2), x2, ld(x2), M)], COL, ROW, out=dw)
            else:
                _generic(N, K, M, dy2, 1, dy2.stride(0), x2, x2.stride(0), 1, dw, K)
        if ctx.has_bias and ctx.needs_input_grad[2]:
            db = torch.empty(1, N, dtype=dy2.dtype, device=dy2.device)
            ones = torch.ones(1, M, dtype=dy2.dtype, device=dy2.device)
            _generic(1, N, M, ones, 0, 1, dy2, dy2.stride(0), 1, db, N)
            db = db.view(N)
        return dx, dw, db


def linear(x: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor] = None) -> torch.Tensor:
    return ForgeLinearFunction.apply(x, weight, bias)
