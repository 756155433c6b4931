"""LoRA-QKV v3 API on MI355X.

Drop-in for kernels/lora_qkv/experiments/v3/lora_qkv_kernel_v3.py of
Forge-researchlab/kernel-POCs: `LoRAQKVFunction` (14 forward arguments,
saves (X, W_q, W_k, W_v, A_q, B_q, A_k, B_k, A_v, B_v), ctx.scalings,
14-tuple backward) and `lora_qkv_v3`.  Same HIP forward/backward as v4.
"""
from __future__ import annotations

import torch

from kernels.lora_qkv._impl import qkv_backward, qkv_forward, split_views, torch_qkv_backward, torch_qkv_forward


class LoRAQKVFunction(torch.autograd.Function):
    """v3 :54-167."""

    @staticmethod
    def forward(ctx, X, W_q, W_k, W_v, A_q, B_q, s_q, A_k, B_k, s_k, A_v, B_v, s_v, W_all=None):
        orig_shape = X.shape
        X2 = X.reshape(-1, X.shape[-1])
        ctx.use_hip = X.dtype != torch.float64
        ctx.lora_aux = {}  # forward products reused by the backward (outside saved_tensors)
        if ctx.use_hip:
            out = qkv_forward(X2, W_q, W_k, W_v, A_q, B_q, s_q, A_k, B_k, s_k, A_v, B_v, s_v, aux=ctx.lora_aux)
            Q, K, V = split_views(out, W_q.shape[0], W_k.shape[0], orig_shape)
        else:
            Q, K, V = torch_qkv_forward(X2, W_q, W_k, W_v, A_q, B_q, s_q, A_k, B_k, s_k, A_v, B_v, s_v)
            if len(orig_shape) == 3:
                Q, K, V = (t.view(orig_shape[0], orig_shape[1], -1) for t in (Q, K, V))
        ctx.save_for_backward(X, W_q, W_k, W_v, A_q, B_q, A_k, B_k, A_v, B_v)
        ctx.scalings = (s_q, s_k, s_v)
        return Q, K, V

    @staticmethod
    def backward(ctx, dQ, dK, dV):
        X, W_q, W_k, W_v, A_q, B_q, A_k, B_k, A_v, B_v = ctx.saved_tensors
        s_q, s_k, s_v = ctx.scalings
        f = lambda t: t.reshape(-1, t.shape[-1])  # noqa: E731
        args = (f(dQ), f(dK), f(dV), f(X), W_q, W_k, W_v, A_q, B_q, s_q, A_k, B_k, s_k, A_v, B_v, s_v)
        if ctx.use_hip:
            dX, dAq, dBq, dAk, dBk, dAv, dBv = qkv_backward(*args, aux=ctx.lora_aux)
        else:
            dX, dAq, dBq, dAk, dBk, dAv, dBv = torch_qkv_backward(*args)
        if X.dim() == 3:
            dX = dX.reshape(X.shape)
        return (dX, None, None, None, dAq, dBq, None, dAk, dBk, None, dAv, dBv, None, None)


def lora_qkv_v3(X, W_q, A_q, B_q, s_q, W_k, A_k, B_k, s_k, W_v, A_v, B_v, s_v, W_all=None):
    """v3 :174-205."""
    return LoRAQKVFunction.apply(X, W_q, W_k, W_v, A_q, B_q, s_q, A_k, B_k, s_k, A_v, B_v, s_v, W_all)


__all__ = ["LoRAQKVFunction", "lora_qkv_v3"]
