"""LoRA-MLP v3 API on MI355X.

Drop-in for kernels/lora_mlp/experiments/v3/lora_mlp_kernel_v3.py of
Forge-researchlab/kernel-POCs: `LoRAMLPv3` (13 forward arguments, same saved
tensors and 13-tuple backward), `lora_mlp_v3` and `fused_lora_swiglu`.
Same fused MFMA pipeline as v6 (kernels/lora_mlp/_impl.py).
"""
from __future__ import annotations

import torch

from kernels.lora_mlp._impl import fused_lora_swiglu, run_backward, run_forward  # noqa: F401


def lora_mlp_v3(X, W_gate, A_gate, B_gate, s_gate, W_up, A_up, B_up, s_up, W_down, A_down, B_down, s_down):
    """v3 :242-254 (no autograd)."""
    params = (W_gate, A_gate, B_gate, s_gate, W_up, A_up, B_up, s_up, W_down, A_down, B_down, s_down)
    return run_forward(X, params, save_eg=False)[0]


class LoRAMLPv3(torch.autograd.Function):
    """v3 :257-358."""

    @staticmethod
    def forward(ctx, X, W_gate, A_gate, B_gate, s_gate, W_up, A_up, B_up, s_up, W_down, A_down, B_down, s_down):
        params = (W_gate, A_gate, B_gate, s_gate, W_up, A_up, B_up, s_up, W_down, A_down, B_down, s_down)
        aux = {}  # LoRA-A products reused by the backward (kept on ctx, outside saved_tensors)
        out, e, g = run_forward(X, params, save_eg=True, aux=aux)
        ctx.lora_aux = aux
        ctx.save_for_backward(A_gate, B_gate, A_up, B_up, A_down, B_down, X, e, g)
        ctx.scales = (s_gate, s_up, s_down)
        ctx.base_weights = (W_gate, W_up, W_down)
        return out

    @staticmethod
    def backward(ctx, dY):
        A_gate, B_gate, A_up, B_up, A_down, B_down, X, e, g = ctx.saved_tensors
        s_gate, s_up, s_down = ctx.scales
        W_gate, W_up, W_down = ctx.base_weights
        batch, seq_len, hd = X.shape
        params = (W_gate, A_gate, B_gate, s_gate, W_up, A_up, B_up, s_up, W_down, A_down, B_down, s_down)
        dX, dAg, dBg, dAu, dBu, dAd, dBd = run_backward(dY, X, e, g, params, aux=ctx.lora_aux)
        return (
            dX.view(batch, seq_len, hd),
            None, dAg, dBg, None,
            None, dAu, dBu, None,
            None, dAd, dBd, None,
        )


__all__ = ["LoRAMLPv3", "lora_mlp_v3", "fused_lora_swiglu"]
