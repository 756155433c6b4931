"""Fused LoRA-GeGLU MLP (Gemma) on MI355X.

The reference has no fused kernel for GeGLU MLPs: its patch adapter computes
`down_proj(geglu(gate_proj(x), up_proj(x)))` through the PEFT submodules and
the GeGLU kernel (forge/forge/patching/kernels/lora.py:170-188) and names a
fully-fused Gemma path as the follow-on.  `LoRAMLPGeGLU` is that path: the
LoRA-MLP pipeline of kernels/lora_mlp/_impl.py (LoRA-B terms as extra K
segments of the base GEMMs, the activation in the GEMM epilogues) with the
GeGLU epilogues, whose activation math is the GeGLU kernel's
(kernels/geglu/geglu.py:104-148) on the bf16 e, g and round(DW):
    h     = round(gelu(e)) g
    d up  = round(DW) round(gelu(e))
    d gate= round(DW) g gelu'(e)
Arguments follow LoRAMLPv6 (X, then per projection W, A, B, s) plus the
GELU form, `approximate` = "tanh" | "none" as in `geglu`.  float64 inputs
take a plain-PyTorch path (gradcheck).  The saved e / g buffers are
overwritten by the backward (not re-entrant), as in LoRAMLPv6.
"""
from __future__ import annotations

import torch

from kernels.lora_mlp._impl import run_backward, run_forward


def _activation(approximate: str) -> str:
    if approximate == "tanh":
        return "gelu_tanh"
    if approximate == "none":
        return "gelu_exact"
    raise ValueError(f"approximate must be 'tanh' or 'none', got {approximate!r}")


class LoRAMLPGeGLU(torch.autograd.Function):
    """Fused LoRA MLP with the GeGLU activation; gradients for X and the six
    LoRA factors (the base weights are frozen)."""

    @staticmethod
    def forward(ctx, X, W_gate, A_gate, B_gate, s_gate, W_up, A_up, B_up, s_up, W_down, A_down, B_down, s_down,
                approximate: str = "tanh"):
        act = _activation(approximate)
        params = (W_gate, A_gate, B_gate, s_gate, W_up, A_up, B_up, s_up, W_down, A_down, B_down, s_down)
        aux = {}
        out, e, g = run_forward(X, params, save_eg=True, aux=aux, activation=act)
        ctx.lora_aux = aux
        ctx.activation = act
        ctx.save_for_backward(A_gate, B_gate, A_up, B_up, A_down, B_down, X, e, g)
        ctx.scales = (s_gate, s_up, s_down)
        ctx.base_weights = (W_gate, W_up, W_down)
        return out

    @staticmethod
    def backward(ctx, dY):
        A_gate, B_gate, A_up, B_up, A_down, B_down, X, e, g = ctx.saved_tensors
        s_gate, s_up, s_down = ctx.scales
        W_gate, W_up, W_down = ctx.base_weights
        params = (W_gate, A_gate, B_gate, s_gate, W_up, A_up, B_up, s_up, W_down, A_down, B_down, s_down)
        dX, dAg, dBg, dAu, dBu, dAd, dBd = run_backward(dY, X, e, g, params, aux=ctx.lora_aux,
                                                        activation=ctx.activation)
        return (
            dX.view(X.shape),
            None, dAg, dBg, None,
            None, dAu, dBu, None,
            None, dAd, dBd, None,
            None,
        )


def lora_mlp_geglu(X, W_gate, A_gate, B_gate, s_gate, W_up, A_up, B_up, s_up, W_down, A_down, B_down, s_down,
                   approximate: str = "tanh"):
    """Forward only (no autograd graph): out with X's leading shape."""
    params = (W_gate, A_gate, B_gate, s_gate, W_up, A_up, B_up, s_up, W_down, A_down, B_down, s_down)
    return run_forward(X, params, save_eg=False, activation=_activation(approximate))[0]
