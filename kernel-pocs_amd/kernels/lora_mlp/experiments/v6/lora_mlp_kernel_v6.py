"""LoRA-MLP v6 API on MI355X.

Drop-in for kernels/lora_mlp/experiments/v6/lora_mlp_kernel_v6.py of
Forge-researchlab/kernel-POCs: `LoRAMLPv6` (same 18 forward arguments, same
`ctx.save_for_backward(A_gate, B_gate, A_up, B_up, A_down, B_down, X, e, g)`,
`ctx.scales`, `ctx.base_weights`, 18-tuple backward), `lora_mlp_v6`,
`LoRAMLPv6Module` (cached stacks, `refresh_packed` / `invalidate_packed`) and
the stacking helpers.  The compute is the fused MFMA pipeline of
kernels/lora_mlp/_impl.py; the optional stacked weights and the side stream
are accepted and not needed (the LoRA-A columns are produced by one
multi-projection GEMM and the LoRA-B terms ride along the base GEMMs), so
results do not depend on them.  float64 inputs take the reference's own
PyTorch path (gradcheck).
"""
from __future__ import annotations

from typing import Optional

import torch
import torch.nn as nn

from kernels.lora_mlp._impl import (  # noqa: F401
    fused_lora_a_stacked,
    fused_lora_swiglu,
    run_backward,
    run_forward,
    stack_down_lora_a,
    stack_gate_lora_a,
    stack_lora_a,
)
from kernels.lora_mlp.experiments.v5.lora_mlp_kernel_v5 import (  # noqa: F401
    lora_mlp_v5_inference,
    merge_lora_weights,
    prepare_inference_weights,
)

# v6 shares v5's merged-weight inference path (reference v6 :158)
lora_mlp_v6_inference = lora_mlp_v5_inference


def fused_lora_swiglu_inplace(e_base, g_base, xa_gate, xa_up, B_gate, B_up, s_gate=1.0, s_up=1.0, save_eg=True):
    """v6 :81-151: e_full/g_full are written over e_base/g_base."""
    return fused_lora_swiglu(e_base, g_base, xa_gate, xa_up, B_gate, B_up, s_gate, s_up, save_eg, inplace=True)


def lora_mlp_v6(X, W_gate, A_gate, B_gate, s_gate, W_up, A_up, B_up, s_up, W_down, A_down, B_down, s_down,
                A_stack=None, W_gate_stack=None, W_down_stack=None, enable_streams=True, side_stream=None):
    """v6 :458-517 (no autograd)."""
    params = (W_gate, A_gate, B_gate, s_gate, W_up, A_up, B_up, s_up, W_down, A_down, B_down, s_down)
    return run_forward(X, params, save_eg=False)[0]


class LoRAMLPv6(torch.autograd.Function):
    """v6 :524-672."""

    @staticmethod
    def forward(ctx, X, W_gate, A_gate, B_gate, s_gate, W_up, A_up, B_up, s_up, W_down, A_down, B_down, s_down,
                A_stack=None, W_gate_stack=None, W_down_stack=None, enable_streams: bool = True,
                side_stream: Optional[torch.cuda.Stream] = None):
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
            None, None, None, None, None,
        )


class LoRAMLPv6Module(nn.Module):
    """v6 :679-784: LoRA MLP module with cached (non-persistent) stacks."""

    def __init__(self, hidden: int, intermediate: int, rank: int, s_gate: float = 1.0, s_up: float = 1.0,
                 s_down: float = 1.0, dtype: torch.dtype = torch.bfloat16, device: str = "cuda",
                 enable_streams: bool = True):
        super().__init__()
        H, I, r = hidden, intermediate, rank

        def W(out_dim, in_dim):
            return torch.randn(out_dim, in_dim, dtype=dtype, device=device) * 0.02

        def A(in_dim):
            return torch.randn(r, in_dim, dtype=dtype, device=device) * 0.02

        def B(out_dim):
            return torch.zeros(out_dim, r, dtype=dtype, device=device)

        self.W_gate = nn.Parameter(W(I, H), requires_grad=False)
        self.W_up = nn.Parameter(W(I, H), requires_grad=False)
        self.W_down = nn.Parameter(W(H, I), requires_grad=False)
        self.A_gate = nn.Parameter(A(H))
        self.B_gate = nn.Parameter(B(I))
        self.A_up = nn.Parameter(A(H))
        self.B_up = nn.Parameter(B(I))
        self.A_down = nn.Parameter(A(I))
        self.B_down = nn.Parameter(B(H))
        self.s_gate, self.s_up, self.s_down = s_gate, s_up, s_down
        self.rank = r
        self.enable_streams = enable_streams
        self.register_buffer("_A_stack_cache", None, persistent=False)
        self.register_buffer("_W_gate_stack_cache", None, persistent=False)
        self.register_buffer("_W_down_stack_cache", None, persistent=False)
        self._cache_valid = False

    def refresh_packed(self) -> None:
        """Marks the cached stacks valid.  The HIP path reads A/W directly,
        so the stacks are built only on request (`build_stacks=True`)."""
        self._cache_valid = True

    def build_stacks(self) -> None:
        with torch.no_grad():
            self._A_stack_cache = stack_lora_a(self.A_gate.data, self.A_up.data)
            self._W_gate_stack_cache = stack_gate_lora_a(self.W_gate.data, self.A_gate.data, self.A_up.data)
            self._W_down_stack_cache = stack_down_lora_a(self.W_down.data, self.A_down.data)
        self._cache_valid = True

    def invalidate_packed(self) -> None:
        self._cache_valid = False
        self._A_stack_cache = None
        self._W_gate_stack_cache = None
        self._W_down_stack_cache = None

    def forward(self, X: torch.Tensor) -> torch.Tensor:
        if not self._cache_valid:
            self.refresh_packed()
        return LoRAMLPv6.apply(
            X, self.W_gate, self.A_gate, self.B_gate, self.s_gate, self.W_up, self.A_up, self.B_up, self.s_up,
            self.W_down, self.A_down, self.B_down, self.s_down, self._A_stack_cache, self._W_gate_stack_cache,
            self._W_down_stack_cache, self.enable_streams, None,
        )


__all__ = [
    "LoRAMLPv6", "LoRAMLPv6Module", "lora_mlp_v6", "stack_lora_a", "stack_gate_lora_a", "stack_down_lora_a",
    "fused_lora_a_stacked", "fused_lora_swiglu_inplace", "lora_mlp_v6_inference", "prepare_inference_weights",
]
