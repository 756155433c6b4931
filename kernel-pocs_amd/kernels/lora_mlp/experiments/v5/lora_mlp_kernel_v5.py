"""LoRA-MLP inference on merged weights (v5 API) on MI355X.

Drop-in for the inference part of
kernels/lora_mlp/experiments/v5/lora_mlp_kernel_v5.py of
Forge-researchlab/kernel-POCs: `merge_lora_weights` (W + s B A),
`prepare_inference_weights` (merged and transposed: gate/up [H, I], down
[I, H]) and `lora_mlp_v5_inference(X, W_gate_eff_T, W_up_eff_T,
W_down_eff_T)`.  The reference runs a cuBLASLt SWISH-epilogue GEMM, a plain
GEMM and a product, or two GEMMs and a SwiGLU kernel (:425-460).  Here a bf16
call is two MFMA GEMMs: the gate/up dual-B GEMM with the SwiGLU epilogue
writes only h = silu(X Wg^T) (X Wu^T) (`forge_lora_mlp_gate_up` with no
LoRA and no e / g outputs), then out = h Wd^T (`forge_gemm`).  Both read
K-contiguous weights: the transposed merged weights are transposed back once
per weight and cached for the weight's lifetime (they are frozen at
inference).  fp32 / fp16 inputs, or widths that are not multiples of 8, run
e, g and out on the generic GEMM and h on the SwiGLU kernel (the
reference's CUDA 12.4 path: silu(e) rounded to the dtype, times g); float64
inputs run the same formula in PyTorch.
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch

from forge_hip import _lib as L
from kernels._lora_ops import COL, ROW, frozen_t, gemm
from kernels.swiglu.swiglu import swiglu_forward


def merge_lora_weights(W: torch.Tensor, A: Optional[torch.Tensor], B: Optional[torch.Tensor],
                       s: float) -> torch.Tensor:
    """lora_mlp_kernel_v5.py:277-286: W_eff = W + s * (B @ A), [out, in]."""
    if A is None or B is None:
        return W
    return W + s * (B @ A)


def prepare_inference_weights(
    W_gate: torch.Tensor, A_gate: Optional[torch.Tensor], B_gate: Optional[torch.Tensor], s_gate: float,
    W_up: torch.Tensor, A_up: Optional[torch.Tensor], B_up: Optional[torch.Tensor], s_up: float,
    W_down: torch.Tensor, A_down: Optional[torch.Tensor], B_down: Optional[torch.Tensor], s_down: float,
) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """lora_mlp_kernel_v5.py:289-316 -> (W_gate_eff^T [H, I], W_up_eff^T
    [H, I], W_down_eff^T [I, H]), contiguous."""
    W_gate_eff = merge_lora_weights(W_gate, A_gate, B_gate, s_gate)
    W_up_eff = merge_lora_weights(W_up, A_up, B_up, s_up)
    W_down_eff = merge_lora_weights(W_down, A_down, B_down, s_down)
    return W_gate_eff.t().contiguous(), W_up_eff.t().contiguous(), W_down_eff.t().contiguous()


def _generic(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """a [M, K] @ b [K, N] (any strides) on forge_gemm_generic, in a's dtype."""
    M, K = a.shape
    N = b.shape[1]
    out = torch.empty(M, N, dtype=a.dtype, device=a.device)
    L.check(L.forge_gemm_generic(M, N, K, L.dtype_code(a.dtype), a.data_ptr(), a.stride(0), a.stride(1),
                                 b.data_ptr(), b.stride(0), b.stride(1), out.data_ptr(), N, L.dtype_code(a.dtype),
                                 1.0, 0.0, None, L.GEMM_ACT_NONE, L.stream_of(out)), "forge_gemm_generic")
    return out


def _mfma_ok(X2, Wg_T, Wd_T) -> bool:
    H, I = Wg_T.shape
    return (X2.dtype == torch.bfloat16 and Wg_T.dtype == torch.bfloat16 and H % 8 == 0 and I % 8 == 0
            and X2.stride(-1) == 1 and X2.stride(0) % 8 == 0 and X2.data_ptr() % 16 == 0 and Wd_T.shape == (I, H))


def lora_mlp_v5_inference(X: torch.Tensor, W_gate_eff_T: torch.Tensor, W_up_eff_T: torch.Tensor,
                          W_down_eff_T: torch.Tensor) -> torch.Tensor:
    """lora_mlp_kernel_v5.py:425-460: out = (silu(X Wg) * (X Wu)) Wd with the
    merged, transposed weights; same outer shape as X."""
    orig_shape = X.shape
    X2 = X.reshape(-1, X.shape[-1])
    if X.dtype == torch.float64:
        e = X2 @ W_gate_eff_T
        g = X2 @ W_up_eff_T
        out = (e * torch.sigmoid(e) * g) @ W_down_eff_T
    else:
        L.require_gpu(X2, W_gate_eff_T, W_up_eff_T, W_down_eff_T)
        if _mfma_ok(X2, W_gate_eff_T, W_down_eff_T):
            M, H = X2.shape
            I = W_gate_eff_T.shape[1]
            Wg, Wu, Wd = frozen_t(W_gate_eff_T), frozen_t(W_up_eff_T), frozen_t(W_down_eff_T)  # [I, H], [I, H], [H, I]
            h = torch.empty(M, I, dtype=torch.bfloat16, device=X2.device)
            L.check(L.forge_lora_mlp_gate_up(M, H, I, 0, X2.data_ptr(), X2.stride(0), Wg.data_ptr(), Wu.data_ptr(), H,
                                             None, 0, None, None, 0, None, None, h.data_ptr(), I, L.ACT_SILU,
                                             L.stream_of(X2)), "forge_lora_mlp_gate_up")
            out = gemm(M, H, [(h, I, Wd, I, I)], ROW, COL)
        else:
            e = _generic(X2, W_gate_eff_T)
            g = _generic(X2, W_up_eff_T)
            h, _, _ = swiglu_forward(e, g)
            out = _generic(h, W_down_eff_T)
    if len(orig_shape) == 3:
        out = out.view(orig_shape[0], orig_shape[1], -1)
    return out


__all__ = ["merge_lora_weights", "prepare_inference_weights", "lora_mlp_v5_inference"]
