"""GEMM with a fused activation epilogue on MI355X.

`matmul_epilogue(A, B, epilogue, alpha, beta, C)` computes
D = epilogue(alpha * A @ B + beta * C), A [M, K] and B [K, N] row-major, with
epilogue "none", "relu", "gelu" (tanh approximation) or "swish" / "silu".
It is the MI355X counterpart of the reference's cuBLASLt SWISH-epilogue
GEMM (kernels/lora_mlp/experiments/v4/cublaslt_silu.cu:9-92 and its Python
wrapper cublaslt_wrapper.py:97-261): bf16 operands run on the MFMA GEMM
(`forge_gemm` with FORGE_EPI_SILU / _RELU / _GELU: the activation is applied
to the fp32 accumulator before the single bf16 rounding); fp32 / fp16
operands, or bf16 shapes the MFMA core does not take (K or N not a multiple
of 8), run on `forge_gemm_generic` with the same activation (its GELU is
the tanh form too).
"""
from __future__ import annotations

from typing import Optional

import torch

from forge_hip import _lib as L

_EPI = {"none": L.EPI_STORE, "relu": L.EPI_RELU, "gelu": L.EPI_GELU, "swish": L.EPI_SILU, "silu": L.EPI_SILU}
_GEN_ACT = {"none": L.GEMM_ACT_NONE, "relu": L.GEMM_ACT_RELU, "gelu": L.GEMM_ACT_GELU, "swish": L.GEMM_ACT_SILU,
            "silu": L.GEMM_ACT_SILU}


def matmul_epilogue(A: torch.Tensor, B: torch.Tensor, epilogue: str = "none", alpha: float = 1.0,
                    beta: float = 0.0, C: Optional[torch.Tensor] = None) -> torch.Tensor:
    """D = epilogue(alpha * A @ B + beta * C) -> new [M, N] tensor in A's dtype."""
    assert A.is_cuda and B.is_cuda and A.is_contiguous() and B.is_contiguous()
    assert A.dtype == B.dtype
    assert A.shape[1] == B.shape[0], f"Shape mismatch: A={A.shape}, B={B.shape}"
    if epilogue not in _EPI:
        raise ValueError(f"epilogue must be one of {sorted(_EPI)}, got {epilogue!r}")
    M, K = A.shape
    N = B.shape[1]
    if beta != 0.0:
        assert C is not None and C.shape == (M, N), "beta != 0 needs C of shape [M, N]"
        D = C.to(A.dtype).contiguous().clone()
    else:
        D = torch.empty(M, N, dtype=A.dtype, device=A.device)
    st = L.stream_of(A)
    mfma_ok = (A.dtype == torch.bfloat16 and K % 8 == 0 and N % 8 == 0 and A.data_ptr() % 16 == 0
               and B.data_ptr() % 16 == 0 and D.data_ptr() % 16 == 0)
    if mfma_ok:
        seg = (L.GemmSegment * 1)(L.GemmSegment(A.data_ptr(), K, B.data_ptr(), N, K))
        L.check(L.forge_gemm(M, N, seg, 1, L.LAYOUT_ROW, L.LAYOUT_ROW, D.data_ptr(), N, L.DTYPE_BF16,
                             float(alpha), float(beta), _EPI[epilogue], 1, st), "forge_gemm")
        return D
    L.check(L.forge_gemm_generic(M, N, K, L.dtype_code(A.dtype), A.data_ptr(), K, 1, B.data_ptr(), N, 1,
                                 D.data_ptr(), N, L.dtype_code(D.dtype), float(alpha), float(beta), None,
                                 _GEN_ACT[epilogue], st), "forge_gemm_generic")
    return D


__all__ = ["matmul_epilogue"]
