"""Unsloth's LoRA-MLP helpers on the HIP kernels.

The reference imports three helpers from its extracted Unsloth baseline
(kernels/lora_mlp/reference/unsloth_baseline.py) into its v5/v6 backwards
(experiments/v6/lora_mlp_kernel_v6.py:66-69, 632-653) and tests
(kernels/lora_mlp/tests/test_lora_mlp.py:24-29).  Same names, arguments,
in-place behaviour and roundings here:

  matmul_lora(X, W, W_quant, A, B, s, out=None)   unsloth_baseline.py:34-55
      X W^T + s (X A^T) B^T.  bf16: one library GEMM with the rank-r term as
      a K segment ([X | s X A^T] [W | B]^T, fp32 accumulation, one rounding;
      the reference rounds the base product before its addmm).  fp32 / fp16:
      the generic GEMM, the same two products.
  swiglu_fg_kernel(e, g)                          unsloth_baseline.py:72-110
      h = round(silu(e)) g: the SwiGLU kernel's forward (forge_swiglu_fwd),
      whose cast order is Unsloth's (f rounded to e's dtype before the product).
  swiglu_DWf_DW_dfg_kernel(DW, e, g)              unsloth_baseline.py:118-168
      in place: DW <- h = f g, e <- df = DW f, g <- de = round(DW g) se (1 + e (1 - se)),
      f = round(e se): forge_lora_mlp_glu_bwd, the fused down-projection
      epilogue's per-element step run on its own.
Quantized weights (W_quant) are not supported, as in the reference's
extraction (unsloth_baseline.py:23-27).
"""
from __future__ import annotations

import torch

from forge_hip import _lib as L
from kernels import _generic_lora as G
from kernels._lora_ops import COL, ROW, as_operand, gemm, ld, lora_a, pad_rank


def matmul_lora(X, W, W_quant, A, B, s, out=None):
    """X @ W^T (+ s (X @ A^T) @ B^T when A is given); 3-D X keeps its batch
    shape (unsloth_baseline.py:34-55)."""
    if W_quant is not None:
        raise NotImplementedError("Quantized weights not supported in standalone benchmark")
    shape = X.shape
    X2 = X.reshape(-1, shape[-1])
    if X2.dtype in G.GENERIC_DTYPES:
        res = G.gmm(X2, W.t())
        if A is not None:
            G.gmm(G.gmm(X2, A.to(X2.dtype).t()), B.to(X2.dtype).t(), out=res, alpha=float(s), beta=1.0)
    else:
        L.require_gpu(X2, W)
        X2 = as_operand(X2)
        Wc = as_operand(W)
        segs = [(X2, ld(X2), Wc, ld(Wc), X2.shape[1])]
        if A is not None:
            A8, B8 = pad_rank(A.to(X2.dtype), B.to(X2.dtype))
            xa = lora_a(X2, [A8], [float(s)])
            B8 = as_operand(B8)
            segs.append((xa, ld(xa), B8, ld(B8), A8.shape[0]))
        res = gemm(X2.shape[0], Wc.shape[0], segs, ROW, COL)
    if out is not None:
        out.view(-1, res.shape[-1]).copy_(res)
        res = out
    return res.view(*shape[:-1], -1) if len(shape) == 3 else res


def swiglu_fg_kernel(e, g):
    """h = round(e sigmoid(e)) g in e's dtype (unsloth_baseline.py:72-110)."""
    batch, seq_len, hd = e.shape
    L.require_gpu(e, g)
    e2 = e.reshape(-1, hd).contiguous()
    g2 = g.reshape(-1, hd).contiguous()
    h = torch.empty(batch, seq_len, hd, dtype=e.dtype, device=e.device)
    L.check(L.forge_swiglu_fwd(L.dtype_code(e.dtype), e2.data_ptr(), g2.data_ptr(), hd, h.data_ptr(), hd,
                               e2.shape[0], hd, 1.0, 1.0, L.stream_of(e2)), "forge_swiglu_fwd")
    return h


def swiglu_DWf_DW_dfg_kernel(DW, e, g):
    """In place on contiguous bf16 [rows, hd] tensors: DW <- h, e <- df,
    g <- de; returns (DW, e, g) (unsloth_baseline.py:118-168)."""
    rows, hd = e.shape
    L.require_gpu(DW, e, g)
    for t in (DW, e, g):
        if t.dtype != torch.bfloat16 or not t.is_contiguous() or t.shape != e.shape:
            raise ValueError("swiglu_DWf_DW_dfg_kernel: DW, e, g must be contiguous bf16 tensors of one shape")
    L.check(L.forge_lora_mlp_glu_bwd(rows, hd, DW.data_ptr(), hd, e.data_ptr(), g.data_ptr(), hd, DW.data_ptr(), hd,
                                     L.ACT_SILU, L.stream_of(e)), "forge_lora_mlp_glu_bwd")
    return DW, e, g


__all__ = ["matmul_lora", "swiglu_fg_kernel", "swiglu_DWf_DW_dfg_kernel"]
