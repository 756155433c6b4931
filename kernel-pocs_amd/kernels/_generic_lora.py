"""LoRA-MLP and LoRA-QKV for fp32 / fp16 inputs on the generic GEMM.

The fused paths (kernels/lora_mlp/_impl.py, kernels/lora_qkv/_impl.py) run
on the bf16 MFMA core.  The reference's entry points also take fp32 (and
fp16) tensors - its tests call lora_mlp_v3 / lora_mlp_v6 / lora_qkv_v2_3 in
fp32 (kernels/lora_mlp/tests/test_lora_mlp.py:507-549, :1348-1456;
kernels/lora_qkv/tests/test_v2_2_v2_3_v3.py) - where its big GEMMs are plain
cuBLAS fp32 products.  This module is that path here: every product is
forge_gemm_generic (fp32 accumulation, one rounding to the storage type, any
strides, so transposed operands are read in place), the activation is the
SwiGLU / GeGLU kernel and RoPE the RoPE kernel, all in the input's dtype.
The math is the reference's PyTorch formulation
(kernels/lora_mlp/reference/lora_mlp_pytorch.py:100-225,
kernels/lora_qkv/reference/lora_qkv_pytorch.py:34-214):
  proj(X) = X W^T + s (X A^T) B^T
  MLP backward: DW = dY Wd + s_d (dY B_d) A_d; (dgate, dup) from the
  activation's backward; LoRA gradients s (dZ B)^T X and s dZ^T (X A^T).
"""
from __future__ import annotations

from typing import Optional

import torch

from forge_hip import _lib as L

GENERIC_DTYPES = (torch.float32, torch.float16)


def check_dtypes(what: str, *ts) -> torch.dtype:
    """The one dtype of the given tensors (None entries skipped)."""
    dts = {t.dtype for t in ts if t is not None}
    if len(dts) != 1:
        raise TypeError(f"{what}: tensors must share one dtype, got {sorted(str(d) for d in dts)}")
    return dts.pop()


def gmm(a: torch.Tensor, b: torch.Tensor, out: Optional[torch.Tensor] = None, alpha: float = 1.0,
        beta: float = 0.0) -> torch.Tensor:
    """alpha * a @ b (+ beta * out): a [M, K], b [K, N] of one dtype with any
    strides (transposed views are read in place), out [M, N] row-major."""
    M, K = a.shape
    N = b.shape[1]
    if out is None:
        out = torch.empty(M, N, dtype=a.dtype, device=a.device)
    if M == 0 or N == 0:
        return out
    if K == 0:
        if beta == 0.0:
            out.zero_()
        else:
            out.mul_(beta)
        return out
    assert out.stride(1) == 1 or N == 1
    L.check(L.forge_gemm_generic(M, N, K, L.dtype_code(a.dtype), a.data_ptr(), a.stride(0), a.stride(1),
                                 b.data_ptr(), b.stride(0), b.stride(1), out.data_ptr(), out.stride(0),
                                 L.dtype_code(out.dtype), float(alpha), float(beta), None, L.GEMM_ACT_NONE,
                                 L.stream_of(out)),
            "forge_gemm_generic")
    return out


def _proj(X, W, A, B, s, out=None):
    """X W^T + s (X A^T) B^T -> (out, xa = X A^T or None)."""
    out = gmm(X, W.t(), out=out)
    xa = None
    if A is not None and B is not None:
        xa = gmm(X, A.t())
        gmm(xa, B.t(), out=out, alpha=s, beta=1.0)
    return out, xa


def _act_fwd(e, g, activation):
    M, n = e.shape
    h = torch.empty_like(e)
    if activation == "silu":
        L.check(L.forge_swiglu_fwd(L.dtype_code(e.dtype), e.data_ptr(), g.data_ptr(), n, h.data_ptr(), n, M, n,
                                   1.0, 1.0, L.stream_of(e)), "forge_swiglu_fwd")
    else:
        L.check(L.forge_geglu_fwd(L.dtype_code(e.dtype), e.data_ptr(), g.data_ptr(), n, h.data_ptr(), n, M, n,
                                  int(activation == "gelu_tanh"), L.stream_of(e)), "forge_geglu_fwd")
    return h


def _act_bwd(DW, e, g, activation):
    """(dup, dgate) of the gated activation at (e, g) for dout = DW."""
    M, n = e.shape
    dgate, dup = torch.empty_like(e), torch.empty_like(e)
    if activation == "silu":
        L.check(L.forge_swiglu_bwd(L.dtype_code(e.dtype), DW.data_ptr(), n, e.data_ptr(), g.data_ptr(), n,
                                   dgate.data_ptr(), dup.data_ptr(), n, M, n, 1.0, 1.0, L.stream_of(e)),
                "forge_swiglu_bwd")
    else:
        L.check(L.forge_geglu_bwd(L.dtype_code(e.dtype), DW.data_ptr(), n, e.data_ptr(), g.data_ptr(), n,
                                  dgate.data_ptr(), dup.data_ptr(), n, M, n, int(activation == "gelu_tanh"),
                                  L.stream_of(e)), "forge_geglu_bwd")
    return dup, dgate


def _c(t):
    return None if t is None else (t if t.stride(-1) == 1 else t.contiguous())


def mlp_forward(X2, W_gate, A_gate, B_gate, s_gate, W_up, A_up, B_up, s_up, W_down, A_down, B_down, s_down,
                save_eg=True, aux=None, activation="silu"):
    """(out [M, H], e, g) as the fused path returns them; aux receives the
    unscaled LoRA-A products (X Ag^T, X Au^T, h Ad^T) for the backward."""
    check_dtypes("LoRA-MLP", X2, W_gate, A_gate, B_gate, W_up, A_up, B_up, W_down, A_down, B_down)
    L.require_gpu(X2, W_gate, W_up, W_down)
    X2 = _c(X2)
    e, xag = _proj(X2, W_gate, A_gate, B_gate, s_gate)
    g, xau = _proj(X2, W_up, A_up, B_up, s_up)
    h = _act_fwd(e, g, activation)
    out, xd = _proj(h, W_down, A_down, B_down, s_down)
    if aux is not None and xag is not None and xd is not None:
        aux.update(generic=True, xag=xag, xau=xau, xd=xd)
    if not save_eg:
        e = g = None
    return out, e, g


def mlp_backward(dY2, X2, e, g, W_gate, A_gate, B_gate, s_gate, W_up, A_up, B_up, s_up, W_down, A_down, B_down,
                 s_down, aux=None, activation="silu"):
    """(dX, dAg, dBg, dAu, dBu, dAd, dBd): lora_mlp_pytorch.py:153-225 with
    the activation's backward from the SwiGLU / GeGLU kernel."""
    dY2, X2, e, g = _c(dY2), _c(X2), _c(e), _c(g)
    DW = gmm(dY2, W_down)                                   # [M, I]
    td = gmm(dY2, B_down)                                   # dY Bd [M, r]
    gmm(td, A_down, out=DW, alpha=s_down, beta=1.0)
    h = _act_fwd(e, g, activation)
    df, de = _act_bwd(DW, e, g, activation)                 # d up, d gate
    dAd = gmm(td.t(), h, alpha=s_down)                      # [r, I]
    xd = aux["xd"] if aux and aux.get("generic") else gmm(h, A_down.t())
    dBd = gmm(dY2.t(), xd, alpha=s_down)                    # [H, r]
    vu, vg = gmm(df, B_up), gmm(de, B_gate)                 # [M, r]
    dAu, dAg = gmm(vu.t(), X2, alpha=s_up), gmm(vg.t(), X2, alpha=s_gate)
    if aux and aux.get("generic"):
        xau, xag = aux["xau"], aux["xag"]
    else:
        xau, xag = gmm(X2, A_up.t()), gmm(X2, A_gate.t())
    dBu, dBg = gmm(df.t(), xau, alpha=s_up), gmm(de.t(), xag, alpha=s_gate)
    dX = gmm(df, W_up)
    gmm(de, W_gate, out=dX, beta=1.0)
    gmm(vu, A_up, out=dX, alpha=s_up, beta=1.0)
    gmm(vg, A_gate, out=dX, alpha=s_gate, beta=1.0)
    return dX, dAg, dBg, dAu, dBu, dAd, dBd


def qkv_forward(X2, W_q, W_k, W_v, A_q, B_q, s_q, A_k, B_k, s_k, A_v, B_v, s_v, rope=None, aux=None):
    """out [M, Hq + 2 Hkv] (Q | K | V columns) as the fused path returns it;
    rope = {cos, sin, positions, head_dim} (tables in X's dtype) rotates Q and K."""
    check_dtypes("LoRA-QKV", X2, W_q, W_k, W_v, A_q, B_q, A_k, B_k, A_v, B_v)
    L.require_gpu(X2, W_q, W_k, W_v)
    X2 = _c(X2)
    M = X2.shape[0]
    Hq, Hkv = W_q.shape[0], W_k.shape[0]
    out = torch.empty(M, Hq + 2 * Hkv, dtype=X2.dtype, device=X2.device)
    xas = []
    for (W, A, B, s), c0, c1 in zip(((W_q, A_q, B_q, s_q), (W_k, A_k, B_k, s_k), (W_v, A_v, B_v, s_v)),
                                    (0, Hq, Hq + Hkv), (Hq, Hq + Hkv, Hq + 2 * Hkv)):
        xas.append(_proj(X2, W, A, B, s, out=out[:, c0:c1])[1])
    if aux is not None and xas[0] is not None:
        aux.update(generic=True, xa=xas)
    if rope is not None:
        D = rope["head_dim"]
        cos, sin, pos = rope["cos"], rope["sin"], rope.get("positions")
        q, k = out[:, :Hq], out[:, Hq:Hq + Hkv]
        L.check(L.forge_rope(L.dtype_code(out.dtype),
                             q.data_ptr(), 0, D, out.stride(0), k.data_ptr(), 0, D, out.stride(0),
                             q.data_ptr(), 0, D, out.stride(0), k.data_ptr(), 0, D, out.stride(0),
                             cos.data_ptr(), 0, cos.stride(0), sin.data_ptr(), 0, sin.stride(0),
                             L.dtype_code(cos.dtype), cos.shape[0],
                             None if pos is None else pos.data_ptr(), 1, Hq // D, Hkv // D, M, D, 0,
                             L.stream_of(out)), "forge_rope")
    return out


def qkv_backward(dQ, dK, dV, X2, W_q, W_k, W_v, A_q, B_q, s_q, A_k, B_k, s_k, A_v, B_v, s_v, aux=None):
    """(dX, dA_q, dB_q, dA_k, dB_k, dA_v, dB_v): lora_qkv_pytorch.py:170-214."""
    X2 = _c(X2)
    dX = None
    grads = []
    xas = aux["xa"] if aux and aux.get("generic") else [None, None, None]
    for dY, W, A, B, s, xa in ((dQ, W_q, A_q, B_q, s_q, xas[0]), (dK, W_k, A_k, B_k, s_k, xas[1]),
                               (dV, W_v, A_v, B_v, s_v, xas[2])):
        dY = _c(dY)
        dX = gmm(dY, W, out=dX, beta=0.0 if dX is None else 1.0)
        dYB = gmm(dY, B)                                    # [M, r]
        gmm(dYB, A, out=dX, alpha=s, beta=1.0)
        xa = xa if xa is not None else gmm(X2, A.t())
        grads += [gmm(dYB.t(), X2, alpha=s), gmm(dY.t(), xa, alpha=s)]
    return (dX, *grads)
