"""LoRA-QKV (GQA-asymmetric widths) on MI355X, optionally fused with RoPE.

Forward (reference `lora_qkv_v2_3`,
kernels/lora_qkv/experiments/v2/lora_qkv_kernel_v2_3.py:177-267):
  1. xa = [sq X Aq^T | sk X Ak^T | sv X Av^T]            forge_lora_a [M, 3r]
  2. out = [Q | K | V] = X [Wq; Wk; Wv]^T + LoRA-B terms: one MFMA GEMM whose
     per-projection K segments carry xa_p B_p^T (one rounding) and whose
     epilogue rotates the Q and K heads in registers   forge_lora_qkv_rope
     (tables or head widths the epilogue cannot take: Q/K stored unrotated,
     then a forge_rope pass over them)
  Q, K, V are returned as column views of `out` (row pitch Hq + 2 Hkv), the
  reference's "strided views of one packed buffer" contract.
Backward (reference `LoRAQKVv4Function.backward`,
kernels/lora_qkv/experiments/v4/lora_qkv_kernel_v4.py:221-336):
  t  = [sq dQ Bq | sk dK Bk | sv dV Bv]                   forge_gemm x3 [M, 3r]
  dA = t^T X (rows split per projection)                 split-K forge_gemm
  dB_p = s_p dY_p^T (X A_p^T)                            split-K forge_gemm
  dX = dQ Wq + dK Wk + dV Wv + sum_p t_p A_p             forge_gemm, 6 K segments
     over the cached W^T and the small A^T (the dX epilogue of the reference,
     lora_qkv_kernel_v4.py:79-163, as K segments: no pass re-reads dX)
With fused RoPE the incoming dQ/dK are first rotated back by -theta
(forge_rope backward) — the chain rule through the rotation.
"""
from __future__ import annotations

from typing import Optional

import torch

from forge_hip import _lib as L
from kernels import _generic_lora as G
from kernels._lora_ops import (COL, ROW, as_operand, frozen_t, gemm, grad_at_b, grad_at_b_group, ld, lora_a,
                               pad_rank, small_t_batch, times_b)


def _w(t):
    return None if t is None else as_operand(t)


# RoPE of the bf16 forward: the QKV GEMM's RoPE epilogue (True, where
# rope_fusable allows) or an in-place forge_rope pass over the stored Q/K
# (False).  Measured cold on MI355X at the BASELINE shape (22954 tokens, Q
# 4096, K/V 1024, same box): GEMM with the RoPE epilogue 994 us, GEMM +
# forge_rope pass 1033 us (the GEMM storing plain Q/K: 952 us).
ROPE_IN_EPILOGUE = True


def qkv_forward(X2, W_q, W_k, W_v, A_q, B_q, s_q, A_k, B_k, s_k, A_v, B_v, s_v,
                rope=None, aux: Optional[dict] = None, a_packed=None, fuse_rope: Optional[bool] = None):
    """Returns out [M, Hq + 2 Hkv] bf16.  rope = {cos, sin, positions, head_dim}
    (tables [P, D]; int64 positions [M], validated by the caller) applies
    RoPE to Q and K: in the GEMM epilogue when fuse_rope (default
    ROPE_IN_EPILOGUE) is set and `rope_fusable` allows it (bf16 tables,
    head_dim 64 / 128, Q and K widths multiples of 256), else by an in-place
    forge_rope pass over the stored Q/K.
    rope may also be a callable that returns that dict (or None): it is
    called once the LoRA-A product is queued, so the host prepares the
    tables while the device already works.
    aux (a dict, optional) receives xa = [sq X Aq^T | sk X Ak^T | sv X Av^T]
    for the backward's B gradients.  fp32 / fp16 inputs run on the generic
    GEMM (kernels/_generic_lora.py; RoPE tables in X's dtype or fp32) and
    return out in X's dtype.  a_packed = [A_q; A_k; A_v] (optional) is read
    as the stacked LoRA-A operand instead of stacking the three."""
    if X2.dtype in G.GENERIC_DTYPES:
        rope = rope() if callable(rope) else rope
        return G.qkv_forward(X2, W_q, W_k, W_v, A_q, B_q, s_q, A_k, B_k, s_k, A_v, B_v, s_v, rope=rope, aux=aux)
    L.require_gpu(X2, W_q, W_k, W_v)
    if A_q is not None and A_q.shape[0] % 8:  # rank padded to a multiple of 8 (exact)
        (A_q, B_q), (A_k, B_k), (A_v, B_v) = (pad_rank(a, b) for a, b in ((A_q, B_q), (A_k, B_k), (A_v, B_v)))
        a_packed = None
    X2 = as_operand(X2)
    has_lora = A_q is not None and B_q is not None
    r = A_q.shape[0] if has_lora else 0
    xa = None
    if has_lora:  # the first launch; the QKV GEMM needs its result
        mats = [A_q, A_k, A_v] if a_packed is None else [a_packed[:r], a_packed[r:2 * r], a_packed[2 * r:]]
        xa = lora_a(X2, mats, [s_q, s_k, s_v])
        if aux is not None:
            aux["xa"] = xa
    if callable(rope):
        rope = rope()
    Wq, Wk, Wv = _w(W_q), _w(W_k), _w(W_v)
    M = X2.shape[0]
    Hq, Hkv = Wq.shape[0], Wk.shape[0]
    out = torch.empty(M, Hq + 2 * Hkv, dtype=torch.bfloat16, device=X2.device)
    Bq = Bk = Bv = None
    if has_lora:
        Bq, Bk, Bv = _w(B_q), _w(B_k), _w(B_v)
    fuse = ROPE_IN_EPILOGUE if fuse_rope is None else fuse_rope
    if rope is not None and not (fuse and rope_fusable(rope, Hq, Hkv)):
        # the GEMM stores Q/K, then a forge_rope pass rotates them in place
        qkv_gemm(X2, Wq, Wk, Wv, xa, Bq, Bk, Bv, r, None, out)
        rope_qk_inplace(out, Hq, Hkv, rope)
    else:
        qkv_gemm(X2, Wq, Wk, Wv, xa, Bq, Bk, Bv, r, rope, out)
    return out


def rope_fusable(rope: dict, Hq: int, Hkv: int) -> bool:
    """Whether forge_lora_qkv_rope can rotate Q/K in its GEMM epilogue: bf16
    tables, head_dim 64 or 128, and Q and K widths that are whole 256-column
    tiles (a tile then holds whole heads of one projection).  Otherwise the
    forward stores Q/K unrotated and rotates them with forge_rope."""
    return (rope["cos"].dtype == torch.bfloat16 and rope["head_dim"] in (64, 128)
            and Hq % 256 == 0 and Hkv % 256 == 0)


def qkv_gemm(X2, Wq, Wk, Wv, xa, Bq, Bk, Bv, r: int, rope: Optional[dict], out: torch.Tensor) -> None:
    """out = [X Wq^T + xa_q Bq^T | X Wk^T + xa_k Bk^T | X Wv^T + xa_v Bv^T]
    (xa = [sq X Aq^T | sk X Ak^T | sv X Av^T], None without LoRA), Q and K
    rotated in the epilogue when rope (bf16 tables) is given: one
    forge_lora_qkv_rope launch.  (Splitting the rows of a last, partly
    filled round of 256 x 256 tiles over K was measured on MI355X at the
    BASELINE shape, 2160 tiles on 256 CUs: no faster, since the chip clocks
    up while fewer CUs are busy.)"""
    M, K = X2.shape
    Hq, Hkv = Wq.shape[0], Wk.shape[0]
    if rope is not None:
        cos, sin = rope["cos"], rope["sin"]
        pos = rope.get("positions")
        hd = rope["head_dim"]
        cos_p, sin_p, cs_ld, cs_rows = cos.data_ptr(), sin.data_ptr(), cos.stride(0), cos.shape[0]
        pos_p = None if pos is None else pos.data_ptr()
        apply = 1
    else:
        cos_p = sin_p = pos_p = None
        cs_ld, cs_rows, hd, apply = 0, 0, 128, 0
    L.check(
        L.forge_lora_qkv_rope(
            M, K, Hq, Hkv, r, X2.data_ptr(), ld(X2), Wq.data_ptr(), Wk.data_ptr(), Wv.data_ptr(), ld(Wq),
            L.ptr(xa), 3 * r, L.ptr(Bq), L.ptr(Bk), L.ptr(Bv), r, out.data_ptr(), ld(out),
            cos_p, sin_p, cs_ld, cs_rows, pos_p, hd, apply, L.stream_of(X2)),
        "forge_lora_qkv_rope",
    )


def rope_qk_inplace(out, Hq, Hkv, rope, backward=False):
    """Rotates the Q and K column blocks of a packed [M, Hq + 2 Hkv] buffer
    in place with forge_rope (tables in out's dtype or fp32)."""
    D = rope["head_dim"]
    cos, sin, pos = rope["cos"], rope["sin"], rope.get("positions")
    M, ldo = out.shape[0], out.stride(0)
    q, k = out[:, :Hq], out[:, Hq:Hq + Hkv]
    L.check(L.forge_rope(L.dtype_code(out.dtype),
                         q.data_ptr(), 0, D, ldo, k.data_ptr(), 0, D, ldo,
                         q.data_ptr(), 0, D, ldo, k.data_ptr(), 0, D, ldo,
                         cos.data_ptr(), 0, cos.stride(0), sin.data_ptr(), 0, sin.stride(0),
                         L.dtype_code(cos.dtype), cos.shape[0],
                         None if pos is None else pos.data_ptr(), 1, Hq // D, Hkv // D, M, D,
                         1 if backward else 0, L.stream_of(out)), "forge_rope")


def qkv_backward(dQ, dK, dV, X2, W_q, W_k, W_v, A_q, B_q, s_q, A_k, B_k, s_k, A_v, B_v, s_v,
                 aux: Optional[dict] = None, pre: Optional[tuple] = None):
    """Returns (dX, dA_q, dB_q, dA_k, dB_k, dA_v, dB_v).  With the forward's
    aux the B gradients reuse its scaled xa instead of re-reading X.  pre =
    (t, B_q^T, B_k^T, B_v^T, A_q^T, A_k^T, A_v^T) from a caller that already
    formed t = s [dQ B_q | dK B_k | dV B_v] (forge_lora_qkv_rope_bwd) and the
    small transposes (rank a multiple of 8)."""
    if X2.dtype in G.GENERIC_DTYPES:
        return G.qkv_backward(dQ, dK, dV, X2, W_q, W_k, W_v, A_q, B_q, s_q, A_k, B_k, s_k, A_v, B_v, s_v, aux=aux)
    if A_q.shape[0] % 8:  # rank padded to a multiple of 8 (exact); the padding's gradients are dropped
        r0 = A_q.shape[0]
        (Aq8, Bq8), (Ak8, Bk8), (Av8, Bv8) = (pad_rank(a, b) for a, b in ((A_q, B_q), (A_k, B_k), (A_v, B_v)))
        dX, dAq, dBq, dAk, dBk, dAv, dBv = qkv_backward(dQ, dK, dV, X2, W_q, W_k, W_v, Aq8, Bq8, s_q, Ak8, Bk8, s_k,
                                                        Av8, Bv8, s_v, aux=aux)
        return (dX, dAq[:r0].contiguous(), dBq[:, :r0].contiguous(), dAk[:r0].contiguous(),
                dBk[:, :r0].contiguous(), dAv[:r0].contiguous(), dBv[:, :r0].contiguous())
    X2 = as_operand(X2)
    dQ, dK, dV = as_operand(dQ), as_operand(dK), as_operand(dV)
    Wq, Wk, Wv = _w(W_q), _w(W_k), _w(W_v)
    M, K = X2.shape
    Hq, Hkv = Wq.shape[0], Wk.shape[0]
    r = A_q.shape[0]
    dev = X2.device
    Aq, Bq, Ak, Bk, Av, Bv = (_w(t) for t in (A_q, B_q, A_k, B_k, A_v, B_v))
    # K-contiguous operands for the 4-wave engine (cached W^T, small A^T / B^T;
    # the rank is a multiple of 8 here): the six small transposes in one launch
    if pre is not None:  # t formed by the caller
        t, BqT, BkT, BvT, AqT, AkT, AvT = pre
    else:
        BqT, BkT, BvT, AqT, AkT, AvT = small_t_batch([Bq, Bk, Bv, Aq, Ak, Av])
        t = torch.empty(M, 3 * r, dtype=torch.bfloat16, device=dev)
    if pre is not None:
        pass
    elif s_q == s_k == s_v:  # [dQ Bq | dK Bk | dV Bv] in one launch (column-ranged segments)
        gemm(M, 3 * r, [(dQ, ld(dQ), BqT, Hq, Hq, 0, r), (dK, ld(dK), BkT, Hkv, Hkv, r, 2 * r),
                        (dV, ld(dV), BvT, Hkv, Hkv, 2 * r, 3 * r)], ROW, COL, out=t, alpha=s_q)
    else:
        times_b(dQ, ld(dQ), Bq, Hq, out=t[:, :r], alpha=s_q, b_t=BqT)
        times_b(dK, ld(dK), Bk, Hkv, out=t[:, r:2 * r], alpha=s_k, b_t=BkT)
        times_b(dV, ld(dV), Bv, Hkv, out=t[:, 2 * r:], alpha=s_v, b_t=BvT)
    dt = A_q.dtype
    dA = grad_at_b(t, 3 * r, X2, ld(X2), 3 * r, K, M, out_dtype=dt)  # [3r, K] (scales included via t)
    if aux is not None and "xa" in aux:
        xa, sc = aux["xa"], (1.0, 1.0, 1.0)            # scaled s_p X A_p^T from the forward
    else:
        xa, sc = lora_a(X2, [Aq, Ak, Av], [1.0, 1.0, 1.0]), (s_q, s_k, s_v)
    if dt == torch.bfloat16 and sc[0] == sc[1] == sc[2]:  # the three B gradients in one launch
        dBq, dBk, dBv = grad_at_b_group([(xa[:, :r], 3 * r, dQ, ld(dQ), Hq), (xa[:, r:2 * r], 3 * r, dK, ld(dK), Hkv),
                                         (xa[:, 2 * r:], 3 * r, dV, ld(dV), Hkv)], r, M, alpha=sc[0])
    else:
        dBq = grad_at_b(dQ, ld(dQ), xa[:, :r], 3 * r, Hq, r, M, alpha=sc[0], out_dtype=dt)
        dBk = grad_at_b(dK, ld(dK), xa[:, r:2 * r], 3 * r, Hkv, r, M, alpha=sc[1], out_dtype=dt)
        dBv = grad_at_b(dV, ld(dV), xa[:, 2 * r:], 3 * r, Hkv, r, M, alpha=sc[2], out_dtype=dt)
    dX = gemm(M, K, [(dQ, ld(dQ), frozen_t(W_q), Hq, Hq), (dK, ld(dK), frozen_t(W_k), Hkv, Hkv),
                     (dV, ld(dV), frozen_t(W_v), Hkv, Hkv), (t[:, :r], 3 * r, AqT, r, r),
                     (t[:, r:2 * r], 3 * r, AkT, r, r), (t[:, 2 * r:], 3 * r, AvT, r, r)],
              ROW, COL)
    return (dX, dA[:r], dBq, dA[r:2 * r], dBk, dA[2 * r:], dBv)


def torch_qkv_forward(X, W_q, W_k, W_v, A_q, B_q, s_q, A_k, B_k, s_k, A_v, B_v, s_v):
    """The reference's plain-PyTorch forward for float64 / no-LoRA inputs
    (kernels/lora_qkv/reference/lora_qkv_pytorch.py:34-121)."""
    def proj(W, A, B, s):
        out = X @ W.t()
        if A is not None and B is not None:
            out = out + s * ((X @ A.t()) @ B.t())
        return out
    return proj(W_q, A_q, B_q, s_q), proj(W_k, A_k, B_k, s_k), proj(W_v, A_v, B_v, s_v)


def torch_qkv_backward(dQ, dK, dV, X, W_q, W_k, W_v, A_q, B_q, s_q, A_k, B_k, s_k, A_v, B_v, s_v):
    """The reference's float64 backward (lora_qkv_pytorch.py:170-214)."""
    dX = dQ @ W_q + dK @ W_k + dV @ W_v
    grads = []
    for dY, A, B, s in ((dQ, A_q, B_q, s_q), (dK, A_k, B_k, s_k), (dV, A_v, B_v, s_v)):
        dYB = dY @ B
        dX = dX + s * (dYB @ A)
        grads += [s * (dYB.t() @ X), s * (dY.t() @ (X @ A.t()))]
    return (dX, *grads)


def pack_weights_all(W_q, A_q, W_k, A_k, W_v, A_v):
    """[W_q; A_q; W_k; A_k; W_v; A_v] (v2_3 :47-76; API parity — the HIP
    forward reads the six matrices directly)."""
    parts = [W_q]
    if A_q is not None:
        parts.append(A_q)
    parts.append(W_k)
    if A_k is not None:
        parts.append(A_k)
    parts.append(W_v)
    if A_v is not None:
        parts.append(A_v)
    return torch.cat(parts, dim=0).contiguous()


def pack_weights_backward(W_q, W_k, W_v):
    """[W_q; W_k; W_v] (v4 :55-63)."""
    return torch.cat([W_q, W_k, W_v], dim=0).contiguous()


def pack_lora_a(A_q, A_k, A_v):
    """[A_q; A_k; A_v] (v4 :66-72)."""
    return torch.cat([A_q, A_k, A_v], dim=0).contiguous()


def split_views(out, Hq, Hkv, orig_shape):
    Q = out[:, :Hq]
    K_ = out[:, Hq:Hq + Hkv]
    V = out[:, Hq + Hkv:Hq + 2 * Hkv]
    if len(orig_shape) == 3:
        Q = Q.view(orig_shape[0], orig_shape[1], Hq)
        K_ = K_.view(orig_shape[0], orig_shape[1], Hkv)
        V = V.view(orig_shape[0], orig_shape[1], Hkv)
    return Q, K_, V
