"""LoRA-QKV v4 API on MI355X (training), plus the fused QKV + RoPE variant.

Drop-in for kernels/lora_qkv/experiments/v4/lora_qkv_kernel_v4.py of
Forge-researchlab/kernel-POCs: `LoRAQKVv4Function` (16 forward arguments,
saves (X, A_q, B_q, A_k, B_k, A_v, B_v, W_dX_packed, A_packed),
ctx.scalings / ctx.dims, 16-tuple backward), `lora_qkv_v4`,
`pack_weights_backward`, `pack_lora_a`.  As in the reference (:209-214) the
packed matrices are built when not given and saved: A_packed = [A_q; A_k;
A_v] is also the forward's stacked LoRA-A operand, and W_dX_packed =
[W_q; W_k; W_v] of the frozen base weights is built once per weight triple
and reused (the HIP backward reads the cached W^T of each weight).

`LoRAQKVRoPEFunction` / `lora_qkv_rope` add the fusion of the caller's RoPE
(forge/forge/patching/kernels/lora.py:250-264 for models without q/k norm):
the Q and K heads are rotated in the GEMM epilogue with per-token positions
(packed variable-length batches), and the backward rotates dQ/dK back before
the v4 backward.  Outputs equal lora_qkv_v4 followed by apply_rope.
"""
from __future__ import annotations

import torch

from forge_hip import _lib as L
from kernels._lora_ops import frozen_cat, small_t_batch
from kernels._positions import check_positions
from kernels.lora_qkv._impl import (  # noqa: F401
    pack_lora_a,
    pack_weights_backward,
    qkv_backward,
    qkv_forward,
    split_views,
    torch_qkv_backward,
    torch_qkv_forward,
)


def _flat(t):
    return t.reshape(-1, t.shape[-1])


# The backward's RoPE pass and its LoRA-B products [dQ B_q | dK B_k | dV B_v]
# in one kernel (forge_lora_qkv_rope_bwd) when the shapes allow (True), else
# a forge_rope pass and a GEMM that reads the gradients again (False).
ROPE_BWD_FUSED = True
_ROPE_BWD_HEADS = {(32, 8), (32, 32), (64, 8), (16, 8), (8, 2), (4, 2)}  # (Q, KV) head counts built


def _rope_bwd_fused(dQ2, dK2, dV2, X2, A_q, B_q, s_q, A_k, B_k, s_k, A_v, B_v, s_v, D, cos2, sin2, pos):
    """(dQu, dKu, pre) from forge_lora_qkv_rope_bwd, or None when the shapes,
    dtypes or scales rule it out; pre is qkv_backward's precomputed t and
    small transposes."""
    from kernels.lora_qkv._impl import _w

    r = A_q.shape[0]
    M, Hq, Hkv = dQ2.shape[0], dQ2.shape[1], dK2.shape[1]
    bf = torch.bfloat16
    tens = (dQ2, dK2, dV2, cos2, sin2)
    if not (ROPE_BWD_FUSED and D == 128 and (Hq // D, Hkv // D) in _ROPE_BWD_HEADS and Hq % D == 0
            and Hkv % D == 0 and r in (16, 32, 48, 64) and s_q == s_k == s_v and M > 0
            and all(t.dtype == bf and t.stride(-1) == 1 and t.stride(0) % 8 == 0 and t.data_ptr() % 16 == 0
                    for t in tens)
            and A_q.dtype == bf and B_q.dtype == bf):
        return None
    Bq, Bk, Bv, Aq, Ak, Av = (_w(t) for t in (B_q, B_k, B_v, A_q, A_k, A_v))
    BqT, BkT, BvT, AqT, AkT, AvT = small_t_batch([Bq, Bk, Bv, Aq, Ak, Av])
    dev = dQ2.device
    dQu = torch.empty(M, Hq, dtype=bf, device=dev)
    dKu = torch.empty(M, Hkv, dtype=bf, device=dev)
    t = torch.empty(M, 3 * r, dtype=bf, device=dev)
    L.check(
        L.forge_lora_qkv_rope_bwd(M, Hq, Hkv, r, D, dQ2.data_ptr(), dQ2.stride(0), dK2.data_ptr(), dK2.stride(0),
                                  dV2.data_ptr(), dV2.stride(0), cos2.data_ptr(), sin2.data_ptr(), cos2.stride(0),
                                  cos2.shape[0], pos.data_ptr() if pos is not None else None,
                                  dQu.data_ptr(), Hq, dKu.data_ptr(), Hkv, BqT.data_ptr(), BkT.data_ptr(),
                                  BvT.data_ptr(), BqT.stride(0), BkT.stride(0), BvT.stride(0), t.data_ptr(), 3 * r,
                                  float(s_q), L.stream_of(dQ2)),
        "forge_lora_qkv_rope_bwd",
    )
    return dQu, dKu, (t, BqT, BkT, BvT, AqT, AkT, AvT)


class LoRAQKVv4Function(torch.autograd.Function):
    """v4 :170-336."""

    @staticmethod
    def forward(ctx, X, W_q, W_k, W_v, A_q, B_q, s_q, A_k, B_k, s_k, A_v, B_v, s_v,
                W_all=None, W_dX_packed=None, A_packed=None):
        use_hip = X.dtype != torch.float64
        orig_shape = X.shape
        X2 = _flat(X)
        ctx.lora_aux = {}  # forward products reused by the backward (outside saved_tensors)
        # the packed matrices of the reference's save contract (:209-214)
        if W_dX_packed is None:
            W_dX_packed = frozen_cat((W_q, W_k, W_v))
        a_stack = None  # a caller's A_packed is only saved; the one built here is the stacked operand
        if A_packed is None:
            A_packed = a_stack = pack_lora_a(A_q.detach(), A_k.detach(), A_v.detach())
        if use_hip:
            out = qkv_forward(X2, W_q, W_k, W_v, A_q, B_q, s_q, A_k, B_k, s_k, A_v, B_v, s_v, aux=ctx.lora_aux,
                              a_packed=a_stack)
            Q, K, V = split_views(out, W_q.shape[0], W_k.shape[0], orig_shape)
        else:
            Q, K, V = torch_qkv_forward(X2, W_q, W_k, W_v, A_q, B_q, s_q, A_k, B_k, s_k, A_v, B_v, s_v)
            if len(orig_shape) == 3:
                Q, K, V = (t.view(orig_shape[0], orig_shape[1], -1) for t in (Q, K, V))
        ctx.save_for_backward(X, A_q, B_q, A_k, B_k, A_v, B_v, W_dX_packed, A_packed)
        ctx.scalings = (s_q, s_k, s_v)
        ctx.dims = (W_q.shape[0], W_k.shape[0], A_q.shape[0])
        ctx.use_triton = use_hip  # name kept from the reference (:217)
        ctx.base_weights = (W_q, W_k, W_v)
        return Q, K, V

    @staticmethod
    def backward(ctx, dQ, dK, dV):
        X, A_q, B_q, A_k, B_k, A_v, B_v, _, _ = ctx.saved_tensors
        s_q, s_k, s_v = ctx.scalings
        W_q, W_k, W_v = ctx.base_weights
        X2 = _flat(X)
        args = (_flat(dQ), _flat(dK), _flat(dV), X2, W_q, W_k, W_v, A_q, B_q, s_q, A_k, B_k, s_k, A_v, B_v, s_v)
        if ctx.use_triton:
            dX, dAq, dBq, dAk, dBk, dAv, dBv = qkv_backward(*args, aux=ctx.lora_aux)
        else:
            dX, dAq, dBq, dAk, dBk, dAv, dBv = torch_qkv_backward(*args)
        if X.dim() == 3:
            dX = dX.reshape(X.shape)
        return (dX, None, None, None, dAq, dBq, None, dAk, dBk, None, dAv, dBv, None, None, None, None)


def lora_qkv_v4(X, W_q, A_q, B_q, s_q, W_k, A_k, B_k, s_k, W_v, A_v, B_v, s_v,
                W_all=None, W_dX_packed=None, A_packed=None):
    """v4 :343-379."""
    return LoRAQKVv4Function.apply(X, W_q, W_k, W_v, A_q, B_q, s_q, A_k, B_k, s_k, A_v, B_v, s_v,
                                   W_all, W_dX_packed, A_packed)


def _rope_rows_backward(d, n_heads, head_dim, cos, sin, positions):
    """Rotates a [M, n_heads*head_dim] gradient (any row pitch) by -theta per
    token with forge_rope; returns a new contiguous tensor."""
    M = d.shape[0]
    out = torch.empty(M, n_heads * head_dim, dtype=d.dtype, device=d.device)
    st = L.stream_of(d)
    ldd = d.stride(0)
    L.check(
        L.forge_rope(L.dtype_code(d.dtype),
                     d.data_ptr(), 0, head_dim, ldd,
                     d.data_ptr(), 0, head_dim, ldd,
                     out.data_ptr(), 0, head_dim, n_heads * head_dim,
                     out.data_ptr(), 0, head_dim, n_heads * head_dim,
                     cos.data_ptr(), 0, cos.stride(0), sin.data_ptr(), 0, sin.stride(0),
                     L.dtype_code(cos.dtype), cos.shape[0],
                     positions.data_ptr() if positions is not None else None,
                     1, n_heads, 0, M, head_dim, 1, st),
        "forge_rope(backward)",
    )
    return out


def _rope_qk_backward(dQ, dK, head_dim, cos, sin, positions):
    """Rotates the [M, Hq] and [M, Hkv] gradients (any row pitches) by -theta
    per token in one forge_rope launch (GQA: Hq/D a multiple of Hkv/D) into
    new contiguous tensors."""
    nq, nk = dQ.shape[1] // head_dim, dK.shape[1] // head_dim
    if nk == 0 or nq % nk != 0:
        return (_rope_rows_backward(dQ, nq, head_dim, cos, sin, positions),
                _rope_rows_backward(dK, nk, head_dim, cos, sin, positions))
    M = dQ.shape[0]
    oq = torch.empty(M, nq * head_dim, dtype=dQ.dtype, device=dQ.device)
    ok = torch.empty(M, nk * head_dim, dtype=dK.dtype, device=dK.device)
    L.check(
        L.forge_rope(L.dtype_code(dQ.dtype),
                     dQ.data_ptr(), 0, head_dim, dQ.stride(0),
                     dK.data_ptr(), 0, head_dim, dK.stride(0),
                     oq.data_ptr(), 0, head_dim, oq.stride(0),
                     ok.data_ptr(), 0, head_dim, ok.stride(0),
                     cos.data_ptr(), 0, cos.stride(0), sin.data_ptr(), 0, sin.stride(0),
                     L.dtype_code(cos.dtype), cos.shape[0],
                     positions.data_ptr() if positions is not None else None,
                     1, nq, nk, M, head_dim, 1, L.stream_of(dQ)),
        "forge_rope(backward)",
    )
    return oq, ok


def _qkv_tables(cos, sin, x_dtype):
    """2-D contiguous cos/sin in one dtype the kernels read as stored:
    X's dtype or fp32 (another dtype, or a mixed pair, is widened to fp32)."""
    cos2, sin2 = cos.reshape(-1, cos.shape[-1]), sin.reshape(-1, sin.shape[-1])
    if not (cos2.dtype == sin2.dtype and cos2.dtype in (x_dtype, torch.float32)):
        cos2, sin2 = cos2.float(), sin2.float()
    return cos2.contiguous(), sin2.contiguous()


class LoRAQKVRoPEFunction(torch.autograd.Function):
    """LoRA-QKV with RoPE fused into the GEMM epilogue.

    forward(ctx, X, W_q, W_k, W_v, A_q, B_q, s_q, A_k, B_k, s_k, A_v, B_v, s_v,
            cos, sin, positions, head_dim) -> (Q_rot, K_rot, V)
    cos/sin: tables [P, head_dim] (rows = positions), read as stored when in
    X's dtype or fp32 (fp32 math either way), else widened to fp32; bf16
    tables with bf16 X rotate in the GEMM epilogue (head_dim 64 or 128, Q and
    K widths multiples of 256), other cases in a forge_rope pass over the
    stored Q/K.  positions: int64 [M] in [0, P)
    (token -> table row; restarts per sequence for packed varlen;
    IndexError otherwise); None means row m for token m."""

    @staticmethod
    def forward(ctx, X, W_q, W_k, W_v, A_q, B_q, s_q, A_k, B_k, s_k, A_v, B_v, s_v, cos, sin, positions,
                head_dim=128):
        orig_shape = X.shape
        X2 = _flat(X)
        if positions is not None:  # validated before any launch
            check_positions(positions, cos.reshape(-1, cos.shape[-1]).shape[0])
        tables = []

        def rope_args():  # called by qkv_forward once the LoRA-A product is queued
            cos2, sin2 = _qkv_tables(cos, sin, X.dtype)
            pos = None
            if positions is not None:
                pos = positions.reshape(-1).to(device=X.device, dtype=torch.int64).contiguous()
            tables.extend((cos2, sin2, pos))
            return {"cos": cos2, "sin": sin2, "positions": pos, "head_dim": int(head_dim)}

        ctx.lora_aux = {}  # forward products reused by the backward (outside saved_tensors)
        out = qkv_forward(X2, W_q, W_k, W_v, A_q, B_q, s_q, A_k, B_k, s_k, A_v, B_v, s_v,
                          rope=rope_args, aux=ctx.lora_aux)
        cos2, sin2, pos = tables
        ctx.save_for_backward(X, A_q, B_q, A_k, B_k, A_v, B_v, cos2, sin2, pos)
        ctx.scalings = (s_q, s_k, s_v)
        ctx.base_weights = (W_q, W_k, W_v)
        ctx.head_dim = int(head_dim)
        return split_views(out, W_q.shape[0], W_k.shape[0], orig_shape)

    @staticmethod
    def backward(ctx, dQ, dK, dV):
        X, A_q, B_q, A_k, B_k, A_v, B_v, cos2, sin2, pos = ctx.saved_tensors
        s_q, s_k, s_v = ctx.scalings
        W_q, W_k, W_v = ctx.base_weights
        D = ctx.head_dim
        dQ2, dK2 = _flat(dQ), _flat(dK)
        dQ2 = dQ2 if dQ2.stride(-1) == 1 else dQ2.contiguous()
        dK2 = dK2 if dK2.stride(-1) == 1 else dK2.contiguous()
        fused = _rope_bwd_fused(dQ2, dK2, _flat(dV), _flat(X), A_q, B_q, s_q, A_k, B_k, s_k, A_v, B_v, s_v, D,
                                cos2, sin2, pos)
        if fused is not None:
            dQu, dKu, pre = fused
        else:
            dQu, dKu = _rope_qk_backward(dQ2, dK2, D, cos2, sin2, pos)
            pre = None
        dX, dAq, dBq, dAk, dBk, dAv, dBv = qkv_backward(dQu, dKu, _flat(dV), _flat(X), W_q, W_k, W_v,
                                                        A_q, B_q, s_q, A_k, B_k, s_k, A_v, B_v, s_v,
                                                        aux=ctx.lora_aux, pre=pre)
        if X.dim() == 3:
            dX = dX.reshape(X.shape)
        return (dX, None, None, None, dAq, dBq, None, dAk, dBk, None, dAv, dBv, None, None, None, None, None)


def lora_qkv_rope(X, W_q, A_q, B_q, s_q, W_k, A_k, B_k, s_k, W_v, A_v, B_v, s_v, cos, sin, positions=None,
                  head_dim=128):
    """LoRA-QKV followed by RoPE on Q and K, fused (see LoRAQKVRoPEFunction)."""
    return LoRAQKVRoPEFunction.apply(X, W_q, W_k, W_v, A_q, B_q, s_q, A_k, B_k, s_k, A_v, B_v, s_v,
                                     cos, sin, positions, head_dim)


__all__ = ["LoRAQKVv4Function", "lora_qkv_v4", "pack_weights_backward", "pack_lora_a",
           "LoRAQKVRoPEFunction", "lora_qkv_rope"]
