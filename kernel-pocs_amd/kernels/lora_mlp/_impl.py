"""LoRA-MLP (LLaMA-style SwiGLU with LoRA on gate/up/down) on MI355X.

Forward  (reference v6 `_v6_forward_impl`,
kernels/lora_mlp/experiments/v6/lora_mlp_kernel_v6.py:335-451):
  1. xa   = [sg X Ag^T | su X Au^T]                  forge_lora_a       [M, 2r]
  2. e = X Wg^T + xa_g Bg^T, g = X Wu^T + xa_u Bu^T, h = glu(e, g)
                                                     forge_lora_mlp_gate_up: one
     MFMA GEMM over the dual gate/up B with the LoRA-B products as K segments
     (one rounding) and the gated activation in its epilogue (h forms in
     registers; e, g are stored for the backward)
  3. xd   = sd h Ad^T                                (ranks up to 64) fp32 partials
     per 128-column tile from forge_lora_mlp_gate_up_v's epilogue, summed by
     forge_splitk_reduce; else forge_lora_a   [M, r]
  4. out  = h Wd^T + xd Bd^T                         forge_gemm, xd Bd^T a K segment
  (the reference sends the base products to cuBLAS, lora_mlp_kernel_v6.py:374-443;
   here every product is the library's own gfx950 GEMM.)

Backward (reference `LoRAMLPv6.backward`, :592-672, Unsloth-style in place;
math of kernels/lora_mlp/reference/lora_mlp_pytorch.py:145-225):
  1. td   = sd dY Bd                                 forge_gemm         [M, r]
  2. DW = dY Wd + td Ad, fused in-place SwiGLU backward:
     (DW, e, g) -> (h, df, de)                       forge_lora_mlp_down_bwd_v
     (ranks up to 64: its epilogue also forms step 4's [df Bu | de Bg] as fp32
     partial sums per 256-column tile from the df, de it holds, and with the
     forward's xa step 4's dBu, dBg as fp32 partial sums per 256-row tile)
  3. dAd = td^T h,  dBd = sd dY^T (h Ad^T)           split-K forge_gemm
  4. vu = su df Bu, vg = sg de Bg                    forge_splitk_reduce of those
                                                     partials (else forge_gemm)  [M, r]
     dAu = vu^T X, dAg = vg^T X, dBu = su df^T (X Au^T), dBg = sg de^T (X Ag^T)
                                                     (dBu, dBg: forge_splitk_reduce of
                                                     step 2's row-tile partials)
  5. dX = df Wu + de Wg + vu Au + vg Ag              forge_gemm, 4 K segments over the
                                                     cached W^T and the small A^T
The saved e/g buffers are overwritten by df/de in step 2 (the reference's
in-place contract: backward is not re-entrant).

activation="gelu_tanh" / "gelu_exact" runs the same pipeline with the GeGLU
epilogues (Gemma MLPs): h = round(gelu(e)) g in the forward and, in step 2,
df = round(DW) round(gelu(e)), de = round(DW) g gelu'(e) - the GeGLU
kernel's forward and backward (kernels/geglu/geglu.py:104-148) on the bf16
e, g and DW, where the reference composes PEFT projections with that kernel
(forge/forge/patching/kernels/lora.py:170-188).
"""
from __future__ import annotations

import math
from typing import Optional, Tuple

import torch
import torch.nn.functional as F

from forge_hip import _lib as L
from kernels import _generic_lora as G
from kernels._lora_ops import (COL, ROW, as_operand, frozen_t, gemm, grad_at_b, grad_at_b_group, ld, lora_a,
                               pad_rank, small_t_batch, times_b)


def _w(t):
    return None if t is None else as_operand(t)


# Rank-r LoRA products formed by the gated-activation epilogues from the
# tensors they hold (True, ranks up to 64), or by GEMMs that read those
# tensors back (False): h Ad^T of the forward in the gate/up epilogue, and
# [df Bu | de Bg] of the backward in the down-projection backward's epilogue
# (SiLU only).  Measured on MI355X at M = 8192, H = 4096, I = 14336, r = 16
# (A/B on one box), the backward's alone: SiLU step 5.32 -> 5.27 ms; GeGLU
# 5.22 -> 5.27 ms, its epilogue's GELU derivative holding enough registers
# that de's stay spills to scratch, so GeGLU keeps the GEMM there.
RANK_IN_EPILOGUE = True
# With RANK_IN_EPILOGUE and the forward's xa, the down-projection backward's
# epilogue also forms the B gradients' token reductions df^T xa_u and
# de^T xa_g (fp32 partial sums per 256-row tile) from the df and de tiles it
# stages for [df Bu | de Bg], instead of a product that re-reads both [M, I]
# tensors (False).
TOKEN_IN_EPILOGUE = True

ACTIVATIONS = {"silu": L.ACT_SILU, "gelu_tanh": L.ACT_GELU_TANH, "gelu_exact": L.ACT_GELU_ERF}


def _act_code(activation: str) -> int:
    try:
        return ACTIVATIONS[activation]
    except KeyError:
        raise ValueError(f"LoRA-MLP activation must be one of {sorted(ACTIVATIONS)}, got {activation!r}") from None


def mlp_forward(X2, W_gate, A_gate, B_gate, s_gate, W_up, A_up, B_up, s_up,
                W_down, A_down, B_down, s_down, save_eg: bool = True, aux: Optional[dict] = None,
                activation: str = "silu"):
    """Returns (out [M, H], e [M, I], g [M, I]) (e, g None unless save_eg).
    aux (a dict, optional) receives the LoRA-A products the backward reuses:
    xa = [sg X Ag^T | su X Au^T] [M, 2r] and xd = sd h Ad^T [M, r]."""
    act = _act_code(activation)
    if X2.dtype in G.GENERIC_DTYPES:
        return G.mlp_forward(X2, W_gate, A_gate, B_gate, s_gate, W_up, A_up, B_up, s_up, W_down, A_down, B_down,
                             s_down, save_eg=save_eg, aux=aux, activation=activation)
    L.require_gpu(X2, W_gate, W_up, W_down)
    if A_gate is not None and A_gate.shape[0] % 8:  # rank padded to a multiple of 8 (exact)
        (A_gate, B_gate), (A_up, B_up), (A_down, B_down) = (
            pad_rank(a, b) for a, b in ((A_gate, B_gate), (A_up, B_up), (A_down, B_down)))
    X2 = as_operand(X2)
    Wg, Wu, Wd = _w(W_gate), _w(W_up), _w(W_down)
    M, H = X2.shape
    I = Wg.shape[0]
    has_lora = A_gate is not None and B_gate is not None
    r = A_gate.shape[0] if has_lora else 0
    dev = X2.device
    xa = None
    Bg = Bu = None
    if has_lora:  # the first launch; the gate/up GEMM needs its result
        xa = lora_a(X2, [A_gate, A_up], [s_gate, s_up])
        Bg, Bu = _w(B_gate), _w(B_up)
    e = torch.empty(M, I, dtype=torch.bfloat16, device=dev)
    g = torch.empty(M, I, dtype=torch.bfloat16, device=dev)
    h = torch.empty(M, I, dtype=torch.bfloat16, device=dev)
    st = L.stream_of(X2)
    down_lora = has_lora and A_down is not None and B_down is not None
    # with ranks up to 64 the gate/up epilogue also forms h Ad^T (step 3) as
    # fp32 partial sums per 128-column tile, from the h it holds
    xd_in_epi = RANK_IN_EPILOGUE and down_lora and r <= 64 and I % 8 == 0
    if xd_in_epi:
        Ad = _w(A_down)
        n_ct = (I + 127) // 128
        xpart = torch.empty(n_ct, M, r, dtype=torch.float32, device=dev)
        L.check(
            L.forge_lora_mlp_gate_up_v(
                M, H, I, r, X2.data_ptr(), ld(X2), Wg.data_ptr(), Wu.data_ptr(), ld(Wg),
                L.ptr(xa), 2 * r, L.ptr(Bg), L.ptr(Bu), r, e.data_ptr(), g.data_ptr(), h.data_ptr(), I, act,
                Ad.data_ptr(), ld(Ad), r, xpart.data_ptr(), st),
            "forge_lora_mlp_gate_up_v",
        )
    else:
        L.check(
            L.forge_lora_mlp_gate_up(
                M, H, I, r, X2.data_ptr(), ld(X2), Wg.data_ptr(), Wu.data_ptr(), ld(Wg),
                L.ptr(xa), 2 * r, L.ptr(Bg), L.ptr(Bu), r, e.data_ptr(), g.data_ptr(), h.data_ptr(), I, act, st),
            "forge_lora_mlp_gate_up",
        )
    segs = [(h, ld(h), Wd, ld(Wd), I)]
    if down_lora:
        if xd_in_epi:  # the column tiles' partial sums, in a fixed order, scaled and rounded once
            xd = torch.empty(M, r, dtype=torch.bfloat16, device=dev)
            L.check(L.forge_splitk_reduce(xpart.data_ptr(), M * r, n_ct, M, r, r, xd.data_ptr(), r, L.DTYPE_BF16,
                                          float(s_down), st), "forge_splitk_reduce")
        else:
            xd = lora_a(h, [A_down], [s_down])
        Bd = _w(B_down)
        segs.append((xd, ld(xd), Bd, ld(Bd), r))
        if aux is not None:
            aux["xa"], aux["xd"] = xa, xd
    out = gemm(M, Wd.shape[0], segs, ROW, COL)
    if not save_eg:
        e = g = None
    return out, e, g


def mlp_backward(dY2, X2, e, g, W_gate, A_gate, B_gate, s_gate, W_up, A_up, B_up, s_up,
                 W_down, A_down, B_down, s_down, aux: Optional[dict] = None, activation: str = "silu"):
    """Returns (dX [M, H], dAg, dBg, dAu, dBu, dAd, dBd).  e and g are
    overwritten with df and de.  With the forward's aux (xa, xd) the
    weight gradients of B reuse those products instead of re-reading X and h;
    xd then comes from the forward's h (fp32 e, g), which differs from the
    backward's recomputed h (bf16-rounded, lora_mlp_pytorch.py:165) only by
    rounding."""
    act = _act_code(activation)
    if X2.dtype in G.GENERIC_DTYPES:
        return G.mlp_backward(dY2, X2, e, g, W_gate, A_gate, B_gate, s_gate, W_up, A_up, B_up, s_up, W_down, A_down,
                              B_down, s_down, aux=aux, activation=activation)
    if A_gate.shape[0] % 8:  # rank padded to a multiple of 8 (exact); the padding's gradients are dropped
        r0 = A_gate.shape[0]
        (Ag8, Bg8), (Au8, Bu8), (Ad8, Bd8) = (
            pad_rank(a, b) for a, b in ((A_gate, B_gate), (A_up, B_up), (A_down, B_down)))
        dX, dAg, dBg, dAu, dBu, dAd, dBd = mlp_backward(dY2, X2, e, g, W_gate, Ag8, Bg8, s_gate, W_up, Au8, Bu8, s_up,
                                                        W_down, Ad8, Bd8, s_down, aux=aux, activation=activation)
        return (dX, dAg[:r0].contiguous(), dBg[:, :r0].contiguous(), dAu[:r0].contiguous(),
                dBu[:, :r0].contiguous(), dAd[:r0].contiguous(), dBd[:, :r0].contiguous())
    dY2 = as_operand(dY2)
    X2 = as_operand(X2)
    Wg, Wu, Wd = _w(W_gate), _w(W_up), _w(W_down)
    M, H = X2.shape
    I = Wg.shape[0]
    r = A_gate.shape[0]
    dev = X2.device
    Ag, Bg, Au, Bu, Ad, Bd = (_w(t) for t in (A_gate, B_gate, A_up, B_up, A_down, B_down))

    # K-contiguous weights (cached W^T, small A^T: the rank is a multiple of
    # 8 here) put the three big GEMMs of the backward on the 4-wave engine.
    # The six small transposes (B^T for the dY B products, A^T for the LoRA
    # segments) are one launch.
    act_ok = RANK_IN_EPILOGUE and act == L.ACT_SILU and r <= 64 and I % 8 == 0
    dt = A_gate.dtype
    # the B gradients' token reductions in the epilogue need xa^T [2r, M]
    # (token-contiguous): one more matrix in the batch of transposes
    tok_epi = (TOKEN_IN_EPILOGUE and act_ok and aux is not None and "xa" in aux and dt == torch.bfloat16
               and M % 8 == 0)
    if tok_epi:
        BdT, AdT, BuT, BgT, AuT, AgT, xaT = small_t_batch([Bd, Ad, Bu, Bg, Au, Ag, aux["xa"]])
    else:
        BdT, AdT, BuT, BgT, AuT, AgT = small_t_batch([Bd, Ad, Bu, Bg, Au, Ag])

    # h, e, g share one pitch
    e, g = as_operand(e), as_operand(g)
    lde = ld(e)
    if ld(g) != lde:
        e, g, lde = e.contiguous(), g.contiguous(), I

    # 1-2: DW = dY Wd + sd (dY Bd) Ad with the GLU backward fused in place
    td = times_b(dY2, ld(dY2), Bd, H, alpha=s_down, b_t=BdT)
    h = torch.empty(M, lde, dtype=torch.bfloat16, device=dev)[:, :I] if lde != I else \
        torch.empty(M, I, dtype=torch.bfloat16, device=dev)
    WdT = frozen_t(W_down)
    # with ranks up to 64 the epilogue also forms [df Bu | de Bg] (step 4) as
    # fp32 partial sums per 256-column tile from the df and de it produces
    # (and, with tok_epi, step 4's dBu, dBg partials per 256-row tile)
    in_epi = act_ok and lde % 8 == 0
    tok_epi = tok_epi and in_epi
    if in_epi:
        n_ct = (I + 255) // 256
        vpart = torch.empty(n_ct, M, 2 * r, dtype=torch.float32, device=dev)
        # dBu, dBg partials per 256-row tile: xa^T rows r..2r are su X Au^T, rows 0..r sg X Ag^T
        n_rt = (M + 255) // 256
        wpart = torch.empty(n_rt, 2, I, r, dtype=torch.float32, device=dev) if tok_epi else None
        L.check(
            L.forge_lora_mlp_down_bwd_v(M, H, I, r, dY2.data_ptr(), ld(dY2), WdT.data_ptr(), ld(WdT), td.data_ptr(),
                                        r, AdT.data_ptr(), ld(AdT), h.data_ptr(), e.data_ptr(), g.data_ptr(), lde,
                                        act, BuT.data_ptr(), BgT.data_ptr(), ld(BuT), r, vpart.data_ptr(),
                                        L.ptr(xaT[r:]) if tok_epi else None, L.ptr(xaT[:r]) if tok_epi else None,
                                        M, L.ptr(wpart), L.stream_of(X2)),
            "forge_lora_mlp_down_bwd_v",
        )
    else:
        L.check(
            L.forge_lora_mlp_down_bwd(M, H, I, r, dY2.data_ptr(), ld(dY2), WdT.data_ptr(), ld(WdT), td.data_ptr(),
                                      r, AdT.data_ptr(), ld(AdT), COL, h.data_ptr(), e.data_ptr(), g.data_ptr(), lde,
                                      act, L.stream_of(X2)),
            "forge_lora_mlp_down_bwd",
        )
    df, de = e, g

    # 3: down-projection LoRA grads
    dAd = grad_at_b(td, r, h, lde, r, I, M, out_dtype=dt)          # [r, I] = (sd dY Bd)^T h
    # with the forward's scaled products the three B gradients are one
    # launch (step 4); otherwise each is its own
    grouped = aux is not None and "xd" in aux and "xa" in aux and dt == torch.bfloat16 and not tok_epi
    if grouped:
        dBd = None
    elif aux is not None and "xd" in aux:
        dBd = grad_at_b(dY2, ld(dY2), aux["xd"], ld(aux["xd"]), H, r, M, out_dtype=dt)  # [H, r] = dY^T (sd h Ad^T)
    else:
        u = lora_a(h, [Ad], [1.0])                                # h Ad^T [M, r]
        dBd = grad_at_b(dY2, ld(dY2), u, r, H, r, M, alpha=s_down, out_dtype=dt)

    # 4: up / gate LoRA grads
    v = torch.empty(M, 2 * r, dtype=torch.bfloat16, device=dev)  # [su df Bu | sg de Bg]
    if in_epi:  # the column tiles' partial sums, in a fixed order, scaled and rounded once
        st = L.stream_of(X2)
        halves = [(0, 2 * r, s_up)] if s_up == s_gate else [(0, r, s_up), (r, r, s_gate)]
        for c0, nc, sc in halves:
            L.check(L.forge_splitk_reduce(vpart.data_ptr() + 4 * c0, M * 2 * r, n_ct, M, nc, 2 * r,
                                          v.data_ptr() + 2 * c0, 2 * r, L.DTYPE_BF16, float(sc), st),
                    "forge_splitk_reduce")
    elif s_up == s_gate:  # both products in one launch (column-ranged segments)
        gemm(M, 2 * r, [(df, lde, BuT, I, I, 0, r), (de, lde, BgT, I, I, r, 2 * r)], ROW, COL, out=v, alpha=s_up)
    else:
        times_b(df, lde, Bu, I, out=v[:, :r], alpha=s_up, b_t=BuT)
        times_b(de, lde, Bg, I, out=v[:, r:], alpha=s_gate, b_t=BgT)
    dA_ug = grad_at_b(v, ld(v), X2, ld(X2), 2 * r, H, M, out_dtype=dt)  # [2r, H]: rows [dAu; dAg]
    if tok_epi:  # the row tiles' partial sums, in a fixed order, rounded once (xa holds the scales)
        st = L.stream_of(X2)
        dBu = torch.empty(I, r, dtype=dt, device=dev)
        dBg = torch.empty(I, r, dtype=dt, device=dev)
        for blk, out in ((0, dBu), (1, dBg)):  # each block's slices are contiguous [I, r] rows
            L.check(L.forge_splitk_reduce(wpart[0, blk].data_ptr(), 2 * I * r, n_rt, I, r, r,
                                          out.data_ptr(), r, L.DTYPE_BF16, 1.0, st), "forge_splitk_reduce")
    elif grouped:
        xa = aux["xa"]                                            # [sg X Ag^T | su X Au^T]
        dBd, dBu, dBg = grad_at_b_group([(aux["xd"], ld(aux["xd"]), dY2, ld(dY2), H), (xa[:, r:], 2 * r, df, lde, I),
                                         (xa[:, :r], 2 * r, de, lde, I)], r, M)
    elif aux is not None and "xa" in aux:
        xa = aux["xa"]                                            # [sg X Ag^T | su X Au^T]
        dBu = grad_at_b(df, lde, xa[:, r:], 2 * r, I, r, M, out_dtype=dt)
        dBg = grad_at_b(de, lde, xa[:, :r], 2 * r, I, r, M, out_dtype=dt)
    else:
        xa_ug = lora_a(X2, [Au, Ag], [1.0, 1.0])                 # [X Au^T | X Ag^T]
        dBu = grad_at_b(df, lde, xa_ug[:, :r], 2 * r, I, r, M, alpha=s_up, out_dtype=dt)
        dBg = grad_at_b(de, lde, xa_ug[:, r:], 2 * r, I, r, M, alpha=s_gate, out_dtype=dt)

    # 5: dX = df Wu + de Wg + v [Au; Ag]: one GEMM over four K segments
    WuT, WgT = frozen_t(W_up), frozen_t(W_gate)
    dX = gemm(M, H, [(df, lde, WuT, I, I), (de, lde, WgT, I, I),
                     (v[:, :r], ld(v), AuT, r, r), (v[:, r:], ld(v), AgT, r, r)], ROW, COL)
    return (dX, dA_ug[r:], dBg, dA_ug[:r], dBu, dAd, dBd)


def _gelu_and_grad(e, activation):
    """(gelu(e), gelu'(e)) for the float64 path, tanh form or exact."""
    if activation == "gelu_tanh":
        c = math.sqrt(2.0 / math.pi)
        t = torch.tanh(c * (e + 0.044715 * e ** 3))
        return 0.5 * e * (1 + t), 0.5 * (1 + t) + 0.5 * e * (1 - t * t) * c * (1 + 3 * 0.044715 * e * e)
    cdf = 0.5 * (1 + torch.erf(e / math.sqrt(2.0)))
    return e * cdf, cdf + e * torch.exp(-0.5 * e * e) / math.sqrt(2 * math.pi)


def torch_forward(X, W_gate, A_gate, B_gate, s_gate, W_up, A_up, B_up, s_up, W_down, A_down, B_down, s_down,
                  activation="silu"):
    """Plain-PyTorch forward the reference uses for float64 (gradcheck)
    inputs (kernels/lora_mlp/experiments/v6/lora_mlp_kernel_v6.py:552-557);
    GELU activations follow the same composition with h = gelu(e) g."""
    e = X @ W_gate.t() + s_gate * ((X @ A_gate.t()) @ B_gate.t())
    g = X @ W_up.t() + s_up * ((X @ A_up.t()) @ B_up.t())
    h = F.silu(e) * g if activation == "silu" else _gelu_and_grad(e, activation)[0] * g
    out = h @ W_down.t() + s_down * ((h @ A_down.t()) @ B_down.t())
    return out, e, g


def torch_backward(dY, X, e, g, W_gate, A_gate, B_gate, s_gate, W_up, A_up, B_up, s_up,
                   W_down, A_down, B_down, s_down, activation="silu"):
    """Plain-PyTorch backward the reference uses for float64 inputs
    (kernels/lora_mlp/experiments/v6/lora_mlp_kernel_v6.py:608-628); GELU
    activations swap silu(e) and its derivative for gelu(e) and gelu'(e)."""
    if activation == "silu":
        sig_e = torch.sigmoid(e.float()).to(e.dtype)
        act_e = e * sig_e
        dact = sig_e * (1.0 + e * (1.0 - sig_e))
    else:
        act_e, dact = _gelu_and_grad(e, activation)
    h = act_e * g
    DW = dY @ W_down + s_down * ((dY @ B_down) @ A_down)
    d_downA = s_down * ((dY @ B_down).t() @ h)
    d_downB = s_down * (dY.t() @ h @ A_down.t())
    df = DW * act_e
    de = DW * g * dact
    d_upA = s_up * ((df @ B_up).t() @ X)
    d_upB = s_up * (df.t() @ X @ A_up.t())
    d_gateA = s_gate * ((de @ B_gate).t() @ X)
    d_gateB = s_gate * (de.t() @ X @ A_gate.t())
    dX = df @ W_up + s_up * ((df @ B_up) @ A_up) + de @ W_gate + s_gate * ((de @ B_gate) @ A_gate)
    return dX, d_gateA, d_gateB, d_upA, d_upB, d_downA, d_downB


def run_forward(X, params, save_eg=True, aux=None, activation="silu"):
    """Dispatch on dtype: float64 -> the reference's PyTorch path, bf16 ->
    the fused MFMA kernels, fp32 / fp16 -> the generic-GEMM kernels
    (kernels/_generic_lora.py).  Returns (out with X's leading shape, e, g);
    aux (a dict) collects the LoRA-A products for run_backward."""
    _act_code(activation)
    if X.dtype == torch.float64:
        Xf = X.reshape(-1, X.shape[-1])
        out, e, g = torch_forward(Xf, *params, activation=activation)
    else:
        if X.dtype != torch.bfloat16 and X.dtype not in G.GENERIC_DTYPES:
            raise TypeError(f"LoRA-MLP kernels take bf16, fp32 or fp16 (float64 via PyTorch), got {X.dtype}")
        out, e, g = mlp_forward(X.reshape(-1, X.shape[-1]), *params, save_eg=save_eg, aux=aux,
                                activation=activation)
    if X.dim() == 3:
        out = out.reshape(X.shape[0], X.shape[1], -1)
        if e is not None:
            e = e.reshape(X.shape[0], X.shape[1], -1)
            g = g.reshape(X.shape[0], X.shape[1], -1)
    return out, e, g


def run_backward(dY, X, e, g, params, aux=None, activation="silu"):
    dY2 = dY.reshape(-1, dY.shape[-1])
    X2 = X.reshape(-1, X.shape[-1])
    e2 = e.reshape(-1, e.shape[-1])
    g2 = g.reshape(-1, g.shape[-1])
    if X.dtype == torch.float64:
        return torch_backward(dY2, X2, e2, g2, *params, activation=activation)
    return mlp_backward(dY2, X2, e2, g2, *params, aux=aux, activation=activation)


def stack_lora_a(A_gate: torch.Tensor, A_up: torch.Tensor) -> torch.Tensor:
    """cat([A_gate, A_up]) [2r, H] (v6 :262-276; kept for API parity — the
    HIP path reads the two A matrices directly)."""
    return torch.cat([A_gate, A_up], dim=0).contiguous()


def stack_gate_lora_a(W_gate, A_gate, A_up):
    """cat([W_gate, A_gate, A_up]) [I+2r, H] (v6 :279-294; API parity)."""
    return torch.cat([W_gate, A_gate, A_up], dim=0).contiguous()


def stack_down_lora_a(W_down, A_down):
    """cat([W_down, A_down]) [H+r, I] (v6 :297-309; API parity)."""
    return torch.cat([W_down, A_down], dim=0).contiguous()


def fused_lora_a_stacked(X: torch.Tensor, A_stack: torch.Tensor, r: int) -> Tuple[torch.Tensor, torch.Tensor]:
    """X @ A_stack^T -> (xa_gate, xa_up) views of one [M, 2r] buffer (v6 :312-330)."""
    if X.dtype in G.GENERIC_DTYPES:
        out = G.gmm(X.reshape(-1, X.shape[-1]), A_stack[:2 * r].t())
        return out[:, :r], out[:, r:2 * r]
    X2 = as_operand(X.reshape(-1, X.shape[-1]))
    out = lora_a(X2, [A_stack[:r], A_stack[r:2 * r]], [1.0, 1.0])
    return out[:, :r], out[:, r:2 * r]


def fused_lora_swiglu(e_base, g_base, xa_gate, xa_up, B_gate, B_up, s_gate=1.0, s_up=1.0, save_eg=False,
                      inplace=False):
    """h = silu(e_base + sg xa_g Bg^T) * (g_base + su xa_u Bu^T)
    (v3 `fused_lora_swiglu` :141-200; v6 in-place variant :81-151 with
    inplace=True writes e_full/g_full over e_base/g_base).
    The rank-r update is one K-segment GEMM with beta=1 over the base tensor;
    the SwiGLU is the HIP SwiGLU kernel."""
    from kernels.swiglu import swiglu_forward

    M, N = e_base.shape
    if xa_gate is not None:
        e_full = e_base if inplace else e_base.clone()
        g_full = g_base if inplace else g_base.clone()
        r = xa_gate.shape[1]
        if e_full.dtype in G.GENERIC_DTYPES:
            G.check_dtypes("fused_lora_swiglu", e_full, g_full, xa_gate, xa_up, B_gate, B_up)
            G.gmm(xa_gate, B_gate.t(), out=e_full, alpha=s_gate, beta=1.0)
            G.gmm(xa_up, B_up.t(), out=g_full, alpha=s_up, beta=1.0)
        else:
            xg, xu = as_operand(xa_gate), as_operand(xa_up)
            Bg, Bu = _w(B_gate), _w(B_up)
            gemm(M, N, [(xg, ld(xg), Bg, ld(Bg), r)], ROW, COL, out=e_full, alpha=s_gate, beta=1.0)
            gemm(M, N, [(xu, ld(xu), Bu, ld(Bu), r)], ROW, COL, out=g_full, alpha=s_up, beta=1.0)
    else:
        e_full, g_full = e_base, g_base
    h = swiglu_forward(e_full, g_full)[0]
    if save_eg:
        return h, e_full, g_full
    return h, None, None
