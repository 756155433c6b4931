"""Fused LoRA-GeGLU MLP (LoRAMLPGeGLU: the LoRA-MLP pipeline with the GeGLU
epilogues, for Gemma MLPs) vs the CPU oracle: oracle/lora_mlp.py with a GELU
activation restates the reference's Gemma composition
(forge/forge/patching/kernels/lora.py:170-188: PEFT projections around
kernels/geglu/geglu.py's geglu), fp32 on the same bf16 values.

Tolerance as for the SwiGLU LoRA-MLP (_parity.close_bf16: 2e-2 relative and
2e-2 of the tensor's rms, cosine > 0.9999).  The GeGLU epilogues evaluate the
standalone GeGLU kernel's math on the bf16 e, g and round(DW), so they are
also checked bit for bit against forge_geglu_fwd / forge_geglu_bwd on the
same tensors (and the GEMM part against forge_gemm on the same operands).
"""
import pytest
import torch

from _parity import close_bf16
from oracle import lora_mlp as orc

NAMES = ["dX", "dA_gate", "dB_gate", "dA_up", "dB_up", "dA_down", "dB_down"]
ACT = {"tanh": "gelu_tanh", "none": "gelu_exact"}


def _params_cuda(params):
    return [t.cuda().requires_grad_(t.shape[0] <= 64 or t.shape[1] <= 64) if isinstance(t, torch.Tensor) else t
            for t in params]


def _run(approximate, X, dY, params):
    from kernels.lora_mlp.geglu_mlp import LoRAMLPGeGLU

    p = _params_cuda(params)
    x = X.cuda().requires_grad_(True)
    out = LoRAMLPGeGLU.apply(x, *p, approximate)
    out.backward(dY.cuda())
    lora = [p[1], p[2], p[5], p[6], p[9], p[10]]
    return out, [x.grad] + [t.grad for t in lora]


@pytest.mark.gpu
@pytest.mark.parametrize("B,S,H,I,r,alpha,xscale", [(2, 128, 512, 1024, 16, 32, 1.0), (1, 200, 256, 768, 8, 16, 1.0),
                                                     (1, 333, 640, 2304, 32, 64, 4.0)])
@pytest.mark.parametrize("approximate", ["tanh", "none"])
def test_lora_mlp_geglu_matches_oracle(B, S, H, I, r, alpha, xscale, approximate):
    gen = torch.Generator().manual_seed(B * S + H + r)
    params = orc.make_params(H, I, r, alpha, gen)
    X = (torch.randn(B, S, H, generator=gen) * xscale).to(torch.bfloat16)
    dY = torch.randn(B, S, H, generator=gen).to(torch.bfloat16)
    ref_out, ref_grads = orc.fwd_bwd(X, dY, params, activation=ACT[approximate])
    print(f"lora_mlp_geglu B={B} S={S} H={H} I={I} r={r} approximate={approximate}", flush=True)
    out, grads = _run(approximate, X, dY, params)
    assert out.shape == (B, S, H) and out.dtype == torch.bfloat16
    close_bf16(out.reshape(-1, H), ref_out, "out")
    for n, a, b in zip(NAMES, grads, ref_grads):
        close_bf16(a.reshape(b.shape), b, n)


@pytest.mark.gpu
@pytest.mark.parametrize("approximate", ["tanh", "none"])
@pytest.mark.parametrize("M,w_layout", [(512, "row"), (333, "row"), (333, "col")])
def test_geglu_epilogues_match_the_geglu_kernel(approximate, M, w_layout):
    """forge_lora_mlp_gate_up's h is forge_geglu_fwd(e, g) on its own stored
    e, g; forge_lora_mlp_down_bwd's (h, d up, d gate) are forge_geglu_fwd and
    forge_geglu_bwd(DW, e, g) with DW the same GEMM through forge_gemm."""
    from forge_hip import _lib as L
    from kernels._lora_ops import COL, ROW, gemm

    torch.manual_seed(M)
    H, I, r = 512, 1280, 16
    tanh = 1 if approximate == "tanh" else 0
    act = L.ACT_GELU_TANH if tanh else L.ACT_GELU_ERF
    bf = dict(device="cuda", dtype=torch.bfloat16)
    X = torch.randn(M, H, **bf) * 2
    Wg, Wu = torch.randn(I, H, **bf) * 0.05, torch.randn(I, H, **bf) * 0.05
    xa = torch.randn(M, 2 * r, **bf)
    Bg, Bu = torch.randn(I, r, **bf) * 0.1, torch.randn(I, r, **bf) * 0.1
    e, g, h = (torch.empty(M, I, **bf) for _ in range(3))
    st = L.stream_of(X)
    print(f"gate_up geglu M={M} approximate={approximate}", flush=True)
    L.check(L.forge_lora_mlp_gate_up(M, H, I, r, X.data_ptr(), H, Wg.data_ptr(), Wu.data_ptr(), H, xa.data_ptr(),
                                     2 * r, Bg.data_ptr(), Bu.data_ptr(), r, e.data_ptr(), g.data_ptr(), h.data_ptr(),
                                     I, act, st), "forge_lora_mlp_gate_up")
    h_ref = torch.empty_like(h)
    L.check(L.forge_geglu_fwd(L.DTYPE_BF16, e.data_ptr(), g.data_ptr(), I, h_ref.data_ptr(), I, M, I, tanh, st),
            "forge_geglu_fwd")
    assert torch.equal(h, h_ref)
    assert e.float().min() < -2 and e.float().max() > 2  # the GELU's tails and its zero-crossing derivative

    dY = torch.randn(M, H, **bf)
    Wd = torch.randn(H, I, **bf) * 0.05
    td = torch.randn(M, r, **bf)
    Ad = torch.randn(r, I, **bf) * 0.1
    if w_layout == "row":
        Wop, Aop, wl = Wd, Ad, ROW
    else:
        Wop, Aop, wl = Wd.t().contiguous(), Ad.t().contiguous(), COL
    DW = gemm(M, I, [(dY, H, Wop, Wop.stride(0), H), (td, r, Aop, Aop.stride(0), r)], ROW, wl)
    e0, g0 = e.clone(), g.clone()
    h_out = torch.empty_like(h)
    print(f"down_bwd geglu M={M} layout={w_layout} approximate={approximate}", flush=True)
    L.check(L.forge_lora_mlp_down_bwd(M, H, I, r, dY.data_ptr(), H, Wop.data_ptr(), Wop.stride(0), td.data_ptr(), r,
                                      Aop.data_ptr(), Aop.stride(0), wl, h_out.data_ptr(), e.data_ptr(), g.data_ptr(),
                                      I, act, st), "forge_lora_mlp_down_bwd")
    dgate, dup = torch.empty_like(h), torch.empty_like(h)
    L.check(L.forge_geglu_bwd(L.DTYPE_BF16, DW.data_ptr(), I, e0.data_ptr(), g0.data_ptr(), I, dgate.data_ptr(),
                              dup.data_ptr(), I, M, I, tanh, st), "forge_geglu_bwd")
    torch.cuda.synchronize()
    assert torch.equal(h_out, h)
    assert torch.equal(e, dup)
    assert torch.equal(g, dgate)


@pytest.mark.gpu
def test_lora_mlp_geglu_forward_only_and_saved_tensors():
    """lora_mlp_geglu (no autograd) matches the autograd forward; the saved
    e / g are the pre-activations with the LoRA terms added."""
    from kernels.lora_mlp.geglu_mlp import LoRAMLPGeGLU, lora_mlp_geglu

    gen = torch.Generator().manual_seed(8)
    H, I, r = 256, 512, 16
    params = orc.make_params(H, I, r, 32, gen)
    X = torch.randn(1, 64, H, generator=gen).to(torch.bfloat16)
    p = _params_cuda(params)
    x = X.cuda().requires_grad_(True)
    out = LoRAMLPGeGLU.apply(x, *p, "none")
    saved = out.grad_fn.saved_tensors
    assert len(saved) == 9 and saved[6].data_ptr() == x.data_ptr()
    pf = [t.float() if isinstance(t, torch.Tensor) else t for t in params]
    ref_out, e_ref, g_ref = orc.forward(X.float().reshape(-1, H), *pf, activation="gelu_exact")
    close_bf16(saved[7].reshape(-1, I), e_ref, "e")
    close_bf16(saved[8].reshape(-1, I), g_ref, "g")
    with torch.no_grad():
        assert torch.equal(lora_mlp_geglu(X.cuda(), *[t.detach() if isinstance(t, torch.Tensor) else t for t in p],
                                          approximate="none"), out.detach())
    with pytest.raises(ValueError, match="approximate"):
        lora_mlp_geglu(X.cuda(), *p, approximate="erf")


def test_lora_mlp_geglu_float64_gradcheck():
    """float64 inputs take the plain-PyTorch formulas (CPU here): the
    hand-written GELU backward against finite differences."""
    from kernels.lora_mlp.geglu_mlp import LoRAMLPGeGLU

    gen = torch.Generator().manual_seed(5)
    H, I, r = 8, 12, 2
    params = [t.double() if isinstance(t, torch.Tensor) else t for t in orc.make_params(H, I, r, 4, gen)]
    for i in (2, 6, 10):  # O(1) LoRA terms, so a wrong LoRA gradient shows
        params[i] = params[i] * 50
    for i in (1, 2, 5, 6, 9, 10):
        params[i].requires_grad_(True)
    X = torch.randn(1, 3, H, dtype=torch.float64, generator=gen, requires_grad=True)
    for approximate in ("tanh", "none"):
        assert torch.autograd.gradcheck(lambda x, *lp: LoRAMLPGeGLU.apply(
            x, params[0], lp[0], lp[1], params[3], params[4], lp[2], lp[3], params[7], params[8], lp[4], lp[5],
            params[11], approximate), (X, params[1], params[2], params[5], params[6], params[9], params[10]))
