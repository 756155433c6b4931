"""LoRA-MLP oracle (test infrastructure only; see oracle/__init__.py).

Restates `matmul_lora`, `lora_swiglu_mlp` and `LoRAMLP`
(kernels/lora_mlp/reference/lora_mlp_pytorch.py:23-225): per projection
XW^T + s (X A^T) B^T, h = silu(e) * g, and the reference's hand-written
backward (:145-225), evaluated on the CPU in the given compute dtype.

activation="gelu_tanh" / "gelu_exact" restates the reference's Gemma MLP
(forge/forge/patching/kernels/lora.py:170-188: PEFT projections, each
XW^T + s (X A^T) B^T, around geglu(gate, up), kernels/geglu/geglu.py): h =
gelu(e) g, and the backward with silu(e), silu'(e) replaced by gelu(e),
gelu'(e) (GELU from oracle.geglu.gelu_and_grad, in float64, cast to the
compute dtype).
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

from oracle.geglu import gelu_and_grad

ACTIVATIONS = ("silu", "gelu_tanh", "gelu_exact")


def _gelu(e, activation):
    act, grad = gelu_and_grad(e, "tanh" if activation == "gelu_tanh" else "none")
    return act.to(e.dtype), grad.to(e.dtype)


def matmul_lora(X, W, A, B, s):
    """lora_mlp_pytorch.py:23-55 (2-D X)."""
    out = X @ W.t()
    if A is not None and B is not None:
        out = out + s * ((X @ A.t()) @ B.t())
    return out


def forward(X, W_gate, A_gate, B_gate, s_gate, W_up, A_up, B_up, s_up, W_down, A_down, B_down, s_down,
            activation="silu"):
    """lora_mlp_pytorch.py:100-104 -> (out, e, g); GELU: lora.py:184-188."""
    assert activation in ACTIVATIONS, activation
    e = matmul_lora(X, W_gate, A_gate, B_gate, s_gate)
    g = matmul_lora(X, W_up, A_up, B_up, s_up)
    h = (F.silu(e) if activation == "silu" else _gelu(e, activation)[0]) * g
    return matmul_lora(h, W_down, A_down, B_down, s_down), e, g


def backward(dY, X, e, g, W_gate, A_gate, B_gate, s_gate, W_up, A_up, B_up, s_up, W_down, A_down, B_down, s_down,
             activation="silu"):
    """lora_mlp_pytorch.py:153-225 -> (dX, dA_gate, dB_gate, dA_up, dB_up, dA_down, dB_down);
    GELU: the same chain with gelu(e), gelu'(e) (geglu.py:104-123)."""
    assert activation in ACTIVATIONS, activation
    if activation == "silu":
        sig_e = torch.sigmoid(e.float()).to(e.dtype)
        act_e = e * sig_e
        dact = sig_e * (1.0 + e * (1.0 - sig_e))
    else:
        act_e, dact = _gelu(e, activation)
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


def lora_grads(dY, X, W_gate, A_gate, B_gate, s_gate, W_up, A_up, B_up, s_up, W_down, A_down, B_down, s_down):
    """The LoRA-parameter part of `forward` + `backward` alone (SiLU,
    lora_mlp_pytorch.py:100-104, 153-211): (dA_gate, dB_gate, dA_up, dB_up,
    dA_down, dB_down).  It skips the output and dX products (two of the five
    [M, H] x [H, I]-sized products), so it runs over the BASELINE token count
    on the CPU."""
    e = matmul_lora(X, W_gate, A_gate, B_gate, s_gate)
    g = matmul_lora(X, W_up, A_up, B_up, s_up)
    sig_e = torch.sigmoid(e.float()).to(e.dtype)
    act_e = e * sig_e
    h = act_e * g
    dYB = dY @ B_down
    DW = dY @ W_down + s_down * (dYB @ A_down)
    d_downA = s_down * (dYB.t() @ h)
    d_downB = s_down * (dY.t() @ (h @ A_down.t()))
    del h
    df = DW * act_e
    de = DW * g * (sig_e * (1.0 + e * (1.0 - sig_e)))
    del DW, e, g, act_e, sig_e
    d_upA = s_up * ((df @ B_up).t() @ X)
    d_upB = s_up * (df.t() @ (X @ A_up.t()))
    d_gateA = s_gate * ((de @ B_gate).t() @ X)
    d_gateB = s_gate * (de.t() @ (X @ A_gate.t()))
    return d_gateA, d_gateB, d_upA, d_upB, d_downA, d_downB


def fwd_bwd(X, dY, params, compute_dtype=torch.float32, activation="silu"):
    """CPU forward + backward; params = (W_gate, A_gate, B_gate, s_gate, ...)."""
    c = lambda t: t.detach().cpu().to(compute_dtype) if isinstance(t, torch.Tensor) else t  # noqa: E731
    p = tuple(c(t) for t in params)
    X2 = c(X).reshape(-1, X.shape[-1])
    dY2 = c(dY).reshape(-1, dY.shape[-1])
    out, e, g = forward(X2, *p, activation=activation)
    grads = backward(dY2, X2, e, g, *p, activation=activation)
    return out, grads


def make_params(H, I, r, alpha, gen, dtype=torch.bfloat16):
    """BASELINE configs[3] initialisation: W ~ N(0, 0.02^2); A Kaiming-uniform
    U(+-1/sqrt(fan_in)) (PEFT default); B ~ N(0, 0.01^2); s = alpha / r."""
    s = alpha / r

    def W(o, i):
        return (torch.randn(o, i, generator=gen) * 0.02).to(dtype)

    def A(i):
        bound = 1.0 / i ** 0.5
        return ((torch.rand(r, i, generator=gen) * 2 - 1) * bound).to(dtype)

    def B(o):
        return (torch.randn(o, r, generator=gen) * 0.01).to(dtype)

    return (W(I, H), A(H), B(I), s, W(I, H), A(H), B(I), s, W(H, I), A(I), B(H), s)


def flops(M, H, I, r):
    """Algorithmic FLOPs of one forward + backward (2 per multiply-add), the
    accounting the published benchmark quotes (5,821,828,169,728 at M=8192, H=4096,
    I=14336, r=16):
      base GEMMs      forward 3 * 2MHI, backward 3 * 2MHI
      LoRA forward    X A^T and xa B^T for gate/up, h Ad^T and xd Bd^T = 6 M r (H + I)
      LoRA backward   with every rank-r product associated through the
                      [M, r] intermediates = M r (16 H + 14 I)"""
    return 12 * M * H * I + 6 * M * r * (H + I) + M * r * (16 * H + 14 * I)
