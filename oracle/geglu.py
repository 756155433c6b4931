"""GeGLU oracle (test infrastructure only; see oracle/__init__.py).

Restates the reference's GeGLU (kernels/geglu/geglu.py) on the CPU:
  forward  out = gelu(gate.float()).to(dtype) * up       (:255-263, :126-148)
  backward dup = dout * gelu(gate).to(dtype),
           dgate = dout * up * gelu'(gate)                (:104-123, :151-182)
with GELU in its tanh form or exact (erf), written out from the formulas,
every intermediate in float64 and one rounding to the storage dtype where
the reference materialises a tensor.
"""
from __future__ import annotations

import math

import torch

SQRT_2_OVER_PI = math.sqrt(2.0 / math.pi)
GELU_CUBIC = 0.044715


def gelu_and_grad(x: torch.Tensor, approximate: str):
    """(gelu(x), gelu'(x)) in float64."""
    x = x.to(torch.float64)
    if approximate == "tanh":
        t = torch.tanh(SQRT_2_OVER_PI * (x + GELU_CUBIC * x ** 3))
        act = 0.5 * x * (1 + t)
        grad = 0.5 * (1 + t) + 0.5 * x * (1 - t * t) * SQRT_2_OVER_PI * (1 + 3 * GELU_CUBIC * x * x)
    else:
        cdf = 0.5 * (1 + torch.erf(x / math.sqrt(2.0)))
        act = x * cdf
        grad = cdf + x * torch.exp(-0.5 * x * x) / math.sqrt(2 * math.pi)
    return act, grad


def geglu_fwd_bwd(gate, up, dout=None, approximate: str = "tanh"):
    """Returns (out, dgate, dup) in gate's dtype (dgate/dup None without dout)."""
    dt = gate.dtype
    g, u = gate.detach().cpu(), up.detach().cpu()
    act, grad = gelu_and_grad(g, approximate)
    act_r = act.to(dt).to(torch.float64)
    out = (act_r * u.to(torch.float64)).to(dt)
    if dout is None:
        return out, None, None
    d = dout.detach().cpu().to(torch.float64)
    dup = (d * act_r).to(dt)
    dgate = (d * u.to(torch.float64) * grad).to(dt)
    return out, dgate, dup
