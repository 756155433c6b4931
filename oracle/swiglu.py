"""SwiGLU oracle (test infrastructure only; see oracle/__init__.py).

Restates `torch_swiglu_reference` / `torch_swiglu_packed_reference`
(kernels/swiglu/swiglu.py:179-198): s = silu(gate.float() * gm).to(dtype);
out = (s * up) * dm, each product materialised in the input dtype.  The
backward is PyTorch autograd of that graph.
"""
from __future__ import annotations

import torch


def swiglu_ref(gate: torch.Tensor, up: torch.Tensor, gate_multiplier: float = 1.0,
               down_multiplier: float = 1.0) -> torch.Tensor:
    """kernels/swiglu/swiglu.py:179-188."""
    silu_gate = torch.nn.functional.silu(gate.float() * float(gate_multiplier)).to(dtype=gate.dtype)
    return (silu_gate * up) * float(down_multiplier)


def swiglu_packed_ref(gate_up: torch.Tensor, gate_multiplier: float = 1.0,
                      down_multiplier: float = 1.0) -> torch.Tensor:
    """kernels/swiglu/swiglu.py:191-198."""
    gate, up = gate_up.chunk(2, dim=-1)
    return swiglu_ref(gate, up, gate_multiplier, down_multiplier)


def swiglu_fwd_bwd(gate, up, dout, gate_multiplier=1.0, down_multiplier=1.0):
    """Forward output and (dgate, dup) by autograd, on CPU."""
    g = gate.detach().cpu().clone().requires_grad_(True)
    u = up.detach().cpu().clone().requires_grad_(True)
    out = swiglu_ref(g, u, gate_multiplier, down_multiplier)
    out.backward(dout.detach().cpu())
    return out.detach(), g.grad, u.grad


def swiglu_packed_fwd_bwd(gate_up, dout, gate_multiplier=1.0, down_multiplier=1.0):
    gu = gate_up.detach().cpu().clone().requires_grad_(True)
    out = swiglu_packed_ref(gu, gate_multiplier, down_multiplier)
    out.backward(dout.detach().cpu())
    return out.detach(), gu.grad
