"""RoPE oracle (test infrastructure only; see oracle/__init__.py).

Restates the HF formula the reference tests RoPE against
(kernels/rope/tests/test_v1.py:49-61): out = x*cos + rotate_half(x)*sin,
evaluated in fp32 and cast back, and the cos/sin builder with a configurable
base (kernels/rope/tests/test_v1.py:68-88).
"""
from __future__ import annotations

import torch


def rotate_half(x: torch.Tensor) -> torch.Tensor:
    """kernels/rope/tests/test_v1.py:49-52."""
    x1 = x[..., : x.shape[-1] // 2]
    x2 = x[..., x.shape[-1] // 2:]
    return torch.cat((-x2, x1), dim=-1)


def hf_apply_rotary_pos_emb(q, k, cos, sin, unsqueeze_dim=1):
    """kernels/rope/tests/test_v1.py:55-61 (q/k (B, H, S, D), cos/sin (B|1, S, D))."""
    cos_u = cos.unsqueeze(unsqueeze_dim)
    sin_u = sin.unsqueeze(unsqueeze_dim)
    return (q * cos_u) + (rotate_half(q) * sin_u), (k * cos_u) + (rotate_half(k) * sin_u)


def cos_sin(positions: torch.Tensor, head_dim: int, base: float, dtype: torch.dtype):
    """kernels/rope/tests/test_v1.py:75-83 for arbitrary (varlen) positions."""
    inv_freq = 1.0 / (base ** (torch.arange(0, head_dim, 2).float() / head_dim))
    freqs = positions.float().unsqueeze(1) * inv_freq.unsqueeze(0)
    emb = torch.cat([freqs, freqs], dim=-1)
    return emb.cos().to(dtype), emb.sin().to(dtype)


def rope_fwd_bwd(q, k, cos, sin, dq_out, dk_out):
    """fp32 forward and autograd backward on CPU; returns values cast to q.dtype
    (the kernel's output dtype) plus the fp32 results."""
    dtype = q.dtype
    qf = q.detach().cpu().float().requires_grad_(True)
    kf = k.detach().cpu().float().requires_grad_(True)
    oq, ok = hf_apply_rotary_pos_emb(qf, kf, cos.detach().cpu().float(), sin.detach().cpu().float())
    (oq * dq_out.detach().cpu().float()).sum().add((ok * dk_out.detach().cpu().float()).sum()).backward()
    return oq.detach().to(dtype), ok.detach().to(dtype), qf.grad.to(dtype), kf.grad.to(dtype)
