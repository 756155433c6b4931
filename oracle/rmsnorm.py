"""RMSNorm oracle (test infrastructure only; see oracle/__init__.py).

Restates the reference's RMSNorm (kernels/rmsnorm/forge_rmsnorm_v2.py:248-276
forward per casting mode, the v2-v4 backward kernel formula
forge_rmsnorm_v4.py:131-184, and v1, forge_rmsnorm_v1.py:32-113) on the CPU:
  rstd = rsqrt(mean(x^2) + eps)                     (float64 here)
  llama: y = (x rstd).to(dtype) * (w + offset)      (product rounded to y's dtype)
  gemma: y = ((x rstd) * (w + offset)).to(dtype)
  none:  y = (x * rstd.to(dtype)).to(dtype) * (w + offset)
  backward (every mode): s = dy (w + offset), dot = sum(s x),
           dx = rstd (s - x rstd^2 dot / H), dw = sum_rows dy x rstd.
"""
from __future__ import annotations

import torch

LLAMA, GEMMA, NONE = 0, 1, 2


def _r(v, dtype):
    return v.to(dtype).to(torch.float64)


def rms_forward(x, w, eps=1e-6, offset=0.0, mode=LLAMA, out_dtype=None):
    """-> (y in out_dtype (default x's), rstd float64 [rows])."""
    dt = x.dtype
    od = out_dtype or dt
    xd = x.detach().cpu().to(torch.float64)
    wd = w.detach().cpu().to(torch.float64)
    rstd = torch.rsqrt(xd.pow(2).mean(-1, keepdim=True) + eps)
    if mode == GEMMA:
        y = (xd * rstd) * (wd + offset)
    else:
        wo = _r(wd + offset, w.dtype)
        if mode == LLAMA:
            y = _r(xd * rstd, dt) * wo
        else:
            y = _r(xd * _r(rstd, dt), dt) * wo
    return y.to(od), rstd.squeeze(-1)


def rms_backward(dy, x, w, offset=0.0, eps=1e-6):
    """-> (dx, dw) float64, the v2-v4 kernel formula with rstd from x."""
    xd = x.detach().cpu().to(torch.float64)
    wd = w.detach().cpu().to(torch.float64)
    d = dy.detach().cpu().to(torch.float64).reshape(xd.shape)
    H = xd.shape[-1]
    rstd = torch.rsqrt(xd.pow(2).mean(-1, keepdim=True) + eps)
    s = d * (wd + offset)
    dot = (s * xd).sum(-1, keepdim=True)
    dx = rstd * (s - xd * rstd * rstd * dot / H)
    dw = (d * xd * rstd).reshape(-1, H).sum(0)
    return dx, dw


def bytes_fwd_bwd(rows: int, cols: int, elem: int = 2) -> int:
    """Algorithmic HBM bytes of one forward + backward with weight gradient:
    forward reads x and writes y; backward reads x and dy and writes dx;
    plus rstd (4 B/row, written and read) and the weight (read twice,
    dw written)."""
    return 5 * rows * cols * elem + 8 * rows + 3 * cols * elem
