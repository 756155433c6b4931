"""RoPE v2 API on MI355X.

Drop-in for kernels/rope/forge_rope_v2.py of Forge-researchlab/kernel-POCs:
`ForgeRoPEv2Function` (the reference's messaged asserts and its
"V2 requires n_q % n_kv == 0" check, `ctx.save_for_backward(cos, sin)`,
out-of-place outputs, backward = rotation by -theta), `apply_rope` and
`ForgeRoPEv2`.  The reference's v2 groups G = n_q / n_kv Q heads with their
K head per Triton program; the HIP kernel (`forge_rope`, csrc/rope.hip)
groups heads by four per work item for every version, with identical values.
"""
from __future__ import annotations

import torch

from kernels.rope.forge_rope_v3 import _rope_backward, rope_forward_checked

_V2_DIVISIBLE = ("V2 requires n_q % n_kv == 0 (got n_q={n_q}, n_kv={n_kv}). "
                 "Use V1 for non-divisible cases.")


def _check_v2_shapes(q, k, cos, sin):
    """kernels/rope/forge_rope_v2.py:143-160 (message texts kept)."""
    assert q.dim() == 4, f"q must be 4D, got shape {tuple(q.shape)}"
    assert k.dim() == 4, f"k must be 4D, got shape {tuple(k.shape)}"
    assert cos.dim() == 3, f"cos must be 3D, got shape {tuple(cos.shape)}"
    assert sin.dim() == 3, f"sin must be 3D, got shape {tuple(sin.shape)}"

    batch, n_q, seq_len, head_dim = q.shape
    n_kv = k.shape[1]

    assert k.shape == (batch, n_kv, seq_len, head_dim), f"k shape {tuple(k.shape)} mismatch"
    assert cos.shape[0] in (1, batch), \
        f"cos.shape[0] must be 1 or batch={batch}, got {cos.shape[0]}"
    assert cos.shape[1] == seq_len and cos.shape[2] == head_dim, \
        f"cos shape {tuple(cos.shape)} mismatch"
    assert sin.shape == cos.shape, \
        f"sin/cos shape mismatch: {tuple(sin.shape)} vs {tuple(cos.shape)}"
    assert head_dim & (head_dim - 1) == 0, f"head_dim must be a power of 2, got {head_dim}"


class ForgeRoPEv2Function(torch.autograd.Function):
    """kernels/rope/forge_rope_v2.py:139-183."""

    @staticmethod
    def forward(ctx, q, k, cos, sin):
        _check_v2_shapes(q, k, cos, sin)
        return rope_forward_checked(ctx, q, k, cos, sin, None, divisible_msg=_V2_DIVISIBLE)

    @staticmethod
    def backward(ctx, dq, dk):
        dq_in, dk_in = _rope_backward(ctx, dq, dk)
        return dq_in, dk_in, None, None


def apply_rope(q: torch.Tensor, k: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor):
    """kernels/rope/forge_rope_v2.py:186-199."""
    return ForgeRoPEv2Function.apply(q, k, cos, sin)


class ForgeRoPEv2(torch.nn.Module):
    """kernels/rope/forge_rope_v2.py:202-209."""

    def __init__(self):
        super().__init__()

    def forward(self, q, k, cos, sin):
        return apply_rope(q, k, cos, sin)


__all__ = ["apply_rope", "ForgeRoPEv2Function", "ForgeRoPEv2"]
