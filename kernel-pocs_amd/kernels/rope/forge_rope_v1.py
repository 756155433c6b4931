"""RoPE v1 API on MI355X.

Drop-in for kernels/rope/forge_rope_v1.py of Forge-researchlab/kernel-POCs:
`ForgeRoPEv1Function` (forward(ctx, q, k, cos, sin) with the reference's
messaged asserts, `ctx.save_for_backward(cos, sin)`, out-of-place outputs,
backward = rotation by -theta), `apply_rope` and `ForgeRoPEv1`.  The rotation
is the same `forge_rope` kernel as v3 (csrc/rope.hip): the reference's v1,
v2 and v3 differ only in how their Triton grids cover the heads, not in the
values, so one HIP kernel serves all three.

v1 has no `n_q % n_kv == 0` requirement (reference :98-124, its grid
rotates K head i in the program of Q head i): any n_kv <= n_q is rotated
here as well.  Unlike the reference's grid, K heads beyond n_q are rotated
too instead of being left unwritten.
"""
from __future__ import annotations

import torch

from kernels.rope.forge_rope_v3 import _rope_backward, rope_forward_checked


def _check_v1_shapes(q, k, cos, sin):
    """kernels/rope/forge_rope_v1.py:131-150 (message texts kept)."""
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
        f"cos shape {tuple(cos.shape)} mismatch (expected (.,{seq_len},{head_dim}))"
    assert sin.shape == cos.shape, \
        f"sin {tuple(sin.shape)} / cos {tuple(cos.shape)} shape mismatch"
    assert head_dim & (head_dim - 1) == 0, f"head_dim must be a power of 2, got {head_dim}"


class ForgeRoPEv1Function(torch.autograd.Function):
    """kernels/rope/forge_rope_v1.py:127-174."""

    @staticmethod
    def forward(ctx, q, k, cos, sin):
        _check_v1_shapes(q, k, cos, sin)
        return rope_forward_checked(ctx, q, k, cos, sin, None, divisible_msg=None)

    @staticmethod
    def backward(ctx, dq, dk):
        dq_in, dk_in = _rope_backward(ctx, dq, dk)
        return dq_in, dk_in, None, None


def apply_rope(q: torch.Tensor, k: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor):
    """kernels/rope/forge_rope_v1.py:177-190."""
    return ForgeRoPEv1Function.apply(q, k, cos, sin)


class ForgeRoPEv1(torch.nn.Module):
    """kernels/rope/forge_rope_v1.py:193-204."""

    def __init__(self):
        super().__init__()

    def forward(self, q, k, cos, sin):
        return apply_rope(q, k, cos, sin)


__all__ = ["apply_rope", "ForgeRoPEv1Function", "ForgeRoPEv1"]
