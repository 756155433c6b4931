"""Fused Q+K rotary embedding with GQA grouping on MI355X.

Drop-in for kernels/rope/forge_rope_v3.py of Forge-researchlab/kernel-POCs:
`ForgeRoPEv3Function` (same asserts, same `ctx.save_for_backward(cos, sin)`,
backward = rotation by -theta), `apply_rope`, `ForgeRoPEv3` and
`get_autotune_cache_for`.  The rotation runs in `forge_rope`
(libforge_hip.so, csrc/rope.hip).

Differences that keep values identical:
  * Inputs with any (batch, head, seq) strides are rotated in place of memory
    order, so HF's `transpose(1, 2)` view of a [B, S, H, D] projection costs
    no `.contiguous()` copy (reference :179-180 copies).  Outputs are allocated
    with `torch.empty_like`, i.e. in the input's memory layout.
  * `apply_rope(..., positions=...)` (optional, int64 [B*S] or [B, S]) selects
    the cos/sin row per token, for packed variable-length sequences; every
    position must lie in [0, cos.shape[-2]) (IndexError otherwise).
  * cos/sin are read as stored: a table in q's dtype or in fp32 goes to the
    kernel unchanged (fp32 math either way, as the reference kernel loads
    the table and computes in fp32); another table dtype is widened to fp32,
    which is exact.
"""
from __future__ import annotations

import math
from typing import Optional

import torch

from forge_hip import _lib as L
from kernels._positions import check_positions

# launch geometry of csrc/rope.hip (fixed; there is no autotuning)
_BLOCK = 256
_HEADS_PER_ITEM = 1


_V3_DIVISIBLE = "V3 requires n_q % n_kv == 0 (got n_q={n_q}, n_kv={n_kv})."


def _rope_launch(q_in, k_in, q_out, k_out, cos, sin, backward_pass: bool, positions=None,
                 divisible_msg=_V3_DIVISIBLE):
    """Replaces `_launch_kernel` (kernels/rope/forge_rope_v3.py:99-132; v2's
    forge_rope_v2.py:103-136 with its own message; v1's forge_rope_v1.py:
    98-124 has no divisibility check)."""
    batch, n_q, seq_len, head_dim = q_in.shape
    n_kv = k_in.shape[1]
    if divisible_msg is not None:
        assert n_q % n_kv == 0, divisible_msg.format(n_q=n_q, n_kv=n_kv)
    L.require_gpu(q_in, k_in, cos, sin)

    # one stride() tuple per tensor: the launch sits on the host's per-step path
    qs, ks, qos, kos, cs, ss = (t.stride() for t in (q_in, k_in, q_out, k_out, cos, sin))
    cos_has_batch = cos.shape[0] == batch
    cos_sb = cs[0] if cos_has_batch else 0
    sin_sb = ss[0] if cos_has_batch else 0
    pos = None
    if positions is not None:
        pos = positions.reshape(-1).to(device=q_in.device, dtype=torch.int64).contiguous()
        assert pos.numel() == batch * seq_len, "positions must have batch*seq_len entries"
    L.check(
        L.forge_rope(
            L.dtype_code(q_in.dtype),
            q_in.data_ptr(), qs[0], qs[1], qs[2],
            k_in.data_ptr(), ks[0], ks[1], ks[2],
            q_out.data_ptr(), qos[0], qos[1], qos[2],
            k_out.data_ptr(), kos[0], kos[1], kos[2],
            cos.data_ptr(), cos_sb, cs[1],
            sin.data_ptr(), sin_sb, ss[1],
            L.dtype_code(cos.dtype), cos.shape[1],
            None if pos is None else pos.data_ptr(),
            batch, n_q, n_kv, seq_len, head_dim, 1 if backward_pass else 0,
            L.stream_of(q_in),
        ),
        "forge_rope",
    )
    return pos


def _unit_last(t: torch.Tensor) -> torch.Tensor:
    return t if t.stride(-1) == 1 else t.contiguous()


def _cos_sin_like(cos: torch.Tensor, q: torch.Tensor) -> torch.Tensor:
    # the reference kernel reads cos/sin as stored and computes in fp32: a
    # table in q's dtype or fp32 is passed as is, any other is widened to
    # fp32 (exact for bf16 / fp16; float64 rounds as the reference's load does)
    if cos.dtype not in (q.dtype, torch.float32):
        cos = cos.to(torch.float32)
    return _unit_last(cos)


def _tables(cos: torch.Tensor, sin: torch.Tensor, q: torch.Tensor):
    cos, sin = _cos_sin_like(cos, q), _cos_sin_like(sin, q)
    if cos.dtype != sin.dtype:  # the kernel reads both tables in one dtype
        cos, sin = cos.float(), sin.float()
    return cos, sin


def get_autotune_cache_for(q, k, cos, sin, backward_pass: bool = False):
    """Diagnostic of kernels/rope/forge_rope_v3.py:135-158.  The HIP kernel has
    one fixed launch shape, reported here in the same dict form."""
    batch, n_q, seq_len, head_dim = q.shape
    n_kv = k.shape[1]
    chunk = 16 // q.element_size()
    items = batch * seq_len * math.ceil((head_dim // 2) / chunk) * math.ceil((n_q + n_kv) / _HEADS_PER_ITEM)
    return {
        "num_warps": _BLOCK // 64,
        "num_stages": 1,
        "all_kwargs": {"block": _BLOCK, "heads_per_item": _HEADS_PER_ITEM, "work_items": items},
    }


def _rope_forward(ctx, q, k, cos, sin, positions):
    """v3's checks (kernels/rope/forge_rope_v3.py:165-176), then the launch."""
    assert q.dim() == 4
    assert k.dim() == 4
    assert cos.dim() == 3 and sin.dim() == 3

    batch, n_q, seq_len, head_dim = q.shape
    n_kv = k.shape[1]

    assert k.shape == (batch, n_kv, seq_len, head_dim)
    assert cos.shape[0] in (1, batch)
    if positions is None:
        assert cos.shape[1] == seq_len and cos.shape[2] == head_dim
    else:
        assert cos.shape[2] == head_dim
    assert sin.shape == cos.shape
    assert head_dim & (head_dim - 1) == 0
    if positions is not None:
        check_positions(positions, cos.shape[1])
    return rope_forward_checked(ctx, q, k, cos, sin, positions, _V3_DIVISIBLE)


def rope_forward_checked(ctx, q, k, cos, sin, positions=None, divisible_msg=_V3_DIVISIBLE):
    """The forward launch shared by the v1 / v2 / v3 Functions once their
    own shape checks have passed: out-of-place outputs in q/k's layout,
    (cos, sin) saved as given."""
    q = _unit_last(q)
    k = _unit_last(k)
    cos_t, sin_t = _tables(cos, sin, q)

    out_q = torch.empty_like(q)
    out_k = torch.empty_like(k)
    pos = _rope_launch(q, k, out_q, out_k, cos_t, sin_t, backward_pass=False, positions=positions,
                       divisible_msg=divisible_msg)
    ctx.save_for_backward(cos, sin)  # the caller's tables, as the reference saves them
    ctx.positions = pos
    ctx.divisible_msg = divisible_msg
    return out_q, out_k


def _rope_backward(ctx, dq, dk):
    cos, sin = ctx.saved_tensors
    dq = _unit_last(dq)
    dk = _unit_last(dk)
    cos, sin = _tables(cos, sin, dq)
    dq_in = torch.empty_like(dq)
    dk_in = torch.empty_like(dk)
    _rope_launch(dq, dk, dq_in, dk_in, cos, sin, backward_pass=True, positions=ctx.positions,
                 divisible_msg=getattr(ctx, "divisible_msg", _V3_DIVISIBLE))
    return dq_in, dk_in


class ForgeRoPEv3Function(torch.autograd.Function):
    """kernels/rope/forge_rope_v3.py:161-200: forward(ctx, q, k, cos, sin),
    saves (cos, sin), backward rotates the incoming grads by -theta."""

    @staticmethod
    def forward(ctx, q, k, cos, sin):
        return _rope_forward(ctx, q, k, cos, sin, None)

    @staticmethod
    def backward(ctx, dq, dk):
        dq_in, dk_in = _rope_backward(ctx, dq, dk)
        return dq_in, dk_in, None, None


class ForgeRoPEPositionsFunction(torch.autograd.Function):
    """Same as ForgeRoPEv3Function with a per-token cos/sin row index
    (int64 positions, B*S entries) for packed variable-length batches."""

    @staticmethod
    def forward(ctx, q, k, cos, sin, positions):
        return _rope_forward(ctx, q, k, cos, sin, positions)

    @staticmethod
    def backward(ctx, dq, dk):
        dq_in, dk_in = _rope_backward(ctx, dq, dk)
        return dq_in, dk_in, None, None, None


def apply_rope(q: torch.Tensor, k: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
               positions: Optional[torch.Tensor] = None):
    """kernels/rope/forge_rope_v3.py:203-210."""
    if positions is None:
        return ForgeRoPEv3Function.apply(q, k, cos, sin)
    return ForgeRoPEPositionsFunction.apply(q, k, cos, sin, positions)


class ForgeRoPEv3(torch.nn.Module):
    """kernels/rope/forge_rope_v3.py:213-218."""

    def __init__(self):
        super().__init__()

    def forward(self, q, k, cos, sin):
        return apply_rope(q, k, cos, sin)


def rope_cos_sin(positions: torch.Tensor, head_dim: int, base: float = 10000.0,
                 dtype: torch.dtype = torch.bfloat16):
    """cos/sin tables (len(positions), head_dim) for a configurable RoPE base,
    built as in kernels/rope/tests/test_v1.py:68-88 (and the HF rotary
    module): inv_freq = 1/base^(arange(0, D, 2)/D), freqs = pos*inv_freq in
    fp32, emb = cat(freqs, freqs), then cos/sin cast to dtype."""
    dev = positions.device
    inv_freq = 1.0 / (base ** (torch.arange(0, head_dim, 2, device=dev).float() / head_dim))
    freqs = positions.float().unsqueeze(1) * inv_freq.unsqueeze(0)
    emb = torch.cat([freqs, freqs], dim=-1)
    return emb.cos().to(dtype), emb.sin().to(dtype)


__all__ = ["apply_rope", "ForgeRoPEv3Function", "ForgeRoPEPositionsFunction", "ForgeRoPEv3", "get_autotune_cache_for",
           "rope_cos_sin"]
