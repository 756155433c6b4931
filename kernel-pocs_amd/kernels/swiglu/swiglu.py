"""SwiGLU forward/backward on MI355X.

Drop-in for kernels/swiglu/swiglu.py of Forge-researchlab/kernel-POCs: the
same public functions, autograd Functions, argument validation (exception
types and messages) and `ctx.save_for_backward` contents.  The elementwise
work runs in `forge_swiglu_fwd` / `forge_swiglu_bwd` (libforge_hip.so,
csrc/swiglu.hip).

Contracts kept from the reference:
  * forward saves the flattened (gate, up) 2-D views (swiglu.py:336-337);
  * the default backward writes dgate/dup INTO those saved buffers, which
    alias the caller's inputs when they were contiguous; preserve_inputs=True
    allocates fresh gradient buffers (swiglu.py:247-248, 310);
  * `swiglu` on a tensor that is not on a GPU returns the module's own PyTorch
    formula `torch_swiglu_reference` (swiglu.py:396-397) — that is the
    reference API for CPU tensors; GPU tensors always take the HIP kernels.
"""
from __future__ import annotations

import numbers

import torch

from forge_hip import _lib as L

MAX_ROW_BLOCK_SIZE = 65536


def _as_float(name: str, value: float) -> float:
    """Scalar check of kernels/swiglu/swiglu.py:11-16."""
    if isinstance(value, torch.Tensor):
        raise TypeError(f"{name} must be a Python scalar, not a tensor")
    if not isinstance(value, numbers.Real):
        raise TypeError(f"{name} must be a real Python scalar")
    return float(value)


def _check_row_size(n_cols: int) -> None:
    """Row-size limit of kernels/swiglu/swiglu.py:19-25 (kept for API parity;
    the HIP kernel itself has no row-size limit)."""
    block = 1 << max(0, (n_cols - 1).bit_length())
    if block > MAX_ROW_BLOCK_SIZE:
        raise RuntimeError(
            f"SwiGLU hidden size {n_cols} requires block size {block}, "
            f"which exceeds the row-wise limit {MAX_ROW_BLOCK_SIZE}."
        )


def _check_same_shape_inputs(gate: torch.Tensor, up: torch.Tensor) -> None:
    """kernels/swiglu/swiglu.py:37-45."""
    if gate.shape != up.shape:
        raise ValueError(f"gate and up must have the same shape, got {gate.shape} and {up.shape}")
    if gate.device != up.device:
        raise ValueError("gate and up must be on the same device")
    if gate.dtype != up.dtype:
        raise TypeError(f"gate and up must have the same dtype, got {gate.dtype} and {up.dtype}")
    if not gate.is_floating_point() or not up.is_floating_point():
        raise TypeError("gate and up must be floating point tensors")


def _check_cuda_dtype(x: torch.Tensor) -> None:
    """kernels/swiglu/swiglu.py:48-50."""
    if x.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        raise TypeError(f"CUDA SwiGLU supports fp16, bf16, and fp32, got {x.dtype}")


def _check_packed_input(gate_up: torch.Tensor) -> None:
    """kernels/swiglu/swiglu.py:53-57."""
    if gate_up.shape[-1] % 2 != 0:
        raise ValueError(f"packed gate_up last dimension must be even, got {gate_up.shape[-1]}")
    if not gate_up.is_floating_point():
        raise TypeError("gate_up must be a floating point tensor")


def torch_swiglu_reference(
    gate: torch.Tensor,
    up: torch.Tensor,
    gate_multiplier: float = 1.0,
    down_multiplier: float = 1.0,
) -> torch.Tensor:
    """The reference's PyTorch formula (kernels/swiglu/swiglu.py:179-188),
    part of its public API: silu(gate.float()*gm).to(dtype) * up * dm."""
    gate_multiplier = _as_float("gate_multiplier", gate_multiplier)
    down_multiplier = _as_float("down_multiplier", down_multiplier)
    silu_gate = torch.nn.functional.silu(gate.float() * gate_multiplier).to(dtype=gate.dtype)
    return (silu_gate * up) * down_multiplier


def torch_swiglu_packed_reference(
    gate_up: torch.Tensor,
    gate_multiplier: float = 1.0,
    down_multiplier: float = 1.0,
) -> torch.Tensor:
    """kernels/swiglu/swiglu.py:191-198."""
    _check_packed_input(gate_up)
    gate, up = gate_up.chunk(2, dim=-1)
    return torch_swiglu_reference(gate, up, gate_multiplier, down_multiplier)


def swiglu_forward(
    gate: torch.Tensor,
    up: torch.Tensor,
    gate_multiplier: float = 1.0,
    down_multiplier: float = 1.0,
):
    """kernels/swiglu/swiglu.py:201-229 -> (out, gate_2d, up_2d)."""
    _check_same_shape_inputs(gate, up)
    _check_cuda_dtype(gate)
    gate_multiplier = _as_float("gate_multiplier", gate_multiplier)
    down_multiplier = _as_float("down_multiplier", down_multiplier)
    L.require_gpu(gate, up)

    original_shape = gate.shape
    n_cols = original_shape[-1]
    _check_row_size(n_cols)
    gate_2d = gate.contiguous().view(-1, n_cols)
    up_2d = up.contiguous().view(-1, n_cols)
    out = torch.empty_like(gate_2d)
    rows = gate_2d.shape[0]
    L.check(
        L.forge_swiglu_fwd(
            L.dtype_code(gate.dtype), gate_2d.data_ptr(), up_2d.data_ptr(), n_cols,
            out.data_ptr(), n_cols, rows, n_cols, gate_multiplier, down_multiplier,
            L.stream_of(gate),
        ),
        "forge_swiglu_fwd",
    )
    return out.view(original_shape), gate_2d, up_2d


def swiglu_backward(
    dout: torch.Tensor,
    gate: torch.Tensor,
    up: torch.Tensor,
    gate_multiplier: float = 1.0,
    down_multiplier: float = 1.0,
    preserve_inputs: bool = False,
):
    """kernels/swiglu/swiglu.py:232-262 -> (dgate, dup).

    gate/up are the saved 2-D buffers; without preserve_inputs the gradients
    are written into them."""
    gate_multiplier = _as_float("gate_multiplier", gate_multiplier)
    down_multiplier = _as_float("down_multiplier", down_multiplier)
    original_shape = dout.shape
    n_cols = original_shape[-1]
    dout_2d = dout.contiguous().view(-1, n_cols)
    dgate = torch.empty_like(gate) if preserve_inputs else gate
    dup = torch.empty_like(up) if preserve_inputs else up
    rows = dout_2d.shape[0]
    L.check(
        L.forge_swiglu_bwd(
            L.dtype_code(gate.dtype), dout_2d.data_ptr(), n_cols, gate.data_ptr(), up.data_ptr(),
            n_cols, dgate.data_ptr(), dup.data_ptr(), n_cols, rows, n_cols,
            gate_multiplier, down_multiplier, L.stream_of(gate),
        ),
        "forge_swiglu_bwd",
    )
    return dgate.view(original_shape), dup.view(original_shape)


def swiglu_packed_forward(
    gate_up: torch.Tensor,
    gate_multiplier: float = 1.0,
    down_multiplier: float = 1.0,
):
    """kernels/swiglu/swiglu.py:265-292 -> (out, gate_up_2d)."""
    _check_packed_input(gate_up)
    _check_cuda_dtype(gate_up)
    gate_multiplier = _as_float("gate_multiplier", gate_multiplier)
    down_multiplier = _as_float("down_multiplier", down_multiplier)
    L.require_gpu(gate_up)

    original_shape = gate_up.shape
    total_cols = original_shape[-1]
    n_cols = total_cols // 2
    _check_row_size(n_cols)
    gate_up_2d = gate_up.contiguous().view(-1, total_cols)
    rows = gate_up_2d.shape[0]
    out = torch.empty((rows, n_cols), device=gate_up.device, dtype=gate_up.dtype)
    es = gate_up.element_size()
    L.check(
        L.forge_swiglu_fwd(
            L.dtype_code(gate_up.dtype), gate_up_2d.data_ptr(), gate_up_2d.data_ptr() + n_cols * es,
            total_cols, out.data_ptr(), n_cols, rows, n_cols, gate_multiplier, down_multiplier,
            L.stream_of(gate_up),
        ),
        "forge_swiglu_fwd(packed)",
    )
    return out.view(*original_shape[:-1], n_cols), gate_up_2d


def swiglu_packed_backward(
    dout: torch.Tensor,
    gate_up: torch.Tensor,
    input_shape: torch.Size,
    gate_multiplier: float = 1.0,
    down_multiplier: float = 1.0,
    preserve_inputs: bool = False,
):
    """kernels/swiglu/swiglu.py:295-323 -> dgate_up (written into gate_up
    unless preserve_inputs)."""
    gate_multiplier = _as_float("gate_multiplier", gate_multiplier)
    down_multiplier = _as_float("down_multiplier", down_multiplier)
    n_cols = dout.shape[-1]
    total_cols = input_shape[-1]
    dout_2d = dout.contiguous().view(-1, n_cols)
    dgate_up = torch.empty_like(gate_up) if preserve_inputs else gate_up
    rows = dout_2d.shape[0]
    es = gate_up.element_size()
    L.check(
        L.forge_swiglu_bwd(
            L.dtype_code(gate_up.dtype), dout_2d.data_ptr(), n_cols,
            gate_up.data_ptr(), gate_up.data_ptr() + n_cols * es, total_cols,
            dgate_up.data_ptr(), dgate_up.data_ptr() + n_cols * es, total_cols,
            rows, n_cols, gate_multiplier, down_multiplier, L.stream_of(gate_up),
        ),
        "forge_swiglu_bwd(packed)",
    )
    return dgate_up.view(input_shape)


class ForgeSwiGLUFunction(torch.autograd.Function):
    """kernels/swiglu/swiglu.py:326-354."""

    @staticmethod
    def forward(
        ctx,
        gate: torch.Tensor,
        up: torch.Tensor,
        gate_multiplier: float = 1.0,
        down_multiplier: float = 1.0,
        preserve_inputs: bool = False,
    ):
        y, gate_2d, up_2d = swiglu_forward(gate, up, gate_multiplier, down_multiplier)
        ctx.save_for_backward(gate_2d, up_2d)
        ctx.gate_multiplier = _as_float("gate_multiplier", gate_multiplier)
        ctx.down_multiplier = _as_float("down_multiplier", down_multiplier)
        ctx.preserve_inputs = bool(preserve_inputs)
        return y

    @staticmethod
    def backward(ctx, dout: torch.Tensor):
        gate, up = ctx.saved_tensors
        dgate, dup = swiglu_backward(
            dout, gate, up, ctx.gate_multiplier, ctx.down_multiplier, ctx.preserve_inputs
        )
        return dgate, dup, None, None, None


class ForgePackedSwiGLUFunction(torch.autograd.Function):
    """kernels/swiglu/swiglu.py:357-385."""

    @staticmethod
    def forward(
        ctx,
        gate_up: torch.Tensor,
        gate_multiplier: float = 1.0,
        down_multiplier: float = 1.0,
        preserve_inputs: bool = False,
    ):
        y, gate_up_2d = swiglu_packed_forward(gate_up, gate_multiplier, down_multiplier)
        ctx.save_for_backward(gate_up_2d)
        ctx.input_shape = gate_up.shape
        ctx.gate_multiplier = _as_float("gate_multiplier", gate_multiplier)
        ctx.down_multiplier = _as_float("down_multiplier", down_multiplier)
        ctx.preserve_inputs = bool(preserve_inputs)
        return y

    @staticmethod
    def backward(ctx, dout: torch.Tensor):
        (gate_up,) = ctx.saved_tensors
        dgate_up = swiglu_packed_backward(
            dout, gate_up, ctx.input_shape, ctx.gate_multiplier, ctx.down_multiplier, ctx.preserve_inputs
        )
        return dgate_up, None, None, None


def swiglu(
    gate: torch.Tensor,
    up: torch.Tensor,
    gate_multiplier: float = 1.0,
    down_multiplier: float = 1.0,
    preserve_inputs: bool = False,
) -> torch.Tensor:
    """kernels/swiglu/swiglu.py:388-398."""
    _check_same_shape_inputs(gate, up)
    if not gate.is_cuda:
        return torch_swiglu_reference(gate, up, gate_multiplier, down_multiplier)
    return ForgeSwiGLUFunction.apply(gate, up, gate_multiplier, down_multiplier, preserve_inputs)


def swiglu_packed(
    gate_up: torch.Tensor,
    gate_multiplier: float = 1.0,
    down_multiplier: float = 1.0,
    preserve_inputs: bool = False,
) -> torch.Tensor:
    """kernels/swiglu/swiglu.py:401-410."""
    _check_packed_input(gate_up)
    if not gate_up.is_cuda:
        return torch_swiglu_packed_reference(gate_up, gate_multiplier, down_multiplier)
    return ForgePackedSwiGLUFunction.apply(gate_up, gate_multiplier, down_multiplier, preserve_inputs)
