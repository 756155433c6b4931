"""GeGLU forward/backward on MI355X.

Drop-in for kernels/geglu/geglu.py of Forge-researchlab/kernel-POCs: the same
public functions, autograd Functions, argument checks (exception types and
messages) and saved tensors.  The elementwise work runs in `forge_geglu_fwd`
/ `forge_geglu_bwd` (libforge_hip.so, csrc/geglu.hip: the gated-linear-unit
engine shared with SwiGLU, with a tanh or exact GELU policy).

Contracts kept from the reference:
  * forward saves the flattened contiguous gate/up (:501-515) or the packed
    2-D gate_up (:523-537);
  * the default backward writes dgate/dup INTO the saved buffers, which alias
    the caller's inputs when they were contiguous; preserve_inputs=True
    allocates fresh gradient buffers (:418-419, 479);
  * `geglu` / `geglu_packed` on tensors that are not on a GPU return the
    module's PyTorch formula (:551-573); GPU tensors always take the HIP path;
  * `geglu_mlp` composes the projections and the GeGLU kernel as the
    reference does (:326-377), with the projections on the library's GEMMs
    (kernels/_linear.py) instead of cuBLAS.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

from forge_hip import _lib as L
from kernels._linear import linear


def _check_same_shape_inputs(gate: torch.Tensor, up: torch.Tensor) -> None:
    """geglu.py:19-27."""
    if gate.shape != up.shape:
        raise ValueError(f"gate and up must have the same shape, got {gate.shape} and {up.shape}")
    if gate.device != up.device:
        raise ValueError("gate and up must be on the same device")
    if gate.dtype != up.dtype:
        raise TypeError(f"gate and up must have the same dtype, got {gate.dtype} and {up.dtype}")
    if not gate.is_floating_point() or not up.is_floating_point():
        raise TypeError("gate and up must be floating point tensors")


def _check_cuda_dtype(x: torch.Tensor) -> None:
    """geglu.py:30-32."""
    if x.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        raise TypeError(f"CUDA GEGLU supports fp16, bf16, and fp32, got {x.dtype}")


def _check_packed_input(gate_up: torch.Tensor) -> None:
    """geglu.py:35-39."""
    if gate_up.shape[-1] % 2 != 0:
        raise ValueError(f"packed gate_up last dimension must be even, got {gate_up.shape[-1]}")
    if not gate_up.is_floating_point():
        raise TypeError("gate_up must be a floating point tensor")


def _check_approximate(approximate: str) -> bool:
    """geglu.py:42-45."""
    if approximate not in {"tanh", "none"}:
        raise ValueError(f"approximate must be 'tanh' or 'none', got {approximate!r}")
    return approximate == "tanh"


def _check_linear_weight(name, weight, in_features, device=None, dtype=None) -> None:
    """geglu.py:48-64."""
    if weight.dim() != 2:
        raise ValueError(f"{name} must be 2D [out_features, in_features], got shape {tuple(weight.shape)}")
    if weight.shape[1] != in_features:
        raise ValueError(f"{name} input features {weight.shape[1]} do not match x last dimension {in_features}")
    if not weight.is_floating_point():
        raise TypeError(f"{name} must be a floating point tensor")
    if device is not None and weight.device != device:
        raise ValueError(f"{name} must be on device {device}, got {weight.device}")
    if dtype is not None and weight.dtype != dtype:
        raise TypeError(f"{name} must have dtype {dtype}, got {weight.dtype}")


def _check_optional_bias(name, bias, out_features, device=None, dtype=None) -> None:
    """geglu.py:67-83."""
    if bias is None:
        return
    if bias.dim() != 1 or bias.shape[0] != out_features:
        raise ValueError(f"{name} must have shape [{out_features}], got {tuple(bias.shape)}")
    if not bias.is_floating_point():
        raise TypeError(f"{name} must be a floating point tensor")
    if device is not None and bias.device != device:
        raise ValueError(f"{name} must be on device {device}, got {bias.device}")
    if dtype is not None and bias.dtype != dtype:
        raise TypeError(f"{name} must have dtype {dtype}, got {bias.dtype}")


def torch_geglu_reference(gate: torch.Tensor, up: torch.Tensor, approximate: str = "tanh") -> torch.Tensor:
    """geglu.py:255-263 (the PyTorch formula; CPU path of `geglu`)."""
    _check_same_shape_inputs(gate, up)
    _check_approximate(approximate)
    activated = torch.nn.functional.gelu(gate.float(), approximate=approximate).to(dtype=gate.dtype)
    return activated * up


def torch_geglu_packed_reference(gate_up: torch.Tensor, approximate: str = "tanh") -> torch.Tensor:
    """geglu.py:266-272."""
    _check_packed_input(gate_up)
    gate, up = gate_up.chunk(2, dim=-1)
    return torch_geglu_reference(gate, up, approximate)


def pack_geglu_gate_up_weight(gate_weight: torch.Tensor, up_weight: torch.Tensor) -> torch.Tensor:
    """geglu.py:275-285: [gate; up] -> one [2I, H] weight."""
    if gate_weight.shape != up_weight.shape:
        raise ValueError(
            f"gate_weight and up_weight must have the same shape, got {gate_weight.shape} and {up_weight.shape}")
    if gate_weight.device != up_weight.device:
        raise ValueError("gate_weight and up_weight must be on the same device")
    if gate_weight.dtype != up_weight.dtype:
        raise TypeError(
            f"gate_weight and up_weight must have the same dtype, got {gate_weight.dtype} and {up_weight.dtype}")
    if gate_weight.dim() != 2:
        raise ValueError(f"gate_weight and up_weight must be 2D, got {gate_weight.dim()}D")
    return torch.cat([gate_weight, up_weight], dim=0).contiguous()


def pack_geglu_gate_up_bias(gate_bias, up_bias):
    """geglu.py:288-305."""
    if gate_bias is None and up_bias is None:
        return None
    if gate_bias is None or up_bias is None:
        raise ValueError("gate_bias and up_bias must either both be None or both be tensors for packed gate+up")
    if gate_bias.dim() != 1 or up_bias.dim() != 1:
        raise ValueError("gate_bias and up_bias must be 1D tensors")
    if gate_bias.shape != up_bias.shape:
        raise ValueError(f"gate_bias and up_bias must have the same shape, got {gate_bias.shape} and {up_bias.shape}")
    if gate_bias.device != up_bias.device:
        raise ValueError("gate_bias and up_bias must be on the same device")
    if gate_bias.dtype != up_bias.dtype:
        raise TypeError(f"gate_bias and up_bias must have the same dtype, got {gate_bias.dtype} and {up_bias.dtype}")
    return torch.cat([gate_bias, up_bias], dim=0).contiguous()


def torch_geglu_mlp_reference(x, gate_weight, up_weight, down_weight, gate_bias=None, up_bias=None, down_bias=None,
                              approximate: str = "tanh") -> torch.Tensor:
    """geglu.py:308-323 (PyTorch baseline)."""
    _check_approximate(approximate)
    gate = F.linear(x, gate_weight, gate_bias)
    up = F.linear(x, up_weight, up_bias)
    hidden = torch_geglu_reference(gate, up, approximate)
    return F.linear(hidden, down_weight, down_bias)


def geglu_mlp(
    x: torch.Tensor,
    down_weight: torch.Tensor,
    gate_weight: torch.Tensor | None = None,
    up_weight: torch.Tensor | None = None,
    packed_gate_up_weight: torch.Tensor | None = None,
    gate_bias: torch.Tensor | None = None,
    up_bias: torch.Tensor | None = None,
    packed_gate_up_bias: torch.Tensor | None = None,
    down_bias: torch.Tensor | None = None,
    approximate: str = "tanh",
    preserve_inputs: bool = False,
) -> torch.Tensor:
    """geglu.py:326-377: down(gelu(gate) * up), packed gate+up when given."""
    _check_approximate(approximate)
    if x.dim() < 2:
        raise ValueError(f"x must have at least 2 dimensions, got shape {tuple(x.shape)}")
    if not x.is_floating_point():
        raise TypeError("x must be a floating point tensor")
    in_features = x.shape[-1]
    if packed_gate_up_weight is not None:
        if gate_weight is not None or up_weight is not None:
            raise ValueError("provide either packed_gate_up_weight or separate gate_weight/up_weight, not both")
        _check_linear_weight("packed_gate_up_weight", packed_gate_up_weight, in_features, x.device, x.dtype)
        if packed_gate_up_weight.shape[0] % 2 != 0:
            raise ValueError(
                f"packed_gate_up_weight output dimension must be even, got {packed_gate_up_weight.shape[0]}")
        intermediate = packed_gate_up_weight.shape[0] // 2
        _check_optional_bias("packed_gate_up_bias", packed_gate_up_bias, packed_gate_up_weight.shape[0], x.device,
                             x.dtype)
        if gate_bias is not None or up_bias is not None:
            raise ValueError("use packed_gate_up_bias with packed_gate_up_weight")
        gate_up = _proj(x, packed_gate_up_weight, packed_gate_up_bias)
        hidden = geglu_packed(gate_up, approximate=approximate, preserve_inputs=preserve_inputs)
    else:
        if gate_weight is None or up_weight is None:
            raise ValueError("separate path requires gate_weight and up_weight")
        _check_linear_weight("gate_weight", gate_weight, in_features, x.device, x.dtype)
        _check_linear_weight("up_weight", up_weight, in_features, x.device, x.dtype)
        if gate_weight.shape != up_weight.shape:
            raise ValueError(
                f"gate_weight and up_weight must have the same shape, got {gate_weight.shape} and {up_weight.shape}")
        intermediate = gate_weight.shape[0]
        _check_optional_bias("gate_bias", gate_bias, intermediate, x.device, x.dtype)
        _check_optional_bias("up_bias", up_bias, intermediate, x.device, x.dtype)
        if packed_gate_up_bias is not None:
            raise ValueError("packed_gate_up_bias requires packed_gate_up_weight")
        gate = _proj(x, gate_weight, gate_bias)
        up = _proj(x, up_weight, up_bias)
        hidden = geglu(gate, up, approximate=approximate, preserve_inputs=preserve_inputs)
    _check_linear_weight("down_weight", down_weight, intermediate, x.device, x.dtype)
    _check_optional_bias("down_bias", down_bias, down_weight.shape[0], x.device, x.dtype)
    return _proj(hidden, down_weight, down_bias)


def _proj(x, weight, bias):
    """nn.Linear: the library GEMMs on a GPU, F.linear for CPU tensors (the
    reference's CPU behaviour)."""
    if not x.is_cuda:
        return F.linear(x, weight, bias)
    return linear(x, weight, bias)


def geglu_forward(gate: torch.Tensor, up: torch.Tensor, approximate: str = "tanh"):
    """geglu.py:380-406 -> (out, gate_flat, up_flat)."""
    _check_same_shape_inputs(gate, up)
    _check_cuda_dtype(gate)
    approximate_tanh = _check_approximate(approximate)
    L.require_gpu(gate, up)
    original_shape = gate.shape
    gate_flat = gate.contiguous().view(-1)
    up_flat = up.contiguous().view(-1)
    out = torch.empty_like(gate_flat)
    n = gate_flat.numel()
    L.check(L.forge_geglu_fwd(L.dtype_code(gate.dtype), gate_flat.data_ptr(), up_flat.data_ptr(), n, out.data_ptr(),
                              n, 1, n, int(approximate_tanh), L.stream_of(gate_flat)), "forge_geglu_fwd")
    return out.view(original_shape), gate_flat, up_flat


def geglu_backward(dout, gate, up, approximate: str = "tanh", preserve_inputs: bool = False):
    """geglu.py:409-437 -> (dgate, dup) in dout's shape; in place by default."""
    approximate_tanh = _check_approximate(approximate)
    original_shape = dout.shape
    dout_flat = dout.contiguous().view(-1)
    n = dout_flat.numel()
    dgate = torch.empty_like(gate) if preserve_inputs else gate
    dup = torch.empty_like(up) if preserve_inputs else up
    L.check(L.forge_geglu_bwd(L.dtype_code(gate.dtype), dout_flat.data_ptr(), n, gate.data_ptr(), up.data_ptr(), n,
                              dgate.data_ptr(), dup.data_ptr(), n, 1, n, int(approximate_tanh),
                              L.stream_of(dout_flat)), "forge_geglu_bwd")
    return dgate.view(original_shape), dup.view(original_shape)


def geglu_packed_forward(gate_up: torch.Tensor, approximate: str = "tanh"):
    """geglu.py:440-467 -> (out [..., H], gate_up_2d)."""
    _check_packed_input(gate_up)
    _check_cuda_dtype(gate_up)
    approximate_tanh = _check_approximate(approximate)
    L.require_gpu(gate_up)
    original_shape = gate_up.shape
    total_cols = original_shape[-1]
    n_cols = total_cols // 2
    gate_up_2d = gate_up.contiguous().view(-1, total_cols)
    rows = gate_up_2d.shape[0]
    out = torch.empty((rows * n_cols,), device=gate_up.device, dtype=gate_up.dtype)
    if rows and n_cols:
        base = gate_up_2d.data_ptr()
        L.check(L.forge_geglu_fwd(L.dtype_code(gate_up.dtype), base, base + n_cols * gate_up.element_size(),
                                  total_cols, out.data_ptr(), n_cols, rows, n_cols, int(approximate_tanh),
                                  L.stream_of(gate_up_2d)), "forge_geglu_fwd")
    return out.view(*original_shape[:-1], n_cols), gate_up_2d


def geglu_packed_backward(dout, gate_up, input_shape, approximate: str = "tanh", preserve_inputs: bool = False):
    """geglu.py:470-498 -> dgate_up in input_shape; in place by default."""
    approximate_tanh = _check_approximate(approximate)
    n_cols = dout.shape[-1]
    total_cols = input_shape[-1]
    dout_2d = dout.contiguous().view(-1, n_cols)
    rows = dout_2d.shape[0]
    dgate_up = torch.empty_like(gate_up) if preserve_inputs else gate_up
    if rows and n_cols:
        es = gate_up.element_size()
        g, d = gate_up.data_ptr(), dgate_up.data_ptr()
        L.check(L.forge_geglu_bwd(L.dtype_code(gate_up.dtype), dout_2d.data_ptr(), n_cols, g, g + n_cols * es,
                                  total_cols, d, d + n_cols * es, total_cols, rows, n_cols, int(approximate_tanh),
                                  L.stream_of(dout_2d)), "forge_geglu_bwd")
    return dgate_up.view(input_shape)


class ForgeGEGLUFunction(torch.autograd.Function):
    """geglu.py:501-520."""

    @staticmethod
    def forward(ctx, gate, up, approximate: str = "tanh", preserve_inputs: bool = False):
        y, gate_flat, up_flat = geglu_forward(gate, up, approximate)
        ctx.save_for_backward(gate_flat, up_flat)
        ctx.approximate = approximate
        ctx.preserve_inputs = bool(preserve_inputs)
        return y

    @staticmethod
    def backward(ctx, dout):
        gate, up = ctx.saved_tensors
        dgate, dup = geglu_backward(dout, gate, up, ctx.approximate, ctx.preserve_inputs)
        return dgate, dup, None, None


class ForgePackedGEGLUFunction(torch.autograd.Function):
    """geglu.py:523-548."""

    @staticmethod
    def forward(ctx, gate_up, approximate: str = "tanh", preserve_inputs: bool = False):
        y, gate_up_2d = geglu_packed_forward(gate_up, approximate)
        ctx.save_for_backward(gate_up_2d)
        ctx.input_shape = gate_up.shape
        ctx.approximate = approximate
        ctx.preserve_inputs = bool(preserve_inputs)
        return y

    @staticmethod
    def backward(ctx, dout):
        (gate_up,) = ctx.saved_tensors
        dgate_up = geglu_packed_backward(dout, gate_up, ctx.input_shape, ctx.approximate, ctx.preserve_inputs)
        return dgate_up, None, None


def geglu(gate: torch.Tensor, up: torch.Tensor, approximate: str = "tanh", preserve_inputs: bool = False):
    """geglu.py:551-561."""
    _check_same_shape_inputs(gate, up)
    _check_approximate(approximate)
    if not gate.is_cuda:
        return torch_geglu_reference(gate, up, approximate)
    return ForgeGEGLUFunction.apply(gate, up, approximate, preserve_inputs)


def geglu_packed(gate_up: torch.Tensor, approximate: str = "tanh", preserve_inputs: bool = False):
    """geglu.py:564-573."""
    _check_packed_input(gate_up)
    _check_approximate(approximate)
    if not gate_up.is_cuda:
        return torch_geglu_packed_reference(gate_up, approximate)
    return ForgePackedGEGLUFunction.apply(gate_up, approximate, preserve_inputs)
