"""SwiGLU parity: HIP kernels (through libforge_hip.so) vs the CPU oracle.

Cases follow the reference's tests/test_swiglu.py:28-145 (shapes, multipliers,
preserve_inputs, dtypes, special values, CPU path, input validation) plus the
BASELINE config (fp32 [2048, 11008]).  Tolerances: fp32 1e-5, fp16/bf16 2e-2.
"""
import pytest
import torch

from forge_hip import _lib as L
from kernels.swiglu import swiglu, swiglu_packed, torch_swiglu_packed_reference, torch_swiglu_reference
from oracle.swiglu import swiglu_fwd_bwd, swiglu_packed_fwd_bwd

TOL = {torch.float32: 1e-5, torch.float16: 2e-2, torch.bfloat16: 2e-2}


def _close(a, b, dtype):
    t = TOL[dtype]
    torch.testing.assert_close(a.cpu(), b.cpu(), atol=t, rtol=t)


@pytest.mark.gpu
@pytest.mark.parametrize("shape", [(2, 8, 128), (1, 3, 257), (4, 5, 1024), (1, 2, 11008)])
@pytest.mark.parametrize("gm, dm", [(1.0, 1.0), (0.7, 1.3)])
@pytest.mark.parametrize("preserve_inputs", [False, True])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_swiglu_forward_backward(shape, gm, dm, preserve_inputs, dtype):
    torch.manual_seed(0)
    gate = torch.randn(*shape, dtype=dtype)
    up = torch.randn(*shape, dtype=dtype)
    dout = torch.randn(*shape, dtype=dtype)
    ref_out, ref_dg, ref_du = swiglu_fwd_bwd(gate, up, dout, gm, dm)

    g = gate.cuda().requires_grad_(True)
    u = up.cuda().requires_grad_(True)
    calls = L.calls
    out = swiglu(g, u, gm, dm, preserve_inputs)
    _close(out, ref_out, dtype)
    out.backward(dout.cuda())
    assert L.calls >= calls + 2  # forward and backward ran in libforge_hip.so
    _close(g.grad, ref_dg, dtype)
    _close(u.grad, ref_du, dtype)
    if preserve_inputs:
        assert torch.equal(g.detach().cpu(), gate)
        assert torch.equal(u.detach().cpu(), up)
    else:
        # reference contract: the saved (aliasing) input buffers now hold the grads
        assert torch.equal(g.detach(), g.grad)
        assert torch.equal(u.detach(), u.grad)


@pytest.mark.gpu
@pytest.mark.parametrize("shape", [(2, 8, 256), (1, 3, 514)])
@pytest.mark.parametrize("gm, dm", [(1.0, 1.0), (1.5, 0.5)])
@pytest.mark.parametrize("preserve_inputs", [False, True])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_swiglu_packed_forward_backward(shape, gm, dm, preserve_inputs, dtype):
    torch.manual_seed(1)
    gate_up = torch.randn(*shape, dtype=dtype)
    dout = torch.randn(*shape[:-1], shape[-1] // 2, dtype=dtype)
    ref_out, ref_dgu = swiglu_packed_fwd_bwd(gate_up, dout, gm, dm)
    gu = gate_up.cuda().requires_grad_(True)
    out = swiglu_packed(gu, gm, dm, preserve_inputs)
    _close(out, ref_out, dtype)
    out.backward(dout.cuda())
    _close(gu.grad, ref_dgu, dtype)
    if preserve_inputs:
        assert torch.equal(gu.detach().cpu(), gate_up)


@pytest.mark.gpu
def test_swiglu_special_values_forward():
    gate = torch.tensor([[[0.0, float("inf"), float("-inf"), float("nan"), 20.0, -20.0]]])
    up = torch.tensor([[[1.0, 2.0, 3.0, 4.0, -1.0, -2.0]]])
    ref = torch_swiglu_reference(gate, up)
    out = swiglu(gate.cuda(), up.cuda(), preserve_inputs=True)
    torch.testing.assert_close(out.cpu(), ref, atol=1e-12, rtol=1e-7, equal_nan=True)


@pytest.mark.gpu
def test_swiglu_baseline_config_fp32():
    """fp32 gate/up/dout [2048, 11008] ~ N(0, 1)."""
    gen = torch.Generator().manual_seed(1234)
    gate = torch.randn(2048, 11008, generator=gen)
    up = torch.randn(2048, 11008, generator=gen)
    dout = torch.randn(2048, 11008, generator=gen)
    ref_out, ref_dg, ref_du = swiglu_fwd_bwd(gate, up, dout)
    g = gate.cuda().requires_grad_(True)
    u = up.cuda().requires_grad_(True)
    out = swiglu(g, u)
    out.backward(dout.cuda())
    _close(out, ref_out, torch.float32)
    _close(g.grad, ref_dg, torch.float32)
    _close(u.grad, ref_du, torch.float32)


@pytest.mark.gpu
def test_swiglu_noncontiguous_input_is_copied_not_aliased():
    torch.manual_seed(3)
    base = torch.randn(64, 256)
    gate = base.cuda().t()  # non-contiguous view
    up = torch.randn(256, 64).cuda()
    g = gate.detach().clone().requires_grad_(False)
    ref_out, _, _ = swiglu_fwd_bwd(gate.cpu(), up.cpu(), torch.ones(256, 64))
    out = swiglu(gate, up)
    _close(out, ref_out, torch.float32)
    assert torch.equal(gate, g)


def test_swiglu_cpu_path_matches_reference():
    """Reference tests/test_swiglu.py:116-131: CPU tensors use the module's
    PyTorch formula (its public API for CPU tensors)."""
    torch.manual_seed(0)
    gate = torch.randn(2, 3, 17, requires_grad=True)
    up = torch.randn(2, 3, 17, requires_grad=True)
    gate_ref = gate.detach().clone().requires_grad_(True)
    up_ref = up.detach().clone().requires_grad_(True)
    out = swiglu(gate, up, gate_multiplier=0.7, down_multiplier=1.3)
    out_ref = torch_swiglu_reference(gate_ref, up_ref, gate_multiplier=0.7, down_multiplier=1.3)
    torch.testing.assert_close(out, out_ref)
    grad = torch.randn_like(out)
    out.backward(grad)
    out_ref.backward(grad)
    torch.testing.assert_close(gate.grad, gate_ref.grad)
    torch.testing.assert_close(up.grad, up_ref.grad)
    packed = torch.randn(2, 6)
    torch.testing.assert_close(swiglu_packed(packed), torch_swiglu_packed_reference(packed))


def test_swiglu_rejects_invalid_inputs():
    """Reference tests/test_swiglu.py:134-145."""
    with pytest.raises(ValueError, match="same shape"):
        swiglu(torch.randn(2, 3), torch.randn(2, 4))
    with pytest.raises(ValueError, match="even"):
        swiglu_packed(torch.randn(2, 5))
    with pytest.raises(TypeError, match="Python scalar"):
        swiglu(torch.randn(2, 3), torch.randn(2, 3), gate_multiplier=torch.tensor(1.0))
