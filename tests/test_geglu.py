"""GeGLU parity: HIP kernels (through libforge_hip.so) vs the CPU oracle.

The reference ships no GeGLU tests; the cases mirror the SwiGLU ones
(shapes with ragged rows, both GELU forms, preserve_inputs and the in-place
aliasing contract, every dtype, packed gate_up, the CPU path, input
validation) and add geglu_mlp against the PyTorch MLP baseline
(geglu.py:308-323).  Tolerances: fp32 1e-5 (the oracle's float64 GELU
against the kernel's fp32 one), fp16/bf16 2e-2.
"""
import pytest
import torch

from oracle.geglu import geglu_fwd_bwd

TOL = {torch.float32: 1e-5, torch.float16: 2e-2, torch.bfloat16: 2e-2}


def _close(a, b, dtype):
    t = TOL[dtype]
    torch.testing.assert_close(a.float().cpu(), b.float().cpu(), atol=t, rtol=t)


@pytest.mark.gpu
@pytest.mark.parametrize("shape", [(2, 8, 128), (1, 3, 257), (4, 5, 1024)])
@pytest.mark.parametrize("approximate", ["tanh", "none"])
@pytest.mark.parametrize("preserve_inputs", [False, True])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_geglu_forward_backward(shape, approximate, preserve_inputs, dtype):
    from forge_hip import _lib as L
    from kernels.geglu import geglu

    torch.manual_seed(0)
    gate = (torch.randn(*shape) * 2).to(dtype)
    up = torch.randn(*shape).to(dtype)
    dout = torch.randn(*shape).to(dtype)
    ref_out, ref_dg, ref_du = geglu_fwd_bwd(gate, up, dout, approximate)
    g = gate.cuda().requires_grad_(True)
    u = up.cuda().requires_grad_(True)
    calls = L.calls
    out = geglu(g, u, approximate, preserve_inputs)
    _close(out, ref_out, dtype)
    out.backward(dout.cuda())
    assert L.calls >= calls + 2
    _close(g.grad, ref_dg, dtype)
    _close(u.grad, ref_du, dtype)
    if preserve_inputs:
        assert torch.equal(g.detach().cpu(), gate)
        assert torch.equal(u.detach().cpu(), up)
    else:  # the saved (aliasing) inputs now hold the gradients
        assert torch.equal(g.detach(), g.grad)
        assert torch.equal(u.detach(), u.grad)


@pytest.mark.gpu
@pytest.mark.parametrize("shape", [(2, 8, 256), (1, 3, 514)])
@pytest.mark.parametrize("approximate", ["tanh", "none"])
@pytest.mark.parametrize("preserve_inputs", [False, True])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_geglu_packed_forward_backward(shape, approximate, preserve_inputs, dtype):
    from kernels.geglu import geglu_packed

    torch.manual_seed(1)
    gate_up = (torch.randn(*shape) * 2).to(dtype)
    h = shape[-1] // 2
    dout = torch.randn(*shape[:-1], h).to(dtype)
    ref_out, ref_dg, ref_du = geglu_fwd_bwd(gate_up[..., :h], gate_up[..., h:], dout, approximate)
    gu = gate_up.cuda().requires_grad_(True)
    out = geglu_packed(gu, approximate, preserve_inputs)
    _close(out, ref_out, dtype)
    out.backward(dout.cuda())
    _close(gu.grad[..., :h], ref_dg, dtype)
    _close(gu.grad[..., h:], ref_du, dtype)
    if not preserve_inputs:
        assert torch.equal(gu.detach(), gu.grad)


@pytest.mark.gpu
def test_geglu_large_bf16_matches_torch_formula():
    """A large bf16 forward against the reference's own PyTorch formula run
    on the GPU."""
    from kernels.geglu import geglu, torch_geglu_reference

    g = torch.Generator(device="cuda").manual_seed(2)
    gate = (torch.randn(2048, 8192, device="cuda", generator=g) * 2).to(torch.bfloat16)
    up = torch.randn(2048, 8192, device="cuda", generator=g).to(torch.bfloat16)
    out = geglu(gate, up, "tanh", preserve_inputs=True)
    ref = torch_geglu_reference(gate, up, "tanh")
    torch.testing.assert_close(out.float(), ref.float(), rtol=2e-2, atol=2e-2)


@pytest.mark.gpu
@pytest.mark.parametrize("packed", [False, True])
@pytest.mark.parametrize("dtype,bias", [(torch.float32, True), (torch.bfloat16, False), (torch.bfloat16, True)])
def test_geglu_mlp_matches_pytorch_baseline(packed, dtype, bias):
    from kernels.geglu import geglu_mlp, pack_geglu_gate_up_bias, pack_geglu_gate_up_weight, torch_geglu_mlp_reference

    g = torch.Generator().manual_seed(5)
    H, I = 64, 96
    x = torch.randn(3, 7, H, generator=g)
    wg, wu = torch.randn(I, H, generator=g) / H ** 0.5, torch.randn(I, H, generator=g) / H ** 0.5
    wd = torch.randn(H, I, generator=g) / I ** 0.5
    bg, bu, bd = (torch.randn(I, generator=g), torch.randn(I, generator=g), torch.randn(H, generator=g)) if bias \
        else (None, None, None)
    dy = torch.randn(3, 7, H, generator=g)

    def dev(t):
        return None if t is None else t.to("cuda", dtype).requires_grad_(True)

    xr, wgr, wur, wdr, bgr, bur, bdr = (None if t is None else t.double().requires_grad_(True)
                                        for t in (x, wg, wu, wd, bg, bu, bd))
    ref = torch_geglu_mlp_reference(xr, wgr, wur, wdr, bgr, bur, bdr, approximate="tanh")
    ref.backward(dy.double())
    xd, wgd, wud, wdd, bgd, bud, bdd = (dev(t) for t in (x, wg, wu, wd, bg, bu, bd))
    if packed:
        wp = pack_geglu_gate_up_weight(wgd.detach(), wud.detach()).requires_grad_(True)
        bp = pack_geglu_gate_up_bias(bgd.detach(), bud.detach()).requires_grad_(True) if bias else None
        out = geglu_mlp(xd, wdd, packed_gate_up_weight=wp, packed_gate_up_bias=bp, down_bias=bdd)
    else:
        out = geglu_mlp(xd, wdd, gate_weight=wgd, up_weight=wud, gate_bias=bgd, up_bias=bud, down_bias=bdd)
    out.backward(dy.to("cuda", dtype))

    def close(a, b):
        # fp32: elementwise; bf16: relative to the tensor's scale (the bf16
        # hidden activations feed reductions whose terms cancel)
        if dtype == torch.float32:
            torch.testing.assert_close(a.double().cpu(), b, rtol=1e-4, atol=1e-4)
        else:
            torch.testing.assert_close(a.double().cpu(), b, rtol=3e-2, atol=3e-2 * float(b.abs().max()))

    close(out, ref.detach())
    close(xd.grad, xr.grad)
    close(wdd.grad, wdr.grad)
    if packed:
        close(wp.grad, torch.cat([wgr.grad, wur.grad]))
    else:
        close(wgd.grad, wgr.grad)
        close(wud.grad, wur.grad)


def test_geglu_cpu_path_and_validation():
    """CPU tensors take the module's PyTorch formula (geglu.py:551-573); the
    argument checks raise the reference's exceptions."""
    from kernels.geglu import geglu, geglu_mlp, geglu_packed, pack_geglu_gate_up_bias, torch_geglu_reference

    gate, up = torch.randn(3, 8), torch.randn(3, 8)
    assert torch.equal(geglu(gate, up, "none"), torch_geglu_reference(gate, up, "none"))
    assert geglu_packed(torch.randn(2, 6)).shape == (2, 3)
    with pytest.raises(ValueError, match="approximate must be 'tanh' or 'none'"):
        geglu(gate, up, "erf")
    with pytest.raises(ValueError, match="gate and up must have the same shape"):
        geglu(gate, up[:, :4])
    with pytest.raises(TypeError, match="gate and up must have the same dtype"):
        geglu(gate, up.double())
    with pytest.raises(ValueError, match="packed gate_up last dimension must be even"):
        geglu_packed(torch.randn(2, 5))
    with pytest.raises(ValueError, match="gate_bias and up_bias must either both be None or both be tensors"):
        pack_geglu_gate_up_bias(torch.zeros(3), None)
    with pytest.raises(ValueError, match="separate path requires gate_weight and up_weight"):
        geglu_mlp(torch.randn(2, 4), torch.randn(4, 4))
    with pytest.raises(ValueError, match="x must have at least 2 dimensions"):
        geglu_mlp(torch.randn(4), torch.randn(4, 4), torch.randn(4, 4), torch.randn(4, 4))
