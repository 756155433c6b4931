"""RMSNorm parity: HIP kernels (csrc/rmsnorm.hip) vs the CPU oracle.

Follows the reference's kernels/rmsnorm/tests/test_v4.py: its shapes (tiny,
Qwen2.5-0.5B, Qwen3-8B short/train, Gemma2 2B/9B, a non-power-of-two row),
dtypes, offset/casting cases and tolerances (diff <= atol + rtol * max|ref|:
bf16 5e-2, fp16 2e-2, fp32 1e-4 / 1e-5); in_place=True bit-identical to
in_place=False; backward against the oracle's gradient; an fp64 gradcheck.
Added here: deterministic weight gradients, rows too wide for the register
path (the column-tiled dw pass, in place and not), a 16-bit input with an
fp32 weight, and the v1 / v2 / v3 entry points of the same kernels.  Row
widths are chosen to reach both engines: the wave-per-row kernels (rows
under 256 vectors, or ragged) and every workgroup-per-row-block shape
(1, 2, 4 and 8 vectors per thread, with row counts that leave a partial
chunk).
"""
import pytest
import torch

from oracle import rmsnorm as orms

pytestmark = pytest.mark.gpu

TOL = {torch.bfloat16: (5e-2, 5e-2), torch.float16: (2e-2, 2e-2), torch.float32: (1e-4, 1e-5),
       torch.float64: (1e-7, 1e-7)}
SHAPES = [(1, 8, 64), (2, 512, 896), (4, 512, 4096), (2, 2048, 4096), (2, 2048, 2304), (2, 2048, 3584),
          (4, 128, 4097)]
OFFSET_CASES = [(0.0, "llama", "ones_plus_noise"), (1.0, "gemma", "near_zero")]
MODES = {"llama": orms.LLAMA, "gemma": orms.GEMMA, "none": orms.NONE}


def _inputs(b, s, h, dt, init, seed=0):
    g = torch.Generator(device="cuda").manual_seed(seed)
    x = torch.randn(b, s, h, device="cuda", dtype=dt, generator=g)
    if init == "ones_plus_noise":
        w = torch.ones(h, device="cuda", dtype=dt) + 0.1 * torch.randn(h, device="cuda", dtype=dt, generator=g)
    else:
        w = 0.05 * torch.randn(h, device="cuda", dtype=dt, generator=g)
    return x, w


def _passes(a, ref, dtype):
    atol, rtol = TOL[dtype]
    diff = (a.double().cpu() - ref.double().cpu()).abs().max().item()
    return diff <= atol + rtol * ref.double().abs().max().item(), diff


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("case", OFFSET_CASES)
def test_forward_matches_oracle(shape, dtype, case):
    from forge_hip import _lib as L
    from kernels.rmsnorm import apply_rmsnorm_v4

    offset, mode, init = case
    x, w = _inputs(*shape, dtype, init)
    ref, _ = orms.rms_forward(x, w, 1e-6, offset, MODES[mode])
    for in_place in (True, False):
        calls = L.calls
        y = apply_rmsnorm_v4(x, w, 1e-6, offset, mode, in_place=in_place)
        assert L.calls > calls
        assert y.shape == x.shape and y.dtype == dtype and not torch.isnan(y).any()
        ok, diff = _passes(y, ref, dtype)
        assert ok, diff


@pytest.mark.parametrize("mode", ["llama", "gemma", "none"])
@pytest.mark.parametrize("h", [1024, 4096])
def test_casting_modes_bf16(mode, h):
    from kernels.rmsnorm import apply_rmsnorm_v4

    x, w = _inputs(3, 100, h, torch.bfloat16, "ones_plus_noise", seed=5)
    y = apply_rmsnorm_v4(x, w, 1e-6, 0.5, mode)
    ref, _ = orms.rms_forward(x, w, 1e-6, 0.5, MODES[mode])
    # the kernel rounds exactly where the oracle does: equal up to rare ties
    assert int((y.cpu() != ref).sum()) <= max(4, y.numel() // 5000)


@pytest.mark.parametrize("shape", [(1, 8, 64), (4, 512, 4096), (2, 2048, 2304), (1, 64, 8192), (4, 128, 4097)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("case", OFFSET_CASES)
def test_in_place_equivalence(shape, dtype, case):
    """in_place=True and in_place=False give bit-identical y, dx and dw (the
    reference's headline v4 check)."""
    from kernels.rmsnorm import apply_rmsnorm_v4

    offset, mode, init = case
    xd, wd = _inputs(*shape, dtype, init, seed=1)
    grad = torch.randn(*shape, device="cuda", dtype=dtype)
    res = []
    for in_place in (True, False):
        x = xd.clone().requires_grad_(True)
        w = wd.clone().requires_grad_(True)
        y = apply_rmsnorm_v4(x, w, 1e-6, offset, mode, in_place=in_place)
        y.backward(grad.clone())
        res.append((y.detach(), x.grad, w.grad))
    for a, b in zip(*res):
        assert torch.equal(a, b)


@pytest.mark.parametrize("shape", [(1, 8, 64), (4, 512, 4096), (2, 2048, 2304), (1, 64, 8192), (4, 128, 4097),
                                   (3, 7, 2048), (1, 5, 16384)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("case", OFFSET_CASES)
@pytest.mark.parametrize("in_place", [False, True])
def test_backward_matches_oracle(shape, dtype, case, in_place):
    from kernels.rmsnorm import apply_rmsnorm_v4

    offset, mode, init = case
    xd, wd = _inputs(*shape, dtype, init, seed=2)
    grad = torch.randn(*shape, device="cuda", dtype=dtype)
    x = xd.clone().requires_grad_(True)
    w = wd.clone().requires_grad_(True)
    apply_rmsnorm_v4(x, w, 1e-6, offset, mode, in_place=in_place).backward(grad.clone())
    rdx, rdw = orms.rms_backward(grad, xd, wd, offset, 1e-6)
    ok, diff = _passes(x.grad, rdx, dtype)
    assert ok, ("dx", diff)
    # dw sums over all rows: scale the tolerance by that reduction's size
    atol, rtol = TOL[dtype]
    dw_diff = (w.grad.double().cpu() - rdw).abs().max().item()
    assert dw_diff <= atol + rtol * rdw.abs().max().item() * (1 if dtype == torch.float32 else 2), ("dw", dw_diff)


@pytest.mark.parametrize("rows_per_chunk, h, dtype", [(4, 2048, torch.bfloat16), (2, 4096, torch.bfloat16),
                                                      (1, 8192, torch.bfloat16), (1, 4096, torch.float32)])
@pytest.mark.parametrize("in_place", [False, True])
def test_backward_chunk_loop_ragged(rows_per_chunk, h, dtype, in_place):
    """The workgroup backward runs at most 512 workgroups, each looping over
    chunks b, b + 512, ... with the next chunk's loads queued before the
    current one is processed.  1324 full chunks plus one single-row chunk:
    workgroups 0..300 take three chunks (the loop's second half, then the
    early exit), the rest two, and the last chunk is ragged.  The forward at
    the same rows ends in a partial chunk too."""
    from kernels.rmsnorm import apply_rmsnorm_v4

    rows = rows_per_chunk * 1324 + 1
    xd, wd = _inputs(1, rows, h, dtype, "ones_plus_noise", seed=4)
    grad = torch.randn(1, rows, h, device="cuda", dtype=dtype)
    x = xd.clone().requires_grad_(True)
    w = wd.clone().requires_grad_(True)
    y = apply_rmsnorm_v4(x, w, 1e-6, 0.0, "llama", in_place=in_place)
    ref_y, _ = orms.rms_forward(xd, wd, 1e-6, 0.0, orms.LLAMA)
    ok, diff = _passes(y, ref_y, dtype)
    assert ok, ("y", diff)
    y.backward(grad.clone())
    rdx, rdw = orms.rms_backward(grad, xd, wd, 0.0, 1e-6)
    ok, diff = _passes(x.grad, rdx, dtype)
    assert ok, ("dx", diff)
    atol, rtol = TOL[dtype]
    dw_diff = (w.grad.double().cpu() - rdw).abs().max().item()
    assert dw_diff <= atol + rtol * rdw.abs().max().item() * (1 if dtype == torch.float32 else 2), ("dw", dw_diff)


@pytest.mark.parametrize("rows, h, dtype", [(8793, 2048, torch.bfloat16), (4397, 4096, torch.bfloat16),
                                            (2349, 8192, torch.bfloat16), (2349, 16384, torch.bfloat16),
                                            (2349, 4096, torch.float32)])
def test_forward_chunk_loop_ragged(rows, h, dtype):
    """The workgroup forward runs a persistent grid (2048 workgroups up to two
    vectors per thread, 1024 beyond; chunks of 2 rows at one vector per
    thread, else 1) with the next chunk's loads queued before the current
    one is processed.  These row counts give the first 301 workgroups three
    chunks and the rest two, and leave a ragged last chunk where chunks
    hold two rows; 16384 bf16 columns run the one-register-set loop."""
    from kernels.rmsnorm import apply_rmsnorm_v4

    xd, wd = _inputs(1, rows, h, dtype, "ones_plus_noise", seed=5)
    y = apply_rmsnorm_v4(xd, wd, 1e-6, 0.0, "llama")
    ref_y, _ = orms.rms_forward(xd, wd, 1e-6, 0.0, orms.LLAMA)
    ok, diff = _passes(y, ref_y, dtype)
    assert ok, ("y", diff)


def test_weight_gradient_is_deterministic():
    from kernels.rmsnorm import apply_rmsnorm_v4

    xd, wd = _inputs(2, 2048, 4096, torch.bfloat16, "ones_plus_noise", seed=3)
    grad = torch.randn(2, 2048, 4096, device="cuda", dtype=torch.bfloat16)
    dws = []
    for _ in range(3):
        x = xd.clone().requires_grad_(True)
        w = wd.clone().requires_grad_(True)
        apply_rmsnorm_v4(x, w, 1e-6, 0.0, "llama", in_place=False).backward(grad.clone())
        dws.append(w.grad.clone())
    assert torch.equal(dws[0], dws[1]) and torch.equal(dws[0], dws[2])


@pytest.mark.parametrize("h", [64, 1024])
def test_fp64_matches_oracle(h):
    """fp64 accumulates in fp64 on both engines (1024 columns: the
    workgroup engine, two vectors per thread)."""
    from kernels.rmsnorm import apply_rmsnorm_v4

    xd, wd = _inputs(2, 16, h, torch.float64, "ones_plus_noise", seed=7)
    grad = torch.randn(2, 16, h, device="cuda", dtype=torch.float64)
    x, w = xd.clone().requires_grad_(True), wd.clone().requires_grad_(True)
    y = apply_rmsnorm_v4(x, w, 1e-6, 1.0, "gemma", in_place=False)
    y.backward(grad)
    ref, _ = orms.rms_forward(xd, wd, 1e-6, 1.0, orms.GEMMA)
    rdx, rdw = orms.rms_backward(grad, xd, wd, 1.0, 1e-6)
    for a, b in ((y, ref), (x.grad, rdx), (w.grad, rdw)):
        torch.testing.assert_close(a.detach().cpu(), b.to(torch.float64), rtol=1e-10, atol=1e-10)


@pytest.mark.parametrize("case", OFFSET_CASES)
def test_gradcheck_fp64(case):
    from kernels.rmsnorm import ForgeRMSNormv4Function

    offset, mode, init = case
    torch.manual_seed(42)
    xs = torch.randn(2, 8, 32, device="cuda", dtype=torch.float64, requires_grad=True)
    ws = (0.5 * (torch.rand(32, device="cuda", dtype=torch.float64) - 0.5) if init == "near_zero"
          else torch.randn(32, device="cuda", dtype=torch.float64) * 0.5).requires_grad_(True)
    assert torch.autograd.gradcheck(lambda a, b: ForgeRMSNormv4Function.apply(a, b, 1e-6, offset, mode, False),
                                    (xs, ws), eps=1e-6, atol=1e-5, rtol=1e-4, fast_mode=True)


def test_fp32_weight_with_bf16_input():
    from kernels.rmsnorm import apply_rmsnorm_v4

    x = torch.randn(64, 2048, device="cuda").to(torch.bfloat16).requires_grad_(True)
    w = (1 + 0.1 * torch.randn(2048, device="cuda")).requires_grad_(True)
    y = apply_rmsnorm_v4(x, w, 1e-6, 0.0, "llama", in_place=False)
    assert y.dtype == torch.bfloat16
    ref, _ = orms.rms_forward(x, w, 1e-6, 0.0, orms.LLAMA)
    assert _passes(y, ref, torch.bfloat16)[0]
    g = torch.randn_like(y)
    y.backward(g)
    rdx, rdw = orms.rms_backward(g, x, w, 0.0, 1e-6)
    assert _passes(x.grad, rdx, torch.bfloat16)[0]
    assert w.grad.dtype == torch.float32
    assert (w.grad.double().cpu() - rdw).abs().max().item() <= 0.1 * rdw.abs().max().item()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("h", [896, 2048])
def test_legacy_versions(dtype, h):
    """v1 (legacy unversioned names), v2 and v3 run on the same kernels."""
    import kernels.rmsnorm as R

    x, w = _inputs(2, 64, h, dtype, "ones_plus_noise", seed=6)
    g = torch.randn(2, 64, h, device="cuda", dtype=dtype)
    ref, _ = orms.rms_forward(x, w, 1e-6, 0.0, orms.LLAMA)
    rdx, rdw = orms.rms_backward(g, x, w, 0.0, 1e-6)
    for fn in (lambda a, b: R.rmsnorm(a, b, 1e-6), lambda a, b: R.apply_rmsnorm_v2(a, b, 1e-6),
               lambda a, b: R.apply_rmsnorm_v3(a, b, 1e-6), lambda a, b: R.ForgeRMSNormFunction.apply(a, b, 1e-6)):
        xa, wa = x.clone().requires_grad_(True), w.clone().requires_grad_(True)
        y = fn(xa, wa)
        assert _passes(y, ref, dtype)[0]
        y.backward(g)
        assert _passes(xa.grad, rdx, dtype)[0]
        assert (wa.grad.double().cpu() - rdw).abs().max().item() <= 0.05 * rdw.abs().max().item() + 1e-4


def test_module_and_cpu_path():
    from kernels.rmsnorm import ForgeRMSNormv4, apply_rmsnorm, torch_rmsnorm_reference_v4

    m = ForgeRMSNormv4(256, eps=1e-5, offset=1.0, casting_mode="gemma", weight_init="zeros", device="cuda")
    x = torch.randn(4, 256, device="cuda")
    ref, _ = orms.rms_forward(x, m.weight, 1e-5, 1.0, orms.GEMMA)
    assert _passes(m(x), ref, torch.float32)[0]
    xc = torch.randn(3, 16)
    assert torch.equal(apply_rmsnorm(xc, torch.ones(16)), torch_rmsnorm_reference_v4(xc, torch.ones(16)))
    with pytest.raises(ValueError, match=r"x.shape\[-1\] \(16\) must equal weight.numel\(\) \(8\)"):
        apply_rmsnorm(xc, torch.ones(8))
    with pytest.raises(ValueError, match="Invalid casting_mode"):
        apply_rmsnorm(x, torch.ones(256, device="cuda"), casting_mode="fp8")
