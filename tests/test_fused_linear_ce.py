"""Fused linear + cross-entropy (HIP) against the CPU oracle.

Cases follow the reference's own tests
(kernels/cross_entropy/tests/test_fused_linear_cross_entropy.py): the small
odd fp32 shapes with and without bias, mean/sum, label smoothing, class
weights, softcap with z-loss, accuracy/predictions, the Liger call order of
the Module, forward-only without grad, an fp32/bf16 dtype smoke test and the
'none' reduction, with the reference's tolerances (fp32 1e-5; bf16 5e-2 /
2e-2).  Added here: the bf16 MFMA path (H % 8 == 0) with a vocabulary that
is and is not a multiple of 8, several token chunks (the weight gradient
accumulated over chunks), token scaling, a grad_output != 1, and the generic
GEMM / token-scaling entry points through the C ABI, and the benchmarked
configuration at its full size against an fp32 torch reference on the GPU.
"""
import pytest
import torch

from oracle import fused_linear_ce as oflce

pytestmark = pytest.mark.gpu

if torch.cuda.is_available():
    from forge_hip import _lib as L
    from kernels.cross_entropy.experiments.v2 import (
        CrossEntropyOutput,
        ForgeFusedLinearCrossEntropyLoss,
        forge_fused_linear_cross_entropy,
    )
    from kernels.cross_entropy.experiments.v2 import fused_linear_cross_entropy as flce_mod

DEV = "cuda"


def _tol(dtype):
    if dtype == torch.bfloat16:
        return 5e-2, 2e-2
    if dtype == torch.float16:
        return 2e-2, 2e-2
    return 1e-5, 1e-5


def _case(bt, h, v, dtype=torch.float32, bias=False, seed=123):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(bt, h, generator=g)
    W = torch.randn(v, h, generator=g) / h ** 0.5
    b = torch.randn(v, generator=g) if bias else None
    t = torch.randint(0, v, (bt,), generator=g)
    xf = x.to(DEV, dtype).requires_grad_(True)
    Wf = W.to(DEV, dtype).requires_grad_(True)
    bf = b.to(DEV, dtype).requires_grad_(True) if bias else None
    return xf, Wf, bf, t.to(DEV)


def _oracle(x, W, b, t, **kw):
    return oflce.fused_linear_ce(x.detach().float(), W.detach().float(), t,
                                 bias=b.detach().float() if b is not None else None, **kw)


def _check_grads(x, W, b, ref, dtype=torch.float32):
    rtol, atol = _tol(dtype)
    torch.testing.assert_close(x.grad.float().cpu(), ref["dX"].float(), rtol=rtol, atol=atol)
    torch.testing.assert_close(W.grad.float().cpu(), ref["dW"].float(), rtol=rtol, atol=atol)
    if b is not None:
        torch.testing.assert_close(b.grad.float().cpu(), ref["db"].float(), rtol=rtol, atol=atol)


@pytest.mark.parametrize("shape", [(10, 32, 73), (21, 48, 129)])
@pytest.mark.parametrize("reduction", ["mean", "sum"])
@pytest.mark.parametrize("bias", [False, True])
def test_matches_oracle(shape, reduction, bias):
    bt, h, v = shape
    x, W, b, t = _case(bt, h, v, bias=bias)
    calls = L.calls
    loss = forge_fused_linear_cross_entropy(x, W, t, bias=b, reduction=reduction)
    assert L.calls > calls  # the HIP path ran
    ref = _oracle(x, W, b, t, reduction=reduction)
    torch.testing.assert_close(loss.cpu().double(), ref["loss"], rtol=1e-5, atol=1e-5)
    loss.backward()
    _check_grads(x, W, b, ref)


@pytest.mark.parametrize("label_smoothing", [0.1, 0.2])
def test_label_smoothing(label_smoothing):
    x, W, b, t = _case(17, 40, 67, bias=True)
    loss = forge_fused_linear_cross_entropy(x, W, t, bias=b, label_smoothing=label_smoothing)
    ref = _oracle(x, W, b, t, label_smoothing=label_smoothing)
    torch.testing.assert_close(loss.cpu().double(), ref["loss"], rtol=1e-5, atol=1e-5)
    loss.backward()
    _check_grads(x, W, b, ref)


def test_class_weight():
    x, W, b, t = _case(13, 36, 59, bias=True)
    cw = torch.rand(59, generator=torch.Generator().manual_seed(3)) + 0.5
    loss = forge_fused_linear_cross_entropy(x, W, t, bias=b, ce_weight=cw.to(DEV))
    ref = _oracle(x, W, b, t, ce_weight=cw.double())
    torch.testing.assert_close(loss.cpu().double(), ref["loss"], rtol=1e-5, atol=1e-5)
    loss.backward()
    _check_grads(x, W, b, ref)


@pytest.mark.parametrize("return_z_loss", [False, True])
def test_softcap_z_loss(return_z_loss):
    x, W, b, t = _case(11, 28, 53, bias=True)
    out = forge_fused_linear_cross_entropy(x, W, t, bias=b, lse_square_scale=1e-4, softcap=30.0,
                                           return_z_loss=return_z_loss)
    ref = _oracle(x, W, b, t, lse_square_scale=1e-4, softcap=30.0)
    loss = out.loss if return_z_loss else out
    torch.testing.assert_close(loss.cpu().double(), ref["loss"], rtol=1e-5, atol=1e-5)
    if return_z_loss:
        torch.testing.assert_close(out.z_loss.cpu().double(), ref["z_loss"], rtol=1e-5, atol=1e-5)
    loss.backward()
    _check_grads(x, W, b, ref)


def test_metrics_match_argmax():
    x, W, b, t = _case(13, 24, 41, bias=True)
    t[::5] = -100
    out = forge_fused_linear_cross_entropy(x, W, t, bias=b, return_token_accuracy=True,
                                           return_predicted_tokens=True)
    ref = _oracle(x, W, b, t)
    assert isinstance(out, CrossEntropyOutput)
    assert torch.equal(out.predicted_tokens.cpu(), ref["predicted"])
    torch.testing.assert_close(out.token_accuracy.cpu().double(), torch.as_tensor(ref["token_accuracy"]).double())
    out.loss.backward()
    _check_grads(x, W, b, ref)


def test_module_liger_call_order():
    x, W, b, t = _case(9, 20, 37, bias=True)
    loss = ForgeFusedLinearCrossEntropyLoss(ignore_index=-100, reduction="mean")(W, x, t, b)
    ref = _oracle(x, W, b, t)
    torch.testing.assert_close(loss.cpu().double(), ref["loss"], rtol=1e-5, atol=1e-5)
    loss.backward()
    _check_grads(x, W, b, ref)


def test_forward_only_no_grad():
    x, W, b, t = _case(8, 24, 47, bias=True)
    x, W, b = x.detach(), W.detach(), b.detach()
    with torch.no_grad():
        loss = forge_fused_linear_cross_entropy(x, W, t, bias=b)
    ref = _oracle(x, W, b, t)
    torch.testing.assert_close(loss.cpu().double(), ref["loss"], rtol=1e-5, atol=1e-5)
    assert not loss.requires_grad


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_dtype_smoke(dtype):
    x, W, b, t = _case(7, 32, 61, dtype=dtype, bias=True)
    loss = forge_fused_linear_cross_entropy(x, W, t, bias=b)
    ref = _oracle(x, W, b, t)
    rtol, atol = _tol(dtype)
    torch.testing.assert_close(loss.float().cpu().double(), ref["loss"], rtol=rtol, atol=atol)
    loss.backward()
    _check_grads(x, W, b, ref, dtype)


def test_none_reduction_forward():
    x, W, b, t = _case(5, 12, 19, bias=True)
    loss = forge_fused_linear_cross_entropy(x, W, t, bias=b, reduction="none")
    ref = _oracle(x, W, b, t, reduction="none")
    torch.testing.assert_close(loss.cpu().double(), ref["loss"], rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("v", [1000, 1003])
@pytest.mark.parametrize("bias", [False, True])
def test_bf16_mfma_path(v, bias):
    """H % 8 == 0: logits, dX and dW on the MFMA GEMMs (V % 8 != 0: padded pitch)."""
    x, W, b, t = _case(320, 256, v, dtype=torch.bfloat16, bias=bias, seed=7)
    t[::7] = -100
    loss = forge_fused_linear_cross_entropy(x, W, t, bias=b, label_smoothing=0.05)
    ref = _oracle(x, W, b, t, label_smoothing=0.05)
    torch.testing.assert_close(loss.float().cpu().double(), ref["loss"], rtol=2e-2, atol=2e-2)
    loss.backward()
    _check_grads(x, W, b, ref, torch.bfloat16)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_several_chunks_match_one(dtype, monkeypatch):
    """Chunks of 256 tokens (weight/bias gradients accumulated in fp32 over
    chunks) against one chunk: equal up to fp32 summation order."""
    x, W, b, t = _case(700, 64, 264, dtype=dtype, bias=True, seed=9)
    t[::3] = -100
    loss1 = forge_fused_linear_cross_entropy(x, W, t, bias=b)
    loss1.backward()
    g1 = [p.grad.clone() for p in (x, W, b)]
    for p in (x, W, b):
        p.grad = None
    monkeypatch.setattr(flce_mod, "_LOGITS_CHUNK_BYTES", 256 * 264 * x.element_size())
    assert flce_mod._chunk_rows(700, 264 * x.element_size()) == 256
    loss3 = forge_fused_linear_cross_entropy(x, W, t, bias=b)
    loss3.backward()
    torch.testing.assert_close(loss3, loss1, rtol=1e-6, atol=1e-6)
    tol = 1e-5 if dtype == torch.float32 else 1e-2
    for p, g in zip((x, W, b), g1):
        torch.testing.assert_close(p.grad.float(), g.float(), rtol=tol, atol=tol)
    ref = _oracle(x, W, b, t)
    _check_grads(x, W, b, ref, dtype)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_token_scaling(dtype):
    x, W, b, t = _case(64, 32, 97, dtype=dtype, bias=True, seed=4)
    t[::6] = -100
    out = forge_fused_linear_cross_entropy(x, W, t, bias=b, use_token_scaling=True, lse_square_scale=1e-3,
                                           softcap=5.0, return_z_loss=True)
    ref = _oracle(x, W, b, t, use_token_scaling=True, lse_square_scale=1e-3, softcap=5.0)
    rtol, atol = _tol(dtype)
    torch.testing.assert_close(out.loss.float().cpu().double(), ref["loss"], rtol=rtol, atol=atol)
    torch.testing.assert_close(out.z_loss.float().cpu().double(), ref["z_loss"], rtol=rtol, atol=atol)
    out.loss.backward()
    _check_grads(x, W, b, ref, dtype)


def test_grad_output_scales_all_gradients():
    x, W, b, t = _case(16, 24, 29, bias=True, seed=2)
    (forge_fused_linear_cross_entropy(x, W, t, bias=b) * 2.5).backward()
    ref = _oracle(x, W, b, t)
    for k in ("dX", "dW", "db"):
        ref[k] = ref[k] * 2.5
    _check_grads(x, W, b, ref)


def test_backward_rejects_non_scalar_grad():
    g = torch.ones(3, device=DEV)
    with pytest.raises(NotImplementedError, match="scalar losses only"):
        flce_mod.fused_linear_cross_entropy_backward(g, None, None, None)


def test_all_ignored_mean_is_zero():
    x, W, b, t = _case(6, 16, 11, bias=True)
    t[:] = -100
    loss = forge_fused_linear_cross_entropy(x, W, t, bias=b)
    assert float(loss) == 0.0
    loss.backward()
    assert float(x.grad.abs().max()) == 0.0 and float(W.grad.abs().max()) == 0.0


# ---------------------------------------------------------------------------
# entry points through the C ABI
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("layout", ["nt", "nn", "tn"])
def test_gemm_generic_layouts(dtype, layout):
    g = torch.Generator().manual_seed(1)
    M, N, K = 67, 45, 131
    A = torch.randn(M, K, generator=g).to(dtype)
    B = torch.randn(K, N, generator=g).to(dtype)
    bias = torch.randn(N, generator=g).to(dtype)
    C0 = torch.randn(M, N, generator=g)
    ref = 0.5 * (A.double() @ B.double()) + 2.0 * C0.double() + bias.double()
    if layout == "nt":    # A [M][K], B given as [N][K]
        a, a_sm, a_sk = A.to(DEV), K, 1
        b, b_sk, b_sn = B.t().contiguous().to(DEV), 1, K
    elif layout == "nn":  # A [M][K], B [K][N]
        a, a_sm, a_sk = A.to(DEV), K, 1
        b, b_sk, b_sn = B.to(DEV), N, 1
    else:                 # A given as [K][M], B [K][N]
        a, a_sm, a_sk = A.t().contiguous().to(DEV), 1, M
        b, b_sk, b_sn = B.to(DEV), N, 1
    C = C0.to(DEV)
    L.check(L.forge_gemm_generic(M, N, K, L.dtype_code(dtype), a.data_ptr(), a_sm, a_sk, b.data_ptr(), b_sk, b_sn,
                                 C.data_ptr(), N, L.DTYPE_F32, 0.5, 2.0, bias.to(DEV).data_ptr(),
                                 L.GEMM_ACT_NONE, L.stream_of(C)), "forge_gemm_generic")
    torch.testing.assert_close(C.cpu().double(), ref, rtol=1e-5, atol=1e-4)


def test_gemm_generic_rejects_bad_arguments():
    assert L.forge_gemm_generic(2, 2, 2, L.DTYPE_F64, None, 2, 1, None, 2, 1, None, 2, L.DTYPE_F32, 1.0, 0.0,
                                None, 0, None) != 0
    assert b"dtype" in L.forge_last_error()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_target_prob_and_row_scale(dtype):
    g = torch.Generator().manual_seed(8)
    x = (torch.randn(9, 50, generator=g) * 3).to(dtype)
    t = torch.randint(0, 50, (9,), generator=g)
    t[2] = -100
    xs = 4.0 * torch.tanh(x.double() / 4.0)
    p = torch.softmax(xs, -1).gather(1, torch.where(t < 0, 0, t).unsqueeze(1)).squeeze(1)
    p[2] = 0
    xd, td = x.to(DEV), t.to(DEV)
    prob = torch.empty(9, device=DEV)
    L.check(L.forge_ce_target_prob(L.dtype_code(dtype), xd.data_ptr(), 50, 9, 50, td.data_ptr(), 1, -100, 4.0,
                                   prob.data_ptr(), L.stream_of(xd)), "forge_ce_target_prob")
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    torch.testing.assert_close(prob.cpu().double(), p, rtol=tol, atol=tol)
    L.check(L.forge_row_scale(L.dtype_code(dtype), xd.data_ptr(), 50, 9, 50, prob.data_ptr(), L.stream_of(xd)),
            "forge_row_scale")
    torch.testing.assert_close(xd.cpu().double(), x.double() * prob.cpu().double().unsqueeze(1),
                               rtol=tol, atol=tol)


def test_bench_shape_one_chunk():
    """The benchmarked configuration at its full size: BT = 8192, H = 4096,
    V = 128256 (Llama-3-8B's lm_head), bf16, 410 ignored targets, mean.  The
    batch is one 2 GiB logits chunk, so dW is the one bf16-output product
    (no fp32 accumulator).  Reference: the same formula in fp32 on the GPU
    (F.linear + F.cross_entropy + autograd on fp32 copies of the bf16
    inputs; too large for the CPU oracle).  Loss within 1e-3 relative;
    gradients within the bf16 tolerance scaled by each gradient's RMS."""
    BT, H, V = 8192, 4096, 128256
    g = torch.Generator(device=DEV).manual_seed(5)
    x = torch.randn(BT, H, device=DEV, generator=g).to(torch.bfloat16).requires_grad_(True)
    W = (torch.randn(V, H, device=DEV, generator=g) / H ** 0.5).to(torch.bfloat16).requires_grad_(True)
    t = torch.randint(0, V, (BT,), device=DEV, generator=g)
    t[torch.randperm(BT, device=DEV, generator=g)[:410]] = -100
    assert flce_mod._chunk_rows(BT, V * 2) == BT  # one chunk
    loss = forge_fused_linear_cross_entropy(x, W, t)
    loss.backward()
    dx, dw = x.grad, W.grad

    xr = x.detach().float().requires_grad_(True)
    Wr = W.detach().float().requires_grad_(True)
    ref = torch.nn.functional.cross_entropy(torch.nn.functional.linear(xr, Wr), t, ignore_index=-100)
    ref.backward()
    assert abs(loss.item() - ref.item()) <= 1e-3 * abs(ref.item())
    for got, want, name in ((dx, xr.grad, "dX"), (dw, Wr.grad, "dW")):
        err = (got.float() - want).abs()
        scale = want.pow(2).mean().sqrt().item()
        assert err.max().item() <= 2e-2 * scale + 2e-2 * want.abs().max().item(), name
        assert err.mean().item() <= 1e-2 * scale, name
        cos = torch.nn.functional.cosine_similarity(got.float().flatten(), want.flatten(), dim=0).item()
        assert cos > 0.9999, (name, cos)
    assert dx[t == -100].abs().max().item() == 0  # ignored rows: dlogits zero-filled, so their dX rows are zero
