"""LoRA-MLP parity: the fused MFMA pipeline (LoRAMLPv6 / LoRAMLPv3 through
libforge_hip.so: the gate/up GEMM with the LoRA-B K segments and the SwiGLU
epilogue, the down-projection GEMM, the down-projection backward GEMM with
the in-place SwiGLU-backward epilogue, the dX GEMM) vs the CPU oracle
(kernels/lora_mlp/reference/lora_mlp_pytorch.py restated, fp32 on the same
bf16 values).

Tolerance (bf16): |a - b| <= 2e-2 * max(1, rms(b)) + 2e-2 |b| elementwise, and
cosine similarity > 0.9999 (the reference's forge/tests/test_lora_mlp.py:56-66
acceptance).  The BASELINE config (M=8192, H=4096, I=14336, r=16) is checked
on token rows of out / dX and on every LoRA gradient over all 8192 tokens
against the oracle.
"""
import pytest
import torch

from kernels.lora_mlp.experiments.v3.lora_mlp_kernel_v3 import LoRAMLPv3, lora_mlp_v3
from kernels.lora_mlp.experiments.v6.lora_mlp_kernel_v6 import LoRAMLPv6, LoRAMLPv6Module, lora_mlp_v6
from oracle import lora_mlp as orc
from _parity import close_bf16 as _close_bf16

NAMES = ["dX", "dA_gate", "dB_gate", "dA_up", "dB_up", "dA_down", "dB_down"]




def _params_cuda(params):
    out = []
    for t in params:
        out.append(t.cuda().requires_grad_(t.shape[0] <= 64 or t.shape[1] <= 64) if isinstance(t, torch.Tensor) else t)
    return out


def _run(fn, X, dY, params):
    p = _params_cuda(params)
    x = X.cuda().requires_grad_(True)
    out = fn(x, *p)
    out.backward(dY.cuda())
    lora = [p[1], p[2], p[5], p[6], p[9], p[10]]
    return out, [x.grad] + [t.grad for t in lora]


@pytest.mark.gpu
@pytest.mark.parametrize("B,S,H,I,r,alpha", [(2, 128, 512, 1024, 16, 32), (1, 200, 256, 768, 8, 16),
                                              (2, 256, 1024, 2816, 64, 128)])
@pytest.mark.parametrize("version", ["v6", "v3"])
def test_lora_mlp_matches_oracle(B, S, H, I, r, alpha, version):
    gen = torch.Generator().manual_seed(B * S + H + r)
    params = orc.make_params(H, I, r, alpha, gen)
    X = torch.randn(B, S, H, generator=gen).to(torch.bfloat16)
    dY = torch.randn(B, S, H, generator=gen).to(torch.bfloat16)
    ref_out, ref_grads = orc.fwd_bwd(X, dY, params)
    fn = (lambda x, *p: LoRAMLPv6.apply(x, *p)) if version == "v6" else (lambda x, *p: LoRAMLPv3.apply(x, *p))
    out, grads = _run(fn, X, dY, params)
    assert out.shape == (B, S, H) and out.dtype == torch.bfloat16
    _close_bf16(out.reshape(-1, H), ref_out, "out")
    for n, a, b in zip(NAMES, grads, ref_grads):
        _close_bf16(a.reshape(b.shape), b, n)


@pytest.mark.gpu
def test_lora_mlp_saved_tensors_contract():
    """save_for_backward = (A_gate, B_gate, A_up, B_up, A_down, B_down, X, e, g)
    with e/g = pre-activations WITH LoRA added (v6 :586)."""
    gen = torch.Generator().manual_seed(3)
    H, I, r = 256, 512, 16
    params = orc.make_params(H, I, r, 32, gen)
    X = torch.randn(1, 64, H, generator=gen).to(torch.bfloat16)
    p = _params_cuda(params)
    x = X.cuda().requires_grad_(True)
    out = LoRAMLPv6.apply(x, *p)
    saved = out.grad_fn.saved_tensors
    assert len(saved) == 9 and saved[6].data_ptr() == x.data_ptr()
    _, e_ref, g_ref = orc.forward(X.float().reshape(-1, H), *[t.float() if isinstance(t, torch.Tensor) else t for t in params])
    _close_bf16(saved[7].reshape(-1, I), e_ref, "e")
    _close_bf16(saved[8].reshape(-1, I), g_ref, "g")


@pytest.mark.gpu
def test_lora_mlp_no_grad_api_and_module():
    gen = torch.Generator().manual_seed(4)
    H, I, r = 256, 512, 16
    params = orc.make_params(H, I, r, 32, gen)
    X = torch.randn(2, 32, H, generator=gen).to(torch.bfloat16)
    ref_out, _, _ = orc.forward(X.float().reshape(-1, H), *[t.float() if isinstance(t, torch.Tensor) else t for t in params])
    p = [t.cuda() if isinstance(t, torch.Tensor) else t for t in params]
    _close_bf16(lora_mlp_v6(X.cuda(), *p).reshape(-1, H), ref_out, "lora_mlp_v6")
    _close_bf16(lora_mlp_v3(X.cuda(), *p).reshape(-1, H), ref_out, "lora_mlp_v3")
    m = LoRAMLPv6Module(H, I, r, dtype=torch.bfloat16, device="cuda")
    y = m(torch.randn(2, 16, H, device="cuda", dtype=torch.bfloat16))
    y.float().sum().backward()
    assert m.A_gate.grad is not None and m.W_gate.grad is None


@pytest.mark.gpu
def test_lora_mlp_fp64_gradcheck_uses_reference_torch_path():
    """v6 :552-557 / tests :1560: float64 goes through the PyTorch formulas."""
    gen = torch.Generator().manual_seed(5)
    H, I, r = 8, 12, 2
    params = [t.double().cuda() if isinstance(t, torch.Tensor) else t for t in orc.make_params(H, I, r, 4, gen)]
    for i in (1, 2, 5, 6, 9, 10):
        params[i].requires_grad_(True)
    X = torch.randn(1, 3, H, dtype=torch.float64, device="cuda", requires_grad=True)
    assert torch.autograd.gradcheck(lambda x, *lp: LoRAMLPv6.apply(
        x, params[0], lp[0], lp[1], params[3], params[4], lp[2], lp[3], params[7], params[8], lp[4], lp[5], params[11]),
        (X, params[1], params[2], params[5], params[6], params[9], params[10]))


@pytest.mark.gpu
def test_lora_mlp_gradients_are_deterministic():
    """Split-K products are reduced in a fixed order (no atomics), so two
    identical fwd+bwd passes give bit-identical outputs and gradients."""
    gen = torch.Generator().manual_seed(77)
    H, I, r = 512, 1536, 16
    params = orc.make_params(H, I, r, 32, gen)
    X = torch.randn(1, 2048, H, generator=gen).to(torch.bfloat16)
    dY = torch.randn(1, 2048, H, generator=gen).to(torch.bfloat16)
    out1, g1 = _run(LoRAMLPv6.apply, X, dY, params)
    out2, g2 = _run(LoRAMLPv6.apply, X, dY, params)
    assert torch.equal(out1, out2)
    for a, b in zip(g1, g2):
        assert torch.equal(a, b)


@pytest.mark.gpu
def test_lora_mlp_baseline_config():
    """X [8192, 4096] ~ N(0,1), W ~ N(0, 0.02^2),
    r=16, alpha=32, A Kaiming-uniform, B ~ N(0, 0.01^2).  out and dX on the
    first and last 128 token rows (a row depends only on the same row of X /
    dY), and all six LoRA gradients, sums over the 8192 tokens, against the
    oracle's lora_grads."""
    gen = torch.Generator().manual_seed(31)
    M, H, I, r = 8192, 4096, 14336, 16
    params = orc.make_params(H, I, r, 32, gen)
    X = torch.randn(1, M, H, generator=gen).to(torch.bfloat16)
    dY = torch.randn(1, M, H, generator=gen).to(torch.bfloat16)
    out, grads = _run(lambda x, *p: LoRAMLPv6.apply(x, *p), X, dY, params)
    rows = torch.cat([torch.arange(128), torch.arange(M - 128, M)])
    ref_out, ref_grads = orc.fwd_bwd(X[:, rows], dY[:, rows], params)
    _close_bf16(out.reshape(-1, H)[rows.cuda()], ref_out, "out rows")
    _close_bf16(grads[0].reshape(-1, H)[rows.cuda()], ref_grads[0], "dX rows")
    del ref_grads
    c = lambda t: t.float() if isinstance(t, torch.Tensor) else t  # noqa: E731
    ref_lora = orc.lora_grads(c(dY).reshape(M, H), c(X).reshape(M, H), *[c(t) for t in params])
    for name, a, b in zip(NAMES[1:], grads[1:], ref_lora):
        _close_bf16(a, b, name + " over 8192 tokens")


@pytest.mark.gpu
@pytest.mark.parametrize("scales", [(2.0, 2.0, 2.0), (1.5, 0.5, 3.0)])
def test_lora_mlp_per_projection_scales(scales):
    """Equal gate / up scales take the one-launch [df B_u | de B_g] product,
    different ones a launch each; both against the oracle."""
    B, S, H, I, r = 2, 300, 512, 1536, 16
    gen = torch.Generator().manual_seed(23)
    params = list(orc.make_params(H, I, r, 2 * r, gen))
    params[3], params[7], params[11] = scales
    X = torch.randn(B, S, H, generator=gen).to(torch.bfloat16)
    dY = torch.randn(B, S, H, generator=gen).to(torch.bfloat16)
    ref_out, ref_grads = orc.fwd_bwd(X, dY, params)
    out, grads = _run(lambda x, *p: LoRAMLPv6.apply(x, *p), X, dY, params)
    _close_bf16(out.reshape(-1, H), ref_out, "out")
    for n, a, b in zip(NAMES, grads, ref_grads):
        _close_bf16(a.reshape(b.shape), b, n)


@pytest.mark.gpu
@pytest.mark.parametrize("r", [4, 12])
@pytest.mark.parametrize("version", ["v6", "v3"])
def test_lora_mlp_rank_not_multiple_of_8(r, version):
    """Ranks the MFMA core's K segments do not take directly (r % 8 != 0) are
    zero-padded inside the bf16 path; outputs and gradients still match the
    oracle, and the LoRA gradients keep the caller's rank."""
    gen = torch.Generator().manual_seed(40 + r)
    B, S, H, I = 1, 150, 256, 512
    params = orc.make_params(H, I, r, 2 * r, gen)
    X = torch.randn(B, S, H, generator=gen).to(torch.bfloat16)
    dY = torch.randn(B, S, H, generator=gen).to(torch.bfloat16)
    ref_out, ref_grads = orc.fwd_bwd(X, dY, params)
    fn = (lambda x, *p: LoRAMLPv6.apply(x, *p)) if version == "v6" else (lambda x, *p: LoRAMLPv3.apply(x, *p))
    out, grads = _run(fn, X, dY, params)
    _close_bf16(out.reshape(-1, H), ref_out, "out")
    for n, a, b in zip(NAMES, grads, ref_grads):
        if n != "dX":  # the LoRA gradients keep the caller's rank
            assert a.shape == b.shape, n
        _close_bf16(a.reshape(b.shape), b, n)


@pytest.mark.gpu
@pytest.mark.parametrize("act", ["silu", "gelu_tanh", "gelu_exact"])
def test_glu_bwd_pass_equals_fused_down_bwd_epilogue(act):
    """forge_lora_mlp_glu_bwd (the backend of swiglu_DWf_DW_dfg_kernel) on D
    equals forge_lora_mlp_down_bwd's in-place epilogue bit for bit when the
    GEMM's DW is exact: W_down = identity and a zero LoRA term make DW = dY,
    so both see the same D."""
    import torch
    from forge_hip import _lib as L
    from kernels.lora_mlp._impl import ACTIVATIONS

    torch.manual_seed(5)
    M, I, r = 1000, 512, 8
    bf = torch.bfloat16
    dY = torch.randn(M, I, device="cuda").to(bf)
    eye = torch.eye(I, device="cuda", dtype=bf)
    td = torch.zeros(M, r, device="cuda", dtype=bf)
    AdT = torch.zeros(I, r, device="cuda", dtype=bf)
    e0 = (torch.randn(M, I, device="cuda") * 2).to(bf)
    g0 = torch.randn(M, I, device="cuda").to(bf)
    code = ACTIVATIONS[act]
    st = L.stream_of(dY)
    e1, g1, h1 = e0.clone(), g0.clone(), torch.empty_like(e0)
    L.check(L.forge_lora_mlp_down_bwd(M, I, I, r, dY.data_ptr(), I, eye.data_ptr(), I, td.data_ptr(), r,
                                      AdT.data_ptr(), r, L.LAYOUT_COL, h1.data_ptr(), e1.data_ptr(), g1.data_ptr(), I,
                                      code, st), "down_bwd")
    # the standalone pass on a padded pitch, e and g side by side in one buffer
    P = 2 * I + 64
    egv = torch.zeros(M, P, device="cuda", dtype=bf)
    egv[:, :I], egv[:, I:2 * I] = e0, g0
    h2 = torch.empty(M, P, device="cuda", dtype=bf)
    L.check(L.forge_lora_mlp_glu_bwd(M, I, dY.data_ptr(), I, egv.data_ptr(), egv[:, I:].data_ptr(), P,
                                     h2.data_ptr(), P, code, st), "glu_bwd")
    torch.cuda.synchronize()
    assert torch.equal(h2[:, :I], h1)
    assert torch.equal(egv[:, :I], e1)
    assert torch.equal(egv[:, I:2 * I], g1)
    assert torch.count_nonzero(egv[:, 2 * I:]) == 0


@pytest.mark.gpu
def test_unsloth_helpers_match_oracle():
    """matmul_lora, swiglu_fg_kernel and the in-place swiglu_DWf_DW_dfg_kernel
    (unsloth_baseline.py:34-55, 72-168) against float64 restatements of
    Unsloth's formulas on the same bf16 values: the GEMM within the bf16 bar,
    the elementwise steps within one bf16 rounding (their fp32 math and cast
    points are Unsloth's)."""
    from kernels.lora_mlp.unsloth_ops import matmul_lora, swiglu_DWf_DW_dfg_kernel, swiglu_fg_kernel

    gen = torch.Generator().manual_seed(61)
    B, S, H, I, r = 2, 96, 256, 512, 12
    params = orc.make_params(H, I, r, 2 * r, gen)
    X = torch.randn(B, S, H, generator=gen).to(torch.bfloat16)
    W, A, Bm, s = params[0], params[1], params[2], params[3]
    got = matmul_lora(X.cuda(), W.cuda(), None, A.cuda(), Bm.cuda(), s)
    assert got.shape == (B, S, I)
    ref = orc.matmul_lora(X.reshape(-1, H).double(), W.double(), A.double(), Bm.double(), s)
    _close_bf16(got.reshape(-1, I), ref.float(), "matmul_lora")
    _close_bf16(matmul_lora(X.cuda().float(), W.cuda().float(), None, A.cuda().float(), Bm.cuda().float(),
                            s).reshape(-1, I), ref.float(), "matmul_lora fp32")

    e = (torch.randn(B, S, I, generator=gen) * 3).to(torch.bfloat16)
    g = torch.randn(B, S, I, generator=gen).to(torch.bfloat16)
    DW = torch.randn(B * S, I, generator=gen).to(torch.bfloat16)
    ed, gd = e.double(), g.double()
    se = torch.sigmoid(ed)
    f = (ed * se).to(torch.bfloat16).double()
    h = swiglu_fg_kernel(e.cuda(), g.cuda())
    torch.testing.assert_close(h.cpu().double(), (f * gd).to(torch.bfloat16).double(), rtol=2 ** -6, atol=1e-6)

    e2, g2, dw2 = e.reshape(-1, I).cuda(), g.reshape(-1, I).cuda(), DW.cuda()
    out = swiglu_DWf_DW_dfg_kernel(dw2, e2, g2)
    assert out[0].data_ptr() == dw2.data_ptr() and out[1].data_ptr() == e2.data_ptr()
    f2, dwd = f.reshape(-1, I), DW.double()
    se2, ed2, gd2 = se.reshape(-1, I), ed.reshape(-1, I), gd.reshape(-1, I)
    dg = (dwd * gd2).to(torch.bfloat16).double()
    exp = [(f2 * gd2), (dwd * f2), dg * se2 * (1 + ed2 * (1 - se2))]
    for name, a, b in zip(("h", "df", "de"), (dw2, e2, g2), exp):
        torch.testing.assert_close(a.cpu().double(), b.to(torch.bfloat16).double(), rtol=2 ** -6, atol=1e-6,
                                   msg=lambda m: f"{name}: {m}")


@pytest.mark.gpu
@pytest.mark.parametrize("M,I,r,act", [(256, 512, 16, "silu"), (300, 776, 8, "silu"), (512, 1280, 64, "silu"),
                                       (130, 264, 24, "silu"), (256, 512, 16, "gelu_tanh"), (130, 264, 24, "gelu_exact")])
def test_down_bwd_rank_partials(M, I, r, act):
    """forge_lora_mlp_down_bwd_v: the same h, df, de as forge_lora_mlp_down_bwd
    (bit for bit), partial sums over its column tiles that add up to
    [df B_u | de B_g], and with w_part partial sums over its row tiles that add
    up to [df^T xa_u | de^T xa_g] (fp32 references on the GPU from the df, de
    it wrote; ragged M, I not a multiple of 256, ranks 8..64, SiLU and both
    GELU forms).  xa^T's pitch is padded past M with NaN, which a read of a
    token outside the tile would carry into the sums."""
    from forge_hip import _lib as L
    from kernels.lora_mlp._impl import ACTIVATIONS

    code = ACTIVATIONS[act]
    torch.manual_seed(M + I + r)
    H = 256
    dev = "cuda"
    bf = torch.bfloat16
    dY = torch.randn(M, H, device=dev).to(bf)
    WdT = (torch.randn(I, H, device=dev) * 0.05).to(bf)       # W_down^T [I][H]
    td = (torch.randn(M, r, device=dev) * 0.1).to(bf)
    AdT = (torch.randn(I, r, device=dev) * 0.1).to(bf)        # A_down^T [I][r]
    e0 = torch.randn(M, I, device=dev).to(bf)
    g0 = torch.randn(M, I, device=dev).to(bf)
    BuT = (torch.randn(r, I, device=dev) * 0.1).to(bf)
    BgT = (torch.randn(r, I, device=dev) * 0.1).to(bf)
    ldx = -(-M // 8) * 8
    xaT = torch.full((2 * r, ldx), float("nan"), device=dev, dtype=bf)   # rows [gate; up], tokens < M valid
    xaT[:, :M] = (torch.randn(2 * r, M, device=dev) * 0.5).to(bf)
    st = L.stream_of(dY)
    outs = []
    n_ct, n_rt = (I + 255) // 256, (M + 255) // 256
    for mode in ("plain", "v", "vw"):
        e, g = e0.clone(), g0.clone()
        h = torch.empty(M, I, device=dev, dtype=bf)
        vpart = torch.full((n_ct, M, 2 * r), float("nan"), device=dev)
        wpart = torch.full((n_rt, 2, I, r), float("nan"), device=dev)
        if mode == "plain":
            L.check(L.forge_lora_mlp_down_bwd(M, H, I, r, dY.data_ptr(), H, WdT.data_ptr(), H, td.data_ptr(), r,
                                              AdT.data_ptr(), r, L.LAYOUT_COL, h.data_ptr(), e.data_ptr(),
                                              g.data_ptr(), I, code, st), "forge_lora_mlp_down_bwd")
        else:
            w = mode == "vw"
            L.check(L.forge_lora_mlp_down_bwd_v(M, H, I, r, dY.data_ptr(), H, WdT.data_ptr(), H, td.data_ptr(), r,
                                                AdT.data_ptr(), r, h.data_ptr(), e.data_ptr(), g.data_ptr(), I,
                                                code, BuT.data_ptr(), BgT.data_ptr(), I, r, vpart.data_ptr(),
                                                xaT[r:].data_ptr() if w else None, xaT[:r].data_ptr() if w else None,
                                                ldx, wpart.data_ptr() if w else None, st),
                    "forge_lora_mlp_down_bwd_v")
        outs.append((h, e, g, vpart, wpart))
    (h0, df0, de0, _, _), (h1, df1, de1, vpart, _), (h2, df2, de2, vpart2, wpart) = outs
    assert torch.equal(h0, h1) and torch.equal(df0, df1) and torch.equal(de0, de1)
    assert torch.equal(h0, h2) and torch.equal(df0, df2) and torch.equal(de0, de2) and torch.equal(vpart, vpart2)
    assert not torch.isnan(vpart).any()
    got = vpart.sum(0)
    want = torch.cat([df1.float() @ BuT.float().t(), de1.float() @ BgT.float().t()], 1)
    torch.testing.assert_close(got, want, rtol=1e-4, atol=1e-3 * want.abs().max().item())
    v = torch.empty(M, 2 * r, device=dev, dtype=bf)
    L.check(L.forge_splitk_reduce(vpart.data_ptr(), M * 2 * r, vpart.shape[0], M, 2 * r, 2 * r, v.data_ptr(), 2 * r,
                                  L.DTYPE_BF16, 1.0, st), "forge_splitk_reduce")
    torch.testing.assert_close(v.float(), want, rtol=1e-2, atol=1e-2 * want.abs().max().item())
    # B gradients' token reductions
    assert not torch.isnan(wpart).any()
    xa = xaT[:, :M].float().t()                                  # [M, 2r]: [xa_g | xa_u]
    want_w = torch.cat([df1.float().t() @ xa[:, r:], de1.float().t() @ xa[:, :r]], 1)   # [I, 2r]
    torch.testing.assert_close(torch.cat([wpart[:, 0].sum(0), wpart[:, 1].sum(0)], 1), want_w, rtol=1e-4,
                               atol=1e-3 * want_w.abs().max().item())
    dB = torch.empty(I, r, device=dev, dtype=bf)
    L.check(L.forge_splitk_reduce(wpart[0, 1].data_ptr(), 2 * I * r, n_rt, I, r, r, dB.data_ptr(), r,
                                  L.DTYPE_BF16, 1.0, st), "forge_splitk_reduce")
    torch.testing.assert_close(dB.float(), want_w[:, r:], rtol=1e-2, atol=1e-2 * want_w.abs().max().item())


@pytest.mark.gpu
@pytest.mark.parametrize("M,I,r,act", [(256, 512, 16, "silu"), (300, 776, 8, "silu"), (512, 1280, 64, "silu"),
                                       (130, 392, 24, "gelu_tanh"), (256, 512, 16, "gelu_exact")])
def test_gate_up_rank_partials(M, I, r, act):
    """forge_lora_mlp_gate_up_v: the same e, g, h as forge_lora_mlp_gate_up
    (bit for bit), and partial sums over its 128-column tiles that add up to
    h A_down^T (fp32 reference on the GPU from the h it wrote; ragged M, I not
    a multiple of 128, ranks 8..64, SiLU and both GELU forms)."""
    from forge_hip import _lib as L
    from kernels.lora_mlp._impl import ACTIVATIONS

    code = ACTIVATIONS[act]
    torch.manual_seed(M + I + r + 1)
    H = 256
    dev = "cuda"
    bf = torch.bfloat16
    X = torch.randn(M, H, device=dev).to(bf)
    Wg = (torch.randn(I, H, device=dev) * 0.05).to(bf)
    Wu = (torch.randn(I, H, device=dev) * 0.05).to(bf)
    xa = (torch.randn(M, 2 * r, device=dev) * 0.1).to(bf)
    Bg = (torch.randn(I, r, device=dev) * 0.1).to(bf)
    Bu = (torch.randn(I, r, device=dev) * 0.1).to(bf)
    Ad = (torch.randn(r, I, device=dev) * 0.1).to(bf)
    st = L.stream_of(X)
    outs = []
    for with_v in (False, True):
        e, g, h = (torch.empty(M, I, device=dev, dtype=bf) for _ in range(3))
        n_ct = (I + 127) // 128
        xpart = torch.full((n_ct, M, r), float("nan"), device=dev)
        common = (M, H, I, r, X.data_ptr(), H, Wg.data_ptr(), Wu.data_ptr(), H, xa.data_ptr(), 2 * r,
                  Bg.data_ptr(), Bu.data_ptr(), r, e.data_ptr(), g.data_ptr(), h.data_ptr(), I, code)
        if with_v:
            L.check(L.forge_lora_mlp_gate_up_v(*common, Ad.data_ptr(), I, r, xpart.data_ptr(), st),
                    "forge_lora_mlp_gate_up_v")
        else:
            L.check(L.forge_lora_mlp_gate_up(*common, st), "forge_lora_mlp_gate_up")
        outs.append((e, g, h, xpart))
    (e0, g0, h0, _), (e1, g1, h1, xpart) = outs
    assert torch.equal(e0, e1) and torch.equal(g0, g1) and torch.equal(h0, h1)
    assert not torch.isnan(xpart).any()
    want = h1.float() @ Ad.float().t()
    torch.testing.assert_close(xpart.sum(0), want, rtol=1e-4, atol=1e-3 * want.abs().max().item())
