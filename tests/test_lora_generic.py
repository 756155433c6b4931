"""LoRA-MLP and LoRA-QKV with fp32 and fp16 inputs: the generic-GEMM path
(kernels/_generic_lora.py) behind the same entry points as the bf16 MFMA
path.  The reference's own tests call these entry points in fp32
(kernels/lora_mlp/tests/test_lora_mlp.py:507-549 lora_mlp_v3, :1348-1456
lora_mlp_v6 with ranks 8-64, :568-583 fused_lora_swiglu, :1316-1329
fused_lora_a_stacked; kernels/lora_qkv/tests/test_v2_2_v2_3_v3.py); the
cases below take their shapes and ranks, plus rank 4 and ragged token counts.

Oracle: oracle/lora_mlp.py and oracle/lora_qkv.py evaluated in float64 on the
same values.  Tolerances: fp32 |a - b| <= 1e-5 |b| + 1e-5 max(1, rms(b));
fp16 2e-2 (the bf16 criterion of _parity.close_bf16).
"""
import pytest
import torch

from _parity import close_bf16
from oracle import lora_mlp as omlp
from oracle import lora_qkv as oqkv
from oracle.rope import cos_sin

MLP_NAMES = ["dX", "dA_gate", "dB_gate", "dA_up", "dB_up", "dA_down", "dB_down"]
QKV_NAMES = ["dX", "dA_q", "dB_q", "dA_k", "dB_k", "dA_v", "dB_v"]


def close(a, b, what, dtype):
    a = a.detach().double().cpu()
    b = b.detach().double().cpu().reshape(a.shape)
    if dtype == torch.float16:
        return close_bf16(a, b, what)
    scale = max(1.0, b.pow(2).mean().sqrt().item())
    torch.testing.assert_close(a, b, rtol=1e-5, atol=1e-5 * scale, msg=lambda m: f"{what}: {m}")


def _mlp_case(H, I, r, dtype, seed, B=2, S=64):
    gen = torch.Generator().manual_seed(seed)
    params = omlp.make_params(H, I, r, 2 * r, gen, dtype=torch.float64)
    X = torch.randn(B, S, H, generator=gen, dtype=torch.float64).to(dtype)
    dY = torch.randn(B, S, H, generator=gen, dtype=torch.float64).to(dtype)
    params = tuple(t.to(dtype) if isinstance(t, torch.Tensor) else t for t in params)
    return params, X, dY


def _mlp_run(apply, X, dY, params):
    p = [t.cuda().requires_grad_(i in (1, 2, 5, 6, 9, 10)) if isinstance(t, torch.Tensor) else t
         for i, t in enumerate(params)]
    x = X.cuda().requires_grad_(True)
    out = apply(x, *p)
    out.backward(dY.cuda())
    return out, [x.grad] + [p[i].grad for i in (1, 2, 5, 6, 9, 10)]


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
@pytest.mark.parametrize("version,r,S", [("v6", 16, 64), ("v3", 16, 64), ("v6", 4, 37), ("v6", 8, 64),
                                         ("v6", 32, 64), ("v3", 64, 64)])
def test_lora_mlp_generic_dtypes_match_oracle(dtype, version, r, S):
    from kernels.lora_mlp.experiments.v3.lora_mlp_kernel_v3 import LoRAMLPv3
    from kernels.lora_mlp.experiments.v6.lora_mlp_kernel_v6 import LoRAMLPv6

    H, I = 128, 256
    params, X, dY = _mlp_case(H, I, r, dtype, seed=r + S)
    ref_out, ref_grads = omlp.fwd_bwd(X, dY, params, compute_dtype=torch.float64)
    fn = LoRAMLPv6 if version == "v6" else LoRAMLPv3
    print(f"lora_mlp {version} {dtype} r={r} S={S}", flush=True)
    out, grads = _mlp_run(lambda x, *p: fn.apply(x, *p), X, dY, params)
    assert out.dtype == dtype and out.shape == X.shape
    close(out.reshape(-1, H), ref_out, "out", dtype)
    for n, a, b in zip(MLP_NAMES, grads, ref_grads):
        assert a.dtype == dtype
        close(a, b, n, dtype)


@pytest.mark.gpu
@pytest.mark.parametrize("approximate", ["tanh", "none"])
def test_lora_mlp_geglu_fp32_matches_oracle(approximate):
    from kernels.lora_mlp.geglu_mlp import LoRAMLPGeGLU

    H, I, r = 128, 256, 16
    params, X, dY = _mlp_case(H, I, r, torch.float32, seed=11)
    act = "gelu_tanh" if approximate == "tanh" else "gelu_exact"
    ref_out, ref_grads = omlp.fwd_bwd(X, dY, params, compute_dtype=torch.float64, activation=act)
    out, grads = _mlp_run(lambda x, *p: LoRAMLPGeGLU.apply(x, *p, approximate), X, dY, params)
    close(out.reshape(-1, H), ref_out, "out", torch.float32)
    for n, a, b in zip(MLP_NAMES, grads, ref_grads):
        close(a, b, n, torch.float32)


@pytest.mark.gpu
def test_lora_mlp_fp32_forward_only_apis():
    """lora_mlp_v3 / lora_mlp_v6 (no autograd), fused_lora_swiglu and
    fused_lora_a_stacked in fp32 (the reference's fp32 cases)."""
    from kernels.lora_mlp.experiments.v3.lora_mlp_kernel_v3 import fused_lora_swiglu, lora_mlp_v3
    from kernels.lora_mlp.experiments.v6.lora_mlp_kernel_v6 import fused_lora_a_stacked, lora_mlp_v6, stack_lora_a

    H, I, r = 128, 256, 16
    params, X, _ = _mlp_case(H, I, r, torch.float32, seed=12)
    ref_out, _, _ = omlp.forward(X.double().reshape(-1, H),
                                 *[t.double() if isinstance(t, torch.Tensor) else t for t in params])
    p = [t.cuda() if isinstance(t, torch.Tensor) else t for t in params]
    for fn in (lora_mlp_v3, lora_mlp_v6):
        close(fn(X.cuda(), *p).reshape(-1, H), ref_out, fn.__name__, torch.float32)

    gen = torch.Generator().manual_seed(13)
    M, N = 256, 512
    e, g = (torch.randn(M, N, generator=gen, dtype=torch.float64) for _ in range(2))
    xg, xu = (torch.randn(M, r, generator=gen, dtype=torch.float64) for _ in range(2))
    Bg, Bu = (torch.randn(N, r, generator=gen, dtype=torch.float64) for _ in range(2))
    ef, gf = e + 0.5 * xg @ Bg.t(), g + 2.0 * xu @ Bu.t()
    ref = ef * torch.sigmoid(ef) * gf
    c = [t.float().cuda() for t in (e, g, xg, xu, Bg, Bu)]
    h, e_full, g_full = fused_lora_swiglu(*c, 0.5, 2.0, save_eg=True)
    close(h, ref, "fused_lora_swiglu", torch.float32)
    close(e_full, ef, "e_full", torch.float32)
    close(g_full, gf, "g_full", torch.float32)

    A_stack = stack_lora_a(p[1], p[5])
    xa_g, xa_u = fused_lora_a_stacked(X.cuda(), A_stack, r)
    Xd = X.double().reshape(-1, H)
    close(xa_g, Xd @ params[1].double().t(), "xa_gate", torch.float32)
    close(xa_u, Xd @ params[5].double().t(), "xa_up", torch.float32)


@pytest.mark.gpu
def test_lora_mlp_mixed_dtypes_are_rejected():
    from kernels.lora_mlp.experiments.v6.lora_mlp_kernel_v6 import LoRAMLPv6

    params, X, _ = _mlp_case(128, 256, 16, torch.float32, seed=14)
    p = [t.cuda() if isinstance(t, torch.Tensor) else t for t in params]
    p[1] = p[1].to(torch.float16)
    with pytest.raises(TypeError, match="one dtype"):
        LoRAMLPv6.apply(X.cuda(), *p)


def _qkv_case(K, Hq, Hkv, r, dtype, seed, T=96):
    gen = torch.Generator().manual_seed(seed)
    params = oqkv.make_params(K, Hq, Hkv, r, 2 * r, gen, dtype=torch.float64)
    X = torch.randn(T, K, generator=gen, dtype=torch.float64).to(dtype)
    d = [torch.randn(T, n, generator=gen, dtype=torch.float64).to(dtype) for n in (Hq, Hkv, Hkv)]
    return tuple(t.to(dtype) if isinstance(t, torch.Tensor) else t for t in params), X, d


def _qkv_params_cuda(params):
    return [t.cuda().requires_grad_(i in (3, 4, 6, 7, 9, 10)) if isinstance(t, torch.Tensor) else t
            for i, t in enumerate(params)]


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
@pytest.mark.parametrize("api", ["v3", "v4"])
def test_lora_qkv_generic_dtypes_match_oracle(dtype, api):
    from kernels.lora_qkv.experiments.v2.lora_qkv_kernel_v2_3 import lora_qkv_v2_3
    from kernels.lora_qkv.experiments.v3.lora_qkv_kernel_v3 import LoRAQKVFunction
    from kernels.lora_qkv.experiments.v4.lora_qkv_kernel_v4 import LoRAQKVv4Function

    K, Hq, Hkv, r = 256, 256, 128, 8
    params, X, (dQ, dK, dV) = _qkv_case(K, Hq, Hkv, r, dtype, seed=21, T=97)
    pd = [t.double() if isinstance(t, torch.Tensor) else t for t in params]
    Xd = X.double()
    ref = oqkv.forward(Xd, *pd)
    ref_grads = oqkv.backward(dQ.double(), dK.double(), dV.double(), Xd, *pd)
    p = _qkv_params_cuda(params)
    x = X.cuda().requires_grad_(True)
    fn = LoRAQKVFunction if api == "v3" else LoRAQKVv4Function
    print(f"lora_qkv {api} {dtype}", flush=True)
    outs = fn.apply(x, *p)
    for a, b, n in zip(outs, ref, "QKV"):
        assert a.dtype == dtype
        close(a, b, n, dtype)
    torch.autograd.backward(outs, (dQ.cuda(), dK.cuda(), dV.cuda()))
    got = [x.grad] + [p[i].grad for i in (3, 4, 6, 7, 9, 10)]
    for n, a, b in zip(QKV_NAMES, got, ref_grads):
        close(a, b, n, dtype)
    with torch.no_grad():  # v2_3 argument order: (X, W_q, A_q, B_q, s_q, W_k, ...)
        o23 = lora_qkv_v2_3(X.cuda(), p[0], p[3], p[4], p[5], p[1], p[6], p[7], p[8], p[2], p[9], p[10], p[11])
    for a, b, n in zip(o23, ref, "QKV"):
        close(a, b, "v2_3 " + n, dtype)


@pytest.mark.gpu
@pytest.mark.parametrize("head_dim", [128, 64])
def test_lora_qkv_rope_fp32_matches_oracle(head_dim):
    """lora_qkv_rope in fp32: the generic QKV products, RoPE by the RoPE
    kernel on fp32 tables, varlen positions; backward through the rotation."""
    from kernels.lora_qkv.experiments.v4.lora_qkv_kernel_v4 import lora_qkv_rope

    lens = [37, 50, 29]
    pos = oqkv.positions_for(lens)
    T, K, Hq, Hkv, r = int(pos.numel()), 256, 512, 256, 16
    params, X, (dQ, dK, dV) = _qkv_case(K, Hq, Hkv, r, torch.float32, seed=22 + head_dim, T=T)
    c, s = cos_sin(torch.arange(64), head_dim, 500000.0, torch.float64)
    (Qr, Kr, Vr), ref_grads = oqkv.qkv_rope_fwd_bwd(X, dQ, dK, dV, params, c[pos], s[pos], head_dim,
                                                    compute_dtype=torch.float64)
    p = _qkv_params_cuda(params)
    x = X.cuda().requires_grad_(True)
    Q, K_, V = lora_qkv_rope(x, p[0], p[3], p[4], p[5], p[1], p[6], p[7], p[8], p[2], p[9], p[10], p[11],
                             c.float().cuda(), s.float().cuda(), pos.cuda(), head_dim)
    for a, b, n in ((Q, Qr, "Q"), (K_, Kr, "K"), (V, Vr, "V")):
        assert a.dtype == torch.float32
        close(a, b, n, torch.float32)
    torch.autograd.backward((Q, K_, V), (dQ.cuda(), dK.cuda(), dV.cuda()))
    got = [x.grad] + [p[i].grad for i in (3, 4, 6, 7, 9, 10)]
    for n, a, b in zip(QKV_NAMES, got, ref_grads):
        close(a, b, n, torch.float32)
