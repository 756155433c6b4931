"""LoRA-MLP merged-weight inference (v5/v6 API) and the activation-epilogue
GEMM that replaces the reference's cuBLASLt SWISH GEMM.

Cases follow kernels/lora_mlp/tests/test_lora_mlp.py:857-888 (inference in
fp32 against the unmerged reference at rtol/atol 1e-4; bf16 against the fp32
reference) with the CPU oracle (oracle/lora_mlp.py, the unmerged
lora_swiglu_mlp) as the checker.  bf16 tolerance: tests/_parity.py
(2e-2 scaled, cosine > 0.9999)."""
import pytest
import torch

from kernels.lora_mlp.experiments.v5.lora_mlp_kernel_v5 import (
    lora_mlp_v5_inference,
    merge_lora_weights,
    prepare_inference_weights,
)
from kernels.lora_mlp.experiments.v6.lora_mlp_kernel_v6 import lora_mlp_v6_inference
from oracle import lora_mlp as orc
from _parity import close_bf16


def test_merge_and_prepare_shapes_cpu():
    gen = torch.Generator().manual_seed(1)
    p = orc.make_params(16, 24, 4, 8, gen, dtype=torch.float64)
    W_eff = merge_lora_weights(p[0], p[1], p[2], p[3])
    torch.testing.assert_close(W_eff, p[0] + p[3] * (p[2] @ p[1]))
    assert merge_lora_weights(p[0], None, p[2], p[3]) is p[0]
    g_t, u_t, d_t = prepare_inference_weights(*p)
    assert g_t.shape == (16, 24) and u_t.shape == (16, 24) and d_t.shape == (24, 16)
    assert g_t.is_contiguous() and d_t.is_contiguous()
    # float64 runs the formula in PyTorch (also on the CPU): equals the unmerged oracle
    X = torch.randn(2, 5, 16, generator=gen, dtype=torch.float64)
    out = lora_mlp_v5_inference(X, g_t, u_t, d_t)
    ref, _, _ = orc.forward(X.reshape(-1, 16), *p)
    torch.testing.assert_close(out.reshape(-1, 16), ref, rtol=1e-10, atol=1e-12)


@pytest.mark.gpu
@pytest.mark.parametrize("B,S,H,I,r", [(2, 128, 256, 512, 16), (1, 300, 512, 1536, 8), (2, 33, 136, 200, 4)])
def test_inference_bf16_matches_unmerged_oracle(B, S, H, I, r):
    """bf16 merged weights: MFMA path (widths multiples of 8) and ragged M;
    H=136, I=200 still take it, out against the unmerged fp32 oracle."""
    gen = torch.Generator().manual_seed(H + I)
    p = orc.make_params(H, I, r, 2 * r, gen)
    X = torch.randn(B, S, H, generator=gen).to(torch.bfloat16)
    ref, _, _ = orc.forward(X.float().reshape(-1, H), *[t.float() if isinstance(t, torch.Tensor) else t for t in p])
    pc = [t.cuda() if isinstance(t, torch.Tensor) else t for t in p]
    wts = prepare_inference_weights(*pc)
    out = lora_mlp_v5_inference(X.cuda(), *wts)
    assert out.shape == (B, S, H) and out.dtype == torch.bfloat16
    close_bf16(out.reshape(-1, H), ref, "inference out")
    assert torch.equal(lora_mlp_v6_inference(X.cuda(), *wts), out)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_inference_fp32_fp16(dtype):
    gen = torch.Generator().manual_seed(7)
    H, I, r = 128, 256, 16
    p = orc.make_params(H, I, r, 32, gen, dtype=torch.float32)
    X = torch.randn(2, 64, H, generator=gen)
    ref, _, _ = orc.forward(X.reshape(-1, H), *p)
    pc = [t.to(dtype).cuda() if isinstance(t, torch.Tensor) else t for t in p]
    out = lora_mlp_v5_inference(X.to(dtype).cuda(), *prepare_inference_weights(*pc))
    if dtype == torch.float32:
        torch.testing.assert_close(out.reshape(-1, H).cpu(), ref, rtol=1e-4, atol=1e-4)
    else:
        torch.testing.assert_close(out.reshape(-1, H).float().cpu(), ref, rtol=2e-2, atol=2e-2)


@pytest.mark.gpu
def test_gate_up_h_only_equals_training_h():
    """The inference call of the gate/up GEMM (no e / g outputs) writes the
    same h, bit for bit, as the training call that also stores e and g."""
    from forge_hip import _lib as L

    gen = torch.Generator().manual_seed(3)
    M, H, I = 300, 512, 768
    X = torch.randn(M, H, generator=gen).to(torch.bfloat16).cuda()
    Wg = (torch.randn(I, H, generator=gen) * 0.02).to(torch.bfloat16).cuda()
    Wu = (torch.randn(I, H, generator=gen) * 0.02).to(torch.bfloat16).cuda()
    e, g, h1, h2 = (torch.empty(M, I, dtype=torch.bfloat16, device="cuda") for _ in range(4))
    st = L.stream_of(X)
    L.check(L.forge_lora_mlp_gate_up(M, H, I, 0, X.data_ptr(), H, Wg.data_ptr(), Wu.data_ptr(), H, None, 0, None,
                                     None, 0, e.data_ptr(), g.data_ptr(), h1.data_ptr(), I, L.ACT_SILU, st), "gate_up")
    L.check(L.forge_lora_mlp_gate_up(M, H, I, 0, X.data_ptr(), H, Wg.data_ptr(), Wu.data_ptr(), H, None, 0, None,
                                     None, 0, None, None, h2.data_ptr(), I, L.ACT_SILU, st), "gate_up h only")
    assert torch.equal(h1, h2)
    assert L.forge_lora_mlp_gate_up(M, H, I, 0, X.data_ptr(), H, Wg.data_ptr(), Wu.data_ptr(), H, None, 0, None,
                                    None, 0, e.data_ptr(), None, h2.data_ptr(), I, L.ACT_SILU, st) != 0


@pytest.mark.gpu
@pytest.mark.parametrize("epilogue", ["none", "swish", "silu", "relu", "gelu"])
@pytest.mark.parametrize("M,K,N", [(512, 256, 768), (1000, 512, 128), (96, 64, 40)])
def test_matmul_epilogue_bf16(epilogue, M, K, N):
    """D = epi(alpha A @ B + beta C) on the MFMA GEMM (big, narrow and small
    tiles) against the fp32 CPU product of the same bf16 values."""
    from kernels.lora_mlp.experiments.v4.cublaslt_wrapper import cublaslt_matmul_epilogue

    gen = torch.Generator().manual_seed(M + N)
    A = torch.randn(M, K, generator=gen).to(torch.bfloat16)
    B = (torch.randn(K, N, generator=gen) / K ** 0.5).to(torch.bfloat16)
    C = torch.randn(M, N, generator=gen).to(torch.bfloat16)
    v = 0.5 * (A.float() @ B.float()) + 0.25 * C.float()
    ref = {"none": v, "swish": torch.nn.functional.silu(v), "silu": torch.nn.functional.silu(v),
           "relu": torch.relu(v), "gelu": torch.nn.functional.gelu(v, approximate="tanh")}[epilogue]
    D = cublaslt_matmul_epilogue(A.cuda(), B.cuda(), epilogue=epilogue, alpha=0.5, beta=0.25, C=C.cuda())
    torch.testing.assert_close(D.float().cpu(), ref, rtol=2e-2, atol=2e-2)


@pytest.mark.gpu
@pytest.mark.parametrize("epilogue", ["none", "silu", "relu", "gelu"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_matmul_epilogue_generic(epilogue, dtype):
    """fp32 / fp16 operands, and bf16 with K and N not multiples of 8, run on
    forge_gemm_generic with the same epilogues as the MFMA path (GELU in its
    tanh form, the reference cuBLASLt epilogue's); checked against the
    float64 product of the same values (fp32: 1e-5; fp16 / bf16 outputs: one
    rounding step of the dtype)."""
    from kernels.lora_mlp.experiments.v4.gemm_epilogue import matmul_epilogue

    gen = torch.Generator().manual_seed(5)
    A = torch.randn(70, 33, generator=gen).to(dtype)
    B = (torch.randn(33, 45, generator=gen) / 33 ** 0.5).to(dtype)
    v = A.double() @ B.double()
    ref = {"none": v, "silu": torch.nn.functional.silu(v), "relu": torch.relu(v),
           "gelu": torch.nn.functional.gelu(v, approximate="tanh")}[epilogue]
    D = matmul_epilogue(A.cuda(), B.cuda(), epilogue=epilogue)
    assert D.dtype == dtype
    tol = 1e-5 if dtype == torch.float32 else (2e-3 if dtype == torch.float16 else 1.6e-2)
    torch.testing.assert_close(D.cpu().double(), ref, rtol=tol, atol=tol)
