"""forge_lora_a_noalloc (split-K LoRA-A products with the library's per-GPU
scratch array instead of a caller workspace) against forge_lora_a with a
PyTorch-allocated workspace: bit-identical outputs on two calls in a row,
the second smaller than the first (the scratch keeps the first call's
partials, which the second must not read), and a clear error, with no
launch, when the partials would not fit."""
import ctypes

import pytest
import torch

from forge_hip import _lib as L


def _case(M, K, r, n_proj, seed):
    g = torch.Generator().manual_seed(seed)
    X = torch.randn(M, K, generator=g).to(torch.bfloat16).cuda()
    A = ((torch.rand(n_proj * r, K, generator=g) * 2 - 1) / K ** 0.5).to(torch.bfloat16).cuda()
    mats = [A[p * r:(p + 1) * r] for p in range(n_proj)]
    scales = [2.0, 0.5, 1.5, 3.0][:n_proj]
    return X, A, mats, scales


def _ptrs(mats, scales):
    n = len(mats)
    return ((ctypes.c_void_p * n)(*[a.data_ptr() for a in mats]), (ctypes.c_float * n)(*scales))


def _with_workspace(X, mats, scales, r, split):
    M, K = X.shape
    n = len(mats)
    out = torch.empty(M, n * r, dtype=torch.bfloat16, device="cuda")
    work = torch.empty(split, M, n * r, dtype=torch.float32, device="cuda")
    p, s = _ptrs(mats, scales)
    L.check(L.forge_lora_a(M, K, r, n, X.data_ptr(), K, p, K, s, out.data_ptr(), n * r, work.data_ptr(), split,
                           L.stream_of(X)), "forge_lora_a")
    return out


def _no_alloc(X, mats, scales, r, split):
    M, K = X.shape
    n = len(mats)
    out = torch.empty(M, n * r, dtype=torch.bfloat16, device="cuda")
    p, s = _ptrs(mats, scales)
    L.check(L.forge_lora_a_noalloc(M, K, r, n, X.data_ptr(), K, p, K, s, out.data_ptr(), n * r, split,
                                   L.stream_of(X)), "forge_lora_a_noalloc")
    return out


@pytest.mark.gpu
def test_lora_a_noalloc_matches_workspace_entry_point():
    # call 1: the LoRA-MLP BASELINE shape (M 8192, K 4096, gate/up r = 16), split 4 -> 4 MiB of partials
    X1, A1, m1, s1 = _case(8192, 4096, 16, 2, seed=1)
    got1 = _no_alloc(X1, m1, s1, 16, 4)
    # call 2, smaller: fewer tokens, K and splits, three projections
    X2, A2, m2, s2 = _case(2048, 1024, 8, 3, seed=2)
    got2 = _no_alloc(X2, m2, s2, 8, 2)
    ref1 = _with_workspace(X1, m1, s1, 16, 4)
    ref2 = _with_workspace(X2, m2, s2, 8, 2)
    torch.cuda.synchronize()
    assert torch.equal(got1, ref1)
    assert torch.equal(got2, ref2)
    # and both are the products they claim to be (bf16 tolerance, fp32 CPU)
    for got, X, A, s, r in ((got1, X1, A1, s1, 16), (got2, X2, A2, s2, 8)):
        ref = (X.float().cpu() @ A.float().cpu().t()) * torch.tensor(s).repeat_interleave(r)
        torch.testing.assert_close(got.float().cpu(), ref, rtol=2e-2, atol=2e-2)
    # split_k 1 takes no scratch at all
    assert torch.equal(_no_alloc(X2, m2, s2, 8, 1), _with_workspace(X2, m2, s2, 8, 1))


@pytest.mark.gpu
def test_lora_a_noalloc_rejects_partials_beyond_the_scratch():
    X, _, mats, scales = _case(16384, 512, 32, 2, seed=3)
    p, s = _ptrs(mats, scales)
    out = torch.empty(16384, 64, dtype=torch.bfloat16, device="cuda")
    # 16 * 16384 * 64 fp32 partials = 64 MiB > 16 MiB
    rc = L.forge_lora_a_noalloc(16384, 512, 32, 2, X.data_ptr(), 512, p, 512, s, out.data_ptr(), 64, 16,
                                L.stream_of(X))
    assert rc != 0
    assert b"exceed" in L.forge_last_error() and str(L.LORA_A_SCRATCH_BYTES).encode() in L.forge_last_error()
