"""LoRA-QKV parity: v2_3 / v3 / v4 APIs and the fused QKV+RoPE entry point
(through libforge_hip.so) vs the CPU oracle
(kernels/lora_qkv/reference/lora_qkv_pytorch.py restated + the caller's RoPE).
Tolerance as in tests/test_lora_mlp.py (bf16 2e-2 scaled, cosine > 0.9999)."""
import pytest
import torch

from kernels.lora_qkv.experiments.v2.lora_qkv_kernel_v2_3 import lora_qkv_v2_3
from kernels.lora_qkv.experiments.v3.lora_qkv_kernel_v3 import LoRAQKVFunction
from kernels.lora_qkv.experiments.v4.lora_qkv_kernel_v4 import (
    LoRAQKVv4Function,
    lora_qkv_rope,
    pack_lora_a,
    pack_weights_backward,
)
from kernels.lora_qkv._impl import qkv_forward, rope_fusable, rope_qk_inplace
from oracle import lora_qkv as orc
from oracle.rope import cos_sin
from _parity import close_bf16 as _close_bf16

NAMES = ["dX", "dA_q", "dB_q", "dA_k", "dB_k", "dA_v", "dB_v"]


def _cuda(params):
    out = []
    for i, t in enumerate(params):
        if isinstance(t, torch.Tensor):
            out.append(t.cuda().requires_grad_(i in (3, 4, 6, 7, 9, 10)))
        else:
            out.append(t)
    return out


@pytest.mark.gpu
@pytest.mark.parametrize("T,K,Hq,Hkv,r", [(256, 512, 512, 128, 16), (300, 256, 512, 256, 64), (128, 1024, 1024, 256, 8)])
@pytest.mark.parametrize("api", ["v4", "v3"])
def test_lora_qkv_matches_oracle(T, K, Hq, Hkv, r, api):
    gen = torch.Generator().manual_seed(T + K + r)
    params = orc.make_params(K, Hq, Hkv, r, 2 * r, gen)
    X = torch.randn(T, K, generator=gen).to(torch.bfloat16)
    dQ = torch.randn(T, Hq, generator=gen).to(torch.bfloat16)
    dK = torch.randn(T, Hkv, generator=gen).to(torch.bfloat16)
    dV = torch.randn(T, Hkv, generator=gen).to(torch.bfloat16)
    f = lambda t: t.float() if isinstance(t, torch.Tensor) else t  # noqa: E731
    pf = [f(t) for t in params]
    Qr, Kr, Vr = orc.forward(X.float(), *pf)
    ref_grads = orc.backward(dQ.float(), dK.float(), dV.float(), X.float(), *pf)
    p = _cuda(params)
    x = X.cuda().requires_grad_(True)
    Fn = LoRAQKVv4Function if api == "v4" else LoRAQKVFunction
    Q, K_, V = Fn.apply(x, *p)
    # outputs are column views of one packed buffer
    assert Q.stride(0) == Hq + 2 * Hkv and K_.data_ptr() == Q.data_ptr() + 2 * Hq
    for a, b, n in ((Q, Qr, "Q"), (K_, Kr, "K"), (V, Vr, "V")):
        _close_bf16(a, b, n)
    torch.autograd.backward((Q, K_, V), (dQ.cuda(), dK.cuda(), dV.cuda()))
    got = [x.grad, p[3].grad, p[4].grad, p[6].grad, p[7].grad, p[9].grad, p[10].grad]
    for n, a, b in zip(NAMES, got, ref_grads):
        _close_bf16(a, b, n)


@pytest.mark.gpu
def test_lora_qkv_v2_3_and_packed_helpers():
    gen = torch.Generator().manual_seed(8)
    T, K, Hq, Hkv, r = 64, 256, 256, 64, 16
    params = orc.make_params(K, Hq, Hkv, r, 32, gen)
    X = torch.randn(2, T // 2, K, generator=gen).to(torch.bfloat16)
    pf = [t.float() if isinstance(t, torch.Tensor) else t for t in params]
    Qr, Kr, Vr = orc.forward(X.float().reshape(-1, K), *pf)
    Wq, Wk, Wv, Aq, Bq, sq, Ak, Bk, sk, Av, Bv, sv = [t.cuda() if isinstance(t, torch.Tensor) else t for t in params]
    Q, K_, V = lora_qkv_v2_3(X.cuda(), Wq, Aq, Bq, sq, Wk, Ak, Bk, sk, Wv, Av, Bv, sv)
    assert Q.shape == (2, T // 2, Hq)
    for a, b, n in ((Q, Qr, "Q"), (K_, Kr, "K"), (V, Vr, "V")):
        _close_bf16(a.reshape(-1, a.shape[-1]), b, n)
    assert torch.equal(pack_weights_backward(Wq, Wk, Wv), torch.cat([Wq, Wk, Wv]))
    assert torch.equal(pack_lora_a(Aq, Ak, Av), torch.cat([Aq, Ak, Av]))


@pytest.mark.gpu
@pytest.mark.parametrize("head_dim", [128, 64])
def test_lora_qkv_rope_fused_matches_composition(head_dim):
    """LoRA-QKV+RoPE (the product path: the QKV GEMM with its RoPE epilogue)
    against the oracle with per-token (varlen) positions, and against the
    composition (the same GEMM storing Q/K, then an in-place forge_rope
    pass), which fuse_rope=False selects."""
    gen = torch.Generator().manual_seed(head_dim)
    lens = [37, 120, 99]
    pos = orc.positions_for(lens)
    T, K, Hq, Hkv, r = int(pos.numel()), 512, 512, 256, 16
    params = orc.make_params(K, Hq, Hkv, r, 32, gen)
    X = torch.randn(T, K, generator=gen).to(torch.bfloat16)
    dQ = torch.randn(T, Hq, generator=gen).to(torch.bfloat16)
    dK = torch.randn(T, Hkv, generator=gen).to(torch.bfloat16)
    dV = torch.randn(T, Hkv, generator=gen).to(torch.bfloat16)
    c, s = cos_sin(torch.arange(256), head_dim, 500000.0, torch.bfloat16)
    (Qr, Kr, Vr), ref_grads = orc.qkv_rope_fwd_bwd(X, dQ, dK, dV, params, c[pos], s[pos], head_dim)
    p = _cuda(params)
    x = X.cuda().requires_grad_(True)
    rope = {"cos": c.cuda(), "sin": s.cuda(), "positions": pos.cuda(), "head_dim": head_dim}
    assert rope_fusable(rope, Hq, Hkv)  # this shape can take the GEMM's RoPE epilogue
    Q, K_, V = lora_qkv_rope(x, p[0], p[3], p[4], p[5], p[1], p[6], p[7], p[8], p[2], p[9], p[10], p[11],
                             c.cuda(), s.cuda(), pos.cuda(), head_dim)
    for a, b, n in ((Q, Qr, "Q"), (K_, Kr, "K"), (V, Vr, "V")):
        _close_bf16(a, b, n)
    # the GEMM's RoPE epilogue against the composition (the same GEMM storing
    # Q/K, then a forge_rope pass); both round the projection to bf16 before
    # rotating, so they differ by at most one bf16 rounding of the rotated value
    args = (x.detach(), p[0], p[1], p[2], p[3].detach(), p[4].detach(), p[5], p[6].detach(), p[7].detach(), p[8],
            p[9].detach(), p[10].detach(), p[11])
    plain = qkv_forward(*args)
    rope_qk_inplace(plain, Hq, Hkv, rope)
    assert torch.equal(qkv_forward(*args, rope=rope, fuse_rope=False), plain)
    fused = qkv_forward(*args, rope=rope)
    assert torch.equal(torch.cat([Q, K_, V], 1), fused)  # the product path is the fused epilogue
    assert torch.equal(fused[:, Hq + Hkv:], plain[:, Hq + Hkv:])  # V is not rotated
    torch.testing.assert_close(fused.float(), plain.float(), rtol=2 ** -7, atol=1e-5)
    torch.autograd.backward((Q, K_, V), (dQ.cuda(), dK.cuda(), dV.cuda()))
    got = [x.grad, p[3].grad, p[4].grad, p[6].grad, p[7].grad, p[9].grad, p[10].grad]
    for n, a, b in zip(NAMES, got, ref_grads):
        _close_bf16(a, b, n)


@pytest.mark.gpu
@pytest.mark.parametrize("head_dim", [128, 64])
def test_qkv_rope_epilogue_paths_agree(head_dim):
    """The fused RoPE epilogue of forge_lora_qkv_rope has a 16-byte staged
    path and a per-element path (taken when the cos/sin rows are not
    8-element aligned); both must give bit-identical Q/K/V."""
    gen = torch.Generator().manual_seed(100 + head_dim)
    T, K, Hq, Hkv, r = 300, 512, 512, 256, 16
    p = _cuda(orc.make_params(K, Hq, Hkv, r, 32, gen))
    X = torch.randn(T, K, generator=gen).to(torch.bfloat16).cuda()
    pos = torch.randint(0, 200, (T,), generator=gen).cuda()
    c, s = (t.cuda() for t in cos_sin(torch.arange(200), head_dim, 10000.0, torch.bfloat16))
    c_odd = torch.zeros(200, head_dim + 2, dtype=torch.bfloat16, device="cuda")[:, :head_dim].copy_(c)
    s_odd = torch.zeros(200, head_dim + 2, dtype=torch.bfloat16, device="cuda")[:, :head_dim].copy_(s)
    args = (X, p[0], p[1], p[2], p[3].detach(), p[4].detach(), p[5], p[6].detach(), p[7].detach(), p[8],
            p[9].detach(), p[10].detach(), p[11])
    vec = qkv_forward(*args, rope={"cos": c, "sin": s, "positions": pos, "head_dim": head_dim}, fuse_rope=True)
    per_elem = qkv_forward(*args, rope={"cos": c_odd, "sin": s_odd, "positions": pos, "head_dim": head_dim},
                           fuse_rope=True)
    assert torch.equal(vec, per_elem)


@pytest.mark.gpu
@pytest.mark.parametrize("M,nq,nkv,r,with_pos", [(300, 32, 8, 64, True), (64, 8, 2, 16, False), (1000, 4, 2, 32, True),
                                                 (31, 8, 2, 48, True), (97, 16, 8, 64, False)])
def test_rope_bwd_rank_kernel(M, nq, nkv, r, with_pos):
    """forge_lora_qkv_rope_bwd: dQ and dK rotated back equal the forge_rope
    backward bit for bit, and t = s [dQu B_q | dKu B_k | dV B_v] matches the
    fp32 product of those rotated rows (one bf16 rounding).  Row pitches are
    padded with NaN past the head columns, which a read outside the heads
    would carry into t; ragged M (partial 32-token tiles), ranks 16..64."""
    from forge_hip import _lib as L
    from kernels.lora_qkv.experiments.v4.lora_qkv_kernel_v4 import _rope_qk_backward

    torch.manual_seed(M + nq + r)
    D, dev, bf = 128, "cuda", torch.bfloat16
    Hq, Hkv = nq * D, nkv * D

    def padded(w):
        t = torch.full((M, w + 8), float("nan"), device=dev, dtype=bf)
        t[:, :w] = torch.randn(M, w, device=dev).to(bf)
        return t

    dq, dk, dv = padded(Hq), padded(Hkv), padded(Hkv)
    P = M + 50
    c, s_ = cos_sin(torch.arange(P), D, 500000.0, bf)
    c, s_ = c.to(dev).contiguous(), s_.to(dev).contiguous()
    pos = torch.randint(0, P, (M,), device=dev, dtype=torch.int64) if with_pos else None
    bt = [(torch.randn(r, w, device=dev) * 0.05).to(bf) for w in (Hq, Hkv, Hkv)]
    dq_out = torch.empty(M, Hq, device=dev, dtype=bf)
    dk_out = torch.empty(M, Hkv, device=dev, dtype=bf)
    t = torch.empty(M, 3 * r, device=dev, dtype=bf)
    scale = 2.0
    L.check(L.forge_lora_qkv_rope_bwd(M, Hq, Hkv, r, D, dq.data_ptr(), Hq + 8, dk.data_ptr(), Hkv + 8,
                                      dv.data_ptr(), Hkv + 8, c.data_ptr(), s_.data_ptr(), D, P,
                                      pos.data_ptr() if pos is not None else None, dq_out.data_ptr(), Hq,
                                      dk_out.data_ptr(), Hkv, bt[0].data_ptr(), bt[1].data_ptr(), bt[2].data_ptr(),
                                      Hq, Hkv, Hkv, t.data_ptr(), 3 * r, scale, L.stream_of(dq)),
            "forge_lora_qkv_rope_bwd")
    ref_q, ref_k = _rope_qk_backward(dq[:, :Hq], dk[:, :Hkv], D, c, s_, pos)
    assert torch.equal(dq_out, ref_q) and torch.equal(dk_out, ref_k)
    want = scale * torch.cat([ref_q.float() @ bt[0].float().t(), ref_k.float() @ bt[1].float().t(),
                              dv[:, :Hkv].float() @ bt[2].float().t()], 1)
    assert not torch.isnan(t).any()
    torch.testing.assert_close(t.float(), want, rtol=1e-2, atol=1e-2 * want.abs().max().item())


@pytest.mark.gpu
def test_lora_qkv_rope_backward_fused_and_unfused_agree():
    """The RoPE autograd backward with the fused RoPE / LoRA-B kernel and
    with the forge_rope pass plus the GEMM: the same gradients within one
    bf16 rounding of t (its products are summed in another order)."""
    import kernels.lora_qkv.experiments.v4.lora_qkv_kernel_v4 as v4

    gen = torch.Generator().manual_seed(11)
    lens = [150, 77, 200]
    pos = orc.positions_for(lens)
    T, K, Hq, Hkv, r, D = int(pos.numel()), 512, 1024, 256, 16, 128
    params = orc.make_params(K, Hq, Hkv, r, 32, gen)
    X = torch.randn(T, K, generator=gen).to(torch.bfloat16)
    dQ = torch.randn(T, Hq, generator=gen).to(torch.bfloat16).cuda()
    dK = torch.randn(T, Hkv, generator=gen).to(torch.bfloat16).cuda()
    dV = torch.randn(T, Hkv, generator=gen).to(torch.bfloat16).cuda()
    c, s = cos_sin(torch.arange(256), D, 500000.0, torch.bfloat16)
    grads = []
    for fused in (True, False):
        v4.ROPE_BWD_FUSED = fused
        try:
            p = _cuda(params)
            x = X.cuda().requires_grad_(True)
            Q, K_, V = lora_qkv_rope(x, p[0], p[3], p[4], p[5], p[1], p[6], p[7], p[8], p[2], p[9], p[10], p[11],
                                     c.cuda(), s.cuda(), pos.cuda(), D)
            torch.autograd.backward((Q, K_, V), (dQ, dK, dV))
            grads.append([x.grad, p[3].grad, p[4].grad, p[6].grad, p[7].grad, p[9].grad, p[10].grad])
        finally:
            v4.ROPE_BWD_FUSED = True
    for n, a, b in zip(NAMES, grads[0], grads[1]):
        torch.testing.assert_close(a.float(), b.float(), rtol=2e-2, atol=2e-2 * b.float().abs().max().item(),
                                   msg=lambda m: f"{n}: {m}")


@pytest.mark.gpu
def test_lora_qkv_fp64_gradcheck_uses_reference_torch_path():
    gen = torch.Generator().manual_seed(9)
    K, Hq, Hkv, r = 8, 8, 4, 2
    params = [t.double().cuda() if isinstance(t, torch.Tensor) else t for t in orc.make_params(K, Hq, Hkv, r, 4, gen)]
    X = torch.randn(5, K, dtype=torch.float64, device="cuda", requires_grad=True)
    lora = [params[i].requires_grad_(True) for i in (3, 4, 6, 7, 9, 10)]

    def f(x, aq, bq, ak, bk, av, bv):
        return LoRAQKVv4Function.apply(x, params[0], params[1], params[2], aq, bq, params[5], ak, bk, params[8],
                                       av, bv, params[11])
    assert torch.autograd.gradcheck(f, (X, *lora))


def _baseline_rows(lens, T, tile=256):
    """Token rows checked at full size: the first and last rows of every
    sequence (and their neighbours), the first rows of the batch, and the
    last partial 256-row GEMM tile."""
    rows = set(range(0, 48))
    start = 0
    for n in lens:
        for r in (start, start + 1, start + 2, start + n - 3, start + n - 2, start + n - 1):
            if 0 <= r < T:
                rows.add(r)
        start += n
    last_tile = (T // tile) * tile
    rows.update(range(max(0, last_tile - 8), min(T, last_tile + 24)))
    rows.update(range(T - 48, T))
    return torch.tensor(sorted(rows))


@pytest.mark.gpu
def test_lora_qkv_rope_baseline_config():
    """BASELINE configs[4] at its own size: hidden 4096, 32 Q / 8 KV heads,
    head_dim 128, r = 64, alpha = 128, RoPE base 500000, 8 packed sequences
    with lengths U[512, 4096] from seed 4 (T = 22954, as bench.py builds it).
    Q/K/V and dX rows depend only on the same token rows, so the oracle runs
    on sequence starts/ends and the last partial tile; the LoRA gradients
    are token sums, so they are checked over ALL tokens against the oracle's
    LoRA-gradient products fed with dQ/dK rotated back by -theta (the
    adjoint rotation, pinned in tests/test_oracle.py)."""
    K, Hq, Hkv, D, r, alpha = 4096, 4096, 1024, 128, 64, 128
    lens = orc.varlen_lengths(8, 512, 4096, seed=4)
    pos = orc.positions_for(lens)
    T = int(pos.numel())
    assert T == 22954
    print(f"lora_qkv_rope baseline: T={T} lens={lens}", flush=True)
    gen = torch.Generator().manual_seed(4)
    params = orc.make_params(K, Hq, Hkv, r, alpha, gen)
    X = torch.randn(T, K, generator=gen).to(torch.bfloat16)
    dQ = torch.randn(T, Hq, generator=gen).to(torch.bfloat16)
    dK = torch.randn(T, Hkv, generator=gen).to(torch.bfloat16)
    dV = torch.randn(T, Hkv, generator=gen).to(torch.bfloat16)
    c, s = cos_sin(torch.arange(max(lens)), D, 500000.0, torch.bfloat16)

    p = _cuda(params)
    x = X.cuda().requires_grad_(True)
    Q, K_, V = lora_qkv_rope(x, p[0], p[3], p[4], p[5], p[1], p[6], p[7], p[8], p[2], p[9], p[10], p[11],
                             c.cuda(), s.cuda(), pos.cuda(), D)
    torch.autograd.backward((Q, K_, V), (dQ.cuda(), dK.cuda(), dV.cuda()))
    torch.cuda.synchronize()

    rows = _baseline_rows(lens, T)
    pr = pos[rows]
    (Qr, Kr, Vr), ref_grads = orc.qkv_rope_fwd_bwd(X[rows], dQ[rows], dK[rows], dV[rows], params,
                                                    c[pr], s[pr], D)
    rc = rows.cuda()
    for a, b, n in ((Q[rc], Qr, "Q rows"), (K_[rc], Kr, "K rows"), (V[rc], Vr, "V rows"),
                    (x.grad[rc], ref_grads[0], "dX rows")):
        _close_bf16(a, b, n)

    # LoRA gradients over every token
    f = lambda t: t.float() if isinstance(t, torch.Tensor) else t  # noqa: E731
    pf = [f(t) for t in params]
    ct, st = c[pos].float(), s[pos].float()
    dQu = orc.rope_rows(dQ.float(), ct, -st, D)
    dKu = orc.rope_rows(dK.float(), ct, -st, D)
    ref_lora = orc.lora_grads(dQu, dKu, dV.float(), X.float(), *pf)
    got = [p[3].grad, p[4].grad, p[6].grad, p[7].grad, p[9].grad, p[10].grad]
    for n, a, b in zip(NAMES[1:], got, ref_lora):
        _close_bf16(a, b, n + " (all tokens)")


def test_lora_qkv_rope_positions_out_of_range_raise():
    """Token positions index the cos/sin rows: out-of-range values raise
    IndexError before any launch (CPU tensors here)."""
    gen = torch.Generator().manual_seed(3)
    params = orc.make_params(64, 128, 128, 4, 8, gen)
    X = torch.randn(5, 64, generator=gen).to(torch.bfloat16)
    c, s = cos_sin(torch.arange(6), 64, 10000.0, torch.bfloat16)
    p = list(params)
    with pytest.raises(IndexError, match=r"\[0, 6\)"):
        lora_qkv_rope(X, p[0], p[3], p[4], p[5], p[1], p[6], p[7], p[8], p[2], p[9], p[10], p[11],
                      c, s, torch.tensor([0, 1, 2, 6, 0]), 64)


@pytest.mark.gpu
def test_lora_qkv_v4_saves_packed_matrices():
    """v4's save_for_backward contract (reference lora_qkv_kernel_v4.py:
    209-214): (X, A_q, B_q, A_k, B_k, A_v, B_v, W_dX_packed, A_packed), with
    the packed matrices built when not given; given ones are saved as is."""
    gen = torch.Generator().manual_seed(12)
    T, K, Hq, Hkv, r = 64, 256, 256, 128, 16
    p = _cuda(orc.make_params(K, Hq, Hkv, r, 32, gen))
    x = torch.randn(T, K, generator=gen).to(torch.bfloat16).cuda().requires_grad_(True)
    Q, _, _ = LoRAQKVv4Function.apply(x, *p)
    saved = Q.grad_fn.saved_tensors
    assert len(saved) == 9
    assert saved[0] is x or torch.equal(saved[0], x)
    assert torch.equal(saved[7], torch.cat([p[0], p[1], p[2]]))
    assert torch.equal(saved[8], torch.cat([p[3], p[6], p[9]]))
    W_dX, A_pack = pack_weights_backward(p[0], p[1], p[2]), pack_lora_a(p[3], p[6], p[9]).detach()
    Q2, _, _ = LoRAQKVv4Function.apply(x, *p, None, W_dX, A_pack)
    s2 = Q2.grad_fn.saved_tensors
    assert s2[7].data_ptr() == W_dX.data_ptr() and s2[8].data_ptr() == A_pack.data_ptr()
    torch.testing.assert_close(Q2, Q, rtol=0, atol=0)


@pytest.mark.gpu
@pytest.mark.parametrize("scales", [(2.0, 2.0, 2.0), (1.5, 0.5, 3.0)])
def test_lora_qkv_per_projection_scales(scales):
    """Equal scales take the one-launch [dQ B_q | dK B_k | dV B_v] product,
    different ones a launch per projection; both against the oracle."""
    T, K, Hq, Hkv, r = 1100, 512, 512, 128, 64
    gen = torch.Generator().manual_seed(17)
    params = list(orc.make_params(K, Hq, Hkv, r, 2 * r, gen))
    params[5], params[8], params[11] = scales
    X = torch.randn(T, K, generator=gen).to(torch.bfloat16)
    dQ = torch.randn(T, Hq, generator=gen).to(torch.bfloat16)
    dK = torch.randn(T, Hkv, generator=gen).to(torch.bfloat16)
    dV = torch.randn(T, Hkv, generator=gen).to(torch.bfloat16)
    f = lambda t: t.float() if isinstance(t, torch.Tensor) else t  # noqa: E731
    pf = [f(t) for t in params]
    ref_grads = orc.backward(dQ.float(), dK.float(), dV.float(), X.float(), *pf)
    p = _cuda(params)
    x = X.cuda().requires_grad_(True)
    Q, K_, V = LoRAQKVv4Function.apply(x, *p)
    torch.autograd.backward((Q, K_, V), (dQ.cuda(), dK.cuda(), dV.cuda()))
    got = [x.grad, p[3].grad, p[4].grad, p[6].grad, p[7].grad, p[9].grad, p[10].grad]
    for n, a, b in zip(NAMES, got, ref_grads):
        _close_bf16(a, b, n)


@pytest.mark.gpu
@pytest.mark.parametrize("Hq,Hkv,head_dim,r,table_dtype", [(256, 128, 64, 16, torch.bfloat16),
                                                            (128, 64, 64, 4, torch.bfloat16),
                                                            (512, 256, 32, 12, torch.bfloat16),
                                                            (256, 128, 128, 8, torch.float32)])
def test_lora_qkv_rope_unfused_shapes_and_ranks(Hq, Hkv, head_dim, r, table_dtype):
    """Q/K widths that are not whole 256-column tiles, head_dim other than 64 /
    128, fp32 tables, and ranks that are not multiples of 8 (zero-padded
    inside): the forward rotates Q/K in a forge_rope pass after the GEMM, and
    everything still matches the oracle."""
    gen = torch.Generator().manual_seed(Hq + Hkv + head_dim + r)
    lens = [70, 33]
    pos = orc.positions_for(lens)
    T, K = int(pos.numel()), 256
    params = orc.make_params(K, Hq, Hkv, r, 2 * r, gen)
    X = torch.randn(T, K, generator=gen).to(torch.bfloat16)
    dQ = torch.randn(T, Hq, generator=gen).to(torch.bfloat16)
    dK = torch.randn(T, Hkv, generator=gen).to(torch.bfloat16)
    dV = torch.randn(T, Hkv, generator=gen).to(torch.bfloat16)
    c, s = cos_sin(torch.arange(128), head_dim, 10000.0, table_dtype)
    (Qr, Kr, Vr), ref_grads = orc.qkv_rope_fwd_bwd(X, dQ, dK, dV, params, c[pos], s[pos], head_dim)
    p = _cuda(params)
    x = X.cuda().requires_grad_(True)
    Q, K_, V = lora_qkv_rope(x, p[0], p[3], p[4], p[5], p[1], p[6], p[7], p[8], p[2], p[9], p[10], p[11],
                             c.cuda(), s.cuda(), pos.cuda(), head_dim)
    for a, b, n in ((Q, Qr, "Q"), (K_, Kr, "K"), (V, Vr, "V")):
        _close_bf16(a, b, n)
    torch.autograd.backward((Q, K_, V), (dQ.cuda(), dK.cuda(), dV.cuda()))
    got = [x.grad, p[3].grad, p[4].grad, p[6].grad, p[7].grad, p[9].grad, p[10].grad]
    for n, a, b in zip(NAMES, got, ref_grads):
        assert a.shape == b.shape, n
        _close_bf16(a, b, n)
