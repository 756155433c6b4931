"""RoPE parity: HIP kernel vs the CPU oracle (HF formula in fp32).

Cases follow kernels/rope/tests/test_v1.py:122-340 (shapes incl. MHA/MQA,
dtypes, backward, fp64 gradcheck, one-hot gradient) plus the BASELINE config
(bf16 Q [4,4096,32,128], K [4,4096,8,128] in B,S,H,D memory passed as the
HF transpose(1,2) view, bases 10000 and 500000) and varlen positions.
Tolerances: fp32 1e-5, bf16/fp16 2e-2 (the oracle is fp32 math rounded once).
"""
import pytest
import torch

from kernels.rope import ForgeRoPEv3Function, apply_rope, rope_cos_sin
from oracle.rope import cos_sin, hf_apply_rotary_pos_emb, rope_fwd_bwd

SHAPES = [
    ("demo_tiny", 2, 4, 2, 16, 64),
    ("qwen25_0p5b_short", 1, 14, 2, 512, 64),
    ("qwen3_8b_short", 4, 32, 8, 512, 128),
    ("qwen3_8b_train", 2, 32, 8, 2048, 128),
    ("mha_no_gqa", 2, 16, 16, 1024, 128),
    ("mqa_extreme", 2, 8, 1, 1024, 128),
]
TOL = {torch.float32: 1e-5, torch.float16: 2e-2, torch.bfloat16: 2e-2, torch.float64: 1e-5}


def _inputs(b, nq, nkv, s, d, dtype, base=10000.0, seed=0, bshd=False, cos_batched=False):
    g = torch.Generator().manual_seed(seed)
    if bshd:
        q = torch.randn(b, s, nq, d, generator=g).to(dtype).transpose(1, 2)
        k = torch.randn(b, s, nkv, d, generator=g).to(dtype).transpose(1, 2)
    else:
        q = torch.randn(b, nq, s, d, generator=g).to(dtype)
        k = torch.randn(b, nkv, s, d, generator=g).to(dtype)
    c, sn = cos_sin(torch.arange(s), d, base, dtype)
    if cos_batched:
        c, sn = c.unsqueeze(0).expand(b, -1, -1).contiguous(), sn.unsqueeze(0).expand(b, -1, -1).contiguous()
    else:
        c, sn = c.unsqueeze(0), sn.unsqueeze(0)
    return q, k, c, sn


def _close(a, b, dtype):
    t = TOL[dtype]
    torch.testing.assert_close(a.cpu(), b.cpu(), atol=t, rtol=t)


@pytest.mark.gpu
@pytest.mark.parametrize("label,b,nq,nkv,s,d", SHAPES)
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_rope_forward_backward(label, b, nq, nkv, s, d, dtype):
    q, k, c, sn = _inputs(b, nq, nkv, s, d, dtype)
    dq = torch.randn(q.shape).to(dtype)
    dk = torch.randn(k.shape).to(dtype)
    rq, rk, rdq, rdk = rope_fwd_bwd(q, k, c, sn, dq, dk)
    qg = q.cuda().requires_grad_(True)
    kg = k.cuda().requires_grad_(True)
    oq, ok = apply_rope(qg, kg, c.cuda(), sn.cuda())
    _close(oq, rq, dtype)
    _close(ok, rk, dtype)
    (oq * dq.cuda()).sum().add((ok * dk.cuda()).sum()).backward()
    _close(qg.grad, rdq, dtype)
    _close(kg.grad, rdk, dtype)


@pytest.mark.gpu
@pytest.mark.parametrize("bshd", [False, True])
@pytest.mark.parametrize("cos_batched", [False, True])
def test_rope_layouts(bshd, cos_batched):
    """Strided (HF transpose) inputs and per-batch cos/sin tables."""
    dtype = torch.bfloat16
    q, k, c, sn = _inputs(2, 8, 2, 64, 128, dtype, bshd=bshd, cos_batched=cos_batched, seed=5)
    rq, rk = hf_apply_rotary_pos_emb(q.float(), k.float(), c.float(), sn.float())
    oq, ok = apply_rope(q.cuda(), k.cuda(), c.cuda(), sn.cuda())
    _close(oq, rq.to(dtype), dtype)
    _close(ok, rk.to(dtype), dtype)
    if bshd:  # output keeps the input's memory layout (no copy was made)
        assert oq.stride() == q.stride()


@pytest.mark.gpu
def test_rope_gradcheck_fp64_and_one_hot():
    """kernels/rope/tests/test_v1.py:273-340: fp64 gradcheck (fp32 math inside)
    and the one-hot analytic check dq_lo = cos, dq_hi = -sin."""
    b, nq, nkv, s, d = 2, 4, 2, 8, 32
    q, k, c, sn = _inputs(b, nq, nkv, s, d, torch.float64)
    q, k, c, sn = q.cuda(), k.cuda(), c.cuda(), sn.cuda()
    q1 = q.clone().requires_grad_(True)
    k1 = k.clone().requires_grad_(True)
    oq, ok = apply_rope(q1, k1, c, sn)
    g = torch.zeros_like(oq)
    g[0, 0, 1, 0] = 1.0
    (oq * g).sum().add((ok * torch.zeros_like(ok)).sum()).backward()
    assert abs(q1.grad[0, 0, 1, 0].item() - c[0, 1, 0].item()) < 1e-5
    assert abs(q1.grad[0, 0, 1, d // 2].item() + sn[0, 1, 0].item()) < 1e-5
    q2 = q.clone().requires_grad_(True)
    k2 = k.clone().requires_grad_(True)
    assert torch.autograd.gradcheck(
        lambda a, b_: ForgeRoPEv3Function.apply(a, b_, c, sn), (q2, k2),
        eps=1e-3, atol=1e-2, rtol=1e-2, nondet_tol=1e-3,
    )


@pytest.mark.gpu
def test_rope_varlen_positions():
    """Packed variable-length sequences: positions restart at 0 per sequence
    and select the cos/sin row per token."""
    lens = [5, 17, 9]
    pos = torch.cat([torch.arange(n) for n in lens])
    T, nq, nkv, d = int(pos.numel()), 4, 2, 128
    dtype = torch.bfloat16
    g = torch.Generator().manual_seed(7)
    q = torch.randn(1, nq, T, d, generator=g).to(dtype)
    k = torch.randn(1, nkv, T, d, generator=g).to(dtype)
    table_c, table_s = cos_sin(torch.arange(32), d, 500000.0, dtype)
    c_tok, s_tok = table_c[pos].unsqueeze(0), table_s[pos].unsqueeze(0)
    rq, rk = hf_apply_rotary_pos_emb(q.float(), k.float(), c_tok.float(), s_tok.float())
    oq, ok = apply_rope(q.cuda(), k.cuda(), table_c.unsqueeze(0).cuda(), table_s.unsqueeze(0).cuda(),
                        positions=pos.cuda())
    _close(oq, rq.to(dtype), dtype)
    _close(ok, rk.to(dtype), dtype)


def test_rope_positions_out_of_range_raise_before_launch():
    """Positions index the cos/sin rows: values outside [0, P) are rejected
    (IndexError) before any launch, here on CPU tensors."""
    from kernels._positions import check_positions

    q = torch.zeros(1, 2, 6, 64)
    k = torch.zeros(1, 1, 6, 64)
    c, s = cos_sin(torch.arange(8), 64, 10000.0, torch.float32)
    c, s = c.unsqueeze(0), s.unsqueeze(0)
    for bad in ([0, 1, 2, 3, 4, 8], [0, -1, 2, 3, 4, 5]):
        with pytest.raises(IndexError, match=r"positions must lie in \[0, 8\)"):
            apply_rope(q, k, c, s, positions=torch.tensor(bad))
    # a valid buffer is checked once per version; writing into it re-checks
    pos = torch.tensor([0, 1, 2, 3, 4, 7])
    check_positions(pos, 8)
    pos[5] = 9
    with pytest.raises(IndexError, match="max 9"):
        check_positions(pos, 8)
    with pytest.raises(TypeError):
        check_positions(torch.zeros(3), 8)


@pytest.mark.gpu
def test_rope_fp32_tables_with_bf16_q_are_read_as_stored():
    """fp32 cos/sin with bf16 q/k: the kernel reads the fp32 table (no bf16
    rounding of cos/sin) and computes in fp32, as the reference kernel does.
    The result equals the fp32-math oracle rounded once (all but a few
    elements bit-equal, the rest within one bf16 ulp), while a bf16-rounded table
    gives a visibly different result."""
    b, nq, nkv, S, d = 2, 8, 2, 256, 128
    g = torch.Generator().manual_seed(21)
    q = torch.randn(b, nq, S, d, generator=g).to(torch.bfloat16)
    k = torch.randn(b, nkv, S, d, generator=g).to(torch.bfloat16)
    c32, s32 = cos_sin(torch.arange(S) * 37, d, 10000.0, torch.float32)  # large angles: cos/sin far from bf16 grid
    dq = torch.randn(q.shape, generator=g).to(torch.bfloat16)
    dk = torch.randn(k.shape, generator=g).to(torch.bfloat16)
    rq, rk, rdq, rdk = rope_fwd_bwd(q, k, c32.unsqueeze(0), s32.unsqueeze(0), dq, dk)
    qg = q.cuda().requires_grad_(True)
    kg = k.cuda().requires_grad_(True)
    oq, ok = apply_rope(qg, kg, c32.unsqueeze(0).cuda(), s32.unsqueeze(0).cuda())
    torch.autograd.backward((oq, ok), (dq.cuda(), dk.cuda()))
    for a, ref in ((oq, rq), (ok, rk), (qg.grad, rdq), (kg.grad, rdk)):
        a = a.detach().cpu()
        diff = (a.float() - ref.float()).abs()
        # one bf16 ulp, plus 1e-5 absolute where x cos - y sin cancels (the
        # fp32 evaluation order then moves a tiny result by more than an ulp)
        ulp = ref.float().abs() * 2.0 ** -7 + 1e-5
        assert bool((diff <= ulp).all())
        assert (a == ref).float().mean().item() > 0.99
    cb, sb = c32.to(torch.bfloat16), s32.to(torch.bfloat16)
    oq_b, _ = apply_rope(q.cuda(), k.cuda(), cb.unsqueeze(0).cuda(), sb.unsqueeze(0).cuda())
    assert (oq_b.cpu() != oq.detach().cpu()).float().mean().item() > 0.05


@pytest.mark.gpu
def test_rope_c_abi_position_outside_table_reads_nothing():
    """Called through the C ABI directly (no host validation), a position
    outside [0, table_rows) gives NaN for that token and reads no table
    memory; every other token is rotated as usual."""
    from forge_hip import _lib as L

    T, nq, nkv, d, P = 64, 4, 2, 128, 40
    g = torch.Generator().manual_seed(5)
    q = torch.randn(1, nq, T, d, generator=g).to(torch.bfloat16).cuda()
    k = torch.randn(1, nkv, T, d, generator=g).to(torch.bfloat16).cuda()
    c, s = (t.cuda() for t in cos_sin(torch.arange(P), d, 10000.0, torch.bfloat16))
    pos = torch.randint(0, P, (T,), generator=g)
    pos[3], pos[60] = P, -2
    pos = pos.cuda()
    oq, ok = torch.empty_like(q), torch.empty_like(k)
    qs, ks = q.stride(), k.stride()
    L.check(L.forge_rope(L.DTYPE_BF16, q.data_ptr(), qs[0], qs[1], qs[2], k.data_ptr(), ks[0], ks[1], ks[2],
                         oq.data_ptr(), qs[0], qs[1], qs[2], ok.data_ptr(), ks[0], ks[1], ks[2],
                         c.data_ptr(), 0, d, s.data_ptr(), 0, d, L.DTYPE_BF16, P, pos.data_ptr(),
                         1, nq, nkv, T, d, 0, L.stream_of(q)), "forge_rope")
    torch.cuda.synchronize()
    bad = torch.zeros(T, dtype=torch.bool)
    bad[3] = bad[60] = True
    assert bool(torch.isnan(oq[0][:, bad.cuda()]).all()) and bool(torch.isnan(ok[0][:, bad.cuda()]).all())
    good = (~bad).cuda()
    pc = pos.clamp(0, P - 1).cpu()
    rq, rk = hf_apply_rotary_pos_emb(q.float().cpu(), k.float().cpu(), c.cpu()[pc].float().unsqueeze(0),
                                     s.cpu()[pc].float().unsqueeze(0))
    _close(oq[:, :, good], rq.to(torch.bfloat16)[:, :, good.cpu()], torch.bfloat16)
    _close(ok[:, :, good], rk.to(torch.bfloat16)[:, :, good.cpu()], torch.bfloat16)


@pytest.mark.gpu
@pytest.mark.parametrize("base", [10000.0, 500000.0])
def test_rope_baseline_config(base):
    """BASELINE configs[1] at full size.  The oracle checks the first 256
    tokens of every batch; every token is checked by the size-independent
    properties: backward(forward(x)) == x and per-pair norm preservation."""
    B, S, NQ, NKV, D = 4, 4096, 32, 8, 128
    dtype = torch.bfloat16
    gen = torch.Generator(device="cuda").manual_seed(11)
    q_bshd = torch.randn(B, S, NQ, D, device="cuda", generator=gen).to(dtype)
    k_bshd = torch.randn(B, S, NKV, D, device="cuda", generator=gen).to(dtype)
    q, k = q_bshd.transpose(1, 2), k_bshd.transpose(1, 2)
    c, sn = cos_sin(torch.arange(S), D, base, dtype)
    c, sn = c.unsqueeze(0).cuda(), sn.unsqueeze(0).cuda()
    oq, ok = apply_rope(q, k, c, sn)
    n = 256
    rq, rk = hf_apply_rotary_pos_emb(q[:, :, :n].float().cpu(), k[:, :, :n].float().cpu(),
                                     c[:, :n].float().cpu(), sn[:, :n].float().cpu())
    _close(oq[:, :, :n], rq.to(dtype), dtype)
    _close(ok[:, :, :n], rk.to(dtype), dtype)
    # inverse rotation: the backward kernel applied to the forward output
    bq, bk = ForgeRoPEv3Function.backward(_Ctx(c, sn), oq, ok)[:2]  # rotation by -theta
    torch.testing.assert_close(bq.float(), q.float(), atol=3e-2, rtol=3e-2)
    torch.testing.assert_close(bk.float(), k.float(), atol=3e-2, rtol=3e-2)
    # norm of each (j, j + D/2) pair is preserved
    def pair_norm(x):
        x = x.float()
        return x[..., : D // 2] ** 2 + x[..., D // 2:] ** 2
    torch.testing.assert_close(pair_norm(oq), pair_norm(q), atol=5e-2, rtol=2e-2)


class _Ctx:
    def __init__(self, c, s):
        self.saved_tensors = (c, s)
        self.positions = None


def test_rope_cos_sin_builder_matches_oracle():
    """The package's configurable-base table builder equals the oracle's
    (kernels/rope/tests/test_v1.py:75-83) on the CPU."""
    for base in (10000.0, 500000.0):
        pos = torch.arange(4096)
        c, s = rope_cos_sin(pos, 128, base, torch.float32)
        rc, rs = cos_sin(pos, 128, base, torch.float32)
        assert torch.equal(c, rc) and torch.equal(s, rs)


# --- v1 / v2 APIs (kernels/rope/forge_rope_v1.py, forge_rope_v2.py): same
# rotation kernel, their own Function names, assert messages and checks ---
from kernels.rope.forge_rope_v1 import ForgeRoPEv1, ForgeRoPEv1Function  # noqa: E402
from kernels.rope.forge_rope_v1 import apply_rope as apply_rope_v1  # noqa: E402
from kernels.rope.forge_rope_v2 import ForgeRoPEv2, ForgeRoPEv2Function  # noqa: E402
from kernels.rope.forge_rope_v2 import apply_rope as apply_rope_v2  # noqa: E402


def test_rope_v1_v2_shape_messages():
    q = torch.zeros(1, 6, 8, 64)
    k = torch.zeros(1, 4, 8, 64)
    c, s = cos_sin(torch.arange(8), 64, 10000.0, torch.float32)
    c, s = c.unsqueeze(0), s.unsqueeze(0)
    with pytest.raises(AssertionError, match=r"V2 requires n_q % n_kv == 0 \(got n_q=6, n_kv=4\)"):
        apply_rope_v2(q, k, c, s)
    with pytest.raises(AssertionError, match="q must be 4D"):
        apply_rope_v1(q[0], k, c, s)
    with pytest.raises(AssertionError, match=r"cos shape \(1, 8, 64\) mismatch \(expected \(.,9,64\)\)"):
        apply_rope_v1(torch.zeros(1, 6, 9, 64), torch.zeros(1, 4, 9, 64), c, s)
    with pytest.raises(AssertionError, match="sin/cos shape mismatch"):
        apply_rope_v2(q[:, :4], k, c, s[:, :4])
    with pytest.raises(AssertionError, match="head_dim must be a power of 2"):
        apply_rope_v1(torch.zeros(1, 2, 8, 48), torch.zeros(1, 2, 8, 48), c[..., :48], s[..., :48])


@pytest.mark.gpu
@pytest.mark.parametrize("version", ["v1", "v2"])
@pytest.mark.parametrize("label,b,nq,nkv,s,d", SHAPES[:3] + SHAPES[4:])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_rope_v1_v2_forward_backward(version, label, b, nq, nkv, s, d, dtype):
    q, k, c, sn = _inputs(b, nq, nkv, s, d, dtype, seed=3)
    dq = torch.randn(q.shape).to(dtype)
    dk = torch.randn(k.shape).to(dtype)
    rq, rk, rdq, rdk = rope_fwd_bwd(q, k, c, sn, dq, dk)
    qg = q.cuda().requires_grad_(True)
    kg = k.cuda().requires_grad_(True)
    fn = apply_rope_v1 if version == "v1" else apply_rope_v2
    oq, ok = fn(qg, kg, c.cuda(), sn.cuda())
    assert type(oq.grad_fn).__name__.startswith("ForgeRoPE" + version + "Function")
    _close(oq, rq, dtype)
    _close(ok, rk, dtype)
    torch.autograd.backward((oq, ok), (dq.cuda(), dk.cuda()))
    _close(qg.grad, rdq, dtype)
    _close(kg.grad, rdk, dtype)


@pytest.mark.gpu
def test_rope_v1_non_divisible_gqa_and_gradcheck():
    """v1 accepts n_q % n_kv != 0 (its reference grid needs no grouping);
    fp64 gradcheck through ForgeRoPEv1Function and the Module form."""
    q, k, c, sn = _inputs(2, 6, 4, 40, 64, torch.bfloat16, seed=9)
    rq, rk = hf_apply_rotary_pos_emb(q.float(), k.float(), c.float(), sn.float())
    oq, ok = ForgeRoPEv1()(q.cuda(), k.cuda(), c.cuda(), sn.cuda())
    _close(oq, rq.to(torch.bfloat16), torch.bfloat16)
    _close(ok, rk.to(torch.bfloat16), torch.bfloat16)
    q, k, c, sn = _inputs(1, 4, 2, 6, 16, torch.float64, seed=10)
    qg = q.cuda().requires_grad_(True)
    kg = k.cuda().requires_grad_(True)
    # fp32 math inside, so the reference test's gradcheck settings (test_v1.py:273-340)
    kw = dict(eps=1e-3, atol=1e-2, rtol=1e-2, nondet_tol=1e-3)
    assert torch.autograd.gradcheck(lambda a, b_: ForgeRoPEv1Function.apply(a, b_, c.cuda(), sn.cuda()), (qg, kg), **kw)
    assert torch.autograd.gradcheck(lambda a, b_: ForgeRoPEv2Function.apply(a, b_, c.cuda(), sn.cuda()), (qg, kg), **kw)
    oq2, _ = ForgeRoPEv2()(qg, kg, c.cuda(), sn.cuda())
    torch.testing.assert_close(oq2, apply_rope(qg, kg, c.cuda(), sn.cuda())[0], rtol=0, atol=0)


@pytest.mark.gpu
def test_rope_64bit_offsets_match_32bit():
    """Index math is 32-bit when every element offset fits and 64-bit
    otherwise: q as a view whose second batch lies 2^31 elements into a
    4.3 GB buffer takes the 64-bit path (forward and backward), and gives
    bit-identical results to the same values in a compact tensor."""
    b, nq, nkv, s, d = 2, 2, 1, 16, 64
    dtype = torch.bfloat16
    g = torch.Generator().manual_seed(11)
    q_small = torch.randn(b, nq, s, d, generator=g).to(dtype).cuda()
    k = torch.randn(b, nkv, s, d, generator=g).to(dtype).cuda()
    dq = torch.randn(b, nq, s, d, generator=g).to(dtype).cuda()
    dk = torch.randn(b, nkv, s, d, generator=g).to(dtype).cuda()
    c, sn = (t.unsqueeze(0).cuda() for t in cos_sin(torch.arange(s), d, 10000.0, dtype))
    stride_b = 2 ** 31
    big = torch.empty(stride_b + nq * s * d, dtype=dtype, device="cuda")
    q_far = big.as_strided((b, nq, s, d), (stride_b, s * d, d, 1))
    q_far.copy_(q_small)
    results = []
    for q in (q_small, q_far):
        qg = q.detach().requires_grad_(True)
        kg = k.clone().requires_grad_(True)
        oq, ok = apply_rope(qg, kg, c, sn)
        (oq * dq).sum().add((ok * dk).sum()).backward()
        results.append([oq.contiguous(), ok, qg.grad.contiguous(), kg.grad])
    del big, q_far
    for a, bb in zip(*results):
        assert torch.equal(a, bb)
