"""Pinning tests for the CPU oracle (oracle/), run with -m "not gpu".

The oracle restates the reference's PyTorch paths; these tests check each of
its functions against something that does not share its formula, chosen so
that a plausible slip (a dropped term, a wrong sign or index, a transposed
operand, a wrong rounding order) fails at least one of them:

  SwiGLU   float64 numpy closed form; analytic derivative; the reference's
           special values (tests/test_swiglu.py:102-113); the exact identity
           dup == dout * silu(gate) (fp32, gm = dm = 1); bf16 rounding order
           checked with an independent round-to-nearest-even in numpy.
  RoPE     rotation as complex multiplication in numpy complex128; pair norm
           preservation; backward(forward(x)) == x; one-hot gradient =
           (cos, -sin) (kernels/rope/tests/test_v1.py:286-307); cos/sin
           against float64 angles; the algorithmic byte count of
           benchmarks/bench_v3.py:333-338.
  CE       float64 brute-force log-softmax loops; F.cross_entropy (the
           reference tests' comparator, test_cross_entropy.py:71-78) for
           every reduction / ignore_index / label smoothing / weight case;
           the z-loss reference of test_cross_entropy.py:263-301; softcap
           chain rule by autograd; gradient row sums; ignore-row semantics
           (cross_entropy_kernel_v2.py:139-151); all-ignored mean -> 0; the
           BASELINE byte count.
  LoRA     the hand-written backward against autograd of the forward
           composition in float64 (gradcheck-style); the forward against a
           numpy float64 composition; BASELINE's FLOP counts; RoPE fused
           into QKV against the adjoint rotation; varlen positions.
"""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import cross_entropy as oce
from oracle import lora_mlp as omlp
from oracle import lora_qkv as oqkv
from oracle import rope as orope
from oracle import swiglu as oswi


def _np_bf16(x: np.ndarray) -> np.ndarray:
    """Round float32 values to bfloat16 (round to nearest, ties to even) by
    bit manipulation, independent of torch's cast."""
    b = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    lsb = (b >> 16) & 1
    r = ((b + 0x7FFF + lsb) >> 16) << 16
    return r.astype(np.uint32).view(np.float32)


# ---------------------------------------------------------------------------
# SwiGLU
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("gm,dm", [(1.0, 1.0), (0.7, 1.3)])
def test_swiglu_forward_matches_float64_closed_form(gm, dm):
    g = torch.Generator().manual_seed(0)
    gate = torch.randn(64, 33, generator=g)
    up = torch.randn(64, 33, generator=g)
    out = oswi.swiglu_ref(gate, up, gm, dm).numpy().astype(np.float64)
    x = gate.numpy().astype(np.float64) * gm
    expect = x / (1.0 + np.exp(-x)) * up.numpy().astype(np.float64) * dm
    np.testing.assert_allclose(out, expect, rtol=2e-6, atol=1e-7)


@pytest.mark.parametrize("gm,dm", [(1.0, 1.0), (0.7, 1.3)])
def test_swiglu_backward_matches_analytic_derivative(gm, dm):
    g = torch.Generator().manual_seed(1)
    gate, up, dout = (torch.randn(16, 40, generator=g, dtype=torch.float64) for _ in range(3))
    # float64 inputs: the oracle computes silu in fp32 (gate.float()), so compare
    # against the float64 derivative with fp32 tolerance
    _, dgate, dup = oswi.swiglu_fwd_bwd(gate, up, dout, gm, dm)
    x = gate.numpy() * gm
    sig = 1.0 / (1.0 + np.exp(-x))
    silu = x * sig
    np.testing.assert_allclose(dup.numpy(), dout.numpy() * dm * silu, rtol=1e-6, atol=1e-7)
    d_silu = sig * (1.0 + x * (1.0 - sig))
    np.testing.assert_allclose(dgate.numpy(), dout.numpy() * dm * up.numpy() * gm * d_silu, rtol=1e-5, atol=1e-6)


def test_swiglu_special_values():
    """tests/test_swiglu.py:102-113: 0, +-inf, nan, +-20."""
    gate = torch.tensor([[0.0, float("inf"), float("-inf"), float("nan"), 20.0, -20.0]])
    up = torch.tensor([[1.0, 2.0, 3.0, 4.0, -1.0, -2.0]])
    out = oswi.swiglu_ref(gate, up)
    assert out[0, 0].item() == 0.0
    assert out[0, 1].item() == float("inf")          # silu(inf) = inf
    assert math.isnan(out[0, 2].item())              # silu(-inf) = -inf * 0 = nan
    assert math.isnan(out[0, 3].item())
    assert out[0, 4].item() == pytest.approx(-20.0 / (1 + math.exp(-20.0)), rel=1e-6)
    assert out[0, 5].item() == pytest.approx(-2.0 * (-20.0 / (1 + math.exp(20.0))), rel=1e-5)


def test_swiglu_dup_identity_fp32():
    g = torch.Generator().manual_seed(2)
    gate, up, dout = (torch.randn(8, 128, generator=g) for _ in range(3))
    _, _, dup = oswi.swiglu_fwd_bwd(gate, up, dout)
    assert torch.equal(dup, dout * F.silu(gate))


def test_swiglu_bf16_rounding_order():
    """swiglu.py:179-188: silu in fp32, rounded to bf16, then the product
    rounded to bf16 (two roundings), then * dm rounded again."""
    g = torch.Generator().manual_seed(3)
    gate = torch.randn(4096, generator=g).to(torch.bfloat16)
    up = torch.randn(4096, generator=g).to(torch.bfloat16)
    out = oswi.swiglu_ref(gate, up, 1.0, 1.5).float().numpy()
    xg = gate.float().numpy().astype(np.float64)
    silu = _np_bf16((xg / (1 + np.exp(-xg))).astype(np.float32))
    prod = _np_bf16((silu.astype(np.float64) * up.float().numpy()).astype(np.float32))
    expect = _np_bf16((prod.astype(np.float64) * 1.5).astype(np.float32))
    # float64 silu vs fp32 silu differ in rare ties: allow a handful of 1-ulp cases
    mismatch = np.count_nonzero(out != expect)
    assert mismatch <= 4, mismatch
    # and a single-rounding variant is measurably different (the order matters)
    single = _np_bf16((xg / (1 + np.exp(-xg)) * up.float().numpy() * 1.5).astype(np.float32))
    assert np.count_nonzero(out != single) > 40


def test_swiglu_packed_matches_split():
    g = torch.Generator().manual_seed(4)
    gu = torch.randn(6, 2 * 24, generator=g)
    dout = torch.randn(6, 24, generator=g)
    out_p, dgu = oswi.swiglu_packed_fwd_bwd(gu, dout, 0.5, 2.0)
    out_s, dg, du = oswi.swiglu_fwd_bwd(gu[:, :24], gu[:, 24:], dout, 0.5, 2.0)
    assert torch.equal(out_p, out_s)
    assert torch.equal(dgu, torch.cat([dg, du], dim=-1))


# ---------------------------------------------------------------------------
# RoPE
# ---------------------------------------------------------------------------
def _rope_case(B=2, Hq=4, Hkv=2, S=16, D=32, base=10000.0, seed=0, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, Hq, S, D, generator=g).to(dtype)
    k = torch.randn(B, Hkv, S, D, generator=g).to(dtype)
    cos, sin = orope.cos_sin(torch.arange(S), D, base, dtype)
    return q, k, cos.unsqueeze(0), sin.unsqueeze(0)


@pytest.mark.parametrize("base", [10000.0, 500000.0])
def test_rope_is_complex_rotation(base):
    q, k, cos, sin = _rope_case(base=base)
    oq, ok = orope.hf_apply_rotary_pos_emb(q, k, cos, sin)
    D = q.shape[-1]
    S = q.shape[2]
    theta = np.arange(S)[:, None] * (base ** (-np.arange(0, D, 2) / D))[None, :]  # (S, D/2) float64
    for x, o in ((q, oq), (k, ok)):
        xn = x.numpy().astype(np.float64)
        z = xn[..., : D // 2] + 1j * xn[..., D // 2:]
        zr = z * np.exp(1j * theta)[None, None]
        expect = np.concatenate([zr.real, zr.imag], axis=-1)
        np.testing.assert_allclose(o.numpy(), expect, rtol=1e-5, atol=2e-5)


def test_rope_preserves_pair_norms_and_inverts():
    q, k, cos, sin = _rope_case(D=64, S=32)
    oq, ok = orope.hf_apply_rotary_pos_emb(q, k, cos, sin)
    D = q.shape[-1]
    n_in = q[..., : D // 2] ** 2 + q[..., D // 2:] ** 2
    n_out = oq[..., : D // 2] ** 2 + oq[..., D // 2:] ** 2
    torch.testing.assert_close(n_out, n_in, rtol=1e-5, atol=1e-5)
    # backward is the transpose rotation: feeding the forward output as the
    # upstream gradient returns the input
    _, _, gq, gk = orope.rope_fwd_bwd(q, k, cos, sin, oq, ok)
    torch.testing.assert_close(gq, q, rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(gk, k, rtol=1e-5, atol=1e-5)


def test_rope_one_hot_gradient():
    """kernels/rope/tests/test_v1.py:286-307: the gradient of out[..., j] w.r.t.
    x is cos_j at j and -sin_j / +sin_j at the partner column."""
    q, k, cos, sin = _rope_case(B=1, Hq=1, Hkv=1, S=4, D=8)
    D = 8
    for j in range(D):
        dq = torch.zeros_like(q)
        dq[..., j] = 1.0
        _, _, gq, _ = orope.rope_fwd_bwd(q, k, cos, sin, dq, torch.zeros_like(k))
        c, s = cos[0, :, j], sin[0, :, j]
        torch.testing.assert_close(gq[0, 0, :, j], c)
        partner = (j + D // 2) % D
        sign = 1.0 if j < D // 2 else -1.0  # d out_lo / d hi = -sin ; d out_hi / d lo = +sin
        torch.testing.assert_close(gq[0, 0, :, partner], -sign * s if j < D // 2 else s)
        others = [i for i in range(D) if i not in (j, partner)]
        assert torch.count_nonzero(gq[0, 0, :, others]) == 0


def test_rope_cos_sin_builder():
    pos = torch.tensor([0, 1, 7, 4095])
    D = 128
    for base in (10000.0, 500000.0):
        c, s = orope.cos_sin(pos, D, base, torch.float32)
        theta = pos.numpy()[:, None].astype(np.float64) * (base ** (-np.arange(0, D, 2) / D))[None, :]
        # freqs are formed in fp32 (as the reference does): ~pos * 6e-8 angle error
        tol = 4096 * 1.2e-7 + 1e-6
        np.testing.assert_allclose(c[:, : D // 2].numpy(), np.cos(theta), atol=tol)
        np.testing.assert_allclose(s[:, : D // 2].numpy(), np.sin(theta), atol=tol)
        assert torch.equal(c[:, : D // 2], c[:, D // 2:]) and torch.equal(s[:, : D // 2], s[:, D // 2:])
    c1, _ = orope.cos_sin(pos, D, 10000.0, torch.float32)
    c2, _ = orope.cos_sin(pos, D, 500000.0, torch.float32)
    assert not torch.equal(c1, c2)  # the base reaches the tables


def test_rope_bytes_known_answer():
    """benchmarks/bench_v3.py:333-338 at the BASELINE shape: 337,641,472 B per direction."""
    B, S, Hq, Hkv, D = 4, 4096, 32, 8, 128
    per_dir = 2 * (B * Hq * S * D + B * Hkv * S * D) * 2 + 2 * S * D * 2
    assert per_dir == 337_641_472


# ---------------------------------------------------------------------------
# Cross-entropy
# ---------------------------------------------------------------------------
def _ce_case(bt=12, V=37, seed=0, scale=2.0):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(bt, V, generator=g) * scale
    t = torch.randint(0, V, (bt,), generator=g)
    return x, t


def test_ce_brute_force_float64():
    x, t = _ce_case()
    t[3] = -100
    loss, _, rows, acc, pred, grad = oce.ce_reference(x, t, reduction="none", compute_dtype=torch.float64)
    xn = x.numpy().astype(np.float64)
    for i in range(x.shape[0]):
        if t[i] == -100:
            assert rows[i].item() == 0.0 and pred[i].item() == -1
            assert np.all(grad[i].numpy() == 0.0)
            continue
        m = max(xn[i])
        s = sum(math.exp(v - m) for v in xn[i])
        lse = m + math.log(s)
        assert rows[i].item() == pytest.approx(lse - xn[i, t[i]], rel=1e-12)
        p = np.array([math.exp(v - lse) for v in xn[i]])
        p[t[i]] -= 1.0
        np.testing.assert_allclose(grad[i].numpy(), p, rtol=1e-10, atol=1e-14)
        assert pred[i].item() == int(np.argmax(xn[i]))


@pytest.mark.parametrize("reduction", ["mean", "sum", "none"])
@pytest.mark.parametrize("ignore_index", [-100, 5])
@pytest.mark.parametrize("label_smoothing", [0.0, 0.1])
@pytest.mark.parametrize("use_weight", [False, True])
def test_ce_matches_torch_cross_entropy(reduction, ignore_index, label_smoothing, use_weight):
    x, t = _ce_case(bt=20, V=31, seed=11)
    t[::4] = ignore_index
    w = torch.rand(31, generator=torch.Generator().manual_seed(5)) + 0.5 if use_weight else None
    loss, _, _, _, _, grad = oce.ce_reference(x, t, weight=w, ignore_index=ignore_index,
                                              label_smoothing=label_smoothing, reduction=reduction,
                                              compute_dtype=torch.float64)
    xr = x.double().requires_grad_(True)
    ref = F.cross_entropy(xr, t, weight=None if w is None else w.double(), ignore_index=ignore_index,
                          reduction=reduction, label_smoothing=label_smoothing)
    torch.testing.assert_close(loss, ref.detach(), rtol=1e-10, atol=1e-12)
    ref.sum().backward()
    torch.testing.assert_close(grad, xr.grad, rtol=1e-10, atol=1e-12)


@pytest.mark.parametrize("reduction", ["mean", "sum", "none"])
@pytest.mark.parametrize("softcap", [None, 20.0])
def test_ce_z_loss_and_softcap_against_test_reference(reduction, softcap):
    """The z-loss/softcap reference of test_cross_entropy.py:263-301, evaluated
    in float64, and the softcap chain rule by autograd."""
    x, t = _ce_case(bt=16, V=29, seed=3, scale=8.0)
    t[2] = -100
    zs = 1e-3
    loss, z, _, _, _, grad = oce.ce_reference(x, t, lse_square_scale=zs, reduction=reduction, softcap=softcap,
                                              compute_dtype=torch.float64)
    xr = x.double().requires_grad_(True)
    xs = softcap * torch.tanh(xr / softcap) if softcap is not None else xr
    ce = F.cross_entropy(xs, t, ignore_index=-100, reduction=reduction)
    mask = t != -100
    zr = torch.where(mask, zs * torch.logsumexp(xs, dim=-1) ** 2, torch.zeros((), dtype=torch.float64))
    if reduction == "mean":
        zr = zr.sum() / mask.sum()
    elif reduction == "sum":
        zr = zr.sum()
    total = ce + zr
    torch.testing.assert_close(loss, total.detach(), rtol=1e-10, atol=1e-12)
    torch.testing.assert_close(z, zr.detach(), rtol=1e-10, atol=1e-12)
    total.sum().backward()
    torch.testing.assert_close(grad, xr.grad, rtol=1e-9, atol=1e-12)


def test_ce_gradient_invariants_and_all_ignored():
    x, t = _ce_case(bt=9, V=50, seed=4)
    t[1] = -100
    _, _, _, _, _, grad = oce.ce_reference(x, t, reduction="sum", compute_dtype=torch.float64)
    valid = t != -100
    assert torch.allclose(grad[valid].sum(-1), torch.zeros(int(valid.sum()), dtype=torch.float64), atol=1e-12)
    assert torch.count_nonzero(grad[~valid]) == 0
    gy = grad[valid].gather(1, t[valid].unsqueeze(1))
    assert (gy < 0).all()
    # all rows ignored, mean: loss 0 and zero gradient (v2 semantics,
    # test_cross_entropy.py:227-237), not NaN
    loss, _, _, _, _, g0 = oce.ce_reference(x, torch.full_like(t, -100), reduction="mean")
    assert loss.item() == 0.0 and torch.count_nonzero(g0) == 0


def test_ce_argmax_ties_first_index():
    x = torch.zeros(2, 10)
    x[:, 3] = 1.0
    x[:, 7] = 1.0
    _, _, _, _, pred, _ = oce.ce_reference(x, torch.tensor([3, 7]), reduction="none")
    assert pred.tolist() == [3, 3]


def test_ce_bytes_known_answer():
    """V (4 n_valid + 2 n_ignored) + 8 N at the BASELINE config: 4,097,588,224 B."""
    assert oce.ce_bytes(128256, 8192 - 410, 410) == 4_097_588_224


def test_ce_planted_mistake_is_caught():
    """A dropped label-smoothing term (a plausible slip) must fail the
    F.cross_entropy comparison used above."""
    x, t = _ce_case(bt=8, V=17, seed=9)
    ref = F.cross_entropy(x.double(), t, label_smoothing=0.2)
    wrong = F.cross_entropy(x.double(), t) * (1 - 0.2)
    assert not torch.allclose(wrong, ref, rtol=1e-6)


# ---------------------------------------------------------------------------
# LoRA-MLP
# ---------------------------------------------------------------------------
def _mlp_params(H=12, I=20, r=3, seed=0):
    g = torch.Generator().manual_seed(seed)
    p = list(omlp.make_params(H, I, r, 2 * r, g, dtype=torch.float64))
    # make the LoRA terms O(1) so a dropped term is visible
    for i in (2, 6, 10):
        p[i] = p[i] * 50
    return tuple(p)


def test_lora_mlp_backward_matches_autograd_float64():
    p = _mlp_params()
    g = torch.Generator().manual_seed(1)
    X = torch.randn(7, 12, generator=g, dtype=torch.float64)
    dY = torch.randn(7, 12, generator=g, dtype=torch.float64)
    out, e, gg = omlp.forward(X, *p)
    grads = omlp.backward(dY, X, e, gg, *p)
    leaves = [X.clone().requires_grad_(True)] + [t.clone().requires_grad_(True) if isinstance(t, torch.Tensor) else t
                                                 for t in p]
    o2, _, _ = omlp.forward(*leaves)
    (o2 * dY).sum().backward()
    # returned order: dX, dA_g, dB_g, dA_u, dB_u, dA_d, dB_d
    expect = [leaves[0].grad, leaves[2].grad, leaves[3].grad, leaves[6].grad, leaves[7].grad, leaves[10].grad,
              leaves[11].grad]
    # the reference rounds sigmoid(e) through float32 even for float64 inputs
    # (lora_mlp_pytorch.py:165), hence fp32-level tolerance; the LoRA terms are
    # O(1) here, so a dropped or mis-signed term misses by orders of magnitude
    for got, exp in zip(grads, expect):
        torch.testing.assert_close(got, exp, rtol=2e-5, atol=2e-6)


@pytest.mark.parametrize("activation", ["gelu_tanh", "gelu_exact"])
def test_lora_mlp_gelu_backward_matches_autograd_float64(activation):
    """The GeGLU MLP oracle (lora.py:170-188 composition): hand-written
    backward against autograd of its forward, and the forward's h against
    torch's own F.gelu; a planted slip (gelu' without its x pdf(x) term) must
    fail the gradient check."""
    p = _mlp_params(seed=6)
    g = torch.Generator().manual_seed(7)
    X = torch.randn(7, 12, generator=g, dtype=torch.float64) * 2
    dY = torch.randn(7, 12, generator=g, dtype=torch.float64)
    out, e, gg = omlp.forward(X, *p, activation=activation)
    grads = omlp.backward(dY, X, e, gg, *p, activation=activation)
    leaves = [X.clone().requires_grad_(True)] + [t.clone().requires_grad_(True) if isinstance(t, torch.Tensor) else t
                                                 for t in p]
    o2, _, _ = omlp.forward(*leaves, activation=activation)
    (o2 * dY).sum().backward()
    expect = [leaves[0].grad, leaves[2].grad, leaves[3].grad, leaves[6].grad, leaves[7].grad, leaves[10].grad,
              leaves[11].grad]
    for got, exp in zip(grads, expect):
        torch.testing.assert_close(got, exp, rtol=1e-9, atol=1e-10)
    approx = "tanh" if activation == "gelu_tanh" else "none"
    h = F.gelu(e, approximate=approx) * gg
    torch.testing.assert_close(out, omlp.matmul_lora(h, *p[8:12]), rtol=1e-12, atol=1e-12)
    assert e.min() < -2 and e.max() > 2

    real = omlp._gelu
    try:
        omlp._gelu = lambda x, a: (real(x, a)[0], (real(x, a)[0] / x))  # Phi(x) only
        wrong = omlp.backward(dY, X, e, gg, *p, activation=activation)
    finally:
        omlp._gelu = real
    assert not torch.allclose(wrong[0], expect[0], rtol=1e-3, atol=1e-4)


def test_lora_mlp_forward_matches_numpy():
    p = _mlp_params(seed=2)
    X = torch.randn(5, 12, generator=torch.Generator().manual_seed(3), dtype=torch.float64)
    out, e, g = omlp.forward(X, *p)
    n = [t.numpy() if isinstance(t, torch.Tensor) else t for t in p]
    Xn = X.numpy()

    def proj(W, A, B, s, Z):
        return Z @ W.T + s * (Z @ A.T) @ B.T

    en = proj(n[0], n[1], n[2], n[3], Xn)
    gn = proj(n[4], n[5], n[6], n[7], Xn)
    h = en / (1 + np.exp(-en)) * gn
    np.testing.assert_allclose(out.numpy(), proj(n[8], n[9], n[10], n[11], h), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(e.numpy(), en, rtol=1e-12)
    np.testing.assert_allclose(g.numpy(), gn, rtol=1e-12)


def test_lora_mlp_flops_known_answer():
    assert omlp.flops(8192, 4096, 14336, 16) == 5_821_828_169_728


def test_lora_mlp_lora_grads_match_autograd_float64():
    """lora_grads (the LoRA-parameter gradients without the out / dX
    products, used at the BASELINE token count) against autograd of the
    forward: every gradient, O(1) LoRA terms so a dropped term or a swapped
    gate / up slot is visible."""
    p = _mlp_params(seed=8)
    g = torch.Generator().manual_seed(9)
    X = torch.randn(9, 12, generator=g, dtype=torch.float64)
    dY = torch.randn(9, 12, generator=g, dtype=torch.float64)
    got = omlp.lora_grads(dY, X, *p)
    leaves = [X.clone().requires_grad_(True)] + [t.clone().requires_grad_(True) if isinstance(t, torch.Tensor) else t
                                                 for t in p]
    o2, _, _ = omlp.forward(*leaves)
    (o2 * dY).sum().backward()
    expect = [leaves[2].grad, leaves[3].grad, leaves[6].grad, leaves[7].grad, leaves[10].grad, leaves[11].grad]
    for a, b in zip(got, expect):
        torch.testing.assert_close(a, b, rtol=2e-5, atol=2e-6)
    assert not torch.allclose(got[0], got[2], rtol=1e-3)  # gate and up differ


# ---------------------------------------------------------------------------
# LoRA-QKV
# ---------------------------------------------------------------------------
def _qkv_params(K=16, Hq=16, Hkv=8, r=4, seed=0):
    g = torch.Generator().manual_seed(seed)
    p = list(oqkv.make_params(K, Hq, Hkv, r, 2 * r, g, dtype=torch.float64))
    for i in (4, 7, 10):
        p[i] = p[i] * 50
    return p


def test_lora_qkv_backward_matches_autograd_float64():
    p = _qkv_params()
    g = torch.Generator().manual_seed(1)
    X = torch.randn(6, 16, generator=g, dtype=torch.float64)
    dQ = torch.randn(6, 16, generator=g, dtype=torch.float64)
    dK = torch.randn(6, 8, generator=g, dtype=torch.float64)
    dV = torch.randn(6, 8, generator=g, dtype=torch.float64)
    grads = oqkv.backward(dQ, dK, dV, X, *p)
    leaves = [X.clone().requires_grad_(True)] + [t.clone().requires_grad_(True) if isinstance(t, torch.Tensor) else t
                                                 for t in p]
    Q, K_, V = oqkv.forward(*leaves)
    ((Q * dQ).sum() + (K_ * dK).sum() + (V * dV).sum()).backward()
    # forward args: X, W_q, W_k, W_v, A_q, B_q, s_q, A_k, B_k, s_k, A_v, B_v, s_v
    expect = [leaves[0].grad, leaves[4].grad, leaves[5].grad, leaves[7].grad, leaves[8].grad, leaves[10].grad,
              leaves[11].grad]
    for got, exp in zip(grads, expect):
        torch.testing.assert_close(got, exp, rtol=1e-10, atol=1e-12)


def test_lora_qkv_forward_matches_numpy():
    p = _qkv_params(seed=4)
    X = torch.randn(5, 16, generator=torch.Generator().manual_seed(5), dtype=torch.float64)
    Q, K_, V = oqkv.forward(X, *p)
    n = [t.numpy() if isinstance(t, torch.Tensor) else t for t in p]
    Xn = X.numpy()
    for out, (W, A, B, s) in ((Q, (n[0], n[3], n[4], n[5])), (K_, (n[1], n[6], n[7], n[8])),
                              (V, (n[2], n[9], n[10], n[11]))):
        np.testing.assert_allclose(out.numpy(), Xn @ W.T + s * (Xn @ A.T) @ B.T, rtol=1e-12, atol=1e-12)


def test_lora_qkv_rope_backward_is_adjoint_rotation():
    """Gradients through the fused RoPE equal the plain QKV backward fed with
    dQ, dK rotated back by -theta (the rotation's transpose)."""
    D = 8
    p = _qkv_params(K=16, Hq=16, Hkv=8, r=4, seed=6)
    g = torch.Generator().manual_seed(7)
    X = torch.randn(5, 16, generator=g, dtype=torch.float64)
    dQ = torch.randn(5, 16, generator=g, dtype=torch.float64)
    dK = torch.randn(5, 8, generator=g, dtype=torch.float64)
    dV = torch.randn(5, 8, generator=g, dtype=torch.float64)
    pos = oqkv.positions_for([3, 2])
    c, s = orope.cos_sin(pos, D, 500000.0, torch.float64)
    _, grads = oqkv.qkv_rope_fwd_bwd(X, dQ, dK, dV, p, c, s, D, compute_dtype=torch.float64)
    dQr = oqkv.rope_rows(dQ, c, -s, D)
    dKr = oqkv.rope_rows(dK, c, -s, D)
    plain = oqkv.backward(dQr, dKr, dV, X, *p)
    for got, exp in zip(grads, plain):
        torch.testing.assert_close(got, exp, rtol=1e-10, atol=1e-12)


def test_lora_qkv_lora_grads_equal_backward_parts():
    """lora_grads is backward's LoRA-parameter part (backward is pinned by
    autograd above); a slip in one of its products (e.g. dB from X instead of
    X A^T) would not keep the shapes and values equal."""
    p = _qkv_params(seed=11)
    g = torch.Generator().manual_seed(12)
    X = torch.randn(7, 16, generator=g, dtype=torch.float64)
    dQ = torch.randn(7, 16, generator=g, dtype=torch.float64)
    dK = torch.randn(7, 8, generator=g, dtype=torch.float64)
    dV = torch.randn(7, 8, generator=g, dtype=torch.float64)
    full = oqkv.backward(dQ, dK, dV, X, *p)
    part = oqkv.lora_grads(dQ, dK, dV, X, *p)
    assert len(part) == 6
    for got, exp in zip(part, full[1:]):
        torch.testing.assert_close(got, exp, rtol=1e-12, atol=1e-12)


def test_lora_qkv_rope_rows_matches_complex_rotation():
    D = 8
    Y = torch.randn(4, 3 * D, generator=torch.Generator().manual_seed(8), dtype=torch.float64)
    pos = torch.tensor([0, 5, 1, 9])
    c, s = orope.cos_sin(pos, D, 10000.0, torch.float64)
    out = oqkv.rope_rows(Y, c, s, D).numpy().reshape(4, 3, D)
    y = Y.numpy().reshape(4, 3, D)
    # multiply each (lo, hi) pair, as a complex number, by w = cos + i sin
    w = c[:, : D // 2].numpy() + 1j * s[:, : D // 2].numpy()
    z = (y[..., : D // 2] + 1j * y[..., D // 2:]) * w[:, None, :]
    np.testing.assert_allclose(out, np.concatenate([z.real, z.imag], -1), rtol=1e-9, atol=1e-9)


def test_lora_qkv_varlen_positions_and_flops():
    assert oqkv.positions_for([3, 2]).tolist() == [0, 1, 2, 0, 1]
    lens = oqkv.varlen_lengths(8, 512, 4096, seed=0)
    assert len(lens) == 8 and all(512 <= n <= 4096 for n in lens)
    assert oqkv.varlen_lengths(8, 512, 4096, seed=0) == lens
    assert oqkv.flops_per_token(4096, 4096, 1024, 64) == 109_314_048


# ---------------------------------------------------------------------------
# fused linear + cross-entropy: pinned against autograd of the torch
# composition F.cross_entropy(F.linear(x, W, b)) in float64 (the reference
# tests' comparator, kernels/cross_entropy/tests/test_fused_linear_cross_entropy.py:64-96)
# ---------------------------------------------------------------------------
from oracle import fused_linear_ce as oflce  # noqa: E402


def _flce_torch(x, W, b, t, ce_weight=None, ignore_index=-100, lse_square_scale=0.0, label_smoothing=0.0,
                reduction="mean", softcap=None, token_scaling=False):
    x = x.clone().requires_grad_(True)
    W = W.clone().requires_grad_(True)
    b = b.clone().requires_grad_(True) if b is not None else None
    logits = F.linear(x, W, b)
    if softcap is not None:
        logits = softcap * torch.tanh(logits / softcap)
    rows = F.cross_entropy(logits, t, weight=ce_weight, ignore_index=ignore_index, reduction="none",
                           label_smoothing=label_smoothing)
    mask = t != ignore_index
    z = torch.where(mask, lse_square_scale * torch.logsumexp(logits, -1) ** 2, torch.zeros_like(rows))
    if reduction == "mean":
        denom = mask.sum() if ce_weight is None else ce_weight[torch.where(mask, t, 0)][mask].sum()
        rows = rows / denom
        z = z / mask.sum()
    rows = rows + z
    if token_scaling:
        p = torch.softmax(logits.detach(), -1).gather(1, torch.where(mask, t, 0).unsqueeze(1)).squeeze(1)
        p = torch.where(mask, p, torch.zeros_like(p))
        rows, z = rows * p, z * p
    loss = rows if reduction == "none" else rows.sum()
    loss.sum().backward()
    return loss.detach(), x.grad, W.grad, (b.grad if b is not None else None)


@pytest.mark.parametrize("case", [
    dict(), dict(reduction="sum"), dict(bias=False), dict(label_smoothing=0.1), dict(ce_weight=True),
    dict(softcap=3.0, lse_square_scale=1e-2), dict(reduction="none"), dict(token_scaling=True),
    dict(token_scaling=True, softcap=2.0, lse_square_scale=1e-3, label_smoothing=0.2),
])
def test_fused_linear_ce_matches_autograd_of_torch_composition(case):
    g = torch.Generator().manual_seed(11)
    bt, h, v = 19, 12, 37
    x = torch.randn(bt, h, generator=g, dtype=torch.float64)
    W = torch.randn(v, h, generator=g, dtype=torch.float64) / h ** 0.5
    b = torch.randn(v, generator=g, dtype=torch.float64) if case.get("bias", True) else None
    t = torch.randint(0, v, (bt,), generator=g)
    t[::4] = -100
    cw = torch.rand(v, generator=g, dtype=torch.float64) + 0.5 if case.get("ce_weight") else None
    kw = dict(ce_weight=cw, lse_square_scale=case.get("lse_square_scale", 0.0),
              label_smoothing=case.get("label_smoothing", 0.0), reduction=case.get("reduction", "mean"),
              softcap=case.get("softcap"))
    ref_loss, ref_dx, ref_dw, ref_db = _flce_torch(x, W, b, t, token_scaling=case.get("token_scaling", False), **kw)
    out = oflce.fused_linear_ce(x, W, t, bias=b, use_token_scaling=case.get("token_scaling", False), **kw)
    torch.testing.assert_close(out["loss"], ref_loss, rtol=1e-10, atol=1e-12)
    torch.testing.assert_close(out["dX"], ref_dx, rtol=1e-10, atol=1e-12)
    torch.testing.assert_close(out["dW"], ref_dw, rtol=1e-10, atol=1e-12)
    if b is not None:
        torch.testing.assert_close(out["db"], ref_db, rtol=1e-10, atol=1e-12)


def test_fused_linear_ce_metrics_and_flops():
    g = torch.Generator().manual_seed(5)
    x = torch.randn(13, 8, generator=g, dtype=torch.float64)
    W = torch.randn(21, 8, generator=g, dtype=torch.float64)
    t = torch.randint(0, 21, (13,), generator=g)
    t[::5] = -100
    out = oflce.fused_linear_ce(x, W, t)
    logits = x @ W.t()
    pred = torch.where(t == -100, torch.full_like(t, -1), logits.argmax(-1))
    assert torch.equal(out["predicted"], pred)
    assert float(out["token_accuracy"]) == pytest.approx(float(((pred == t) & (t != -100)).sum() / (t != -100).sum()))
    assert oflce.flops(8192, 4096, 128256) == 6 * 8192 * 4096 * 128256 == 25_821_343_383_552


# ---------------------------------------------------------------------------
# GeGLU: the formula restatement against torch's own GELU (forward) and
# autograd of F.gelu (derivative), in float64
# ---------------------------------------------------------------------------
from oracle import geglu as ogeglu  # noqa: E402


@pytest.mark.parametrize("approximate", ["tanh", "none"])
def test_geglu_oracle_matches_torch_gelu_and_autograd(approximate):
    g = torch.Generator().manual_seed(3)
    x = (torch.randn(4096, generator=g, dtype=torch.float64) * 3).requires_grad_(True)
    act, grad = ogeglu.gelu_and_grad(x.detach(), approximate)
    ref = F.gelu(x, approximate=approximate)
    ref.sum().backward()
    torch.testing.assert_close(act, ref.detach(), rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(grad, x.grad, rtol=1e-10, atol=1e-12)


@pytest.mark.parametrize("approximate", ["tanh", "none"])
def test_geglu_oracle_fp32_matches_autograd_of_reference_formula(approximate):
    """fp32 storage: out = gelu(gate) * up and its autograd gradients."""
    g = torch.Generator().manual_seed(4)
    gate = torch.randn(64, 33, generator=g, dtype=torch.float64)
    up = torch.randn(64, 33, generator=g, dtype=torch.float64)
    dout = torch.randn(64, 33, generator=g, dtype=torch.float64)
    gv, uv = gate.clone().requires_grad_(True), up.clone().requires_grad_(True)
    (F.gelu(gv, approximate=approximate) * uv).backward(dout)
    out, dgate, dup = ogeglu.geglu_fwd_bwd(gate, up, dout, approximate)
    torch.testing.assert_close(out, F.gelu(gate, approximate=approximate) * up, rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(dgate, gv.grad, rtol=1e-10, atol=1e-12)
    torch.testing.assert_close(dup, uv.grad, rtol=1e-10, atol=1e-12)


def test_geglu_oracle_bf16_rounds_activation_before_product():
    """bf16: the activation is rounded before the product (a single-rounding
    variant differs), and dup uses the rounded activation."""
    g = torch.Generator().manual_seed(6)
    gate = (torch.randn(8192, generator=g) * 2).to(torch.bfloat16)
    up = torch.randn(8192, generator=g).to(torch.bfloat16)
    out, _, _ = ogeglu.geglu_fwd_bwd(gate, up, None, "tanh")
    ref = F.gelu(gate.float(), approximate="tanh").to(torch.bfloat16) * up  # the reference formula
    # the oracle's float64 activation and the reference's fp32 one differ only
    # by a bf16 rounding step, or in the far negative tail where fp32's
    # 1 + tanh cancels (|gelu| < 1e-4 there)
    err = (out.float() - ref.float()).abs()
    assert bool((err <= out.float().abs() * 2 ** -7 + 1e-4).all())
    assert bool(((out == ref) | (err <= out.float().abs() * 2 ** -7) | (gate.float() < -3.5)).all())
    single = (F.gelu(gate.double(), approximate="tanh") * up.double()).to(torch.bfloat16)
    assert int((single != out).sum()) > 50


# ---------------------------------------------------------------------------
# RMSNorm: forward against torch's F.rms_norm, backward against autograd, in
# float64; the casting-mode rounding points in bf16
# ---------------------------------------------------------------------------
from oracle import rmsnorm as orms  # noqa: E402


@pytest.mark.parametrize("offset", [0.0, 1.0])
def test_rmsnorm_oracle_matches_torch_rms_norm_and_autograd(offset):
    g = torch.Generator().manual_seed(9)
    x = torch.randn(6, 5, 40, generator=g, dtype=torch.float64).requires_grad_(True)
    w = (torch.randn(40, generator=g, dtype=torch.float64) * 0.3).requires_grad_(True)
    dy = torch.randn(6, 5, 40, generator=g, dtype=torch.float64)
    ref = F.rms_norm(x, (40,), w + offset, eps=1e-6)
    ref.backward(dy)
    for mode in (orms.LLAMA, orms.GEMMA, orms.NONE):  # no rounding at float64
        y, _ = orms.rms_forward(x, w, 1e-6, offset, mode)
        torch.testing.assert_close(y, ref.detach(), rtol=1e-12, atol=1e-12)
    dx, dw = orms.rms_backward(dy, x, w, offset, 1e-6)
    torch.testing.assert_close(dx, x.grad, rtol=1e-10, atol=1e-12)
    torch.testing.assert_close(dw, w.grad, rtol=1e-10, atol=1e-12)


def test_rmsnorm_oracle_casting_modes_round_where_the_reference_does():
    """bf16: llama rounds the normalised row before the weight product, gemma
    rounds once at the end, none rounds rstd first; each differs from the
    others on random data, and llama equals the reference tests' formula."""
    g = torch.Generator().manual_seed(10)
    x = torch.randn(64, 96, generator=g).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(96, generator=g)).to(torch.bfloat16)
    ys = [orms.rms_forward(x, w, 1e-6, 0.0, m)[0] for m in (orms.LLAMA, orms.GEMMA, orms.NONE)]
    assert not torch.equal(ys[0], ys[1]) and not torch.equal(ys[0], ys[2])
    xf = x.float()
    ref_llama = (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-6)).to(torch.bfloat16) * w
    assert int((ys[0] != ref_llama).sum()) <= 3  # float64 vs fp32 rstd: ties only


def test_rmsnorm_oracle_scale_invariance_and_bytes():
    g = torch.Generator().manual_seed(11)
    x = torch.randn(4, 32, generator=g, dtype=torch.float64)
    w = torch.randn(32, generator=g, dtype=torch.float64)
    y1, _ = orms.rms_forward(x, w, 0.0)
    y2, _ = orms.rms_forward(x * 37.0, w, 0.0)
    torch.testing.assert_close(y1, y2, rtol=1e-12, atol=1e-12)
    assert orms.bytes_fwd_bwd(8192, 4096) == 5 * 8192 * 4096 * 2 + 8 * 8192 + 3 * 4096 * 2
