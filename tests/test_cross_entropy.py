"""Cross-entropy parity: HIP kernel (through libforge_hip.so) vs the CPU oracle.

Cases follow kernels/cross_entropy/tests/test_cross_entropy.py:97-400 (shapes,
reductions, dtypes, ignore_index incl. a valid class id, label smoothing,
non-unit upstream grad, no-grad forward, all-ignored rows, all-ignored mean
-> 0, out-of-bounds targets, class weights, z-loss, softcap, accuracy and
predicted tokens) plus the BASELINE config (bf16 [8192, 128256], 5% ignored).

Tolerances: loss within 1e-3 relative (fp32 internal value) and exact
rounding to the logits dtype; gradients fp32 1e-5, bf16/fp16 2e-2; labels,
ignore rows, predicted tokens and accuracy bit-exact.
"""
import ctypes

import pytest
import torch

from forge_hip import _lib as L
from kernels.cross_entropy.experiments.v2 import CrossEntropyOutput, forge_cross_entropy
from kernels.cross_entropy.experiments.v2.cross_entropy_kernel_v2 import _cross_entropy_forward_impl
from oracle.cross_entropy import ce_reference

GTOL = {torch.float32: 1e-5, torch.float16: 2e-2, torch.bfloat16: 2e-2}
LTOL = {torch.float32: 1e-5, torch.float16: 1e-3, torch.bfloat16: 1e-3}


def _case(bt, vocab, dtype, scalar=1.0, seed=0):
    g = torch.Generator().manual_seed(seed)
    logits = (torch.randn(bt, vocab, generator=g) * scalar).to(dtype)
    target = torch.randint(0, vocab, (bt,), generator=g)
    return logits, target


def _run(logits, target, **kw):
    x = logits.cuda().requires_grad_(True)
    out = forge_cross_entropy(x, target.cuda(), **kw)
    return x, out


def _check(logits, target, reduction="mean", upstream=None, **kw):
    dtype = logits.dtype
    ref_kw = {k: v for k, v in kw.items() if not k.startswith("return_")}
    if ref_kw.get("weight") is not None:
        ref_kw["weight"] = ref_kw["weight"].cpu()
    ref_loss, ref_z, ref_rows, ref_acc, ref_pred, ref_grad = ce_reference(logits, target, reduction=reduction,
                                                                           **ref_kw)
    x, out = _run(logits, target, reduction=reduction, **kw)
    loss = out.loss if isinstance(out, CrossEntropyOutput) else out
    assert loss.dtype == dtype
    t = LTOL[dtype]
    torch.testing.assert_close(loss.float().cpu(), ref_loss.float(), rtol=max(t, 4e-3) if dtype != torch.float32 else t,
                               atol=t)
    grad = upstream if upstream is not None else torch.ones_like(loss)
    loss.backward(gradient=grad.cuda() if upstream is not None else grad)
    if upstream is not None:
        ref_grad = ref_grad * (upstream.float().unsqueeze(1) if upstream.dim() > 0 else upstream.float())
    gt = GTOL[dtype]
    torch.testing.assert_close(x.grad.float().cpu(), ref_grad.float(), rtol=gt, atol=gt)
    return out


@pytest.mark.gpu
@pytest.mark.parametrize("bt,vocab", [(16, 128), (21, 257), (128, 4096)])
@pytest.mark.parametrize("reduction", ["mean", "sum", "none"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_correctness_matches_oracle(bt, vocab, reduction, dtype):
    logits, target = _case(bt, vocab, dtype)
    _check(logits, target, reduction=reduction)
    if dtype != torch.float32 and reduction != "none":
        # the fp32 value before the final cast is within 1e-3 relative
        ref_loss = ce_reference(logits, target, reduction=reduction)[0]
        loss32 = _cross_entropy_forward_impl(logits.cuda(), target.cuda(), None, -100, 0.0, 0.0, reduction,
                                             None, False)[0]
        torch.testing.assert_close(loss32.cpu(), ref_loss, rtol=1e-3, atol=1e-6)
        assert loss32.to(dtype).item() == _run(logits, target, reduction=reduction)[1].item()


@pytest.mark.gpu
@pytest.mark.parametrize("bt,vocab,ignore_index", [(16, 128, -100), (21, 257, -123), (32, 512, 2)])
@pytest.mark.parametrize("reduction", ["mean", "sum", "none"])
def test_ignore_index(bt, vocab, ignore_index, reduction):
    logits, target = _case(bt, vocab, torch.float32)
    target[::3] = ignore_index
    _check(logits, target, reduction=reduction, ignore_index=ignore_index)


@pytest.mark.gpu
@pytest.mark.parametrize("label_smoothing", [0.1, 0.2])
@pytest.mark.parametrize("reduction", ["mean", "sum", "none"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_label_smoothing(label_smoothing, reduction, dtype):
    logits, target = _case(16, 129, dtype)
    _check(logits, target, reduction=reduction, label_smoothing=label_smoothing)


@pytest.mark.gpu
@pytest.mark.parametrize("ignore_index,label_smoothing", [(-100, 0.1), (3, 0.2)])
@pytest.mark.parametrize("reduction", ["mean", "sum", "none"])
def test_label_smoothing_with_ignore_index(ignore_index, label_smoothing, reduction):
    logits, target = _case(15, 97, torch.float32)
    target[::3] = ignore_index
    _check(logits, target, reduction=reduction, ignore_index=ignore_index, label_smoothing=label_smoothing)


@pytest.mark.gpu
@pytest.mark.parametrize("reduction", ["mean", "sum", "none"])
def test_not_last_layer_grad_output(reduction):
    logits, target = _case(12, 113, torch.float32)
    upstream = torch.rand(12) * 3.0 if reduction == "none" else torch.tensor(2.5)
    _check(logits, target, reduction=reduction, upstream=upstream)


@pytest.mark.gpu
@pytest.mark.parametrize("reduction", ["mean", "sum", "none"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_forward_only_no_grad(reduction, dtype):
    logits, target = _case(10, 64, dtype)
    ref_loss = ce_reference(logits, target, reduction=reduction)[0]
    with torch.no_grad():
        out = forge_cross_entropy(logits.cuda(), target.cuda(), reduction=reduction)
    torch.testing.assert_close(out.float().cpu(), ref_loss.float(), rtol=2e-3, atol=1e-5)
    assert not out.requires_grad
    with pytest.raises(RuntimeError, match="does not require grad"):
        out.backward(gradient=torch.ones_like(out))


@pytest.mark.gpu
@pytest.mark.parametrize("reduction", ["sum", "none"])
def test_all_ignored_rows_have_zero_gradient(reduction):
    logits, target = _case(8, 32, torch.float32)
    target.fill_(-100)
    x, out = _run(logits, target, reduction=reduction)
    out.backward(gradient=torch.ones_like(out))
    assert torch.count_nonzero(x.grad) == 0
    assert torch.count_nonzero(out) == 0


@pytest.mark.gpu
def test_all_ignored_mean_is_zero_not_nan():
    logits, target = _case(8, 32, torch.float32)
    target.fill_(-100)
    x, out = _run(logits, target, ignore_index=-100, reduction="mean")
    torch.testing.assert_close(out.cpu(), torch.zeros((), dtype=torch.float32))
    out.backward()
    assert torch.count_nonzero(x.grad) == 0


@pytest.mark.gpu
@pytest.mark.parametrize("bad_target", [-1, 128])
@pytest.mark.parametrize("vocab,dtype", [(128, torch.float32), (4096, torch.bfloat16)])
def test_out_of_bounds_target_raises(bad_target, vocab, dtype):
    """The reference asserts the masked target range before launching
    (cross_entropy_kernel_v2.py:382-387).  Here the kernel is queued before
    the host reads the range, so it must leave the logits untouched when the
    range check fails (both engines: fp32 -> streaming, bf16 -> resident)."""
    logits = torch.randn(8, vocab, device="cuda").to(dtype)
    before = logits.clone()
    target = torch.randint(0, vocab, (8,), device="cuda")
    target[2] = vocab if bad_target == 128 else bad_target
    x = logits.requires_grad_(True)
    with pytest.raises((AssertionError, IndexError), match="out of bounds"):
        forge_cross_entropy(x, target)
    torch.cuda.synchronize()
    assert torch.equal(logits.detach(), before)


@pytest.mark.gpu
def test_c_abi_skips_rows_with_out_of_range_targets():
    """Called directly (no stats), forge_ce_fwd leaves a row whose target is
    outside [0, V) untouched and processes the others."""
    BT, V = 4, 256
    x = torch.randn(BT, V, device="cuda")
    ref_x = x.clone()
    t = torch.tensor([3, V + 5, -7, 10], device="cuda")
    loss = torch.full((BT,), -1.0, device="cuda")
    rc = L.forge_ce_fwd(0, x.data_ptr(), V, BT, V, t.data_ptr(), 1, None, loss.data_ptr(), None, None, None, -100,
                        2.0, 2.0, 0.0, 0.0, 0.0, 0.0, L.CE_HAS_GRADIENTS, None, L.stream_of(x))
    assert rc == 0
    torch.cuda.synchronize()
    assert torch.equal(x[1], ref_x[1]) and torch.equal(x[2], ref_x[2])
    assert loss[1].item() == -1.0 and loss[2].item() == -1.0
    _, _, rows, _, _, g = ce_reference(ref_x[[0, 3]].cpu(), t[[0, 3]].cpu(), reduction="none")
    torch.testing.assert_close(loss[[0, 3]].cpu(), rows, rtol=1e-5, atol=1e-6)
    torch.testing.assert_close(x[[0, 3]].cpu(), g, rtol=1e-5, atol=1e-6)


def _reduce_call(x, t, flags, loss1d, loss_sum, z1d=None, z_sum=None, cast=None, z_cast=None, ignore=-100):
    """forge_ce_fwd_reduce through the C-ABI, then forge_ce_stats_wait;
    returns the host statistics [n_valid, min, max, in_range]."""
    BT, V = x.shape
    ticket = ctypes.c_uint64()
    st = L.stream_of(x)
    L.check(L.forge_ce_fwd_reduce(L.dtype_code(x.dtype), x.data_ptr(), x.stride(0), BT, V, t.data_ptr(), 1,
                                  loss1d.data_ptr(), L.ptr(z1d), None, None, ignore, 1e-4 if z1d is not None else 0.0,
                                  0.0, 0.0, flags, L.ptr(loss_sum), L.ptr(z_sum), L.ptr(cast), L.ptr(z_cast),
                                  L.dtype_code(cast.dtype) if cast is not None else L.DTYPE_F32,
                                  ctypes.byref(ticket), st), "forge_ce_fwd_reduce")
    stats = (ctypes.c_int64 * 4)()
    L.check(L.forge_ce_stats_wait(ticket.value, stats, st), "forge_ce_stats_wait")
    return list(stats)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype,vocab", [(torch.bfloat16, 4096), (torch.float32, 300)])
def test_fwd_reduce_sum_statistics_and_slot_reuse(dtype, vocab):
    """forge_ce_fwd_reduce (one launch: statistics, rows, dlogits, reduced
    loss).  The host statistics are the targets' count and masked range; the
    reduced loss is the fixed-order fp32 sum of the per-row losses the launch
    also writes (checked against a float64 sum of them, and against the
    oracle), and it is bit-identical over 70 calls: more than the library's 64
    call slots, so every slot is reused and its done count must have been
    reset by the previous launch on it.  bf16 [*, 4096] runs the resident
    engine, fp32 the streaming one."""
    BT = 301
    logits, target = _case(BT, vocab, dtype, scalar=2.0, seed=7)
    target[::9] = -100
    n_valid = int((target != -100).sum())
    masked = torch.where(target != -100, target, torch.zeros_like(target))
    ref_loss, ref_z, ref_rows, _, _, ref_grad = ce_reference(logits, target, reduction="mean", lse_square_scale=1e-4)
    t = target.cuda()
    flags = L.CE_HAS_GRADIENTS | L.CE_REDUCTION_MEAN | L.CE_RETURN_Z_LOSS
    sums = set()
    for i in range(70):
        x = logits.cuda()
        loss1d = torch.empty(BT, device="cuda")
        z1d = torch.empty(BT, device="cuda")
        s, zs = torch.empty((), device="cuda"), torch.empty((), device="cuda")
        cast = torch.empty((), dtype=torch.bfloat16, device="cuda")
        stats = _reduce_call(x, t, flags, loss1d, s, z1d, zs, cast)
        assert stats == [n_valid, int(masked.min()), int(masked.max()), 1]
        torch.cuda.synchronize()
        sums.add((s.item(), zs.item(), cast.float().item()))
        if i == 0:
            torch.testing.assert_close(s.double().cpu(), loss1d.double().sum().cpu(), rtol=1e-6, atol=0)
            torch.testing.assert_close(zs.double().cpu(), z1d.double().sum().cpu(), rtol=1e-6, atol=0)
            assert cast.item() == s.to(torch.bfloat16).item()
            torch.testing.assert_close(loss1d.cpu(), ref_rows.float(), rtol=1e-4, atol=1e-6)
            torch.testing.assert_close(s.cpu(), ref_loss.float(), rtol=1e-4, atol=0)
            torch.testing.assert_close(x.float().cpu(), ref_grad.float(), rtol=GTOL[dtype], atol=GTOL[dtype])
    assert len(sums) == 1


@pytest.mark.gpu
@pytest.mark.parametrize("dtype,vocab", [(torch.bfloat16, 4096), (torch.float32, 300)])
def test_fwd_reduce_out_of_range_touches_nothing_and_next_call_is_clean(dtype, vocab):
    """A target out of range: the launch reports in_range = 0 and a masked
    min / max that names it, leaves the logits untouched, writes its sum as 0,
    and still resets
    its slot: the following calls (all 64 slots, then this one's again) give
    the correct loss."""
    BT = 64
    logits, target = _case(BT, vocab, dtype, seed=3)
    bad = target.clone()
    bad[5] = vocab + 3
    x = logits.cuda()
    loss1d, s = torch.empty(BT, device="cuda"), torch.empty((), device="cuda")
    stats = _reduce_call(x, bad.cuda(), L.CE_HAS_GRADIENTS | L.CE_REDUCTION_MEAN, loss1d, s)
    assert stats[0] == BT and stats[2] == vocab + 3 and stats[3] == 0
    torch.cuda.synchronize()
    assert torch.equal(x.cpu(), logits)
    assert s.item() == 0.0  # the sum of a refused launch is written as 0
    ref_loss = ce_reference(logits, target, reduction="sum")[0]
    for _ in range(65):
        x = logits.cuda()
        stats = _reduce_call(x, target.cuda(), 0, loss1d, s)
        assert stats[3] == 1
        torch.testing.assert_close(s.cpu(), ref_loss.float(), rtol=1e-4, atol=0)


@pytest.mark.gpu
def test_fwd_reduce_concurrent_streams():
    """Calls on two streams at once use different call slots: both sums are
    right."""
    BT, V = 2048, 4096
    la, ta = _case(BT, V, torch.bfloat16, seed=11)
    lb, tb = _case(BT, V, torch.bfloat16, seed=12)
    ra = ce_reference(la, ta, reduction="sum")[0]
    rb = ce_reference(lb, tb, reduction="sum")[0]
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    xa, xb, tga, tgb = la.cuda(), lb.cuda(), ta.cuda(), tb.cuda()
    out = []
    torch.cuda.synchronize()
    for _ in range(4):
        res = []
        for x, t, s in ((xa.clone(), tga, s1), (xb.clone(), tgb, s2)):
            with torch.cuda.stream(s):
                l1, sm = torch.empty(BT, device="cuda"), torch.empty((), device="cuda")
                ticket = ctypes.c_uint64()
                L.check(L.forge_ce_fwd_reduce(2, x.data_ptr(), V, BT, V, t.data_ptr(), 1, l1.data_ptr(), None, None,
                                              None, -100, 0.0, 0.0, 0.0, 0, sm.data_ptr(), None, None, None,
                                              L.DTYPE_F32, ctypes.byref(ticket), L.stream_of(x)), "reduce")
                res.append((ticket.value, sm, s))
        for ticket, sm, s in res:
            st = (ctypes.c_int64 * 4)()
            L.check(L.forge_ce_stats_wait(ticket, st, s.cuda_stream), "wait")
        torch.cuda.synchronize()
        out.append((res[0][1].cpu(), res[1][1].cpu()))
    for a, b in out:
        torch.testing.assert_close(a, ra.float(), rtol=1e-4, atol=0)
        torch.testing.assert_close(b, rb.float(), rtol=1e-4, atol=0)


@pytest.mark.gpu
@pytest.mark.parametrize("reduction", ["mean", "sum", "none"])
def test_class_weights(reduction):
    logits, target = _case(8, 73, torch.float32)
    weight = torch.rand(73, generator=torch.Generator().manual_seed(4))
    _check(logits, target, reduction=reduction, weight=weight.cuda())


@pytest.mark.gpu
@pytest.mark.parametrize("reduction", ["mean", "sum", "none"])
@pytest.mark.parametrize("return_z_loss", [False, True])
def test_z_loss(reduction, return_z_loss):
    logits, target = _case(10, 67, torch.float32)
    out = _check(logits, target, reduction=reduction, lse_square_scale=1e-4, return_z_loss=return_z_loss)
    if return_z_loss:
        ref_z = ce_reference(logits, target, reduction=reduction, lse_square_scale=1e-4)[1]
        torch.testing.assert_close(out.z_loss.cpu(), ref_z, rtol=1e-5, atol=1e-5)


@pytest.mark.gpu
@pytest.mark.parametrize("reduction", ["mean", "sum", "none"])
@pytest.mark.parametrize("softcap", [30.0, 40.0])
def test_softcap(reduction, softcap):
    logits, target = _case(10, 67, torch.float32, scalar=3.0)
    _check(logits, target, reduction=reduction, softcap=softcap)


@pytest.mark.gpu
def test_weight_with_label_smoothing_and_ignore_index():
    logits, target = _case(10, 83, torch.float32)
    target[::3] = -100
    weight = torch.rand(83, generator=torch.Generator().manual_seed(9))
    _check(logits, target, weight=weight.cuda(), ignore_index=-100, label_smoothing=0.1)


@pytest.mark.gpu
@pytest.mark.parametrize("return_z_loss", [False, True])
def test_token_accuracy_and_predicted_tokens(return_z_loss):
    logits, target = _case(13, 41, torch.float32)
    target[::4] = -100
    _, _, _, ref_acc, ref_pred, _ = ce_reference(logits, target, lse_square_scale=1e-4)
    out = forge_cross_entropy(logits.cuda().requires_grad_(True), target.cuda(), ignore_index=-100,
                              lse_square_scale=1e-4, return_z_loss=return_z_loss,
                              return_token_accuracy=True, return_predicted_tokens=True)
    assert isinstance(out, CrossEntropyOutput)
    assert torch.equal(out.predicted_tokens.cpu(), ref_pred)
    assert out.token_accuracy.item() == ref_acc.item()


@pytest.mark.gpu
def test_argmax_ties_take_first_index():
    logits = torch.zeros(4, 300)
    logits[:, 7] = 5.0
    logits[:, 250] = 5.0
    target = torch.tensor([7, 250, 1, -100])
    out = forge_cross_entropy(logits.cuda(), target.cuda(), return_predicted_tokens=True,
                              return_token_accuracy=True)
    assert out.predicted_tokens.cpu().tolist() == [7, 7, 7, -1]
    assert out.token_accuracy.item() == pytest.approx(1.0 / 3.0)


@pytest.mark.gpu
def test_strided_rows_and_inplace_contract():
    """Row stride > V (a column slice of a wider buffer) and the in-place
    dlogits contract: the returned gradient is the caller's logits storage."""
    buf = torch.randn(16, 160, generator=torch.Generator().manual_seed(2)).cuda()
    logits = buf[:, :128].requires_grad_(False)
    target = torch.randint(0, 128, (16,), generator=torch.Generator().manual_seed(3)).cuda()
    x = logits.detach().requires_grad_(True)
    ref_loss, _, _, _, _, ref_grad = ce_reference(logits.cpu(), target.cpu())
    loss = forge_cross_entropy(x, target)
    torch.testing.assert_close(loss.cpu(), ref_loss, rtol=1e-5, atol=1e-6)
    loss.backward()
    torch.testing.assert_close(x.grad.cpu(), ref_grad, rtol=1e-5, atol=1e-6)
    # dlogits were written over the caller's logits; the padding columns are untouched
    assert torch.equal(buf[:, :128], x.grad)
    assert torch.equal(buf[:, 128:].cpu(), torch.randn(16, 160, generator=torch.Generator().manual_seed(2))[:, 128:])


@pytest.mark.gpu
def test_baseline_config_bf16():
    """BASELINE configs[2] at its own size: bf16 [8192, 128256] ~ N(0, 2^2),
    exactly 5% (410) rows ignored, mean over the non-ignored rows (the
    benchmarked call).  The oracle runs over every row in 512-row chunks with
    reduction='sum'; the full mean is the sum of the chunk sums over the
    global n_valid, and the mean's dlogits are the sum-gradients / n_valid, so
    both the loss and every dlogits row are checked against the oracle.  The
    loss is compared in fp32 (1e-3 relative); the returned bf16 scalar must be
    that value rounded once (a bf16 ulp at ~13.8 is 4.5e-3 relative).
    Ignored rows must be exactly zero and predictions are not requested."""
    BT, V = 8192, 128256
    gen = torch.Generator().manual_seed(2024)
    logits = (torch.randn(BT, V, generator=gen) * 2.0).to(torch.bfloat16)
    target = torch.randint(0, V, (BT,), generator=gen)
    ign = torch.randperm(BT, generator=gen)[:410]
    target[ign] = -100
    n_valid = BT - 410

    x = logits.cuda().requires_grad_(True)
    tg = target.cuda()
    loss = forge_cross_entropy(x, tg)  # reduction="mean"
    loss.backward()
    g = x.grad  # the dlogits, written over the caller's logits
    assert g.data_ptr() == x.data_ptr()
    assert torch.count_nonzero(g[ign.cuda()]) == 0

    ref_sum = torch.zeros((), dtype=torch.float64)
    chunk = 512
    for r0 in range(0, BT, chunk):
        rl, _, _, _, _, rg = ce_reference(logits[r0:r0 + chunk], target[r0:r0 + chunk], reduction="sum")
        ref_sum += rl.double()
        # mean's dlogits * n_valid == the sum's dlogits (grad_output = 1)
        got = g[r0:r0 + chunk].float().cpu() * n_valid
        torch.testing.assert_close(got, rg, rtol=2e-2, atol=2e-2,
                                   msg=lambda m, r0=r0: f"dlogits rows {r0}..: {m}")
    ref_mean = (ref_sum / n_valid).float()
    # the loss in fp32 (before the rounding to the logits dtype) within 1e-3
    # of the oracle, and the returned bf16 loss is that value rounded once
    with torch.no_grad():
        loss32, _, _, _, _ = _cross_entropy_forward_impl(logits.cuda(), tg, None, -100, 0.0, 0.0, "mean", None,
                                                         False)
    torch.testing.assert_close(loss32.cpu(), ref_mean, rtol=1e-3, atol=0)
    assert loss.dtype == torch.bfloat16
    assert loss.float().item() == loss32.to(torch.bfloat16).float().item()


# Resident-row engine (2-byte logits, 16-byte aligned rows, no weight /
# softcap / accuracy / predictions): a row is held on chip as up to 8 vectors
# per thread in LDS plus NR in registers (NR buckets 8 / 16 / 24, 512
# threads, 8 values a vector), so V <= 32 * 512 * 8 = 131072.  These vocab
# sizes hit each bucket and its edges, the exact maximum, and the first size
# past it (streaming engine); the target sits in the first and last columns
# of some rows.
RESIDENT_V = [4096, 32768, 50000, 65536, 65544, 98304, 128256, 131072, 131080]


@pytest.mark.gpu
@pytest.mark.parametrize("vocab", RESIDENT_V)
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_resident_engine_buckets(vocab, dtype):
    logits, target = _case(6, vocab, dtype, scalar=2.0, seed=vocab)
    target[0], target[1], target[2] = 0, vocab - 1, -100
    _check(logits, target, reduction="sum", ignore_index=-100)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_resident_engine_negative_rows_and_features(dtype):
    """Rows whose every logit is negative take the float max pass (the packed
    int16 max only orders non-negative values); label smoothing and z-loss
    run in the resident engine too; a dominant logit leaves most p tiny."""
    logits, target = _case(5, 50000, dtype, seed=7)
    logits[0] = -logits[0].abs() - 1.0
    logits[1] = -torch.rand(50000) * 0.01 - 30.0
    logits[2, 123] = 60.0
    target[2] = 123
    _check(logits, target, reduction="mean", label_smoothing=0.1, lse_square_scale=1e-4, return_z_loss=True)


@pytest.mark.gpu
def test_resident_engine_fp16_gradients_are_unbiased():
    """fp16 logits on the resident engine: p is held as fp16 between passes
    and rounded to nearest, so each dlogit is within two fp16 roundings of
    the fp32 oracle (|rel| <= 2^-10 for normal values) and the signed error
    averages to ~0.  Round-toward-zero storage would bias every value low by
    ~2^-12 on average, far outside the mean bound."""
    logits, target = _case(64, 32768, torch.float16, scalar=3.0, seed=41)
    _, _, _, _, _, ref_grad = ce_reference(logits, target, reduction="sum")
    x, loss = _run(logits, target, reduction="sum")
    loss.backward()
    got = x.grad.float().cpu()
    sel = ref_grad.abs() >= 2.0 ** -13  # fp16 normal range after the final rounding
    rel = (got[sel] - ref_grad[sel]) / ref_grad[sel].abs()
    assert sel.sum().item() > 20_000
    assert rel.abs().max().item() <= 2.0 ** -10 * 1.01
    assert abs(rel.mean().item()) < 3e-5
