"""Cross-entropy v1 API (kernels/cross_entropy/experiments/v1) against the
CPU oracle, following kernels/cross_entropy/tests/test_cross_entropy.py's
v1 cases: reductions, label smoothing, ignore_index, dtypes, the all-ignored
mean (NaN loss, zero gradients: v1's own semantics), host-side target
validation (IndexError), the F.cross_entropy compatibility path, and the
backward's grad_output handling.  Tolerances as for v2: fp32 1e-5, bf16 /
fp16 2e-2 on dlogits, loss 1e-3 relative (v1 rounds each row loss to the
logits dtype before summing)."""
import pytest
import torch
import torch.nn.functional as F

from kernels.cross_entropy.experiments.v1 import forge_cross_entropy
from kernels.cross_entropy.experiments.v1.cross_entropy_kernel_v1 import ForgeCrossEntropyFunction
from oracle.cross_entropy import ce_reference

GTOL = {torch.float32: 1e-5, torch.float16: 2e-2, torch.bfloat16: 2e-2}


def _case(bt, vocab, dtype, seed=0, scalar=2.0):
    g = torch.Generator().manual_seed(seed)
    logits = (torch.randn(bt, vocab, generator=g) * scalar).to(dtype)
    target = torch.randint(0, vocab, (bt,), generator=g)
    return logits, target


def test_v1_argument_errors_and_cpu_path():
    logits, target = _case(4, 32, torch.float32)
    with pytest.raises(ValueError, match="reduction must be one of"):
        forge_cross_entropy(logits, target, reduction="avg")
    with pytest.raises(ValueError, match="label_smoothing must be between 0.0 and 1.0"):
        forge_cross_entropy(logits, target, label_smoothing=1.5)
    # CPU tensors take the F.cross_entropy compatibility path
    x = logits.clone().requires_grad_(True)
    torch.testing.assert_close(forge_cross_entropy(x, target, label_smoothing=0.1),
                               F.cross_entropy(logits, target, label_smoothing=0.1))


@pytest.mark.gpu
@pytest.mark.parametrize("reduction", ["mean", "sum", "none"])
@pytest.mark.parametrize("label_smoothing", [0.0, 0.1])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_v1_matches_oracle(reduction, label_smoothing, dtype):
    logits, target = _case(37, 4099, dtype, seed=len(reduction) * 10 + int(label_smoothing * 10))
    target[::5] = -100
    ref_loss, _, ref_rows, _, _, ref_grad = ce_reference(logits, target, reduction=reduction,
                                                         label_smoothing=label_smoothing)
    x = logits.cuda().requires_grad_(True)
    loss = forge_cross_entropy(x, target.cuda(), reduction=reduction, label_smoothing=label_smoothing)
    assert loss.dtype == dtype
    t = 1e-5 if dtype == torch.float32 else 1e-3
    torch.testing.assert_close(loss.float().cpu(), ref_loss.float(), rtol=max(t, 4e-3 if dtype != torch.float32 else t),
                               atol=t)
    up = torch.randn(37) if reduction == "none" else None
    if up is None:
        loss.backward()
    else:
        loss.backward(up.to(dtype).cuda())
        ref_grad = ref_grad * up.to(dtype).float().unsqueeze(1)
    torch.testing.assert_close(x.grad.float().cpu(), ref_grad.float(), rtol=GTOL[dtype], atol=GTOL[dtype])
    assert torch.count_nonzero(x.grad[::5]) == 0


@pytest.mark.gpu
def test_v1_all_ignored_mean_is_nan_with_zero_gradients():
    """v1 returns torch.sum(loss_1d) / 0 = NaN for a mean over no targets
    (cross_entropy_kernel_v1.py:309-315); v2 returns 0."""
    logits, target = _case(8, 512, torch.bfloat16)
    target[:] = -100
    x = logits.cuda().requires_grad_(True)
    loss = forge_cross_entropy(x, target.cuda())
    assert torch.isnan(loss).item()
    loss.backward()
    assert torch.count_nonzero(x.grad) == 0
    assert forge_cross_entropy(logits.cuda(), target.cuda(), reduction="sum").item() == 0.0


@pytest.mark.gpu
def test_v1_target_validation_and_weight_path():
    logits, target = _case(6, 100, torch.float32)
    target[2] = 100
    with pytest.raises(IndexError, match="Target 100 is out of bounds. Expected < 100"):
        forge_cross_entropy(logits.cuda(), target.cuda())
    target[2] = -3
    with pytest.raises(IndexError, match="Target -3 is out of bounds. Expected >= 0"):
        forge_cross_entropy(logits.cuda(), target.cuda())
    target[2] = 7
    w = torch.rand(100)
    got = forge_cross_entropy(logits.cuda(), target.cuda(), weight=w.cuda())  # F.cross_entropy path
    torch.testing.assert_close(got.cpu(), F.cross_entropy(logits, target, weight=w), rtol=1e-5, atol=1e-6)


@pytest.mark.gpu
def test_v1_inplace_contract_and_scalar_grad_output():
    """dlogits are written over the logits (the saved buffer is the caller's
    storage); a scalar grad_output != 1 scales them in place."""
    logits, target = _case(16, 1000, torch.float32, seed=4)
    x = logits.cuda().requires_grad_(True)
    loss = ForgeCrossEntropyFunction.apply(x, target.cuda(), -100, "sum", 0.0)
    (saved,) = loss.grad_fn.saved_tensors
    assert saved.data_ptr() == x.data_ptr()
    loss.backward(torch.tensor(0.5, device="cuda"))
    _, _, _, _, _, ref_grad = ce_reference(logits, target, reduction="sum")
    torch.testing.assert_close(x.grad.cpu(), ref_grad * 0.5, rtol=1e-5, atol=1e-6)
    # the scaling ran in place on the caller's logits storage (autograd may
    # hand the leaf a copy of that buffer as .grad)
    assert torch.equal(x.detach(), x.grad)
