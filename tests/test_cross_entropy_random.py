"""Seeded random sweep of forge_cross_entropy (the v2 drop-in) against the CPU
oracle: random row counts and vocabulary sizes (both row engines, their
bucket edges and ragged tails), fp32 / bf16 / fp16 logits, ignored rows
(none, some, all; ignore_index -100 or a class id), class weights, label
smoothing, z-loss, softcap, every reduction, and upstream gradients other
than 1."""
import random

import pytest
import torch

from kernels.cross_entropy.experiments.v2 import CrossEntropyOutput, forge_cross_entropy
from oracle.cross_entropy import ce_reference

GTOL = {torch.float32: 1e-5, torch.float16: 2e-2, torch.bfloat16: 2e-2}
LTOL = {torch.float32: 1e-5, torch.float16: 1e-3, torch.bfloat16: 1e-3}
VOCABS = [1, 2, 7, 64, 127, 513, 1000, 4095, 4096, 4097, 8192, 12289, 32000]


def _case(rng: random.Random, gen: torch.Generator):
    V = rng.choice(VOCABS + [rng.randint(2, 20000)])
    bt = rng.randint(1, max(1, min(300, 2_000_000 // V)))
    dtype = rng.choice([torch.float32, torch.bfloat16, torch.float16])
    scale = rng.choice([1.0, 4.0])
    shift = rng.choice([0.0, 0.0, -20.0])  # all-negative rows take the kernels' float max pass
    logits = (torch.randn(bt, V, generator=gen) * scale + shift).to(dtype)
    target = torch.randint(0, V, (bt,), generator=gen)
    ignore_index = rng.choice([-100, -100, min(3, V - 1)])
    frac = rng.choice([0.0, 0.1, 0.5, 1.0])
    if frac > 0:
        mask = torch.rand(bt, generator=gen) < frac
        target[mask] = ignore_index
    kw = dict(ignore_index=ignore_index, reduction=rng.choice(["mean", "sum", "none"]))
    if rng.random() < 0.3:
        kw["label_smoothing"] = 0.1
    if rng.random() < 0.3:
        kw["lse_square_scale"] = 1e-4
    if rng.random() < 0.25:
        kw["softcap"] = 30.0
    weight = torch.rand(V, generator=gen) + 0.1 if rng.random() < 0.25 else None
    upstream = None
    if rng.random() < 0.3:
        upstream = (torch.rand(bt, generator=gen) + 0.5) if kw["reduction"] == "none" else torch.tensor(0.75)
    return logits, target, weight, kw, upstream


def _check_one(logits, target, weight, kw, upstream):
    dtype = logits.dtype
    ref_loss, _, _, _, _, ref_grad = ce_reference(logits, target, weight=weight, **kw)
    x = logits.cuda().requires_grad_(True)
    out = forge_cross_entropy(x, target.cuda(), weight=None if weight is None else weight.cuda(), **kw)
    loss = out.loss if isinstance(out, CrossEntropyOutput) else out
    assert loss.dtype == dtype
    t = LTOL[dtype]
    torch.testing.assert_close(loss.float().cpu(), ref_loss.float(), rtol=max(t, 4e-3) if dtype != torch.float32 else t,
                               atol=t)
    if upstream is None:
        loss.backward(torch.ones_like(loss))
    else:
        loss.backward(upstream.to(dtype).cuda())
        g = upstream.to(dtype).float()
        ref_grad = ref_grad * (g.unsqueeze(1) if g.dim() > 0 else g)
    gt = GTOL[dtype]
    torch.testing.assert_close(x.grad.float().cpu(), ref_grad.float(), rtol=gt, atol=gt)


@pytest.mark.gpu
@pytest.mark.parametrize("seed", [3, 17])
def test_cross_entropy_random_sweep(seed):
    rng = random.Random(seed)
    gen = torch.Generator().manual_seed(seed)
    for i in range(40):
        logits, target, weight, kw, upstream = _case(rng, gen)
        desc = (f"case {i}: shape {tuple(logits.shape)} {logits.dtype} weight={weight is not None} "
                f"upstream={None if upstream is None else tuple(upstream.shape)} {kw}")
        try:
            _check_one(logits, target, weight, kw, upstream)
        except AssertionError as e:
            raise AssertionError(f"{desc}\n{e}") from None
