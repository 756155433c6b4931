"""Seeded random sweep of the fused linear + cross-entropy drop-in against the
float64 oracle: random token counts, hidden sizes (multiples of 8 on the MFMA
path, others on the generic GEMM) and vocabulary sizes, fp32 / bf16, bias,
ignored rows, class weights, label smoothing, z-loss, softcap, token scaling,
both reductions, and logits chunks small enough to split the batch."""
import random

import pytest
import torch

from oracle import fused_linear_ce as oflce

pytestmark = pytest.mark.gpu


def _tol(dtype):
    return (5e-2, 2e-2) if dtype == torch.bfloat16 else (1e-5, 1e-5)


@pytest.mark.parametrize("seed", [6, 27])
def test_fused_linear_ce_random_sweep(seed, monkeypatch):
    from kernels.cross_entropy.experiments.v2 import CrossEntropyOutput, forge_fused_linear_cross_entropy
    from kernels.cross_entropy.experiments.v2 import fused_linear_cross_entropy as flce_mod

    rng = random.Random(seed)
    gen = torch.Generator().manual_seed(seed)
    default_chunk = flce_mod._LOGITS_CHUNK_BYTES
    for i in range(16):
        bt = rng.choice([1, rng.randint(1, 64), rng.randint(1, 600)])
        h = rng.choice([8, 32, 64, 100, 256, rng.randint(1, 300)])
        v = rng.choice([2, 73, 257, 1000, rng.randint(2, 2000)])
        dtype = rng.choice([torch.float32, torch.bfloat16])
        bias = rng.random() < 0.5
        kw = {"reduction": rng.choice(["mean", "sum"])}
        if rng.random() < 0.3:
            kw["label_smoothing"] = 0.1
        if rng.random() < 0.3:
            kw["lse_square_scale"] = 1e-3
        if rng.random() < 0.25:
            kw["softcap"] = 5.0
        if rng.random() < 0.25 and kw["reduction"] == "mean":
            kw["use_token_scaling"] = True
        weight = torch.rand(v, generator=gen) + 0.1 if rng.random() < 0.2 and "use_token_scaling" not in kw else None
        chunked = rng.random() < 0.4
        x = torch.randn(bt, h, generator=gen)
        W = torch.randn(v, h, generator=gen) / h ** 0.5
        b = torch.randn(v, generator=gen) if bias else None
        t = torch.randint(0, v, (bt,), generator=gen)
        t[torch.rand(bt, generator=gen) < rng.choice([0.0, 0.2])] = -100
        desc = f"case {i}: bt={bt} h={h} v={v} {dtype} bias={bias} weight={weight is not None} chunked={chunked} {kw}"
        xd = x.to("cuda", dtype).requires_grad_(True)
        Wd = W.to("cuda", dtype).requires_grad_(True)
        bd = b.to("cuda", dtype).requires_grad_(True) if bias else None
        ref = oflce.fused_linear_ce(xd.detach().float(), Wd.detach().float(), t,
                                    bias=None if b is None else bd.detach().float(),
                                    ce_weight=None if weight is None else weight.double(), **kw)
        monkeypatch.setattr(flce_mod, "_LOGITS_CHUNK_BYTES",
                            max(1, rng.randint(1, 64)) * v * xd.element_size() if chunked else default_chunk)
        out = forge_fused_linear_cross_entropy(xd, Wd, t.cuda(), bias=bd,
                                               ce_weight=None if weight is None else weight.cuda(), **kw)
        loss = out.loss if isinstance(out, CrossEntropyOutput) else out
        rtol, atol = _tol(dtype)
        try:
            torch.testing.assert_close(loss.float().cpu().double(), ref["loss"], rtol=rtol, atol=atol)
            loss.backward()
            torch.testing.assert_close(xd.grad.float().cpu(), ref["dX"].float(), rtol=rtol, atol=atol)
            torch.testing.assert_close(Wd.grad.float().cpu(), ref["dW"].float(), rtol=rtol, atol=atol)
            if bias:
                torch.testing.assert_close(bd.grad.float().cpu(), ref["db"].float(), rtol=rtol, atol=atol)
        except AssertionError as e:
            raise AssertionError(f"{desc}\n{e}") from None
