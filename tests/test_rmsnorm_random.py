"""Seeded random sweep of the RMSNorm drop-in (v4 forward and backward, both
in-place modes) against the CPU oracle: random row counts and widths (both
engines, odd widths and scalar tails), bf16 / fp16 / fp32 inputs, fp32
weights with 2-byte inputs, every casting mode, offsets and eps."""
import random

import pytest
import torch

from oracle import rmsnorm as orms

TOL = {torch.bfloat16: (5e-2, 5e-2), torch.float16: (2e-2, 2e-2), torch.float32: (1e-4, 1e-5)}
MODES = {"llama": orms.LLAMA, "gemma": orms.GEMMA, "none": orms.NONE}


def _passes(a, ref, dtype, scale=1.0):
    atol, rtol = TOL[dtype]
    diff = (a.double().cpu() - ref.double().cpu()).abs().max().item()
    return diff <= atol + rtol * scale * ref.double().abs().max().item(), diff


@pytest.mark.gpu
@pytest.mark.parametrize("seed", [8, 19])
def test_rmsnorm_random_sweep(seed):
    from kernels.rmsnorm import apply_rmsnorm_v4

    rng = random.Random(seed)
    g = torch.Generator(device="cuda").manual_seed(seed)
    for i in range(30):
        rows = rng.choice([1, rng.randint(1, 64), rng.randint(1, 3000)])
        h = rng.choice([1, 7, 64, 896, 2048, 4096, 4097, 8192, rng.randint(1, 12000)])
        dtype = rng.choice([torch.bfloat16, torch.float16, torch.float32])
        wdtype = torch.float32 if dtype != torch.float32 and rng.random() < 0.25 else dtype
        mode = rng.choice(["llama", "gemma", "none"])
        offset = rng.choice([0.0, 1.0])
        eps = rng.choice([1e-6, 1e-5])
        in_place = rng.random() < 0.5
        desc = f"case {i}: rows={rows} h={h} {dtype} weight={wdtype} mode={mode} offset={offset} eps={eps} in_place={in_place}"
        x0 = torch.randn(rows, h, device="cuda", generator=g).to(dtype)
        w0 = (torch.ones(h, device="cuda") * (1.0 - offset) + 0.1 * torch.randn(h, device="cuda", generator=g)).to(wdtype)
        dy = torch.randn(rows, h, device="cuda", generator=g).to(dtype)
        ref_y, _ = orms.rms_forward(x0, w0, eps, offset, MODES[mode])
        rdx, rdw = orms.rms_backward(dy, x0, w0, offset, eps)
        x = x0.clone().requires_grad_(True)
        w = w0.clone().requires_grad_(True)
        y = apply_rmsnorm_v4(x, w, eps, offset, mode, in_place=in_place)
        ok, diff = _passes(y, ref_y, dtype)
        assert ok, f"{desc}: y {diff}"
        y.backward(dy.clone())
        ok, diff = _passes(x.grad, rdx, dtype)
        assert ok, f"{desc}: dx {diff}"
        # dw sums over every row: a looser relative bound for 2-byte inputs
        ok, diff = _passes(w.grad, rdw, dtype, 1.0 if dtype == torch.float32 else 2.0)
        assert ok, f"{desc}: dw {diff}"
