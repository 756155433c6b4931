"""Seeded random sweep of the SwiGLU and GeGLU drop-ins (separate and packed
gate/up, forward and the in-place backward) against the CPU oracles: random
leading shapes and row widths (odd widths and scalar tails included), fp32 /
bf16 / fp16, SwiGLU gate/down multipliers, tanh and exact GELU, and both
preserve_inputs modes."""
import random

import pytest
import torch

from kernels.geglu import geglu, geglu_packed
from kernels.swiglu import swiglu, swiglu_packed
from oracle.geglu import geglu_fwd_bwd
from oracle.swiglu import swiglu_fwd_bwd, swiglu_packed_fwd_bwd

TOL = {torch.float32: 1e-5, torch.float16: 2e-2, torch.bfloat16: 2e-2}


def _close(a, b, dtype, what):
    t = TOL[dtype]
    torch.testing.assert_close(a.float().cpu(), b.float().cpu(), atol=t, rtol=t, msg=lambda m: f"{what}: {m}")


def _one(rng: random.Random, gen: torch.Generator):
    kind = rng.choice(["swiglu", "geglu"])
    packed = rng.random() < 0.4
    dtype = rng.choice([torch.float32, torch.bfloat16, torch.float16])
    if kind == "geglu" and packed and dtype == torch.float16:
        dtype = torch.bfloat16
    lead = [rng.randint(1, 6) for _ in range(rng.choice([1, 2]))]
    h = rng.choice([1, 7, 8, 63, 64, 257, rng.randint(1, 3000)])
    preserve = rng.random() < 0.5
    desc = f"{kind} packed={packed} {dtype} lead={lead} h={h} preserve={preserve}"
    dout = torch.randn(*lead, h, generator=gen).to(dtype)
    if kind == "swiglu":
        gm, dm = rng.choice([(1.0, 1.0), (0.7, 1.3)])
        desc += f" gm={gm} dm={dm}"
        if packed:
            gu_host = torch.randn(*lead, 2 * h, generator=gen).to(dtype)
            ref_out, ref_grad = swiglu_packed_fwd_bwd(gu_host, dout, gm, dm)
            gu = gu_host.cuda().requires_grad_(True)
            out = swiglu_packed(gu, gm, dm, preserve)
            out.backward(dout.cuda())
            return [(out, ref_out, "out"), (gu.grad, ref_grad, "d gate_up")], dtype, desc
        gate, up = torch.randn(*lead, h, generator=gen).to(dtype), torch.randn(*lead, h, generator=gen).to(dtype)
        ref_out, ref_dg, ref_du = swiglu_fwd_bwd(gate, up, dout, gm, dm)
        g, u = gate.cuda().requires_grad_(True), up.cuda().requires_grad_(True)
        out = swiglu(g, u, gm, dm, preserve)
        out.backward(dout.cuda())
        return [(out, ref_out, "out"), (g.grad, ref_dg, "d gate"), (u.grad, ref_du, "d up")], dtype, desc
    approximate = rng.choice(["tanh", "none"])
    desc += f" approximate={approximate}"
    gate = (torch.randn(*lead, h, generator=gen) * 2).to(dtype)
    up = torch.randn(*lead, h, generator=gen).to(dtype)
    ref_out, ref_dg, ref_du = geglu_fwd_bwd(gate, up, dout, approximate)
    if packed:
        gu = torch.cat([gate, up], -1).cuda().requires_grad_(True)
        out = geglu_packed(gu, approximate, preserve)
        out.backward(dout.cuda())
        return [(out, ref_out, "out"), (gu.grad[..., :h], ref_dg, "d gate"), (gu.grad[..., h:], ref_du, "d up")], \
            dtype, desc
    g, u = gate.cuda().requires_grad_(True), up.cuda().requires_grad_(True)
    out = geglu(g, u, approximate, preserve)
    out.backward(dout.cuda())
    return [(out, ref_out, "out"), (g.grad, ref_dg, "d gate"), (u.grad, ref_du, "d up")], dtype, desc


@pytest.mark.gpu
@pytest.mark.parametrize("seed", [2, 31])
def test_glu_random_sweep(seed):
    rng = random.Random(seed)
    gen = torch.Generator().manual_seed(seed)
    for i in range(40):
        pairs, dtype, desc = _one(rng, gen)
        try:
            for got, want, what in pairs:
                _close(got, want, dtype, what)
        except AssertionError as e:
            raise AssertionError(f"case {i}: {desc}\n{e}") from None
