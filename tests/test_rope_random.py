"""Seeded random sweep of the v3 RoPE drop-in (`apply_rope`, forward and
backward) against the float32 HF formula on the CPU: random batch, GQA
ratios (including MQA and non-power-of-two ratios), sequence lengths,
head_dim 16..256, bf16 / fp16 / fp32, [B, H, S, D] tensors or transposed
[B, S, H, D] views, per-batch tables, fp32 tables with 2-byte q / k, and
varlen positions into a longer table."""
import random

import pytest
import torch

from kernels.rope import apply_rope
from oracle.rope import cos_sin, rope_fwd_bwd

TOL = {torch.float32: 1e-5, torch.float16: 2e-2, torch.bfloat16: 2e-2}


def _case(rng: random.Random, gen: torch.Generator):
    b = rng.choice([1, 1, 2, 3])
    nkv = rng.choice([1, 2, 4, 8])
    nq = nkv * rng.choice([1, 2, 3, 4, 7])
    s = rng.choice([1, rng.randint(1, 64), rng.randint(1, 600)])
    d = rng.choice([16, 32, 64, 128, 128, 256])
    dtype = rng.choice([torch.bfloat16, torch.float16, torch.float32])
    bshd = rng.random() < 0.3
    mode = rng.choice(["plain", "batched", "positions"])
    base = rng.choice([10000.0, 500000.0])
    tdtype = torch.float32 if dtype != torch.float32 and rng.random() < 0.3 else dtype
    if bshd:
        q = torch.randn(b, s, nq, d, generator=gen).to(dtype).transpose(1, 2)
        k = torch.randn(b, s, nkv, d, generator=gen).to(dtype).transpose(1, 2)
    else:
        q = torch.randn(b, nq, s, d, generator=gen).to(dtype)
        k = torch.randn(b, nkv, s, d, generator=gen).to(dtype)
    pos = None
    if mode == "positions":
        P = rng.randint(1, 2 * s + 1)
        pos = torch.randint(0, P, (b * s,), generator=gen)
        tc, ts = cos_sin(torch.arange(P), d, base, tdtype)
        cos, sin = tc.unsqueeze(0), ts.unsqueeze(0)                    # [1, P, D] table
        ref_c, ref_s = tc[pos].view(b, s, d), ts[pos].view(b, s, d)   # per-token rows
    else:
        tc, ts = cos_sin(torch.arange(s), d, base, tdtype)
        if mode == "batched":
            cos, sin = tc.unsqueeze(0).expand(b, -1, -1).contiguous(), ts.unsqueeze(0).expand(b, -1, -1).contiguous()
        else:
            cos, sin = tc.unsqueeze(0), ts.unsqueeze(0)
        ref_c, ref_s = cos, sin
    desc = (f"b={b} nq={nq} nkv={nkv} s={s} d={d} {dtype} bshd={bshd} mode={mode} base={base} "
            f"tables={tdtype}")
    return q, k, cos, sin, pos, ref_c, ref_s, desc


def _close(a, b, dtype):
    t = TOL[dtype]
    torch.testing.assert_close(a.float().cpu(), b.float().cpu(), atol=t, rtol=t)


@pytest.mark.gpu
@pytest.mark.parametrize("seed", [5, 29])
def test_rope_random_sweep(seed):
    rng = random.Random(seed)
    gen = torch.Generator().manual_seed(seed)
    for i in range(40):
        q, k, cos, sin, pos, ref_c, ref_s, desc = _case(rng, gen)
        dtype = q.dtype
        dq = torch.randn(q.shape, generator=gen).to(dtype)
        dk = torch.randn(k.shape, generator=gen).to(dtype)
        rq, rk, rdq, rdk = rope_fwd_bwd(q, k, ref_c, ref_s, dq, dk)
        qg = q.cuda().requires_grad_(True)
        kg = k.cuda().requires_grad_(True)
        try:
            oq, ok = apply_rope(qg, kg, cos.cuda(), sin.cuda(), positions=None if pos is None else pos.cuda())
            (oq * dq.cuda()).sum().add((ok * dk.cuda()).sum()).backward()
            _close(oq, rq, dtype)
            _close(ok, rk, dtype)
            _close(qg.grad, rdq, dtype)
            _close(kg.grad, rdk, dtype)
        except AssertionError as e:
            raise AssertionError(f"case {i}: {desc}\n{e}") from None
