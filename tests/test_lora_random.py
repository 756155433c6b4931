"""Seeded random sweep of the fused LoRA drop-ins against the float32 oracles,
forward and backward: LoRA-MLP (v6 and v3) over random token counts, hidden
and intermediate sizes and ranks (multiples of 8 and not), and LoRA-QKV (v4,
v3, and QKV + RoPE with varlen positions and bf16 or fp32 tables) over random
token counts, hidden sizes, GQA widths, head_dim 64 / 128 and ranks."""
import random

import pytest
import torch

from _parity import close_bf16
from kernels.lora_mlp.experiments.v3.lora_mlp_kernel_v3 import LoRAMLPv3
from kernels.lora_mlp.experiments.v6.lora_mlp_kernel_v6 import LoRAMLPv6
from kernels.lora_qkv.experiments.v3.lora_qkv_kernel_v3 import LoRAQKVFunction
from kernels.lora_qkv.experiments.v4.lora_qkv_kernel_v4 import LoRAQKVv4Function, lora_qkv_rope
from oracle import lora_mlp as omlp
from oracle import lora_qkv as oqkv
from oracle.rope import cos_sin


def _mlp_case(rng, gen, i):
    M = rng.choice([1, rng.randint(1, 64), rng.randint(1, 400)])
    H = rng.choice([128, 256, 384, 512])
    I = rng.choice([256, 512, 768, 1344])
    r = rng.choice([4, 8, 12, 16, 32, 64])
    alpha = rng.choice([r, 2 * r, 16])
    version = rng.choice(["v6", "v3"])
    desc = f"LoRA-MLP case {i}: M={M} H={H} I={I} r={r} alpha={alpha} {version}"
    params = omlp.make_params(H, I, r, alpha, gen)
    X = torch.randn(1, M, H, generator=gen).to(torch.bfloat16)  # [batch, seq, hidden], as the reference's API
    dY = torch.randn(1, M, H, generator=gen).to(torch.bfloat16)
    ref_out, ref_grads = omlp.fwd_bwd(X, dY, params)
    p = [t.cuda().requires_grad_(t.shape[0] <= 64 or t.shape[1] <= 64) if isinstance(t, torch.Tensor) else t
         for t in params]
    x = X.cuda().requires_grad_(True)
    Fn = LoRAMLPv6 if version == "v6" else LoRAMLPv3
    out = Fn.apply(x, *p)
    out.backward(dY.cuda())
    got = [x.grad] + [t.grad for t in (p[1], p[2], p[5], p[6], p[9], p[10])]
    names = ["dX", "dA_gate", "dB_gate", "dA_up", "dB_up", "dA_down", "dB_down"]
    return desc, [("out", out, ref_out)] + list(zip(names, got, ref_grads))


def _qkv_case(rng, gen, i):
    T = rng.choice([1, rng.randint(1, 64), rng.randint(1, 400)])
    K = rng.choice([128, 256, 512])
    D = rng.choice([64, 128])
    Hkv = D * rng.choice([1, 2])
    Hq = Hkv * rng.choice([1, 2, 4])
    r = rng.choice([4, 8, 12, 16, 24, 64])
    api = rng.choice(["v4", "v3", "rope", "rope"])
    params = oqkv.make_params(K, Hq, Hkv, r, 2 * r, gen)
    X = torch.randn(T, K, generator=gen).to(torch.bfloat16)
    dQ = torch.randn(T, Hq, generator=gen).to(torch.bfloat16)
    dK = torch.randn(T, Hkv, generator=gen).to(torch.bfloat16)
    dV = torch.randn(T, Hkv, generator=gen).to(torch.bfloat16)
    p = [t.cuda().requires_grad_(j in (3, 4, 6, 7, 9, 10)) if isinstance(t, torch.Tensor) else t
         for j, t in enumerate(params)]
    x = X.cuda().requires_grad_(True)
    desc = f"LoRA-QKV case {i}: T={T} K={K} Hq={Hq} Hkv={Hkv} D={D} r={r} {api}"
    if api == "rope":
        # packed varlen sequences: positions restart per sequence, into a longer table
        lens, left = [], T
        while left > 0:
            n = min(left, rng.randint(1, 200))
            lens.append(n)
            left -= n
        pos = oqkv.positions_for(lens)
        tdtype = rng.choice([torch.bfloat16, torch.float32])
        c, s = cos_sin(torch.arange(256), D, rng.choice([10000.0, 500000.0]), tdtype)
        desc += f" tables={tdtype} seqs={len(lens)}"
        (Qr, Kr, Vr), ref_grads = oqkv.qkv_rope_fwd_bwd(X, dQ, dK, dV, params, c[pos], s[pos], D)
        Q, K_, V = lora_qkv_rope(x, p[0], p[3], p[4], p[5], p[1], p[6], p[7], p[8], p[2], p[9], p[10], p[11],
                                 c.cuda(), s.cuda(), pos.cuda(), D)
    else:
        pf = [t.float() if isinstance(t, torch.Tensor) else t for t in params]
        Qr, Kr, Vr = oqkv.forward(X.float(), *pf)
        ref_grads = oqkv.backward(dQ.float(), dK.float(), dV.float(), X.float(), *pf)
        Fn = LoRAQKVv4Function if api == "v4" else LoRAQKVFunction
        Q, K_, V = Fn.apply(x, *p)
    torch.autograd.backward((Q, K_, V), (dQ.cuda(), dK.cuda(), dV.cuda()))
    got = [x.grad, p[3].grad, p[4].grad, p[6].grad, p[7].grad, p[9].grad, p[10].grad]
    names = ["dX", "dA_q", "dB_q", "dA_k", "dB_k", "dA_v", "dB_v"]
    return desc, [("Q", Q, Qr), ("K", K_, Kr), ("V", V, Vr)] + list(zip(names, got, ref_grads))


@pytest.mark.gpu
@pytest.mark.parametrize("which", ["mlp", "qkv"])
@pytest.mark.parametrize("seed", [13, 41])
def test_lora_random_sweep(which, seed):
    rng = random.Random(seed)
    gen = torch.Generator().manual_seed(seed)
    for i in range(12):
        desc, checks = (_mlp_case if which == "mlp" else _qkv_case)(rng, gen, i)
        try:
            for name, got, want in checks:
                close_bf16(got.reshape(want.shape), want, name)
        except AssertionError as e:
            raise AssertionError(f"{desc}\n{e}") from None
