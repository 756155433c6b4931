"""LoRA-QKV oracle (test infrastructure only; see oracle/__init__.py).

Restates `lora_qkv_forward` and `LoRAQKV`
(kernels/lora_qkv/reference/lora_qkv_pytorch.py:34-214) on the CPU, and the
caller's QKV -> RoPE composition (forge/forge/patching/kernels/lora.py:250-264:
view(T, H, d) -> transpose -> apply_rotary_pos_emb) with per-token positions
for packed variable-length sequences.
"""
from __future__ import annotations

import torch

from oracle.rope import hf_apply_rotary_pos_emb


def forward(X, W_q, W_k, W_v, A_q, B_q, s_q, A_k, B_k, s_k, A_v, B_v, s_v):
    """lora_qkv_pytorch.py:34-121."""
    def proj(W, A, B, s):
        out = X @ W.t()
        if A is not None and B is not None:
            out = out + s * ((X @ A.t()) @ B.t())
        return out
    return proj(W_q, A_q, B_q, s_q), proj(W_k, A_k, B_k, s_k), proj(W_v, A_v, B_v, s_v)


def backward(dQ, dK, dV, X, W_q, W_k, W_v, A_q, B_q, s_q, A_k, B_k, s_k, A_v, B_v, s_v):
    """lora_qkv_pytorch.py:170-214 -> (dX, dA_q, dB_q, dA_k, dB_k, dA_v, dB_v)."""
    dX = dQ @ W_q + dK @ W_k + dV @ W_v
    out = []
    for dY, A, B, s in ((dQ, A_q, B_q, s_q), (dK, A_k, B_k, s_k), (dV, A_v, B_v, s_v)):
        dYB = dY @ B
        dX = dX + s * (dYB @ A)
        out += [s * (dYB.t() @ X), s * (dY.t() @ (X @ A.t()))]
    return (dX, *out)


def rope_rows(Y, cos_tok, sin_tok, head_dim):
    """RoPE on a [T, n*head_dim] projection with per-token cos/sin [T, D]."""
    T = Y.shape[0]
    y = Y.reshape(T, -1, head_dim).transpose(0, 1).unsqueeze(0)  # (1, n, T, D)
    out, _ = hf_apply_rotary_pos_emb(y, y[:, :1], cos_tok.unsqueeze(0), sin_tok.unsqueeze(0))
    return out[0].transpose(0, 1).reshape(T, -1)


def qkv_rope_fwd_bwd(X, dQ, dK, dV, params, cos_tok, sin_tok, head_dim, compute_dtype=torch.float32):
    """Forward with RoPE on Q/K and the backward by autograd (CPU)."""
    c = lambda t: t.detach().cpu().to(compute_dtype) if isinstance(t, torch.Tensor) else t  # noqa: E731
    p = [c(t) for t in params]
    for i in (3, 4, 6, 7, 9, 10):  # LoRA A/B need grads
        p[i] = p[i].requires_grad_(True)
    Xc = c(X).requires_grad_(True)
    Q, K, V = forward(Xc, *p)
    cq, sq = c(cos_tok), c(sin_tok)
    Qr, Kr = rope_rows(Q, cq, sq, head_dim), rope_rows(K, cq, sq, head_dim)
    (Qr * c(dQ)).sum().add((Kr * c(dK)).sum()).add((V * c(dV)).sum()).backward()
    grads = (Xc.grad, p[3].grad, p[4].grad, p[6].grad, p[7].grad, p[9].grad, p[10].grad)
    return (Qr.detach(), Kr.detach(), V.detach()), grads


def make_params(K, Hq, Hkv, r, alpha, gen, dtype=torch.bfloat16):
    """BASELINE configs[4] initialisation: W ~ N(0, 0.02^2), A Kaiming-uniform,
    B ~ N(0, 0.01^2), s = alpha / r.  Order matches LoRAQKV.forward."""
    s = alpha / r

    def W(o):
        return (torch.randn(o, K, generator=gen) * 0.02).to(dtype)

    def A():
        bound = 1.0 / K ** 0.5
        return ((torch.rand(r, K, generator=gen) * 2 - 1) * bound).to(dtype)

    def B(o):
        return (torch.randn(o, r, generator=gen) * 0.01).to(dtype)

    return (W(Hq), W(Hkv), W(Hkv), A(), B(Hq), s, A(), B(Hkv), s, A(), B(Hkv), s)


def varlen_lengths(n_seq, lo, hi, seed):
    """Sequence lengths U[lo, hi] from a seed."""
    g = torch.Generator().manual_seed(seed)
    return torch.randint(lo, hi + 1, (n_seq,), generator=g).tolist()


def positions_for(lengths):
    return torch.cat([torch.arange(n) for n in lengths])


def flops_per_token(K, Hq, Hkv, r):
    """Algorithmic FLOPs per token of one forward + backward, the published
    benchmark's accounting (109,314,048 at K=4096, Hq=4096, Hkv=1024, r=64):
    forward 2KN + 6Kr + 2rN, backward 2NK + 2Nr + 18Kr + 2Nr, N = Hq + 2Hkv."""
    N = Hq + 2 * Hkv
    return 4 * K * N + 6 * r * N + 24 * K * r


def lora_grads(dQ, dK, dV, X, W_q, W_k, W_v, A_q, B_q, s_q, A_k, B_k, s_k, A_v, B_v, s_v):
    """The LoRA-parameter part of `backward` alone (lora_qkv_pytorch.py:
    196-211): (dA_q, dB_q, dA_k, dB_k, dA_v, dB_v) with dA = s (dY B)^T X and
    dB = s dY^T (X A^T).  It skips backward's [T, K] dX products, so it runs
    over tens of thousands of tokens on the CPU."""
    out = []
    for dY, A, B, s in ((dQ, A_q, B_q, s_q), (dK, A_k, B_k, s_k), (dV, A_v, B_v, s_v)):
        out += [s * ((dY @ B).t() @ X), s * (dY.t() @ (X @ A.t()))]
    return tuple(out)
