"""LoRA-QKV v2_3 API on MI355X.

Drop-in for kernels/lora_qkv/experiments/v2/lora_qkv_kernel_v2_3.py of
Forge-researchlab/kernel-POCs: `pack_weights_all` and `lora_qkv_v2_3`
(forward only; Q, K, V returned as column views of one [M, Hq + 2 Hkv]
buffer).  `W_all` is accepted for API parity; the MFMA GEMM reads the six
weight matrices directly, so no packed copy is needed.
"""
from __future__ import annotations

import torch

from kernels.lora_qkv._impl import pack_weights_all, qkv_forward, split_views, torch_qkv_forward  # noqa: F401


def lora_qkv_v2_3(X, W_q, A_q, B_q, s_q, W_k, A_k, B_k, s_k, W_v, A_v, B_v, s_v, W_all=None):
    """v2_3 :177-267."""
    orig_shape = X.shape
    X2 = X.reshape(-1, X.shape[-1])
    if X.dtype == torch.float64:
        Q, K, V = torch_qkv_forward(X2, W_q, W_k, W_v, A_q, B_q, s_q, A_k, B_k, s_k, A_v, B_v, s_v)
        if len(orig_shape) == 3:
            Q, K, V = (t.view(orig_shape[0], orig_shape[1], -1) for t in (Q, K, V))
        return Q, K, V
    out = qkv_forward(X2, W_q, W_k, W_v, A_q, B_q, s_q, A_k, B_k, s_k, A_v, B_v, s_v)
    return split_views(out, W_q.shape[0], W_k.shape[0], orig_shape)


__all__ = ["pack_weights_all", "lora_qkv_v2_3"]
