"""Shared parity criteria for the bf16 GEMM-based kernels."""
import torch


def close_bf16(a, b, what=""):
    """bf16 parity: |a - b| <= 2e-2 * max(1, rms(b)) + 2e-2 * |b| elementwise,
    and cosine similarity > 0.9999."""
    a = a.detach().float().cpu()
    b = b.detach().float().cpu()
    scale = max(1.0, b.pow(2).mean().sqrt().item())
    torch.testing.assert_close(a, b, rtol=2e-2, atol=2e-2 * scale, msg=lambda m: f"{what}: {m}")
    cos = torch.nn.functional.cosine_similarity(a.flatten(), b.flatten(), dim=0).item()
    assert cos > 0.9999, f"{what}: cosine {cos}"
