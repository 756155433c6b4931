"""The Python drop-in boundary: import paths, names and host-side argument
checks that the reference performs before any launch (CPU tests), plus the
HF-signature RoPE adapter on the GPU.

Import surface: reference forge/forge/kernels/{swiglu,rope,cross_entropy,
lora_mlp,lora_qkv}.py re-export the POC modules; callers and the reference's
tests import from both places, so both must resolve to the same objects.
"""
import importlib

import pytest
import torch

REEXPORTS = {
    "forge.kernels.swiglu": ("kernels.swiglu", [
        "ForgePackedSwiGLUFunction", "ForgeSwiGLUFunction", "swiglu", "swiglu_backward", "swiglu_forward",
        "swiglu_packed", "swiglu_packed_backward", "swiglu_packed_forward", "torch_swiglu_packed_reference",
        "torch_swiglu_reference"]),
    "forge.kernels.rope": ("kernels.rope.forge_rope_v3", ["apply_rope", "ForgeRoPEv3", "ForgeRoPEv3Function"]),
    "forge.kernels.rmsnorm": ("kernels.rmsnorm", [
        "ForgeRMSNormFunction", "apply_rmsnorm", "rmsnorm", "rmsnorm_backward", "rmsnorm_forward",
        "torch_rmsnorm_reference"]),
    "forge.kernels.geglu": ("kernels.geglu", [
        "ForgeGEGLUFunction", "ForgePackedGEGLUFunction", "geglu", "geglu_backward", "geglu_forward", "geglu_packed",
        "geglu_packed_backward", "geglu_packed_forward", "torch_geglu_packed_reference", "torch_geglu_reference"]),
    "forge.kernels.cross_entropy": ("kernels.cross_entropy.experiments.v2", [
        "CrossEntropyOutput", "ForgeCrossEntropyFunction", "ForgeCrossEntropyLoss", "forge_cross_entropy",
        "ForgeFusedLinearCrossEntropyFunction", "ForgeFusedLinearCrossEntropyLoss",
        "forge_fused_linear_cross_entropy", "fused_linear_cross_entropy_backward",
        "fused_linear_cross_entropy_forward"]),
    "forge.kernels.lora_mlp": ("kernels.lora_mlp.experiments.v6.lora_mlp_kernel_v6", [
        "LoRAMLPv6", "LoRAMLPv6Module", "lora_mlp_v6", "stack_lora_a"]),
    "forge.kernels.lora_qkv": ("kernels.lora_qkv.experiments.v4.lora_qkv_kernel_v4", [
        "LoRAQKVv4Function", "lora_qkv_v4", "pack_lora_a", "pack_weights_backward"]),
}


@pytest.mark.parametrize("pkg", sorted(REEXPORTS))
def test_reexports_resolve_to_the_same_objects(pkg):
    mod = importlib.import_module(pkg)
    src_name, names = REEXPORTS[pkg]
    src = importlib.import_module(src_name)
    for n in names:
        assert getattr(mod, n) is getattr(src, n), n
        assert n in mod.__all__, n


def test_lora_reexports_include_v3_contracts():
    mlp = importlib.import_module("forge.kernels.lora_mlp")
    qkv = importlib.import_module("forge.kernels.lora_qkv")
    for n in ("LoRAMLPv3", "lora_mlp_v3", "fused_lora_swiglu"):
        assert callable(getattr(mlp, n))
    for n in ("LoRAQKVFunction", "lora_qkv_v3", "pack_weights_all"):
        assert callable(getattr(qkv, n))


# ---------------------------------------------------------------------------
# host-side checks (same exception types and messages as the reference)
# ---------------------------------------------------------------------------
def test_rope_shape_assertions():
    """kernels/rope/forge_rope_v3.py:161-200: 4-D q/k, 3-D cos/sin, matching
    shapes, cos batch 1 or B, power-of-two head_dim, n_q % n_kv == 0."""
    from kernels.rope.forge_rope_v3 import apply_rope

    q = torch.randn(1, 4, 8, 16)
    k = torch.randn(1, 2, 8, 16)
    cs = torch.randn(1, 8, 16)
    with pytest.raises(AssertionError):
        apply_rope(q[0], k, cs, cs)                       # 3-D q
    with pytest.raises(AssertionError):
        apply_rope(q, k, cs[0], cs[0])                    # 2-D cos
    with pytest.raises(AssertionError):
        apply_rope(q, torch.randn(1, 2, 8, 8), cs, cs)    # k head_dim mismatch
    with pytest.raises(AssertionError):
        apply_rope(q, k, torch.randn(3, 8, 16), torch.randn(3, 8, 16))  # cos batch 3 vs B 1
    with pytest.raises(AssertionError):
        apply_rope(torch.randn(1, 4, 8, 12), torch.randn(1, 2, 8, 12), torch.randn(1, 8, 12),
                   torch.randn(1, 8, 12))                 # head_dim 12 not a power of two
    with pytest.raises(AssertionError, match="n_q % n_kv"):
        apply_rope(torch.randn(1, 3, 8, 16), k, cs, cs)


def test_cross_entropy_loss_module_assertions():
    """cross_entropy_kernel_v2.py:646-660: label_smoothing in [0, 1], reduction
    in {mean, sum, none}."""
    from kernels.cross_entropy.experiments.v2 import ForgeCrossEntropyLoss

    with pytest.raises(AssertionError, match="label_smoothing"):
        ForgeCrossEntropyLoss(label_smoothing=1.5)
    with pytest.raises(AssertionError, match="reduction"):
        ForgeCrossEntropyLoss(reduction="avg")
    ForgeCrossEntropyLoss(label_smoothing=0.0, reduction="none")


def test_fused_linear_ce_argument_checks():
    """fused_linear_cross_entropy.py:59-84 and :441-447: the shape checks
    raise ValueError, the flag and Module checks AssertionError, all before
    any device work (so they hold on the CPU too)."""
    from kernels.cross_entropy.experiments.v2 import (
        ForgeFusedLinearCrossEntropyLoss,
        fused_linear_cross_entropy_forward as fwd,
    )

    x, W, t = torch.zeros(4, 8), torch.zeros(5, 8), torch.zeros(4, dtype=torch.int64)
    with pytest.raises(AssertionError, match="return_z_loss must be True or False"):
        fwd(x, W, t, return_z_loss=1)
    with pytest.raises(ValueError, match=r"_input must be 2D \(B\*T, H\)"):
        fwd(x.view(2, 2, 8), W, t)
    with pytest.raises(ValueError, match=r"weight must be 2D \(V, H\)"):
        fwd(x, W.view(-1), t)
    with pytest.raises(ValueError, match=r"target must be 1D \(B\*T,\)"):
        fwd(x, W, t.view(2, 2))
    with pytest.raises(ValueError, match="weight.shape\\[1\\] must match _input.shape\\[1\\]; got 4 != 8"):
        fwd(x, torch.zeros(5, 4), t)
    with pytest.raises(ValueError, match="target length must match _input rows; got 3 != 4"):
        fwd(x, W, t[:3])
    with pytest.raises(ValueError, match=r"bias must have shape \(5,\); got \(4,\)"):
        fwd(x, W, t, bias=torch.zeros(4))
    with pytest.raises(AssertionError, match="label_smoothing must be between 0.0 and 1.0"):
        ForgeFusedLinearCrossEntropyLoss(label_smoothing=-0.1)
    with pytest.raises(AssertionError, match="supports reduction='mean', 'sum', or 'none'"):
        ForgeFusedLinearCrossEntropyLoss(reduction="avg")
    with pytest.raises(AssertionError, match="softcap must greater than 0.0 or None"):
        ForgeFusedLinearCrossEntropyLoss(softcap=0.0)


# ---------------------------------------------------------------------------
# the HF-signature adapter on the GPU
# ---------------------------------------------------------------------------
@pytest.mark.gpu
@pytest.mark.parametrize("pre_unsqueezed", [False, True])
def test_forge_apply_rotary_pos_emb_matches_hf(pre_unsqueezed):
    """forge/forge/kernels/rope.py:19-36: cos/sin (B, S, D), or pre-unsqueezed
    (B, 1, S, D) which is squeezed back; outputs match the HF formula."""
    from forge.kernels.rope import forge_apply_rotary_pos_emb
    from oracle.rope import cos_sin, hf_apply_rotary_pos_emb

    g = torch.Generator().manual_seed(0)
    B, Hq, Hkv, S, D = 2, 8, 2, 64, 128
    q = torch.randn(B, S, Hq, D, generator=g).to(torch.bfloat16).transpose(1, 2)  # HF view of BSHD
    k = torch.randn(B, S, Hkv, D, generator=g).to(torch.bfloat16).transpose(1, 2)
    c, s = cos_sin(torch.arange(S), D, 500000.0, torch.bfloat16)
    c, s = c.unsqueeze(0).expand(B, S, D).contiguous(), s.unsqueeze(0).expand(B, S, D).contiguous()
    ref_q, ref_k = hf_apply_rotary_pos_emb(q.float(), k.float(), c.float(), s.float())
    cc, ss = (c.unsqueeze(1), s.unsqueeze(1)) if pre_unsqueezed else (c, s)
    oq, ok = forge_apply_rotary_pos_emb(q.cuda(), k.cuda(), cc.cuda(), ss.cuda(), position_ids=None, unsqueeze_dim=1)
    assert oq.shape == q.shape and ok.shape == k.shape
    torch.testing.assert_close(oq.float().cpu(), ref_q.to(torch.bfloat16).float(), rtol=2e-2, atol=2e-2)
    torch.testing.assert_close(ok.float().cpu(), ref_k.to(torch.bfloat16).float(), rtol=2e-2, atol=2e-2)
