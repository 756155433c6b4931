"""RoPE re-export and the HF-signature adapter (reference
forge/forge/kernels/rope.py:12-43)."""
from kernels.rope.forge_rope_v3 import ForgeRoPEv3, ForgeRoPEv3Function, apply_rope


def forge_apply_rotary_pos_emb(q, k, cos, sin, position_ids=None, unsqueeze_dim=1):
    """Drop-in for transformers' module-level `apply_rotary_pos_emb`
    (reference forge/forge/kernels/rope.py:19-36).

    cos/sin arrive already indexed to the sequence, (batch, seq, head_dim), or
    pre-unsqueezed to 4-D along `unsqueeze_dim`; the 4-D form is squeezed back
    because `apply_rope` broadcasts over heads itself.  `position_ids` is
    accepted for signature compatibility and not used (the same contract as
    the reference).  Returns (q_rot, k_rot) with q's and k's shapes.
    """
    if cos.dim() == 4:
        cos = cos.squeeze(unsqueeze_dim)
        sin = sin.squeeze(unsqueeze_dim)
    return apply_rope(q, k, cos, sin)


__all__ = ["apply_rope", "ForgeRoPEv3", "ForgeRoPEv3Function", "forge_apply_rotary_pos_emb"]
