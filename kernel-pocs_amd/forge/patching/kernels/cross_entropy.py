"""Module-level replacement of torch.nn.functional.cross_entropy (reference
forge/forge/patching/kernels/cross_entropy.py:15-49)."""
from __future__ import annotations

from typing import Optional

import torch
import torch.nn.functional as torch_F

from forge.kernels.cross_entropy import forge_cross_entropy

_TORCH_CROSS_ENTROPY = torch_F.cross_entropy  # bound at import, before any patch replaces it


def forge_cross_entropy_replacement(input: torch.Tensor, target: torch.Tensor, weight: Optional[torch.Tensor] = None,
                                    size_average=None, ignore_index: int = -100, reduce=None, reduction: str = "mean",
                                    label_smoothing: float = 0.0):
    """F.cross_entropy's signature.  2-D GPU logits without the legacy
    size_average / reduce arguments run the HIP cross-entropy; anything else
    (CPU tensors, [N, C, d...] inputs, legacy arguments) calls PyTorch's."""
    if size_average is not None or reduce is not None or input.dim() != 2 or not input.is_cuda:
        return _TORCH_CROSS_ENTROPY(input, target, weight=weight, size_average=size_average,
                                    ignore_index=ignore_index, reduce=reduce, reduction=reduction,
                                    label_smoothing=label_smoothing)
    return forge_cross_entropy(input, target, weight=weight, ignore_index=ignore_index,
                               label_smoothing=label_smoothing, reduction=reduction)
