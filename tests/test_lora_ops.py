"""Host-side helpers of the LoRA modules (CPU): the cached transpose of a
frozen base weight must never serve stale data."""
import gc

import torch

from kernels import _lora_ops as ops


def test_frozen_t_is_cached_and_invalidated():
    w = torch.randn(24, 40)
    t1 = ops.frozen_t(w)
    assert torch.equal(t1, w.t()) and t1.is_contiguous()
    assert ops.frozen_t(w) is t1                      # second call: the cached copy
    w.add_(1.0)                                       # in-place change bumps _version
    t2 = ops.frozen_t(w)
    assert t2 is not t1 and torch.equal(t2, w.t())
    w.data = torch.randn(24, 40)                      # new storage under the same object
    t3 = ops.frozen_t(w)
    assert torch.equal(t3, w.t())
    other = torch.randn(24, 40)
    assert torch.equal(ops.frozen_t(other), other.t())
    n = len(ops._T_CACHE)
    del other
    gc.collect()
    assert len(ops._T_CACHE) == n - 1                 # entry dropped with its weight


def test_small_t():
    a = torch.randn(16, 64)
    assert torch.equal(ops.small_t(a), a.t()) and ops.small_t(a).is_contiguous()
