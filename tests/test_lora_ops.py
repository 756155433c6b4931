"""Host-side helpers of the LoRA modules: the cached transpose of a frozen
base weight must never serve stale data (CPU), and clear_caches() makes
writes through `.data` visible (GPU)."""
import gc

import pytest
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


@pytest.mark.gpu
def test_clear_caches_after_data_writes():
    """A write through `.data` (checkpoint load, PEFT-style merge) bumps
    neither tensor._version nor data_ptr, so the cached W^T copies the
    backwards use (frozen_t) and the stacked QKV weight (frozen_cat) cannot
    see it; clear_caches() is the documented call after such writes.  After
    it, LoRA-MLP and LoRA-QKV gradients and outputs equal those of a run on
    fresh tensors holding the new weights, bit for bit."""
    from kernels._lora_ops import clear_caches, frozen_cat, frozen_t
    from kernels.lora_mlp.experiments.v6.lora_mlp_kernel_v6 import LoRAMLPv6
    from kernels.lora_qkv.experiments.v4.lora_qkv_kernel_v4 import LoRAQKVv4Function
    from oracle import lora_mlp as orc_mlp
    from oracle import lora_qkv as orc_qkv

    gen = torch.Generator().manual_seed(31)
    H, I, r = 256, 512, 16

    def mlp_run(params, X, dY):
        p = [t.cuda().requires_grad_(t.shape[0] <= 64 or t.shape[1] <= 64) if isinstance(t, torch.Tensor) else t
             for t in params]
        return p, mlp_grads(p, X, dY)

    def mlp_grads(p, X, dY):
        for t in p:
            if isinstance(t, torch.Tensor):
                t.grad = None
        x = X.cuda().requires_grad_(True)
        out = LoRAMLPv6.apply(x, *p)
        out.backward(dY.cuda())
        return [out.detach().clone(), x.grad.clone()] + [t.grad.clone() for t in (p[1], p[2], p[5], p[6], p[9], p[10])]

    params = orc_mlp.make_params(H, I, r, 2 * r, gen)
    X = torch.randn(1, 64, H, generator=gen).to(torch.bfloat16)  # [batch, seq, hidden]
    dY = torch.randn(1, 64, H, generator=gen).to(torch.bfloat16)
    p, _ = mlp_run(params, X, dY)  # fills frozen_t for the three base weights
    deltas = [torch.randn(t.shape, generator=gen).to(torch.bfloat16) * 0.02 for t in (p[0], p[4], p[8])]
    for w, dlt in zip((p[0], p[4], p[8]), deltas):
        v, ptr = w._version, w.data_ptr()
        w.data += dlt.cuda()
        assert w._version == v and w.data_ptr() == ptr  # invisible to the cache keys
    stale_t = frozen_t(p[0])
    assert not torch.equal(stale_t.t(), p[0])  # the cached copy predates the write
    clear_caches()
    got = mlp_grads(p, X, dY)
    fresh = [t.detach().clone() if isinstance(t, torch.Tensor) else t for t in p]
    _, want = mlp_run([t.cpu() if isinstance(t, torch.Tensor) else t for t in fresh], X, dY)
    for a, b in zip(got, want):
        assert torch.equal(a, b)

    T, K, Hq, Hkv = 64, 256, 256, 128
    qp = [t.cuda() if isinstance(t, torch.Tensor) else t for t in orc_qkv.make_params(K, Hq, Hkv, r, 2 * r, gen)]
    x = torch.randn(T, K, generator=gen).to(torch.bfloat16).cuda()
    LoRAQKVv4Function.apply(x, *qp)  # fills frozen_cat((W_q, W_k, W_v))
    qp[0].data += 0.5
    clear_caches()
    assert torch.equal(frozen_cat((qp[0], qp[1], qp[2])), torch.cat([qp[0], qp[1], qp[2]]))
    Q1, K1, V1 = LoRAQKVv4Function.apply(x, *qp)
    Q2, K2, V2 = LoRAQKVv4Function.apply(x, *[t.clone() if isinstance(t, torch.Tensor) else t for t in qp])
    assert torch.equal(Q1, Q2) and torch.equal(K1, K2) and torch.equal(V1, V2)
