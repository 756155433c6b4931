"""HIP graph capture of the library's launches (torch.cuda.graph): SwiGLU
forward + backward, a LoRA-MLP forward + backward step, and the allocation-
free LoRA-A product (forge_lora_a_noalloc).  Each graph is replayed several
times with new inputs copied into its static buffers eagerly between the
replays, and every replay must equal the eager result bit for bit (the
library records kernels only: no memset or memcpy nodes)."""
import ctypes

import pytest
import torch

from forge_hip import _lib as L

pytestmark = pytest.mark.gpu


def _capture(step, warmup=2):
    """Warms step() up on a side stream, then captures one call; returns
    (graph, its static outputs)."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(warmup):
            step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = step()
    return g, out


def test_swiglu_graph_replays():
    from kernels.swiglu import swiglu

    gate = torch.randn(512, 4096, device="cuda", requires_grad=True)
    up = torch.randn(512, 4096, device="cuda", requires_grad=True)
    dout = torch.randn(512, 4096, device="cuda")

    def step():
        gate.grad = up.grad = None
        out = swiglu(gate, up, 1.0, 1.0, True)
        out.backward(dout)
        return out, gate.grad, up.grad

    g, static = _capture(step)
    for i in range(3):
        with torch.no_grad():
            gate.copy_(torch.randn_like(gate))
            up.copy_(torch.randn_like(up))
            dout.copy_(torch.randn_like(dout))
        g.replay()
        torch.cuda.synchronize()
        got = [t.clone() for t in static]
        ref = step()
        torch.cuda.synchronize()
        for a, b in zip(got, ref):
            assert torch.equal(a, b), f"replay {i}"


def test_lora_mlp_graph_replays():
    from kernels.lora_mlp.experiments.v6.lora_mlp_kernel_v6 import LoRAMLPv6
    from oracle import lora_mlp as orc

    gen = torch.Generator().manual_seed(5)
    params = [t.cuda() if isinstance(t, torch.Tensor) else t for t in orc.make_params(512, 1024, 16, 32, gen)]
    lora = [params[i].requires_grad_(True) for i in (1, 2, 5, 6, 9, 10)]
    x = torch.randn(1, 600, 512, device="cuda").to(torch.bfloat16).requires_grad_(True)
    dy = torch.randn(1, 600, 512, device="cuda").to(torch.bfloat16)

    def step():
        for t in [x] + lora:
            t.grad = None
        out = LoRAMLPv6.apply(x, *params)
        out.backward(dy)
        return [out, x.grad] + [t.grad for t in lora]

    g, static = _capture(step)
    for i in range(3):
        with torch.no_grad():
            x.copy_(torch.randn_like(x, dtype=torch.float32).to(torch.bfloat16))
            dy.copy_(torch.randn_like(dy, dtype=torch.float32).to(torch.bfloat16))
        g.replay()
        torch.cuda.synchronize()
        got = [t.clone() for t in static]
        ref = step()
        torch.cuda.synchronize()
        for j, (a, b) in enumerate(zip(got, ref)):
            assert torch.equal(a, b), f"replay {i}, output {j}"


def test_lora_a_noalloc_graph_replays():
    M, K, r, n = 4096, 2048, 16, 2
    X = torch.randn(M, K, device="cuda").to(torch.bfloat16)
    A = (torch.randn(n * r, K, device="cuda") * 0.02).to(torch.bfloat16)
    ptrs = (ctypes.c_void_p * n)(*[A[p * r:].data_ptr() for p in range(n)])
    sc = (ctypes.c_float * n)(2.0, 0.5)
    out = torch.empty(M, n * r, dtype=torch.bfloat16, device="cuda")
    split = 4

    def step():
        L.check(L.forge_lora_a_noalloc(M, K, r, n, X.data_ptr(), K, ptrs, K, sc, out.data_ptr(), n * r, split,
                                       L.stream_of(X)), "forge_lora_a_noalloc")
        return out

    def eager_ref():
        ref = torch.empty_like(out)
        work = torch.empty(split, M, n * r, dtype=torch.float32, device="cuda")
        L.check(L.forge_lora_a(M, K, r, n, X.data_ptr(), K, ptrs, K, sc, ref.data_ptr(), n * r, work.data_ptr(),
                               split, L.stream_of(X)), "forge_lora_a")
        return ref

    g, static = _capture(step)
    for i in range(3):
        X.copy_(torch.randn(M, K, device="cuda").to(torch.bfloat16))
        g.replay()
        torch.cuda.synchronize()
        got = static.clone()
        ref = eager_ref()
        torch.cuda.synchronize()
        assert torch.equal(got, ref), f"replay {i}"
