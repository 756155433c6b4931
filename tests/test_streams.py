"""Every entry point runs on the caller's current stream.  Each case makes a
side stream current (default priority), has a slow producer on it write the
op's input (a large matmul, then the copy into the input buffer), then calls
the op on that stream: an op that launched on another stream would read the
input before the producer wrote it.  Results are checked against the same op
run on the default stream after a synchronisation."""
import pytest
import torch

pytestmark = pytest.mark.gpu


def _slow_fill(dst: torch.Tensor, src: torch.Tensor):
    """On the current stream: ~1 ms of matmuls, then dst <- src (so dst
    holds garbage until the stream reaches the copy)."""
    a = torch.randn(4096, 4096, device="cuda")
    for _ in range(4):
        a = a @ a * 1e-3
    dst.copy_(src + 0 * a[0, 0].to(src.dtype))


def _on_side_stream(make_inputs, op):
    """(result on a side stream behind a slow producer, result on the default stream)."""
    torch.manual_seed(0)
    srcs = make_inputs()
    torch.cuda.synchronize()
    ref = op(*[s.clone() for s in srcs])
    torch.cuda.synchronize()
    bufs = [torch.full_like(s, float("nan")) if s.is_floating_point() else torch.zeros_like(s) for s in srcs]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for b, s in zip(bufs, srcs):
            _slow_fill(b, s)
        got = op(*bufs)
    torch.cuda.synchronize()
    return got, ref


def _same(got, ref):
    got = got if isinstance(got, (tuple, list)) else (got,)
    ref = ref if isinstance(ref, (tuple, list)) else (ref,)
    for a, b in zip(got, ref):
        assert torch.equal(a, b)


def test_swiglu_and_rope_on_side_stream():
    from kernels.rope import apply_rope, rope_cos_sin
    from kernels.swiglu import swiglu

    got, ref = _on_side_stream(lambda: (torch.randn(64, 4096, device="cuda"), torch.randn(64, 4096, device="cuda")),
                               lambda g, u: swiglu(g, u, 1.0, 1.0, True))
    _same(got, ref)
    c, s = rope_cos_sin(torch.arange(128, device="cuda"), 128, 10000.0, torch.bfloat16)

    def rope(q, k):
        return apply_rope(q, k, c.unsqueeze(0), s.unsqueeze(0))

    got, ref = _on_side_stream(lambda: (torch.randn(2, 8, 128, 128, device="cuda").to(torch.bfloat16),
                                        torch.randn(2, 2, 128, 128, device="cuda").to(torch.bfloat16)), rope)
    _same(got, ref)


def test_cross_entropy_on_side_stream():
    from kernels.cross_entropy.experiments.v2 import forge_cross_entropy

    def ce(logits, target):
        x = logits.requires_grad_(True)
        loss = forge_cross_entropy(x, target)
        loss.backward()
        return loss.detach(), x.grad

    got, ref = _on_side_stream(lambda: ((torch.randn(256, 32000, device="cuda") * 2).to(torch.bfloat16),
                                        torch.randint(0, 32000, (256,), device="cuda")), ce)
    _same(got, ref)


def test_lora_mlp_and_gemm_on_side_stream():
    from kernels.lora_mlp.experiments.v6.lora_mlp_kernel_v6 import LoRAMLPv6
    from oracle import lora_mlp as orc

    gen = torch.Generator().manual_seed(3)
    params = [t.cuda() if isinstance(t, torch.Tensor) else t for t in orc.make_params(256, 512, 16, 32, gen)]

    def mlp(x):
        return LoRAMLPv6.apply(x, *params)

    got, ref = _on_side_stream(lambda: (torch.randn(1, 300, 256, device="cuda").to(torch.bfloat16),), mlp)
    _same(got, ref)
