"""Patch adapters (forge/patching/kernels): the PEFT-LoRA factories that run
the fused LoRA-MLP and LoRA-QKV(+RoPE) kernels, the basic module adapters,
the cross-entropy replacement and the fused linear-CE CausalLM forward.

Reference contracts: forge/forge/patching/kernels/lora.py:16-312 (skip
policy, activation detection, forward signatures), basic.py:24-126,
cross_entropy.py:15-49, fused_linear_ce.py:16-140.

peft is not installed here, so `LoraLinear` below reproduces the attribute
layout and forward of peft.tuners.lora.Linear that the adapters read
(base_layer, lora_A / lora_B ModuleDicts, scaling, lora_dropout,
active_adapters, disable_adapters, merged; result = base(x) +
lora_B(lora_A(dropout(x))) * scaling).  The models are Hugging Face's own
Llama / Qwen3 / Qwen2 / Gemma2 modules from tiny configs with random
weights (no checkpoint).

GPU parity: the patched (fused) forward and backward are compared with an
fp32 copy of the same modules, next to the unpatched bf16 PEFT path: the
fused error may not exceed twice the PEFT path's, or 1% of the tensor's
scale.
"""
import copy

import pytest
import torch
import torch.nn as nn

transformers = pytest.importorskip("transformers")

from transformers import Gemma2Config, LlamaConfig, Qwen2Config, Qwen3Config  # noqa: E402
import transformers.models.gemma2.modeling_gemma2 as MG  # noqa: E402
import transformers.models.llama.modeling_llama as ML  # noqa: E402
import transformers.models.qwen2.modeling_qwen2 as MQ2  # noqa: E402
import transformers.models.qwen3.modeling_qwen3 as MQ3  # noqa: E402

ARCH = {
    "llama": (LlamaConfig, ML, "Llama", {}),
    "qwen3": (Qwen3Config, MQ3, "Qwen3", {}),
    "qwen2": (Qwen2Config, MQ2, "Qwen2", {}),
    "gemma2": (Gemma2Config, MG, "Gemma2", {"hidden_activation": "gelu_pytorch_tanh", "query_pre_attn_scalar": 128,
                                             "attn_logit_softcapping": 50.0}),
}


class LoraLinear(nn.Module):
    """peft.tuners.lora.Linear's layout and forward (see the module docstring)."""

    def __init__(self, base: nn.Linear, r=16, alpha=32, dropout=0.0, lora_dtype=None, adapter="default"):
        super().__init__()
        self.base_layer = base
        dev, dt = base.weight.device, lora_dtype or base.weight.dtype
        self.lora_A = nn.ModuleDict({adapter: nn.Linear(base.in_features, r, bias=False, device=dev, dtype=dt)})
        self.lora_B = nn.ModuleDict({adapter: nn.Linear(r, base.out_features, bias=False, device=dev, dtype=dt)})
        with torch.no_grad():  # peft starts B at zero; a non-zero B makes the LoRA term count
            self.lora_B[adapter].weight.normal_(0.0, 0.05)
        self.lora_dropout = nn.ModuleDict({adapter: nn.Dropout(dropout) if dropout > 0 else nn.Identity()})
        self.scaling = {adapter: alpha / r}
        self.active_adapters = [adapter]
        self.disable_adapters = False
        self.merged = False
        base.weight.requires_grad_(False)
        if base.bias is not None:
            base.bias.requires_grad_(False)

    def forward(self, x):
        out = self.base_layer(x)
        for name in self.active_adapters:
            a, b = self.lora_A[name], self.lora_B[name]
            lx = self.lora_dropout[name](x.to(a.weight.dtype))
            out = out + (b(a(lx)) * self.scaling[name]).to(out.dtype)
        return out


def _cls(mod, suffix):
    return next(getattr(mod, k) for k in dir(mod) if k.endswith(suffix) and not k.startswith("_"))


def build(arch, part, dtype=torch.float32, device="cpu", lora=True, lora_dtype=None, seed=0, **cfg_over):
    """(module, rotary) of `arch`; part "mlp" or "attn"; projections wrapped
    in LoraLinear when lora."""
    C, M, _, extra = ARCH[arch]
    cfg = dict(hidden_size=512, intermediate_size=1024, num_attention_heads=4, num_key_value_heads=2, head_dim=128,
               vocab_size=1000, attn_implementation="eager", **extra)
    cfg.update(cfg_over)
    c = C(**cfg)
    torch.manual_seed(seed)
    if part == "mlp":
        m = _cls(M, "MLP")(c)
        names = ("gate_proj", "up_proj", "down_proj")
    else:
        m = _cls(M, "Attention")(c, 0)
        names = ("q_proj", "k_proj", "v_proj")
    m = m.to(device=device, dtype=dtype)
    if lora:
        for n in names:
            setattr(m, n, LoraLinear(getattr(m, n), lora_dtype=lora_dtype))
    rot = _cls(M, "RotaryEmbedding")(c).to(device)
    return m, rot


def lora_params(m):
    return [p for n, p in m.named_parameters() if "lora_" in n]


def patch(m, kernel):
    from forge.patching import FORWARD_MAKERS

    m.forward = FORWARD_MAKERS[kernel](m, {})
    return m


# ---------------------------------------------------------------------------
# CPU: patch-time policy, fallback identity, registry
# ---------------------------------------------------------------------------
def test_skip_policy():
    """lora.py:53-124: no adapter, disabled or merged adapter, dropout > 0,
    an unknown activation, a biased GeGLU projection -> ForgeSkipPatch."""
    from forge.patching import FORWARD_MAKERS, ForgeSkipPatch

    mk_mlp, mk_qkv = FORWARD_MAKERS["lora_mlp"], FORWARD_MAKERS["lora_qkv"]
    plain, _ = build("llama", "mlp", lora=False)
    with pytest.raises(ForgeSkipPatch, match="no active PEFT LoRA adapter"):
        mk_mlp(plain, {})
    attn, _ = build("llama", "attn", lora=False)
    with pytest.raises(ForgeSkipPatch):
        mk_qkv(attn, {})
    for attr in ("disable_adapters", "merged"):
        m, _ = build("llama", "mlp")
        setattr(m.up_proj, attr, True)
        with pytest.raises(ForgeSkipPatch, match="disabled or merged"):
            mk_mlp(m, {})
    m, _ = build("llama", "mlp")
    m.down_proj.lora_dropout["default"] = nn.Dropout(0.1)
    with pytest.raises(ForgeSkipPatch, match="dropout"):
        mk_mlp(m, {})
    m, _ = build("llama", "mlp", hidden_act="relu")
    with pytest.raises(ForgeSkipPatch, match="cannot infer activation"):
        mk_mlp(m, {})
    g, _ = build("gemma2", "mlp")
    g.gate_proj.base_layer.bias = nn.Parameter(torch.zeros(1024), requires_grad=False)
    with pytest.raises(ForgeSkipPatch, match="bias-free"):
        mk_mlp(g, {})
    # an adapter named only by `active_adapter` (a callable) is found
    m, _ = build("llama", "mlp")
    for p in (m.gate_proj, m.up_proj, m.down_proj):
        del p.active_adapters
        p.active_adapter = lambda: "default"
    mk_mlp(m, {})


@pytest.mark.parametrize("arch", ["llama", "qwen3", "qwen2", "gemma2"])
def test_cpu_calls_take_the_reference_path(arch):
    """On CPU tensors every call falls back to the submodule path, which must
    reproduce the unpatched HF + PEFT module exactly, forward and backward."""
    x = torch.randn(2, 9, 512)
    for part, kernel in (("mlp", "lora_mlp"), ("attn", "lora_qkv")):
        m, rot = build(arch, part)
        ref = copy.deepcopy(m)
        pe = rot(x, torch.arange(9)[None].expand(2, 9))
        args = (pe, None) if part == "attn" else ()
        xa, xb = x.clone().requires_grad_(True), x.clone().requires_grad_(True)
        o_ref = ref(xa, *args)
        o_ref = o_ref[0] if part == "attn" else o_ref
        patch(m, kernel)
        o = m(xb, *args)
        o = o[0] if part == "attn" else o
        torch.testing.assert_close(o, o_ref, rtol=1e-5, atol=1e-6)
        g = torch.randn_like(o)
        o_ref.backward(g)
        o.backward(g)
        torch.testing.assert_close(xb.grad, xa.grad, rtol=1e-5, atol=1e-6)
        for p, q in zip(lora_params(m), lora_params(ref)):
            torch.testing.assert_close(p.grad, q.grad, rtol=1e-5, atol=1e-6)


def test_call_time_conditions_on_cpu(tmp_path):
    """live_lora rejects what the fused kernels cannot reproduce: CPU tensors,
    a trainable base weight, a biased base, a merged adapter; DTensor weights
    are recognised (one-rank gloo group)."""
    import torch.distributed as dist
    from torch.distributed.device_mesh import init_device_mesh
    from torch.distributed.tensor import Replicate, distribute_tensor

    from forge.patching.kernels.lora import _is_dtensor, live_lora

    m, _ = build("llama", "mlp")
    assert live_lora(m.gate_proj) is None  # CPU
    assert not _is_dtensor(m.gate_proj.base_layer.weight)
    if not dist.is_initialized():
        dist.init_process_group("gloo", store=dist.FileStore(str(tmp_path / "store"), 1), rank=0, world_size=1)
    try:
        mesh = init_device_mesh("cpu", (1,))
        dt = distribute_tensor(m.gate_proj.base_layer.weight.detach(), mesh, [Replicate()])
        assert _is_dtensor(dt)
    finally:
        dist.destroy_process_group()


def test_registry_and_basic_adapters():
    from forge.patching import FORWARD_MAKERS

    assert sorted(FORWARD_MAKERS) == ["embedding", "fused_linear_ce", "geglu", "lora_mlp", "lora_qkv", "rmsnorm",
                                      "swiglu"]
    emb = FORWARD_MAKERS["embedding"]
    assert emb.__forge_stub__ and emb.__forge_kernel_name__ == "embedding"
    with pytest.raises(NotImplementedError, match="not implemented yet"):
        emb(nn.Embedding(4, 4), {})(torch.zeros(1, dtype=torch.long))
    m, _ = build("llama", "mlp", lora=False)
    with pytest.raises(NotImplementedError, match="only supports activation='silu'"):
        FORWARD_MAKERS["swiglu"](m, {"activation": "gelu"})
    with pytest.raises(NotImplementedError, match="cannot infer GELU variant"):
        FORWARD_MAKERS["geglu"](m, {})
    x = torch.randn(3, 512)
    ref = m(x)
    assert torch.allclose(FORWARD_MAKERS["swiglu"](m, {})(x), ref, rtol=1e-5, atol=1e-6)
    g, _ = build("gemma2", "mlp", lora=False)
    assert torch.allclose(FORWARD_MAKERS["geglu"](g, {})(x), g(x), rtol=1e-5, atol=1e-6)


def test_cross_entropy_replacement_cpu_fallback():
    import torch.nn.functional as F

    from forge.patching.kernels.cross_entropy import forge_cross_entropy_replacement

    logits, target = torch.randn(6, 11), torch.randint(0, 11, (6,))
    assert torch.equal(forge_cross_entropy_replacement(logits, target), F.cross_entropy(logits, target))
    x3, t2 = torch.randn(2, 11, 3), torch.randint(0, 11, (2, 3))
    assert torch.equal(forge_cross_entropy_replacement(x3, t2, label_smoothing=0.1),
                       F.cross_entropy(x3, t2, label_smoothing=0.1))


# ---------------------------------------------------------------------------
# GPU: the fused paths
# ---------------------------------------------------------------------------
def _err(a, b):
    return (a.detach().double() - b.detach().double()).abs().max().item()


def _check(fused, peft, ref, what):
    ef, ep, scale = _err(fused, ref), _err(peft, ref), ref.detach().abs().max().item()
    assert ef <= max(2 * ep, 1e-2 * scale), (what, ef, ep, scale)


def _run(m, x, args, part, g):
    xx = x.clone().requires_grad_(True)
    o = m(xx, *args)
    o = o[0] if part == "attn" else o
    o.backward(g.to(o.dtype))
    return o, xx.grad, [p.grad for p in lora_params(m)]


def _parity(arch, part, kernel, B=2, S=37, cos_batch=None, lora_dtype=None, expect_fused=True, **cfg):
    from forge_hip import _lib as L

    from forge.patching.kernels import lora as LA

    m, rot = build(arch, part, dtype=torch.bfloat16, device="cuda", lora_dtype=lora_dtype, **cfg)
    m32 = copy.deepcopy(m).float()
    peft = copy.deepcopy(m)
    gen = torch.Generator(device="cuda").manual_seed(1)
    x = torch.randn(B, S, 512, device="cuda", generator=gen)
    pos = torch.arange(S, device="cuda")[None].expand(cos_batch or B, S)
    cos, sin = rot(x, pos)
    args32 = ((cos.float(), sin.float()), None) if part == "attn" else ()
    args16 = ((cos.to(torch.bfloat16), sin.to(torch.bfloat16)), None) if part == "attn" else ()
    g = torch.randn(B, S, 512, device="cuda", generator=gen)
    r32 = _run(m32, x, args32, part, g)
    rp = _run(peft, x.to(torch.bfloat16), args16, part, g)
    patch(m, kernel)
    xb = x.to(torch.bfloat16)
    if expect_fused is not None:
        fused = (LA.mlp_fused_args(m, xb) if part == "mlp" else LA.qkv_fused_args(m, xb)) is not None
        assert fused == expect_fused
    calls = L.calls
    rf = _run(m, xb, args16, part, g)
    if expect_fused is not False:
        assert L.calls > calls
    _check(rf[0], rp[0], r32[0], "out")
    _check(rf[1], rp[1], r32[1], "dx")
    for i, (a, b, c) in enumerate(zip(rf[2], rp[2], r32[2])):
        assert a.dtype == b.dtype
        _check(a, b, c, f"lora grad {i}")
    return m


@pytest.mark.gpu
@pytest.mark.parametrize("arch", ["llama", "qwen2", "qwen3"])
@pytest.mark.parametrize("S", [37, 64])
def test_lora_mlp_fused(arch, S):
    _parity(arch, "mlp", "lora_mlp", S=S)


@pytest.mark.gpu
@pytest.mark.parametrize("act", ["gelu_pytorch_tanh", "gelu"])
def test_lora_mlp_geglu_fused(act):
    """Gemma2 (GeGLU, tanh or exact GELU): the fused LoRA-GeGLU MLP in place of
    the reference's PEFT projections + GeGLU kernel (lora.py:170-197)."""
    _parity("gemma2", "mlp", "lora_mlp", hidden_activation=act)


@pytest.mark.gpu
def test_lora_mlp_geglu_fallback_keeps_the_projection_path():
    """A GeGLU MLP whose width the fused kernel cannot take runs the
    reference's composition (PEFT projections + the GeGLU kernel)."""
    _parity("gemma2", "mlp", "lora_mlp", expect_fused=False, intermediate_size=1020)


@pytest.mark.gpu
@pytest.mark.parametrize("arch,cos_batch", [("llama", None), ("llama", 1), ("gemma2", None)])
def test_lora_qkv_fused_rope(arch, cos_batch):
    """No q/k norm: one GEMM with RoPE in its epilogue (cos/sin per token, or
    a batch-1 table shared through positions); Gemma2 adds the softcap."""
    from forge.patching.kernels.lora import rope_tables

    m = _parity(arch, "attn", "lora_qkv", cos_batch=cos_batch)
    x = torch.zeros(2, 37, 512, device="cuda", dtype=torch.bfloat16)
    cos = torch.zeros(cos_batch or 2, 37, 128, device="cuda", dtype=torch.bfloat16)
    assert rope_tables(cos, cos, x, 128, 512, 256) is not None
    assert m.head_dim == 128


@pytest.mark.gpu
def test_lora_qkv_fused_without_rope_for_qk_norm():
    """Qwen3: q_norm/k_norm sit between the projection and RoPE, so the fused
    QKV GEMM runs without RoPE and the model's norms and RoPE follow."""
    _parity("qwen3", "attn", "lora_qkv")


@pytest.mark.gpu
def test_call_time_fallbacks_on_gpu():
    """Biased projections (Qwen2 attention), a trainable base weight and
    unsupported widths take the submodule path; fp32 LoRA factors stay fused
    and get fp32 gradients."""
    from forge.patching.kernels import lora as LA

    _parity("qwen2", "attn", "lora_qkv", expect_fused=False)  # q/k/v biases
    _parity("llama", "mlp", "lora_mlp", lora_dtype=torch.float32, expect_fused=True)
    m, _ = build("llama", "mlp", dtype=torch.bfloat16, device="cuda")
    m.up_proj.base_layer.weight.requires_grad_(True)
    patch(m, "lora_mlp")
    x = torch.randn(2, 8, 512, device="cuda", dtype=torch.bfloat16)
    assert LA.mlp_fused_args(m, x) is None
    m(x).float().sum().backward()
    assert m.up_proj.base_layer.weight.grad is not None
    m, _ = build("llama", "mlp", dtype=torch.bfloat16, device="cuda", intermediate_size=1020)
    assert LA.mlp_fused_args(m, x) is None  # I % 8 != 0
    patch(m, "lora_mlp")
    assert m(x).shape == x.shape


@pytest.mark.gpu
def test_cross_entropy_replacement_gpu():
    import torch.nn.functional as F
    from forge_hip import _lib as L

    from forge.patching.kernels.cross_entropy import forge_cross_entropy_replacement

    logits = torch.randn(64, 1000, device="cuda")
    target = torch.randint(0, 1000, (64,), device="cuda")
    target[::7] = -100
    calls = L.calls
    out = forge_cross_entropy_replacement(logits, target, label_smoothing=0.1)
    assert L.calls > calls
    torch.testing.assert_close(out, F.cross_entropy(logits, target, label_smoothing=0.1), rtol=1e-5, atol=1e-5)


@pytest.mark.gpu
@pytest.mark.parametrize("num_items", [None, 50])
def test_fused_linear_ce_causal_lm(num_items):
    """Training with labels: loss through the fused lm_head + CE (no logits);
    loss and gradients match the unpatched model's lm_head + loss_function."""
    from transformers import LlamaForCausalLM

    from forge.patching import FORWARD_MAKERS

    cfg = LlamaConfig(hidden_size=256, intermediate_size=512, num_attention_heads=2, num_key_value_heads=1,
                      head_dim=128, num_hidden_layers=1, vocab_size=1024, attn_implementation="eager")
    torch.manual_seed(0)
    ref = LlamaForCausalLM(cfg).to("cuda", torch.bfloat16).train()
    mod = copy.deepcopy(ref)
    mod.forward = FORWARD_MAKERS["fused_linear_ce"](mod, {})
    ids = torch.randint(0, 1024, (2, 33), device="cuda")
    labels = ids.clone()
    labels[0, :5] = -100
    kw = {} if num_items is None else {"num_items_in_batch": num_items}
    o_ref = ref(input_ids=ids, labels=labels, **kw)
    o = mod(input_ids=ids, labels=labels, **kw)
    assert o.logits is None and o_ref.logits is not None
    torch.testing.assert_close(o.loss.float(), o_ref.loss.float(), rtol=2e-2, atol=2e-2)
    o.loss.backward()
    o_ref.loss.backward()
    for (n, p), (_, q) in zip(mod.named_parameters(), ref.named_parameters()):
        scale = q.grad.abs().max().item()
        assert _err(p.grad, q.grad) <= 3e-2 * scale + 1e-6, n
    mod.eval()
    out = mod(input_ids=ids)  # no labels: logits through lm_head, as unpatched
    torch.testing.assert_close(out.logits, ref.eval()(input_ids=ids).logits)
