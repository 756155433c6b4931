"""PEFT-LoRA patch adapters that run the fused LoRA kernels.

Reference: forge/forge/patching/kernels/lora.py:126-312.  The reference's
factories validate the PEFT wrappers at patch time and then route every call
through the PEFT submodules (`module.gate_proj(x)`, `module.q_proj(h)`, ...)
so that FSDP2's all-gather hooks see each weight access: closing over raw
weights captured at patch time breaks once FSDP2 turns them into DTensor
shards.  That safety cost them the fused kernels.

These factories keep the reference's patch-time contract (same skip rules,
same ForgeSkipPatch sentinel, same forward signatures) and regain the fusion
without capturing anything at patch time: on every call they read the live
tensors off the submodules (`linear.base_layer.weight`, `lora_A[adapter]`,
...) and take the fused path only when that is exact for this call:

  * every weight is a plain CUDA tensor (not a DTensor shard: under FSDP2 the
    wrapped layer's pre-forward hook has already swapped in the unsharded
    parameters, which is what the call-time read sees);
  * the base Linear is bf16, frozen (the fused kernels return no base-weight
    gradient) and bias-free; the adapter is active, not merged or disabled,
    with identity dropout; bf16 or fp32 LoRA factors (fp32 ones are cast to
    bf16 for the kernels, and autograd returns fp32 gradients through the
    cast);
  * the widths are ones the kernels take (multiples of 8; the fused RoPE
    epilogue needs head_dim 64 or 128 and projection widths that are
    multiples of 256, with a full-width cos/sin table).

Otherwise the call takes the reference's submodule path, so a patched module
is never less general than the reference's.

Fused paths:
  * SiLU MLP (Qwen/Llama): LoRAMLPv6 (gate/up GEMMs with the LoRA-B terms as
    extra K segments, SwiGLU in the epilogue, down GEMM with its LoRA term).
  * GeGLU MLP (Gemma): LoRAMLPGeGLU, the same pipeline with the GeGLU
    epilogues - the fully-fused Gemma path the reference leaves as a
    follow-on (its adapter composes PEFT projections with the GeGLU kernel,
    which stays the fallback here).
  * Attention without q/k norms (Llama, Qwen2 bias-free, Gemma2):
    LoRAQKVRoPEFunction - one GEMM for Q|K|V with the LoRA terms, RoPE applied
    to Q and K in its epilogue (replaces view -> transpose ->
    apply_rotary_pos_emb, lora.py:240-264).  With q/k norms (Qwen3) the norm
    sits between the projection and RoPE, so the fused QKV GEMM runs without
    RoPE and the model's own norm and apply_rotary_pos_emb follow.
"""
from __future__ import annotations

import importlib
from typing import NamedTuple, Optional

import torch

from .common import ForgeSkipPatch

# ---------------------------------------------------------------------------
# patch-time inspection of a PEFT LoRA Linear (same policy as lora.py:16-95)
# ---------------------------------------------------------------------------


def _base(linear):
    return getattr(linear, "base_layer", linear)


def _linear_base_weight(linear):
    return getattr(_base(linear), "weight", None)


def _linear_base_bias(linear):
    return getattr(_base(linear), "bias", None)


def _active_lora_adapter(linear) -> Optional[str]:
    """Name of the first active adapter present in both lora_A and lora_B
    (lora.py:26-42): `active_adapters` (or `active_adapter`, possibly a
    callable or a single name); all of lora_A's adapters when none is set."""
    lora_a, lora_b = getattr(linear, "lora_A", None), getattr(linear, "lora_B", None)
    if not lora_a or not lora_b:
        return None
    names = getattr(linear, "active_adapters", None)
    if names is None:
        names = getattr(linear, "active_adapter", None)
    if callable(names):
        names = names()
    if isinstance(names, str):
        names = [names]
    if not names:
        names = list(lora_a.keys())
    return next((n for n in names if n in lora_a and n in lora_b), None)


def _is_identity_dropout(dropout) -> bool:
    """lora.py:45-50: None, nn.Identity or p == 0."""
    return dropout is None or isinstance(dropout, torch.nn.Identity) or float(getattr(dropout, "p", 0.0)) == 0.0


def _adapter_dropout(linear, adapter):
    """The adapter's dropout module.  PEFT keeps them in an nn.ModuleDict,
    which has no .get (the reference's `dropouts.get(adapter) if
    hasattr(dropouts, "get")` therefore never sees one): look the adapter up
    by key, so the documented rule (dropout must be 0) is enforced."""
    drops = getattr(linear, "lora_dropout", None)
    if drops is None:
        return None
    try:
        return drops[adapter] if adapter in drops else None
    except TypeError:
        return None


def _adapter_state_ok(linear, adapter) -> Optional[str]:
    """None when the adapter can be fused, else the reason it cannot."""
    if adapter is None:
        return "no active PEFT LoRA adapter"
    if getattr(linear, "disable_adapters", False) or getattr(linear, "merged", False):
        return "LoRA adapter is disabled or merged"
    if not _is_identity_dropout(_adapter_dropout(linear, adapter)):
        return "LoRA dropout must be 0.0 for exact fused patching"
    return None


def _check_lora_active(linear) -> None:
    """lora.py:77-91: raise ForgeSkipPatch unless `linear` carries an active,
    unmerged adapter with identity dropout."""
    why = _adapter_state_ok(linear, _active_lora_adapter(linear))
    if why is not None:
        raise ForgeSkipPatch(why)


def _lora_tensors(linear, *, allow_bias: bool = False):
    """lora.py:53-74: (W, A, B, scaling, bias) of the active adapter, or
    ForgeSkipPatch (also for a biased base Linear unless allow_bias)."""
    adapter = _active_lora_adapter(linear)
    why = _adapter_state_ok(linear, adapter)
    if why is not None:
        raise ForgeSkipPatch(why)
    bias = _linear_base_bias(linear)
    if bias is not None and not allow_bias:
        raise ForgeSkipPatch("LoRA Forge kernels currently require bias-free base Linear modules")
    scaling = getattr(linear, "scaling", {}).get(adapter, 1.0)
    return (_linear_base_weight(linear), linear.lora_A[adapter].weight, linear.lora_B[adapter].weight,
            float(scaling), bias)


_SILU_ACTS = {"silu", None}  # HF Qwen MLPs default to SiLU
_GELU_TANH_ACTS = {"gelu_pytorch_tanh", "gelu_new"}
_GELU_EXACT_ACTS = {"gelu", "gelu_python"}


def _detect_mlp_activation(module) -> str:
    """lora.py:99-124: "silu" | "gelu_tanh" | "gelu_exact" from the HF config
    attached to the MLP; ForgeSkipPatch when unrecognised."""
    cfg = getattr(module, "config", None)
    act = None
    if cfg is not None:
        act = getattr(cfg, "hidden_activation", None) or getattr(cfg, "hidden_act", None)
    if act in _SILU_ACTS:
        return "silu"
    if act in _GELU_TANH_ACTS:
        return "gelu_tanh"
    if act in _GELU_EXACT_ACTS:
        return "gelu_exact"
    raise ForgeSkipPatch(
        f"LoRA MLP fused kernel cannot infer activation from {act!r}; fall back to per-projection patching")


# ---------------------------------------------------------------------------
# call-time view of the live tensors
# ---------------------------------------------------------------------------
_DTENSOR = None


def _is_dtensor(t) -> bool:
    global _DTENSOR
    if _DTENSOR is None:
        try:
            from torch.distributed.tensor import DTensor
        except Exception:  # torch built without distributed
            DTensor = ()
        _DTENSOR = DTensor
    return bool(_DTENSOR) and isinstance(t, _DTENSOR)


class LiveLoRA(NamedTuple):
    W: torch.Tensor   # [out, in] frozen base weight (bf16)
    A: torch.Tensor   # [r, in]
    B: torch.Tensor   # [out, r]
    s: float          # LoRA scaling


def live_lora(linear) -> Optional[LiveLoRA]:
    """The tensors of `linear` as they are at this call, or None when the
    fused kernels cannot reproduce its forward exactly (see the module
    docstring for the conditions)."""
    adapter = _active_lora_adapter(linear)
    if _adapter_state_ok(linear, adapter) is not None:
        return None
    base = _base(linear)
    if getattr(base, "bias", None) is not None:
        return None
    W = getattr(base, "weight", None)
    A, B = linear.lora_A[adapter].weight, linear.lora_B[adapter].weight
    for t in (W, A, B):
        if t is None or _is_dtensor(t) or not t.is_cuda:
            return None
    if W.dtype != torch.bfloat16 or W.requires_grad or W.dim() != 2:
        return None
    if A.dtype not in (torch.bfloat16, torch.float32) or B.dtype != A.dtype:
        return None
    r = A.shape[0]
    if A.shape[1] != W.shape[1] or B.shape != (W.shape[0], r) or r % 8 != 0:
        return None
    return LiveLoRA(W, A, B, float(getattr(linear, "scaling", {}).get(adapter, 1.0)))


def _bf16(t):
    # differentiable cast: fp32 LoRA factors get their fp32 gradient back
    return t if t.dtype == torch.bfloat16 else t.to(torch.bfloat16)


def _fusable_input(x) -> bool:
    return x.is_cuda and x.dtype == torch.bfloat16 and not _is_dtensor(x) and x.shape[-1] % 8 == 0


def mlp_fused_args(module, x):
    """(gate, up, down) LiveLoRA of a gated MLP when the fused LoRA-MLP takes
    this call, else None."""
    if not _fusable_input(x):
        return None
    g, u, d = live_lora(module.gate_proj), live_lora(module.up_proj), live_lora(module.down_proj)
    if g is None or u is None or d is None:
        return None
    H, I, r = x.shape[-1], g.W.shape[0], g.A.shape[0]
    if g.W.shape != (I, H) or u.W.shape != (I, H) or d.W.shape != (H, I) or I % 8 != 0:
        return None
    if u.A.shape[0] != r or d.A.shape[0] != r:
        return None
    return g, u, d


def qkv_fused_args(module, x):
    """(q, k, v) LiveLoRA when the fused LoRA-QKV takes this call, else None."""
    if not _fusable_input(x) or x.dim() != 3:
        return None
    q, k, v = live_lora(module.q_proj), live_lora(module.k_proj), live_lora(module.v_proj)
    if q is None or k is None or v is None:
        return None
    K, r, D = x.shape[-1], q.A.shape[0], module.head_dim
    if q.W.shape[1] != K or k.W.shape[1] != K or v.W.shape != k.W.shape:
        return None
    if k.A.shape[0] != r or v.A.shape[0] != r:
        return None
    if q.W.shape[0] % D or k.W.shape[0] % D or q.W.shape[0] % 8 or k.W.shape[0] % 8:
        return None
    return q, k, v


def rope_tables(cos, sin, x, head_dim, hq, hkv):
    """(cos [P, D], sin [P, D], positions [B*S] or None) for the fused RoPE
    epilogue from HF's position embeddings (cos/sin [B or 1, S, D], one row
    per token), or None when the epilogue cannot take them (partial rotary,
    head_dim other than 64/128, widths not multiples of 256)."""
    if head_dim not in (64, 128) or hq % 256 or hkv % 256:
        return None
    if cos.dim() != 3 or cos.shape != sin.shape or cos.shape[-1] != head_dim:
        return None
    B, S = x.shape[0], x.shape[1]
    if cos.shape[1] != S or cos.shape[0] not in (1, B) or not cos.is_cuda:
        return None
    if cos.shape[0] == B:
        return cos.reshape(B * S, head_dim), sin.reshape(B * S, head_dim), None
    pos = torch.arange(B * S, device=x.device, dtype=torch.int64) % S  # every batch row reuses table rows 0..S-1
    return cos[0], sin[0], pos


# ---------------------------------------------------------------------------
# factories
# ---------------------------------------------------------------------------


def make_lora_mlp_forward(module, config):
    """PEFT LoRA MLP.forward -> fused LoRA-MLP with the SwiGLU (SiLU) or GeGLU
    (GELU, tanh or exact) epilogues; lora.py:126-197.

    Patch time: the activation must be recognised; SiLU needs an active
    adapter on each projection (lora.py:166-168), GeGLU extractable bias-free
    adapters (lora.py:189-191).  Call time: the fused kernel when
    `mlp_fused_args` accepts the live tensors, else the submodules (with the
    SwiGLU / GeGLU kernel for the activation, as in the reference)."""
    activation = _detect_mlp_activation(module)

    if activation == "silu":
        from forge.kernels.lora_mlp import LoRAMLPv6
        from forge.kernels.swiglu import swiglu

        for proj in (module.gate_proj, module.up_proj, module.down_proj):
            _check_lora_active(proj)

        def forward(x):
            fused = mlp_fused_args(module, x)
            if fused is None:
                return module.down_proj(swiglu(module.gate_proj(x), module.up_proj(x)))
            g, u, d = fused
            X3 = x if x.dim() == 3 else x.reshape(1, -1, x.shape[-1])
            out = LoRAMLPv6.apply(X3, g.W, _bf16(g.A), _bf16(g.B), g.s, u.W, _bf16(u.A), _bf16(u.B), u.s,
                                  d.W, _bf16(d.A), _bf16(d.B), d.s)
            return out.reshape(*x.shape[:-1], out.shape[-1])

        return forward

    from forge.kernels.geglu import geglu
    from forge.kernels.lora_mlp import LoRAMLPGeGLU

    for proj in (module.gate_proj, module.up_proj, module.down_proj):
        _lora_tensors(proj)
    approximate = "tanh" if activation == "gelu_tanh" else "none"

    def forward(x):
        fused = mlp_fused_args(module, x)
        if fused is None:
            return module.down_proj(geglu(module.gate_proj(x), module.up_proj(x), approximate=approximate))
        g, u, d = fused
        X3 = x if x.dim() == 3 else x.reshape(1, -1, x.shape[-1])
        out = LoRAMLPGeGLU.apply(X3, g.W, _bf16(g.A), _bf16(g.B), g.s, u.W, _bf16(u.A), _bf16(u.B), u.s,
                                 d.W, _bf16(d.A), _bf16(d.B), d.s, approximate)
        return out.reshape(*x.shape[:-1], out.shape[-1])

    return forward


def _sliding_window(module):
    """lora.py:271-279: the layer's own window, else Qwen's config rule."""
    window = getattr(module, "sliding_window", None)
    cfg = getattr(module, "config", None)
    if window is None and cfg is not None:
        if (getattr(cfg, "use_sliding_window", False) and getattr(cfg, "sliding_window", None) is not None
                and module.layer_idx >= getattr(cfg, "max_window_layers", 0)):
            window = cfg.sliding_window
    return window


def _attention_interface(module, modeling, kwargs):
    """lora.py:281-289: eager unless the config names another implementation
    (sdpa with output_attentions falls back to eager, with HF's warning)."""
    impl = module.config._attn_implementation
    if impl == "eager":
        return modeling.eager_attention_forward
    if impl == "sdpa" and kwargs.get("output_attentions", False):
        modeling.logger.warning_once(
            "`torch.nn.functional.scaled_dot_product_attention` does not support `output_attentions=True`. "
            "Falling back to eager attention.")
        return modeling.eager_attention_forward
    return modeling.ALL_ATTENTION_FUNCTIONS[impl]


def _qkv_states(module, modeling, hidden_states, cos, sin):
    """(query, key, value) as [B, heads, S, D] with RoPE applied to query and
    key: fused when the live tensors allow it, else the reference's chain."""
    from kernels.lora_qkv.experiments.v4.lora_qkv_kernel_v4 import LoRAQKVRoPEFunction, LoRAQKVv4Function

    D = module.head_dim
    hidden_shape = (*hidden_states.shape[:-1], -1, D)
    has_norm = hasattr(module, "q_norm") or hasattr(module, "k_norm")
    fused = qkv_fused_args(module, hidden_states)
    if fused is not None:
        q, k, v = fused
        tables = None if has_norm else rope_tables(cos, sin, hidden_states, D, q.W.shape[0], k.W.shape[0])
        lora = (q.W, k.W, v.W, _bf16(q.A), _bf16(q.B), q.s, _bf16(k.A), _bf16(k.B), k.s,
                _bf16(v.A), _bf16(v.B), v.s)
        if tables is not None:
            Q, K, V = LoRAQKVRoPEFunction.apply(hidden_states, *lora, *tables, D)
            return (Q.view(hidden_shape).transpose(1, 2), K.view(hidden_shape).transpose(1, 2),
                    V.view(hidden_shape).transpose(1, 2))
        Q, K, V = LoRAQKVv4Function.apply(hidden_states, *lora, None, None, None)
    else:
        Q, K, V = module.q_proj(hidden_states), module.k_proj(hidden_states), module.v_proj(hidden_states)
    Q, K, V = Q.view(hidden_shape), K.view(hidden_shape), V.view(hidden_shape)
    if hasattr(module, "q_norm"):
        Q = module.q_norm(Q)
    if hasattr(module, "k_norm"):
        K = module.k_norm(K)
    Q, K, V = Q.transpose(1, 2), K.transpose(1, 2), V.transpose(1, 2)
    Q, K = modeling.apply_rotary_pos_emb(Q, K, cos, sin)
    return Q, K, V


def make_lora_qkv_forward(module, config):
    """PEFT LoRA attention forward with fused Q/K/V (+RoPE), per
    lora.py:200-312: same signature (past_key_value or past_key_values,
    cache_position, **kwargs), KV-cache update, sliding window, attention
    interface selection, Gemma2's softcap, o_proj through its submodule."""
    for proj in (module.q_proj, module.k_proj, module.v_proj):
        _check_lora_active(proj)
    modeling = importlib.import_module(module.__class__.__module__)

    def forward(hidden_states, position_embeddings, attention_mask, past_key_value=None, past_key_values=None,
                cache_position=None, **kwargs):
        kv_cache = past_key_values if past_key_values is not None else past_key_value
        input_shape = hidden_states.shape[:-1]
        cos, sin = position_embeddings
        query, key, value = _qkv_states(module, modeling, hidden_states, cos, sin)
        if kv_cache is not None:
            key, value = kv_cache.update(key, value, module.layer_idx,
                                         {"sin": sin, "cos": cos, "cache_position": cache_position})
        extra = {}
        softcap = getattr(module, "attn_logit_softcapping", None)
        if softcap is not None:
            extra["softcap"] = softcap
        attn_output, attn_weights = _attention_interface(module, modeling, kwargs)(
            module, query, key, value, attention_mask,
            dropout=0.0 if not module.training else module.attention_dropout,
            scaling=module.scaling, sliding_window=_sliding_window(module), **extra, **kwargs)
        attn_output = attn_output.reshape(*input_shape, -1).contiguous()
        return module.o_proj(attn_output), attn_weights

    return forward


__all__ = ["LiveLoRA", "live_lora", "make_lora_mlp_forward", "make_lora_qkv_forward", "mlp_fused_args",
           "qkv_fused_args", "rope_tables"]
