"""Module-forward adapters for the elementwise and normalisation kernels
(reference forge/forge/patching/kernels/basic.py:24-126): each closes over
the module itself (never a tensor), so live weights and PEFT wrappers are
read at call time."""
from __future__ import annotations


def make_rmsnorm_forward(module, config):
    """RMSNorm.forward -> apply_rmsnorm (basic.py:24-50).  config: offset
    (0.0 Llama/Qwen, 1.0 Gemma), casting_mode (default "gemma" when offset is
    1.0 else "llama"), in_place (default: not for Gemma's residual-paired
    norms, whose dY feeds a second backward consumer)."""
    from forge.kernels.rmsnorm import apply_rmsnorm

    offset = float(config.get("offset", 0.0))
    casting_mode = config.get("casting_mode", "gemma" if offset == 1.0 else "llama")
    in_place = bool(config.get("in_place", offset != 1.0))
    eps = float(getattr(module, "variance_epsilon", getattr(module, "eps", 1e-6)))

    def forward(hidden_states):
        return apply_rmsnorm(hidden_states, module.weight, eps=eps, offset=offset, casting_mode=casting_mode,
                             in_place=in_place)

    return forward


_GELU_EXACT = {"gelu", "gelu_python"}
_GELU_TANH = {"gelu_pytorch_tanh", "gelu_new"}


def make_geglu_forward(module, config):
    """Gemma MLP.forward -> down_proj(geglu(gate_proj(x), up_proj(x)))
    (basic.py:53-90).  The GELU form comes from config["approximate"] or the
    HF config's hidden_activation / hidden_act; NotImplementedError when
    neither names a known form."""
    from forge.kernels.geglu import geglu

    approximate = config.get("approximate")
    if approximate is None:
        cfg = getattr(module, "config", None)
        act = None
        if cfg is not None:
            act = getattr(cfg, "hidden_activation", None) or getattr(cfg, "hidden_act", None)
        if act in _GELU_EXACT:
            approximate = "none"
        elif act in _GELU_TANH:
            approximate = "tanh"
        else:
            raise NotImplementedError(
                f"forge.patch: geglu kernel cannot infer GELU variant for hidden_activation={act!r}. "
                f"Pass approximate='tanh' or approximate='none' via the mapping config to override.")

    def forward(x):
        return module.down_proj(geglu(module.gate_proj(x), module.up_proj(x), approximate=approximate))

    return forward


def make_swiglu_forward(module, config):
    """Qwen/Llama MLP.forward -> down_proj(swiglu(gate_proj(x), up_proj(x)))
    (basic.py:93-107); only activation "silu"."""
    activation = config.get("activation", "silu")
    if activation != "silu":
        raise NotImplementedError(
            f"forge.patch: swiglu kernel only supports activation='silu', got {activation!r}. "
            f"Route this module to the 'geglu' kernel instead.")
    from forge.kernels.swiglu import swiglu

    def forward(x):
        return module.down_proj(swiglu(module.gate_proj(x), module.up_proj(x)))

    return forward


def make_not_implemented(kernel_name: str, why: str):
    """A declared-but-unwired kernel (basic.py:110-126): the factory is
    flagged as a stub (a patch loop skips it unless asked for it by name) and
    its forward raises NotImplementedError."""

    def factory(module, config):
        def forward(*args, **kwargs):
            raise NotImplementedError(
                f"Forge kernel {kernel_name!r} is not implemented yet ({why}). "
                f"Use forge.patch(model, kernels=[<built kernels only>]) to skip it.")

        return forward

    factory.__forge_stub__ = True
    factory.__forge_kernel_name__ = kernel_name
    factory.__forge_reason__ = why
    return factory
