"""LoRA-MLP re-export (reference forge/forge/kernels/lora_mlp.py:22-41): the
v3 contract (13 inputs) and the v6 contract (stacked LoRA-A, streams), plus
the fused GeGLU variant for Gemma MLPs (no reference counterpart: the
reference's Gemma adapter composes PEFT projections with the GeGLU kernel)."""
from kernels.lora_mlp.experiments.v3.lora_mlp_kernel_v3 import LoRAMLPv3, fused_lora_swiglu, lora_mlp_v3
from kernels.lora_mlp.experiments.v6.lora_mlp_kernel_v6 import LoRAMLPv6, LoRAMLPv6Module, lora_mlp_v6, stack_lora_a
from kernels.lora_mlp.geglu_mlp import LoRAMLPGeGLU, lora_mlp_geglu

__all__ = [
    "LoRAMLPv3", "lora_mlp_v3", "fused_lora_swiglu",
    "LoRAMLPv6", "lora_mlp_v6", "LoRAMLPv6Module", "stack_lora_a",
    "LoRAMLPGeGLU", "lora_mlp_geglu",
]
