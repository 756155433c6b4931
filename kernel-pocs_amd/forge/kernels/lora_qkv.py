"""LoRA-QKV re-export (reference forge/forge/kernels/lora_qkv.py:15-31)."""
from kernels.lora_qkv.experiments.v2.lora_qkv_kernel_v2_3 import pack_weights_all
from kernels.lora_qkv.experiments.v3.lora_qkv_kernel_v3 import LoRAQKVFunction, lora_qkv_v3
from kernels.lora_qkv.experiments.v4.lora_qkv_kernel_v4 import (
    LoRAQKVv4Function,
    lora_qkv_v4,
    pack_lora_a,
    pack_weights_backward,
)

__all__ = [
    "LoRAQKVFunction", "lora_qkv_v3", "pack_weights_all",
    "LoRAQKVv4Function", "lora_qkv_v4",
    "pack_weights_backward", "pack_lora_a",
]
