"""Re-exports of the hot-path kernels (reference forge/forge/kernels/__init__.py):

    forge.kernels.swiglu         ForgeSwiGLUFunction, swiglu, ...  (kernels/swiglu)
    forge.kernels.geglu          ForgeGEGLUFunction, geglu, ...    (kernels/geglu)
    forge.kernels.rope           apply_rope, ForgeRoPEv3, forge_apply_rotary_pos_emb
    forge.kernels.cross_entropy  ForgeCrossEntropyFunction, forge_cross_entropy,
                                 ForgeFusedLinearCrossEntropyFunction, ...
    forge.kernels.lora_mlp       LoRAMLPv3 / LoRAMLPv6 and helpers
    forge.kernels.lora_qkv       LoRAQKVFunction / LoRAQKVv4Function and helpers
"""
