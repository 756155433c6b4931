"""Drop-in MI355X replacements for the reference's `kernels.*` package.

Module paths, function/class names, signatures and autograd contracts mirror
Forge-researchlab/kernel-POCs `kernels/{swiglu,rope,cross_entropy,lora_mlp,
lora_qkv}`; the device work runs in libforge_hip.so (hand-written gfx950 HIP).
"""
