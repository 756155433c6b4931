"""Package-level entry points of the hot path (the reference's `forge` package
surface for it): `forge.kernels.{swiglu,rope,cross_entropy,lora_mlp,lora_qkv}`
re-export the drop-in modules under `kernels/`, as the reference's
forge/forge/kernels/*.py do, so callers that import from either place resolve.
"""
