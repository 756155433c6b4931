"""Patch adapters that route Hugging Face / PEFT module forwards into the
HIP kernels (reference forge/forge/patching/kernels/).  Only the adapter
factories and their registry are provided; the model traversal and
restoration loop of the reference's patching/core.py is not part of this
package, so callers assign `module.forward = FORWARD_MAKERS[name](module,
config)` themselves (keeping the original for restoration)."""
from .kernels import FORWARD_MAKERS, ForgeSkipPatch

__all__ = ["FORWARD_MAKERS", "ForgeSkipPatch"]
