"""Shared sentinel of the patch adapters (reference
forge/forge/patching/kernels/common.py:1-6)."""
from __future__ import annotations


class ForgeSkipPatch(RuntimeError):
    """Raised by an adapter factory when its kernel does not apply to the
    module it was offered; the patch loop then tries the next candidate."""
