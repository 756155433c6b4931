"""Validation of caller-supplied RoPE positions (cos/sin row indices).

Varlen RoPE (`apply_rope(..., positions=)`, `lora_qkv_rope`) indexes the
cos/sin tables with caller data.  The kernels read no table memory for an
out-of-range position (that token's outputs become NaN), and the wrappers
raise before launching: `check_positions` reads the positions' min/max (one
host sync) and remembers the result for that tensor object at its current
version, so a positions buffer reused across steps (and the backward of the
same call) is checked once.
"""
from __future__ import annotations

import weakref

import torch

# id(tensor) -> (weak reference, version, rows needed); tensors compare
# elementwise, so they cannot be mapping keys themselves
_checked: dict = {}


def check_positions(positions: torch.Tensor, table_rows: int, what: str = "positions") -> None:
    """Raises IndexError unless every entry lies in [0, table_rows)."""
    if positions.dtype.is_floating_point or positions.dtype == torch.bool:
        raise TypeError(f"{what} must be an integer tensor (got {positions.dtype})")
    key = id(positions)
    hit = _checked.get(key)
    if hit is not None and hit[0]() is positions and hit[1] == positions._version and hit[2] <= table_rows:
        return
    if positions.numel() == 0:
        need = 0
    else:
        lo, hi = (int(v) for v in torch.aminmax(positions.detach()))
        if lo < 0 or hi >= table_rows:
            raise IndexError(
                f"{what} must lie in [0, {table_rows}) (the cos/sin table rows); got min {lo}, max {hi}")
        need = hi + 1

    def _drop(_ref, key=key):
        _checked.pop(key, None)

    _checked[key] = (weakref.ref(positions, _drop), positions._version, need)
