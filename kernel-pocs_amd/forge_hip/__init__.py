"""MI355X (gfx950) kernel library behind the drop-in `kernels.*` modules."""
from . import _lib  # noqa: F401  (raises ImportError if libforge_hip.so is not built)
from ._lib import LIB_PATH, check, dtype_code, ptr, require_gpu, stream_of  # noqa: F401

__all__ = ["LIB_PATH", "check", "dtype_code", "ptr", "require_gpu", "stream_of"]
