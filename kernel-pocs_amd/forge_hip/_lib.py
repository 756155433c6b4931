"""ctypes binding of libforge_hip.so (the gfx950 kernel library).

The C ABI is declared in include/forge_hip.h.  PyTorch provides device
memory and the current stream; every call passes raw data pointers, element
strides and the stream handle.  A non-zero status becomes a RuntimeError with
the library's message.

The library must be built (python kernel-pocs_amd/build.py, or
__graft_entry__.build()); importing this module without it raises ImportError,
so no kernel path can silently run without the HIP code.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

import torch  # loads the HIP runtime (libamdhip64.so.7) that the library links against

LIB_PATH = Path(os.environ.get("FORGE_HIP_LIB", Path(__file__).resolve().parent / "libforge_hip.so"))

if not LIB_PATH.exists():
    raise ImportError(
        f"libforge_hip.so not found at {LIB_PATH}; build it with "
        "`python kernel-pocs_amd/build.py` (hipcc, gfx950)"
    )

_lib = ctypes.CDLL(str(LIB_PATH))

c_i64 = ctypes.c_int64
c_int = ctypes.c_int
c_f32 = ctypes.c_float
c_vp = ctypes.c_void_p

DTYPE_F32, DTYPE_F16, DTYPE_BF16, DTYPE_F64 = 0, 1, 2, 3
LAYOUT_ROW, LAYOUT_COL = 0, 1
EPI_STORE, EPI_ATOMIC_F32, EPI_SILU, EPI_RELU, EPI_GELU = 0, 1, 2, 3, 4
GEMM_ACT_NONE, GEMM_ACT_SILU, GEMM_ACT_RELU, GEMM_ACT_GELU = 0, 1, 2, 3
ACT_SILU, ACT_GELU_TANH, ACT_GELU_ERF = 0, 1, 2

CE_HAS_GRADIENTS = 1
CE_HAS_WEIGHT = 2
CE_HAS_SOFTCAP = 4
CE_RETURN_Z_LOSS = 8
CE_RETURN_ACCURACY = 16
CE_RETURN_PREDICTED = 32
CE_REDUCTION_MEAN = 64

_TORCH_DTYPE = {
    torch.float32: DTYPE_F32,
    torch.float16: DTYPE_F16,
    torch.bfloat16: DTYPE_BF16,
    torch.float64: DTYPE_F64,
}


class GemmSegment(ctypes.Structure):
    """Mirror of forge_gemm_segment."""

    _fields_ = [
        ("a", c_vp),
        ("lda", c_i64),
        ("b", c_vp),
        ("ldb", c_i64),
        ("k", c_i64),
        ("n_lo", c_i64),  # output columns [n_lo, n_hi); 0, 0 = every column
        ("n_hi", c_i64),
    ]


def _decl(name, argtypes, restype=c_int):
    fn = getattr(_lib, name)
    fn.argtypes = argtypes
    fn.restype = restype
    return fn


forge_version = _decl("forge_version", [], ctypes.c_char_p)
forge_last_error = _decl("forge_last_error", [], ctypes.c_char_p)
forge_arch_ok = _decl("forge_arch_ok", [])
forge_swiglu_fwd = _decl(
    "forge_swiglu_fwd", [c_int, c_vp, c_vp, c_i64, c_vp, c_i64, c_i64, c_i64, c_f32, c_f32, c_vp]
)
forge_swiglu_bwd = _decl(
    "forge_swiglu_bwd",
    [c_int, c_vp, c_i64, c_vp, c_vp, c_i64, c_vp, c_vp, c_i64, c_i64, c_i64, c_f32, c_f32, c_vp],
)
forge_geglu_fwd = _decl("forge_geglu_fwd", [c_int, c_vp, c_vp, c_i64, c_vp, c_i64, c_i64, c_i64, c_int, c_vp])
forge_geglu_bwd = _decl(
    "forge_geglu_bwd", [c_int, c_vp, c_i64, c_vp, c_vp, c_i64, c_vp, c_vp, c_i64, c_i64, c_i64, c_int, c_vp]
)
forge_rope = _decl(
    "forge_rope",
    [c_int]
    + [c_vp, c_i64, c_i64, c_i64] * 4
    + [c_vp, c_i64, c_i64] * 2
    + [c_int, c_i64]
    + [c_vp, c_i64, c_i64, c_i64, c_i64, c_i64, c_int, c_vp],
)
forge_ce_fwd = _decl(
    "forge_ce_fwd",
    [c_int, c_vp, c_i64, c_i64, c_i64, c_vp, c_i64, c_vp, c_vp, c_vp, c_vp, c_vp, c_i64]
    + [c_f32] * 6
    + [c_int, c_vp, c_vp],
)
forge_ce_target_stats = _decl("forge_ce_target_stats", [c_vp, c_i64, c_i64, c_i64, c_i64, c_vp, c_vp])
forge_ce_fwd_reduce = _decl(
    "forge_ce_fwd_reduce",
    [c_int, c_vp, c_i64, c_i64, c_i64, c_vp, c_i64, c_vp, c_vp, c_vp, c_vp, c_i64]
    + [c_f32] * 3
    + [c_int, c_vp, c_vp, c_vp, c_vp, c_int, ctypes.POINTER(ctypes.c_uint64), c_vp],
)
forge_ce_stats_wait = _decl("forge_ce_stats_wait", [ctypes.c_uint64, ctypes.POINTER(c_i64), c_vp])
forge_splitk_reduce = _decl("forge_splitk_reduce", [c_vp, c_i64, c_int, c_i64, c_i64, c_i64, c_vp, c_i64, c_int, c_f32, c_vp])
forge_ce_scale = _decl("forge_ce_scale", [c_int, c_vp, c_i64, c_i64, c_i64, c_vp, c_int, c_vp])
forge_sum_f32 = _decl("forge_sum_f32", [c_vp, c_i64, c_vp, c_vp, c_int, c_vp])
forge_gemm = _decl(
    "forge_gemm",
    [c_i64, c_i64, ctypes.POINTER(GemmSegment), c_int, c_int, c_int, c_vp, c_i64, c_int, c_f32, c_f32, c_int, c_int, c_vp],
)
forge_lora_mlp_gate_up = _decl(
    "forge_lora_mlp_gate_up",
    [c_i64] * 4 + [c_vp, c_i64, c_vp, c_vp, c_i64, c_vp, c_i64, c_vp, c_vp, c_i64, c_vp, c_vp, c_vp, c_i64, c_int, c_vp],
)
forge_lora_mlp_down_bwd = _decl(
    "forge_lora_mlp_down_bwd",
    [c_i64] * 4 + [c_vp, c_i64, c_vp, c_i64, c_vp, c_i64, c_vp, c_i64, c_int, c_vp, c_vp, c_vp, c_i64, c_int, c_vp],
)
forge_lora_qkv_rope = _decl(
    "forge_lora_qkv_rope",
    [c_i64] * 5
    + [c_vp, c_i64, c_vp, c_vp, c_vp, c_i64, c_vp, c_i64, c_vp, c_vp, c_vp, c_i64, c_vp, c_i64]
    + [c_vp, c_vp, c_i64, c_i64, c_vp, c_i64, c_int, c_vp],
)

forge_lora_a = _decl(
    "forge_lora_a",
    [c_i64, c_i64, c_i64, c_int, c_vp, c_i64, ctypes.POINTER(c_vp), c_i64, ctypes.POINTER(c_f32), c_vp, c_i64,
     c_vp, c_int, c_vp],
)

forge_lora_a_noalloc = _decl(
    "forge_lora_a_noalloc",
    [c_i64, c_i64, c_i64, c_int, c_vp, c_i64, ctypes.POINTER(c_vp), c_i64, ctypes.POINTER(c_f32), c_vp, c_i64,
     c_int, c_vp],
)
LORA_A_SCRATCH_BYTES = 16 * 1024 * 1024

forge_ce_target_prob = _decl(
    "forge_ce_target_prob", [c_int, c_vp, c_i64, c_i64, c_i64, c_vp, c_i64, c_i64, c_f32, c_vp, c_vp]
)
forge_row_scale = _decl("forge_row_scale", [c_int, c_vp, c_i64, c_i64, c_i64, c_vp, c_vp])
forge_gemm_generic = _decl(
    "forge_gemm_generic",
    [c_i64, c_i64, c_i64, c_int, c_vp, c_i64, c_i64, c_vp, c_i64, c_i64, c_vp, c_i64, c_int, c_f32, c_f32, c_vp, c_int,
     c_vp],
)

forge_rmsnorm_fwd = _decl(
    "forge_rmsnorm_fwd",
    [c_int, c_int, c_int, c_vp, c_i64, c_vp, c_vp, c_i64, c_vp, c_i64, c_i64, ctypes.c_double, ctypes.c_double,
     c_int, c_vp],
)
forge_rmsnorm_bwd = _decl(
    "forge_rmsnorm_bwd",
    [c_int, c_int, c_vp, c_i64, c_vp, c_i64, c_vp, c_vp, c_vp, c_i64, c_vp, c_vp, c_i64, c_i64, ctypes.c_double,
     c_int, c_vp],
)
forge_lora_mlp_gate_up_v = _decl(
    "forge_lora_mlp_gate_up_v",
    [c_i64, c_i64, c_i64, c_i64, c_vp, c_i64, c_vp, c_vp, c_i64, c_vp, c_i64, c_vp, c_vp, c_i64, c_vp, c_vp, c_vp,
     c_i64, c_int, c_vp, c_i64, c_i64, c_vp, c_vp])
forge_lora_mlp_down_bwd_v = _decl(
    "forge_lora_mlp_down_bwd_v",
    [c_i64, c_i64, c_i64, c_i64, c_vp, c_i64, c_vp, c_i64, c_vp, c_i64, c_vp, c_i64, c_vp, c_vp, c_vp, c_i64, c_int,
     c_vp, c_vp, c_i64, c_i64, c_vp, c_vp, c_vp, c_i64, c_vp, c_vp])
forge_lora_qkv_rope_bwd = _decl(
    "forge_lora_qkv_rope_bwd",
    [c_i64, c_i64, c_i64, c_i64, c_i64, c_vp, c_i64, c_vp, c_i64, c_vp, c_i64, c_vp, c_vp, c_i64, c_i64, c_vp,
     c_vp, c_i64, c_vp, c_i64, c_vp, c_vp, c_vp, c_i64, c_i64, c_i64, c_vp, c_i64, c_f32, c_vp])
forge_lora_mlp_glu_bwd = _decl("forge_lora_mlp_glu_bwd", [c_i64, c_i64, c_vp, c_i64, c_vp, c_vp, c_i64, c_vp, c_i64,
                                                          c_int, c_vp])
forge_rmsnorm_bwd_workspace = _decl("forge_rmsnorm_bwd_workspace", [c_int, c_i64, c_i64], c_i64)
forge_zero = _decl("forge_zero", [c_vp, c_i64, c_vp])
forge_copy = _decl("forge_copy", [c_vp, c_vp, c_i64, c_vp])
forge_transpose_2b = _decl("forge_transpose_2b", [c_vp, c_i64, c_i64, c_i64, c_vp, c_i64, c_vp])
forge_transpose_2b_batch = _decl("forge_transpose_2b_batch", [c_int, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp])
TRANSPOSE_BATCH_MAX = 8
forge_cast_f32_bf16 = _decl("forge_cast_f32_bf16", [c_vp, c_i64, c_vp, c_i64, c_i64, c_i64, c_vp])

# Every symbol include/forge_hip.h declares (checked by the CPU test suite).
EXPORTED = [
    "forge_version", "forge_last_error", "forge_arch_ok",
    "forge_swiglu_fwd", "forge_swiglu_bwd", "forge_geglu_fwd", "forge_geglu_bwd", "forge_rope",
    "forge_ce_fwd", "forge_ce_target_stats", "forge_ce_fwd_reduce", "forge_ce_stats_wait", "forge_ce_scale",
    "forge_sum_f32",
    "forge_gemm", "forge_lora_mlp_gate_up", "forge_lora_mlp_gate_up_v", "forge_lora_mlp_down_bwd", "forge_lora_mlp_down_bwd_v", "forge_lora_mlp_glu_bwd",
    "forge_lora_qkv_rope", "forge_lora_qkv_rope_bwd",
    "forge_lora_a", "forge_lora_a_noalloc", "forge_zero", "forge_copy", "forge_cast_f32_bf16", "forge_splitk_reduce",
    "forge_ce_target_prob", "forge_row_scale", "forge_gemm_generic", "forge_transpose_2b", "forge_transpose_2b_batch",
    "forge_rmsnorm_fwd", "forge_rmsnorm_bwd", "forge_rmsnorm_bwd_workspace",
]

# Number of successful library calls (tests use it to prove the HIP path ran).
calls = 0


def check(status: int, what: str) -> None:
    global calls
    if status != 0:
        msg = forge_last_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed (status {status}): {msg}")
    calls += 1


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _TORCH_DTYPE[dtype]
    except KeyError:
        raise TypeError(f"unsupported dtype {dtype}") from None


def stream_of(t: torch.Tensor) -> int:
    """Handle of torch's current stream on t's device (launches are async on
    it).  The raw accessor skips building a Stream object (2 us -> 0.1 us per
    launch on the host)."""
    return torch._C._cuda_getCurrentRawStream(t.device.index)


def ptr(t):
    return None if t is None else t.data_ptr()


def require_gpu(*tensors: torch.Tensor) -> None:
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise RuntimeError("forge_hip kernels need tensors on a ROCm GPU device")
