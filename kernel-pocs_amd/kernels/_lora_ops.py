"""Host-side helpers shared by the LoRA-MLP and LoRA-QKV modules.

Thin wrappers over the MFMA GEMM entry points of libforge_hip.so
(csrc/gemm.hip, csrc/lora.hip).  Operands are bf16 with unit stride in the
last dimension and 16-byte aligned rows; every wrapper checks that and calls
the library on torch's current stream.  Every product, the plain base-weight
ones included (which the reference sends to cuBLAS,
kernels/lora_mlp/experiments/v6/lora_mlp_kernel_v6.py:374-443, 650-652), is
the library's own gfx950 GEMM.

Caches: frozen_t keeps one W^T per frozen base weight and frozen_cat one
stacked copy per weight triple (the LoRA-QKV v4 save contract).  An entry is
rebuilt when its weight is freed, modified through autograd-visible
in-place ops (tensor._version) or given new storage (data_ptr).  Writes
that bypass both (``w.data.copy_(...)``, ``w.data += delta``) are invisible
to that check: call clear_caches() after them.
"""
from __future__ import annotations

import ctypes
import weakref
from typing import Optional, Sequence, Tuple

import torch

from forge_hip import _lib as L

ROW, COL = L.LAYOUT_ROW, L.LAYOUT_COL


def as_operand(t: torch.Tensor) -> torch.Tensor:
    """A 2-D bf16 operand the kernels can read: unit last stride, row pitch a
    multiple of 8 elements, 16-byte aligned base.  Copies only if needed."""
    if t.dtype != torch.bfloat16:
        raise TypeError(f"LoRA kernels compute in bf16, got {t.dtype}")
    if t.dim() != 2:
        t = t.reshape(-1, t.shape[-1])
    ok = t.stride(-1) == 1 and (t.shape[0] <= 1 or t.stride(0) % 8 == 0) and t.data_ptr() % 16 == 0
    return t if ok else t.contiguous()


def ld(t: torch.Tensor) -> int:
    return t.stride(0) if t.dim() == 2 and t.shape[0] > 1 else t.shape[-1]


def skinny_split(M: int, N: int, K: int, k_contiguous: bool = True) -> int:
    """Split-K factor for a skinny output.  A K-contiguous A (k_contiguous)
    runs on 64-row tiles as wide as the output (64, 128 or 256 columns): with >= 256
    of them (one per CU) no split is needed, the fp32 partial pass would only
    add traffic; fewer tiles split K towards ~512 workgroups.  Token-major
    operands run on 256 x 32 / 256 x 64 tiles, which alone give only M/256
    workgroups per column tile: aim for ~512 (two workgroups on each of the
    256 CUs)."""
    k_tiles = max(1, (K + 63) // 64)
    if k_contiguous:
        tile_n = 64 if N <= 64 else 128 if N <= 128 else 192 if N <= 192 else 256  # (B as [N][K])
        tiles = max(1, (M + 63) // 64) * max(1, (N + tile_n - 1) // tile_n)
        if tiles >= 256:
            return 1
    else:
        tile_n = 32 if N <= 32 else 64
        tiles = max(1, (M + 255) // 256) * max(1, (N + tile_n - 1) // tile_n)
    return max(1, min(16, -(-512 // tiles), k_tiles // 4))


def _segments(segs) -> ctypes.Array:
    """forge_gemm_segment array from (A, lda, B, ldb, K) tuples, optionally
    extended by (n_lo, n_hi): the output columns the segment applies to."""
    arr = (L.GemmSegment * len(segs))()
    for i, sg in enumerate(segs):
        a, lda, b, ldb, k = sg[:5]
        n_lo, n_hi = (int(sg[5]), int(sg[6])) if len(sg) > 5 else (0, 0)
        arr[i] = L.GemmSegment(a.data_ptr(), int(lda), b.data_ptr(), int(ldb), int(k), n_lo, n_hi)
    return arr


def gemm(M: int, N: int, segs: Sequence[Tuple[torch.Tensor, int, torch.Tensor, int, int]], a_layout: int,
         b_layout: int, out: Optional[torch.Tensor] = None, alpha: float = 1.0, beta: float = 0.0,
         out_dtype=torch.bfloat16, atomic: bool = False, split_k: int = 1, device=None) -> torch.Tensor:
    """C[M, N] = alpha * sum_s A_s @ B_s (+ beta C).  segs: (A, lda, B, ldb, K),
    or (A, lda, B, ldb, K, n_lo, n_hi) for a segment that applies to output
    columns [n_lo, n_hi) only (B's first row is column n_lo).  atomic=True accumulates into a zero-initialised fp32 C over split_k
    K partitions.  A skinny bf16 output (N <= 64, beta = 0) is split over K
    into fp32 partial slices, then summed in a fixed order and rounded."""
    dev = device if device is not None else segs[0][0].device
    K = sum(int(sg[4]) for sg in segs)
    if not atomic and beta == 0.0 and N <= 64 and M >= 1024 and (out is None or out.dtype == torch.bfloat16):
        split = skinny_split(M, N, K, a_layout == ROW)
        if split > 1:
            if out is None:
                out = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
            return split_gemm(M, N, segs, a_layout, b_layout, split, out, alpha, dev)
    if out is None:
        if atomic:
            out = torch.empty(M, N, dtype=torch.float32, device=dev)
            L.check(L.forge_zero(out.data_ptr(), out.numel() * 4, L.stream_of(out)), "forge_zero")
        else:
            out = torch.empty(M, N, dtype=out_dtype, device=dev)
    arr = _segments(segs)
    c_dtype = L.DTYPE_F32 if out.dtype == torch.float32 else L.DTYPE_BF16
    L.check(
        L.forge_gemm(M, N, arr, len(segs), a_layout, b_layout, out.data_ptr(), ld(out), c_dtype, float(alpha),
                     float(beta), L.EPI_ATOMIC_F32 if atomic else L.EPI_STORE, int(split_k), L.stream_of(out)),
        "forge_gemm",
    )
    return out


def split_gemm(M: int, N: int, segs, a_layout: int, b_layout: int, split: int, out: torch.Tensor,
               alpha: float = 1.0, device=None) -> torch.Tensor:
    """out = alpha * sum_s A_s @ B_s with K split `split` ways: each split
    writes fp32 partials to its slice of a [split, M, N] workspace and
    forge_splitk_reduce sums them in a fixed order (deterministic) and rounds
    once to out's dtype."""
    dev = device if device is not None else out.device
    parts = torch.empty(split, M, N, dtype=torch.float32, device=dev)
    arr = _segments(segs)
    st = L.stream_of(parts)
    L.check(L.forge_gemm(M, N, arr, len(segs), a_layout, b_layout, parts.data_ptr(), N, L.DTYPE_F32, float(alpha),
                         0.0, L.EPI_STORE, int(split), st), "forge_gemm")
    L.check(L.forge_splitk_reduce(parts.data_ptr(), M * N, int(split), M, N, N, out.data_ptr(), ld(out),
                                  L.dtype_code(out.dtype), 1.0, st), "forge_splitk_reduce")
    return out


def pad_rank(A: Optional[torch.Tensor], B: Optional[torch.Tensor]):
    """Zero-pads a LoRA pair (A [r, K], B [N, r]) to the next rank that is a
    multiple of 8, which the MFMA core's K segments need.  The added rows of
    A and columns of B are zero, so every product and every gradient of the
    original rows / columns is unchanged (the extra terms add exact zeros)."""
    if A is None or B is None or A.shape[0] % 8 == 0:
        return A, B
    extra = -A.shape[0] % 8
    return torch.nn.functional.pad(A, (0, 0, 0, extra)), torch.nn.functional.pad(B, (0, extra))


def _row_stacked(mats: Sequence[torch.Tensor]) -> bool:
    """True when mats are consecutive row blocks of one buffer (same pitch)."""
    r, pitch, base = mats[0].shape[0], ld(mats[0]), mats[0].data_ptr()
    return all(ld(a) == pitch and a.data_ptr() == base + p * r * pitch * a.element_size()
               for p, a in enumerate(mats))


def lora_a(x: torch.Tensor, mats: Sequence[torch.Tensor], scales: Sequence[float],
           out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """[s_p * x @ A_p^T for p] concatenated along columns -> [M, n*r] bf16."""
    M, K = x.shape
    r = mats[0].shape[0]
    n = len(mats)
    mats = [as_operand(a) for a in mats]
    if n > 1 and not _row_stacked(mats):
        # one [n r, K] buffer (contiguous: A_p is rows p r .. p r + r - 1):
        # the kernel then streams x once per column tile
        stack = torch.cat([a.detach() for a in mats], 0)
        lda = ld(stack)
        addrs = [stack.data_ptr() + p * r * lda * stack.element_size() for p in range(n)]
    else:
        lda = ld(mats[0])
        addrs = [a.data_ptr() for a in mats]
    if out is None:
        out = torch.empty(M, n * r, dtype=torch.bfloat16, device=x.device)
    ptrs = (ctypes.c_void_p * n)(*addrs)
    sc = (ctypes.c_float * n)(*[float(s) for s in scales])
    split = skinny_split(M, n * r, K) if M >= 1024 else 1
    work = torch.empty(split, M, n * r, dtype=torch.float32, device=x.device) if split > 1 else None
    L.check(
        L.forge_lora_a(M, K, r, n, x.data_ptr(), ld(x), ptrs, lda, sc, out.data_ptr(), ld(out),
                       L.ptr(work), split, L.stream_of(x)),
        "forge_lora_a",
    )
    return out


_T_CACHE = {}


def frozen_t(w: torch.Tensor, pitch_multiple: int = 1) -> torch.Tensor:
    """Contiguous W^T of a frozen base weight, kept for the weight's lifetime.

    The backward GEMMs contract over the weight's output dimension, which is
    not contiguous in the nn.Linear layout; with W^T they become K-contiguous
    and run on the LDS-DMA engine.  The copy is made once per weight (LoRA
    freezes the base weights) and dropped when the weight is freed, changed
    in place (tensor._version) or given new storage (data_ptr).
    pitch_multiple > 1 returns [in, out_pad] with out_pad the next multiple
    (columns past `out` are zero), for GEMMs that read K in 8-element chunks.
    """
    key = (id(w), pitch_multiple)
    ent = _T_CACHE.get(key)
    if ent is not None:
        ref, ver, ptr, wt = ent
        if ref() is w and ver == w._version and ptr == w.data_ptr():
            return wt
    n_out = w.shape[0]
    pad = -(-n_out // pitch_multiple) * pitch_multiple
    if pad == n_out:
        wt = w.detach().t().contiguous()
    else:
        wt = torch.zeros(w.shape[1], pad, dtype=w.dtype, device=w.device)
        wt[:, :n_out].copy_(w.detach().t())

    def _drop(_ref, key=key):
        _T_CACHE.pop(key, None)

    _T_CACHE[key] = (weakref.ref(w, _drop), w._version, w.data_ptr(), wt)
    return wt


_CAT_CACHE = {}


def clear_caches() -> None:
    """Drops every cached W^T (frozen_t) and stacked weight copy
    (frozen_cat).  Needed after a write to a frozen base weight that
    autograd does not see (through ``.data``: checkpoint loads, PEFT-style
    merges); the next call rebuilds the copies from the current weights."""
    _T_CACHE.clear()
    _CAT_CACHE.clear()


def frozen_cat(ws: Sequence[torch.Tensor]) -> torch.Tensor:
    """torch.cat(ws, 0) of frozen base weights, kept like frozen_t: made once
    and reused while every weight is alive, unmodified (tensor._version) and
    on the same storage (data_ptr)."""
    key = tuple(id(w) for w in ws)
    ent = _CAT_CACHE.get(key)
    if ent is not None:
        refs, vers, ptrs, cat = ent
        if all(r() is w and v == w._version and p == w.data_ptr() for r, v, p, w in zip(refs, vers, ptrs, ws)):
            return cat
    cat = torch.cat([w.detach() for w in ws], 0)

    def _drop(_ref, key=key):
        _CAT_CACHE.pop(key, None)

    _CAT_CACHE[key] = (tuple(weakref.ref(w, _drop) for w in ws), tuple(w._version for w in ws),
                       tuple(w.data_ptr() for w in ws), cat)
    return cat


def small_t(a: torch.Tensor) -> torch.Tensor:
    """A^T contiguous for a rank-r LoRA matrix (r x features: a few hundred KB)."""
    return a.detach().t().contiguous()


def small_t_batch(mats: Sequence[torch.Tensor]) -> list:
    """small_t of each 2-byte matrix in one launch (forge_transpose_2b_batch)
    instead of one copy kernel each; the transposes share one buffer."""
    if len(mats) > L.TRANSPOSE_BATCH_MAX or any(m.dtype != torch.bfloat16 or m.dim() != 2 for m in mats):
        return [small_t(m) for m in mats]
    mats = [as_operand(m.detach()) for m in mats]
    sizes = [m.numel() for m in mats]
    # each transposed matrix starts on a 16-byte boundary of the shared buffer
    offs, o = [], 0
    for n in sizes:
        offs.append(o)
        o += -(-n // 8) * 8
    buf = torch.empty(o, dtype=mats[0].dtype, device=mats[0].device)
    outs = [buf[off:off + n].view(m.shape[1], m.shape[0]) for off, n, m in zip(offs, sizes, mats)]
    k = len(mats)
    src = (ctypes.c_void_p * k)(*[m.data_ptr() for m in mats])
    dst = (ctypes.c_void_p * k)(*[t.data_ptr() for t in outs])
    ld_src = (ctypes.c_int64 * k)(*[ld(m) for m in mats])
    rows = (ctypes.c_int64 * k)(*[m.shape[0] for m in mats])
    cols = (ctypes.c_int64 * k)(*[m.shape[1] for m in mats])
    ld_dst = (ctypes.c_int64 * k)(*[m.shape[0] for m in mats])
    L.check(L.forge_transpose_2b_batch(k, src, ld_src, rows, cols, dst, ld_dst, L.stream_of(buf)),
            "forge_transpose_2b_batch")
    return outs


def times_b(x: torch.Tensor, ldx: int, b: torch.Tensor, k: int, out: Optional[torch.Tensor] = None,
            alpha: float = 1.0, b_t: Optional[torch.Tensor] = None) -> torch.Tensor:
    """alpha * x @ b for a rank-r LoRA B [k, r], from a transposed copy
    B^T [r, k] (a few hundred KB; b_t if the caller made it already): with
    both operands K-contiguous the narrow tiles stream x faster than when
    they read B [k][r] as stored (measured cold on MI355X: [8192, 14336] x
    [14336, 16] 68.5 -> 51.1 us, [22954, 4096] x [4096, 64] 70.0 -> 52.8 us)."""
    M = x.shape[0]
    bt = b_t if b_t is not None else small_t(b)
    return gemm(M, b.shape[1], [(x, ldx, bt, k, k)], ROW, COL, out=out, alpha=alpha)


def split_k_for(k: int, tiles: int, target_wgs: int = 512, min_tiles_per_split: int = 4) -> int:
    """Split count for a reduction over k (= tokens) with `tiles` output tiles:
    aim for ~target_wgs workgroups, keep >= min_tiles_per_split K-tiles each."""
    k_tiles = max(1, (k + 63) // 64)
    split = max(1, min(target_wgs // max(1, tiles), k_tiles // min_tiles_per_split))
    return split


def grad_at_b(a_t: torch.Tensor, lda: int, b: torch.Tensor, ldb: int, rows: int, cols: int, k: int,
              alpha: float = 1.0, out_dtype=torch.float32) -> torch.Tensor:
    """alpha * A^T @ B where A is stored [k][rows] and B [k][cols] (both
    row-major over the reduction dim k): the LoRA weight-gradient shape
    (rank x features or features x rank, reduced over tokens).  Split over k
    into fp32 partials, reduced in a fixed order, returned as [rows, cols] in
    out_dtype (rounded once)."""
    tiles_m = max(1, (rows + 255) // 256) if rows > 64 else 1
    tiles_n = max(1, (cols + 255) // 256) if cols > 64 else 1
    # 256 x 256 tiles (both sides > 64) run one workgroup per CU, the skinny
    # token-major tiles two: aim for ~1 resp. ~2 workgroups per CU (measured
    # cold: [192, 4096] over 22954 tokens 113 us at 32 splits, 86 us at 16)
    big = rows > 64 and cols > 64
    split = split_k_for(k, tiles_m * tiles_n, target_wgs=256 if big else 512)
    out = torch.empty(rows, cols, dtype=out_dtype, device=a_t.device)
    return split_gemm(rows, cols, [(a_t, lda, b, ldb, k)], COL, ROW, split, out, alpha)


def grad_at_b_group(pairs: Sequence[Tuple[torch.Tensor, int, torch.Tensor, int, int]], r: int, k: int,
                    alpha: float = 1.0) -> list:
    """[alpha * D_p^T @ U_p for each pair] (each [w_p, r] bf16), where U_p is
    stored [k][r] (pitch ldu) and D_p [k][w_p] (pitch ldd), both token-major:
    the LoRA B gradients of one backward in one launch.  Computed transposed,
    out^T [r, sum w_p] = [U_p^T D_p], as one product with column-ranged
    segments split over k (fp32 partials, fixed-order reduction, one
    rounding), then the blocks transposed in one launch (measured cold on
    MI355X, the three LoRA-QKV B gradients at T = 22954, r = 64: 138 -> 82 us
    against a launch per projection).  pairs: (U_p, ldu, D_p, ldd, w_p)."""
    widths = [int(p[4]) for p in pairs]
    N = sum(widths)
    dev = pairs[0][0].device
    split = split_k_for(k, ((r + 31) // 32) * ((N + 255) // 256), target_wgs=512)
    segs, lo = [], 0
    for (u, ldu, d, ldd, w) in pairs:
        segs.append((u, ldu, d, ldd, k, lo, lo + w))
        lo += w
    out_t = torch.empty(r, N, dtype=torch.bfloat16, device=dev)
    split_gemm(r, N, segs, COL, ROW, split, out_t, alpha)
    blocks, lo = [], 0
    for w in widths:
        blocks.append(out_t[:, lo:lo + w])
        lo += w
    return small_t_batch(blocks)
