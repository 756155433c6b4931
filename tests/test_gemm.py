"""MFMA GEMM core parity (forge_gemm through the C ABI) vs a float32 matmul
of the same bf16 operands on the CPU.

Covers every operand layout, the tile configurations (big, skinny-N and
the 64 x 64 narrow tiles of K-contiguous products up to N = 256, skinny-M,
and the token-major LDS-DMA variants of each), ragged M/N edges, multi-segment K (the LoRA K-extension), beta,
fp32 output and split-K with the atomic epilogue.  Tolerance: bf16 output
2e-2 relative to the output scale; fp32 output 1e-3 (bf16 inputs, fp32
accumulation, different summation order).
"""
import ctypes

import pytest
import torch

from forge_hip import _lib as L


def _operand(rows, k, layout, gen):
    """Returns (device tensor as stored, logical [rows, k] fp32 CPU matrix)."""
    x = torch.randn(rows, k, generator=gen).to(torch.bfloat16)
    stored = x if layout == L.LAYOUT_ROW else x.t().contiguous()
    return stored.cuda(), x.float()


def _gemm(M, N, segs_host, a_layout, b_layout, c, c_dtype, alpha=1.0, beta=0.0, epi=L.EPI_STORE, split_k=1):
    arr = (L.GemmSegment * len(segs_host))()
    for i, (a, lda, b, ldb, k) in enumerate(segs_host):
        arr[i] = L.GemmSegment(a.data_ptr(), lda, b.data_ptr(), ldb, k)
    L.check(L.forge_gemm(M, N, arr, len(segs_host), a_layout, b_layout, c.data_ptr(), c.stride(0), c_dtype,
                         alpha, beta, epi, split_k, L.stream_of(c)), "forge_gemm")


# B layouts: COL = weight [N][K] (K contiguous), ROW = [K][N]
def _b_operand(n, k, layout, gen):
    w = torch.randn(n, k, generator=gen).to(torch.bfloat16)  # logical B^T = [N][K]
    stored = w if layout == L.LAYOUT_COL else w.t().contiguous()
    return stored.cuda(), w.float().t()  # logical B [K][N]


@pytest.mark.gpu
@pytest.mark.parametrize("M,N,K", [(256, 256, 64), (296, 520, 264), (64, 1000, 136), (1000, 40, 512),
                                   (16, 704, 1024), (2048, 2048, 512), (1000, 192, 264), (1000, 200, 72), (600, 128, 200),
                                   (2000, 160, 520)])
@pytest.mark.parametrize("a_layout", [0, 1])
@pytest.mark.parametrize("b_layout", [0, 1])
def test_gemm_layouts(M, N, K, a_layout, b_layout):
    gen = torch.Generator().manual_seed(M * 7 + N + K)
    a, A = _operand(M, K, a_layout, gen)
    b, B = _b_operand(N, K, b_layout, gen)
    lda = K if a_layout == L.LAYOUT_ROW else M
    ldb = K if b_layout == L.LAYOUT_COL else N
    c = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
    _gemm(M, N, [(a, lda, b, ldb, K)], a_layout, b_layout, c, L.DTYPE_BF16)
    ref = A @ B
    scale = ref.abs().max()
    torch.testing.assert_close(c.float().cpu() / scale, ref / scale, atol=2e-2, rtol=0)
    # fp32 output is tighter
    c32 = torch.empty(M, N, dtype=torch.float32, device="cuda")
    _gemm(M, N, [(a, lda, b, ldb, K)], a_layout, b_layout, c32, L.DTYPE_F32)
    torch.testing.assert_close(c32.cpu(), ref, atol=1e-3 * scale.item(), rtol=1e-3)


@pytest.mark.gpu
def test_gemm_segments_beta_alpha():
    """C = alpha * (A0 B0 + A1 B1) + beta * C with a rank-16 second segment."""
    gen = torch.Generator().manual_seed(5)
    M, N, K0, K1 = 384, 320, 256, 16
    a0, A0 = _operand(M, K0, 0, gen)
    a1, A1 = _operand(M, K1, 0, gen)
    b0, B0 = _b_operand(N, K0, 1, gen)
    b1, B1 = _b_operand(N, K1, 1, gen)
    c0 = torch.randn(M, N, generator=gen)
    c = c0.cuda().contiguous()
    _gemm(M, N, [(a0, K0, b0, K0, K0), (a1, K1, b1, K1, K1)], 0, 1, c, L.DTYPE_F32, alpha=0.5, beta=2.0)
    ref = 0.5 * (A0 @ B0 + A1 @ B1) + 2.0 * c0
    torch.testing.assert_close(c.cpu(), ref, atol=2e-3, rtol=1e-3)


@pytest.mark.gpu
@pytest.mark.parametrize("split,T", [(1, 2048), (4, 2048), (7, 2048), (3, 1001)])
def test_gemm_split_k_atomic(split, T):
    """LoRA-A-gradient shape: [r, H] = T^T @ X with K = tokens (any count)."""
    gen = torch.Generator().manual_seed(split)
    r, H = 16, 512
    t, Tm = _operand(r, T, 1, gen)  # A = T^T stored as [T][r]
    x_stored = torch.randn(T, H, generator=gen).to(torch.bfloat16)
    c = torch.zeros(r, H, dtype=torch.float32, device="cuda")
    _gemm(r, H, [(t, r, x_stored.cuda(), H, T)], 1, 0, c, L.DTYPE_F32, epi=L.EPI_ATOMIC_F32, split_k=split)
    ref = Tm @ x_stored.float()
    torch.testing.assert_close(c.cpu(), ref, atol=1e-3 * ref.abs().max().item(), rtol=1e-3)


@pytest.mark.gpu
@pytest.mark.parametrize("N,ldc,b_layout", [(300, 304, 1), (300, 301, 1), (512, 520, 1), (512, 520, 0),
                                            (304, 304, 0)])  # a [K][N] B (layout 0) needs N % 8 == 0
def test_gemm_bf16_epilogue_paths(N, ldc, b_layout):
    """bf16 output through the staged (LDS, 16-byte vector) epilogue and the
    per-element one: an N tail that is not a multiple of 8 (scalar tail of the
    staged path), an output pitch that is not a multiple of 8 (per-element
    path), alpha and beta (C read back) on both, untouched padding columns."""
    gen = torch.Generator().manual_seed(N + ldc)
    M, K = 520, 192
    a, A = _operand(M, K, 0, gen)
    b, B = _b_operand(N, K, b_layout, gen)
    ldb = K if b_layout == 1 else N
    c0 = torch.randn(M, ldc, generator=gen).to(torch.bfloat16)
    buf = c0.cuda()
    c = buf[:, :N]
    _gemm(M, N, [(a, K, b, ldb, K)], 0, b_layout, c, L.DTYPE_BF16, alpha=0.75, beta=0.5)
    ref = 0.75 * (A @ B) + 0.5 * c0[:, :N].float()
    scale = ref.abs().max()
    torch.testing.assert_close(c.float().cpu() / scale, ref / scale, atol=2e-2, rtol=0)
    assert torch.equal(buf[:, N:].cpu(), c0[:, N:])


def test_gemm_rejects_bad_segments_without_gpu():
    """Argument validation happens on the host before any launch."""
    seg = (L.GemmSegment * 1)()
    seg[0] = L.GemmSegment(16, 8, 16, 8, 12)  # K not a multiple of 8 with a K-contiguous A
    rc = L.forge_gemm(8, 8, seg, 1, 0, 1, 16, 8, L.DTYPE_BF16, 1.0, 0.0, L.EPI_STORE, 1, None)
    assert rc == 1 and b"multiple of 8" in L.forge_last_error()
    rc = L.forge_gemm(8, 8, seg, 0, 0, 1, 16, 8, L.DTYPE_BF16, 1.0, 0.0, L.EPI_STORE, 1, None)
    assert rc == 1


@pytest.mark.gpu
@pytest.mark.parametrize("dtype,code", [(torch.float32, 0), (torch.bfloat16, 2)])
@pytest.mark.parametrize("rows,cols,n_split", [(37, 52, 5), (16, 14336, 9), (3, 7, 1)])
def test_splitk_reduce_sums_partials_in_order(dtype, code, rows, cols, n_split):
    """forge_splitk_reduce: alpha * sum over split slices, fixed order,
    rounded once; both the 4-wide and the scalar paths (cols % 4)."""
    gen = torch.Generator().manual_seed(rows * cols + n_split)
    parts = torch.randn(n_split, rows, cols, generator=gen)
    out = torch.empty(rows, cols, dtype=dtype, device="cuda")
    p = parts.cuda()
    L.check(L.forge_splitk_reduce(p.data_ptr(), rows * cols, n_split, rows, cols, cols, out.data_ptr(), cols, code,
                                  0.5, L.stream_of(p)), "forge_splitk_reduce")
    acc = torch.zeros(rows, cols)
    for z in range(n_split):
        acc = acc + parts[z]
    ref = (0.5 * acc).to(dtype)
    assert torch.equal(out.cpu(), ref)


@pytest.mark.gpu
def test_gemm_split_k_partials_match_single_pass():
    """EPI_STORE with an fp32 C and split_k > 1 writes one partial slice per
    split; their sum equals the unsplit product."""
    gen = torch.Generator().manual_seed(11)
    M, N, K, split = 1024, 32, 2048, 6
    a, A = _operand(M, K, 0, gen)
    b, B = _b_operand(N, K, 1, gen)
    parts = torch.empty(split, M, N, dtype=torch.float32, device="cuda")
    _gemm(M, N, [(a, K, b, K, K)], 0, 1, parts.view(split * M, N), L.DTYPE_F32, split_k=split)
    ref = A @ B
    torch.testing.assert_close(parts.sum(0).cpu(), ref, atol=1e-3 * ref.abs().max().item(), rtol=1e-3)


@pytest.mark.gpu
@pytest.mark.parametrize("a_layout,b_layout,N,ldc", [(0, 1, 520, 520), (0, 1, 300, 304), (0, 1, 300, 301),
                                                     (1, 0, 520, 520), (1, 0, 296, 304), (1, 0, 296, 301)])
def test_gemm_fp32_beta_epilogue(a_layout, b_layout, N, ldc):
    """fp32 C with beta (the staged 16-byte epilogue when the pitch allows,
    the per-element one otherwise) on both engines (LDS-DMA for A ROW x B COL,
    register path for A^T x [K][N] B)."""
    gen = torch.Generator().manual_seed(21)
    M, K = 296, 264
    a, af = _operand(M, K, a_layout, gen)
    b, bf = _b_operand(N, K, b_layout, gen)
    c0 = torch.randn(M, ldc, generator=gen)
    c = c0.cuda()
    lda = a.shape[1]
    ldb = b.shape[1]
    _gemm(M, N, [(a, lda, b, ldb, K)], a_layout, b_layout, c, L.DTYPE_F32, alpha=0.5, beta=-1.5)
    ref = 0.5 * (af @ bf) - 1.5 * c0[:, :N]
    torch.testing.assert_close(c[:, :N].cpu(), ref, rtol=1e-3, atol=1e-3 * float(ref.abs().max()))
    assert torch.equal(c[:, N:].cpu(), c0[:, N:])  # pitch padding untouched


@pytest.mark.gpu
@pytest.mark.parametrize("rows,cols,ld_in,ld_out", [(64, 64, 64, 64), (300, 1003, 1008, 304), (7, 129, 129, 9),
                                                    (4096, 1024, 1024, 4096), (130, 1000, 1000, 136),
                                                    (200, 1030, 1040, 208), (1024, 4096, 4104, 1032)])
def test_transpose_2b(rows, cols, ld_in, ld_out):
    """dst = src^T for 2-byte elements: the 64 x 64 tile kernel (small or
    unaligned cases) and the 64 x 256 one with transposing LDS reads (aligned
    cases of 2^16 elements and more, partial tiles in both dimensions and
    rows not a multiple of 8); pitch padding untouched."""
    gen = torch.Generator().manual_seed(4)
    src = torch.randn(rows, ld_in, generator=gen).to(torch.bfloat16).cuda()
    dst = torch.full((cols, ld_out), 7.0, dtype=torch.bfloat16).cuda()
    L.check(L.forge_transpose_2b(src.data_ptr(), ld_in, rows, cols, dst.data_ptr(), ld_out, L.stream_of(src)),
            "forge_transpose_2b")
    assert torch.equal(dst[:, :rows].cpu(), src[:, :cols].t().cpu())
    assert bool((dst[:, rows:] == 7.0).all())  # pitch padding untouched


@pytest.mark.gpu
def test_transpose_2b_batch_matches_single_transposes():
    """One launch, matrices of different shapes, pitches and alignments (a
    zero-size one included); every output equals src^T and pitch padding is
    untouched."""
    import ctypes

    gen = torch.Generator().manual_seed(5)
    shapes = [(16, 14336, 14336, 16), (4096, 64, 64, 4096), (7, 129, 130, 9), (0, 5, 5, 0), (300, 1003, 1008, 304),
              (64, 64, 64, 64)]
    srcs = [torch.randn(r, ldi, generator=gen).to(torch.bfloat16).cuda() for r, _, ldi, _ in shapes]
    dsts = [torch.full((c, max(ldo, 1)), 7.0, dtype=torch.bfloat16).cuda() for _, c, _, ldo in shapes]
    n = len(shapes)
    arr = lambda t, vals: (t * n)(*vals)  # noqa: E731
    L.check(L.forge_transpose_2b_batch(
        n, arr(ctypes.c_void_p, [s.data_ptr() for s in srcs]), arr(ctypes.c_int64, [s[2] for s in shapes]),
        arr(ctypes.c_int64, [s[0] for s in shapes]), arr(ctypes.c_int64, [s[1] for s in shapes]),
        arr(ctypes.c_void_p, [d.data_ptr() for d in dsts]), arr(ctypes.c_int64, [s[3] for s in shapes]),
        L.stream_of(srcs[0])), "forge_transpose_2b_batch")
    for (r, c, _, ldo), s, d in zip(shapes, srcs, dsts):
        assert torch.equal(d[:, :r].cpu(), s[:, :c].t().cpu())
        assert bool((d[:, r:] == 7.0).all())


def test_transpose_2b_batch_rejects_bad_arguments_without_gpu():
    import ctypes

    one = lambda t, v: (t * 1)(v)  # noqa: E731
    rc = L.forge_transpose_2b_batch(9, None, None, None, None, None, None, None)
    assert rc == 1 and b"matrices" in L.forge_last_error()
    rc = L.forge_transpose_2b_batch(1, one(ctypes.c_void_p, 16), one(ctypes.c_int64, 4), one(ctypes.c_int64, 8),
                                    one(ctypes.c_int64, 8), one(ctypes.c_void_p, 16), one(ctypes.c_int64, 8), None)
    assert rc == 1 and b"pitch" in L.forge_last_error()


@pytest.mark.gpu
@pytest.mark.parametrize("M,r,split", [(2048, 16, 1), (2048, 16, 4), (300, 64, 1), (700, 64, 2), (1000, 8, 3)])
def test_gemm_column_ranged_segments(M, r, split):
    """Independent products side by side in one launch: out[:, p r:(p+1) r] =
    A_p B_p^T with a different K per product (segments restricted to their
    columns), against float32 matmuls of the same bf16 operands; with split-K
    the fp32 partials are summed by forge_splitk_reduce.  At r = 64 each
    product has column tiles of its own, dispatched heaviest first (K = 512,
    136, 128: a reordered grid)."""
    gen = torch.Generator().manual_seed(6)
    Ks = [512, 128, 136]
    As = [torch.randn(M, k, generator=gen).to(torch.bfloat16) for k in Ks]
    Bs = [torch.randn(r, k, generator=gen).to(torch.bfloat16) for k in Ks]  # B^T [r][K] (layout COL)
    N = r * len(Ks)
    segs = (L.GemmSegment * len(Ks))()
    dA, dB = [a.cuda() for a in As], [b.cuda() for b in Bs]
    for p, (a, b, k) in enumerate(zip(dA, dB, Ks)):
        segs[p] = L.GemmSegment(a.data_ptr(), k, b.data_ptr(), k, k, p * r, (p + 1) * r)
    ref = torch.cat([a.float() @ b.float().t() for a, b in zip(As, Bs)], 1)
    if split == 1:
        c = torch.zeros(M, N, dtype=torch.bfloat16).cuda()
        L.check(L.forge_gemm(M, N, segs, len(Ks), L.LAYOUT_ROW, L.LAYOUT_COL, c.data_ptr(), N, L.DTYPE_BF16, 1.0,
                             0.0, L.EPI_STORE, 1, L.stream_of(c)), "forge_gemm")
        got = c.float().cpu()
    else:
        parts = torch.empty(split, M, N).cuda()
        L.check(L.forge_gemm(M, N, segs, len(Ks), L.LAYOUT_ROW, L.LAYOUT_COL, parts.data_ptr(), N, L.DTYPE_F32,
                             1.0, 0.0, L.EPI_STORE, split, L.stream_of(parts)), "forge_gemm")
        got = parts.sum(0).cpu()
    scale = ref.abs().max()
    torch.testing.assert_close(got / scale, ref / scale, atol=2e-2, rtol=0)


def test_gemm_rejects_pitches_beyond_32bit_tile_offsets_without_gpu():
    """Operand offsets inside a tile are 32-bit: a pitch whose 256 rows reach
    2^31 bytes is refused before any launch instead of reading wrong rows."""
    limit = (1 << 31) // (256 * 2) - 1
    seg = (L.GemmSegment * 1)()
    seg[0] = L.GemmSegment(16, limit - limit % 8 + 8, 16, 64, 64)  # lda just above the limit
    rc = L.forge_gemm(64, 64, seg, 1, 0, 1, 16, 64, L.DTYPE_BF16, 1.0, 0.0, L.EPI_STORE, 1, None)
    assert rc == 1 and b"leading dimension above" in L.forge_last_error()
    seg[0] = L.GemmSegment(16, 64, 16, limit - limit % 8 + 8, 64)  # ldb
    rc = L.forge_gemm(64, 64, seg, 1, 0, 1, 16, 64, L.DTYPE_BF16, 1.0, 0.0, L.EPI_STORE, 1, None)
    assert rc == 1 and b"leading dimension above" in L.forge_last_error()


def test_gemm_rejects_bad_column_ranges_without_gpu():
    seg = (L.GemmSegment * 1)()
    seg[0] = L.GemmSegment(16, 8, 16, 8, 8, 4, 40)  # [4, 40) outside N = 32
    rc = L.forge_gemm(64, 32, seg, 1, 0, 1, 16, 32, L.DTYPE_BF16, 1.0, 0.0, L.EPI_STORE, 1, None)
    assert rc == 1 and b"columns" in L.forge_last_error()
    seg[0] = L.GemmSegment(16, 8, 16, 8, 8, 8, 8)  # empty range with n_lo != 0
    rc = L.forge_gemm(64, 32, seg, 1, 0, 1, 16, 32, L.DTYPE_BF16, 1.0, 0.0, L.EPI_STORE, 1, None)
    assert rc == 1
