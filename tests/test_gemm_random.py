"""Seeded random sweep of forge_gemm against float32 matmuls of the same bf16
operands on the CPU: random M, N, K (every tile configuration and its
partial tiles), both A and B layouts, one to three K segments, column-ranged
segments of unequal K (which reorders the column tiles), fp32 output with
split-K partial slices, bf16 output, alpha and beta."""
import random

import pytest
import torch

from forge_hip import _lib as L


def _case(rng: random.Random, gen: torch.Generator):
    al, bl = rng.choice([0, 0, 0, 1]), rng.choice([1, 1, 1, 0])
    M = rng.choice([rng.randint(1, 300), rng.randint(1, 3000), rng.choice([64, 96, 256, 512, 2048])])
    N = rng.choice([rng.randint(1, 260), rng.randint(1, 900), rng.choice([16, 32, 48, 64, 128, 192, 256, 512])])
    if al == L.LAYOUT_COL:  # A^T tiles are fetched as 8-row blocks
        M = (M + 7) // 8 * 8
    if bl == L.LAYOUT_ROW:  # so are [K][N] B tiles
        N = (N + 7) // 8 * 8
    nseg = rng.choice([1, 1, 2, 3])
    ranged = bl == L.LAYOUT_COL and nseg > 1 and N >= nseg and rng.random() < 0.6
    bounds = [0] + sorted(rng.sample(range(1, N), nseg - 1)) + [N] if ranged else None
    out_f32 = rng.random() < 0.4
    split = rng.choice([1, 1, 2, 3]) if out_f32 else 1
    alpha = rng.choice([1.0, 0.5, 1.75])
    beta = rng.choice([0.0, 0.0, 0.5]) if split == 1 else 0.0
    segs, keep, ref = [], [], torch.zeros(M, N)
    for s in range(nseg):
        K = 8 * rng.randint(1, 128)
        lo, hi = (bounds[s], bounds[s + 1]) if ranged else (0, N)
        A = torch.randn(M, K, generator=gen).to(torch.bfloat16)
        Bt = torch.randn(hi - lo, K, generator=gen).to(torch.bfloat16)  # logical B^T
        a = (A if al == L.LAYOUT_ROW else A.t().contiguous()).cuda()
        b = (Bt if bl == L.LAYOUT_COL else Bt.t().contiguous()).cuda()
        keep += [a, b]
        lda = K if al == L.LAYOUT_ROW else M
        ldb = K if bl == L.LAYOUT_COL else hi - lo
        segs.append(L.GemmSegment(a.data_ptr(), lda, b.data_ptr(), ldb, K, lo if ranged else 0,
                                  hi if ranged else 0))
        ref[:, lo:hi] += A.float() @ Bt.float().t()
    c0 = torch.randn(M, N, generator=gen)
    if out_f32:
        c = c0.clone().cuda() if split == 1 else torch.full((split, M, N), float("nan")).cuda()
        dtype = L.DTYPE_F32
    else:
        c = c0.to(torch.bfloat16).cuda()
        dtype = L.DTYPE_BF16
    arr = (L.GemmSegment * nseg)(*segs)
    L.check(L.forge_gemm(M, N, arr, nseg, al, bl, c.data_ptr(), N, dtype, alpha, beta, L.EPI_STORE, split,
                         L.stream_of(c)), "forge_gemm")
    got = (c.sum(0) if split > 1 else c).float().cpu()
    c_in = c0 if out_f32 else c0.to(torch.bfloat16).float()
    want = alpha * ref + (beta * c_in if beta else 0.0)
    scale = max(1.0, want.abs().max().item())
    err = ((got - want).abs().max() / scale).item()
    tol = 2e-3 if out_f32 else 2e-2
    desc = (f"M={M} N={N} a_layout={al} b_layout={bl} segments={nseg} ranged={ranged} "
            f"fp32={out_f32} split={split} alpha={alpha} beta={beta}")
    return err <= tol, f"{desc}: max error {err:.3e} (tolerance {tol:g} of max |C|)"


@pytest.mark.gpu
@pytest.mark.parametrize("seed", [7, 11, 23])
def test_gemm_random_sweep(seed):
    rng = random.Random(seed)
    gen = torch.Generator().manual_seed(seed)
    bad = []
    for _ in range(100):
        ok, msg = _case(rng, gen)
        if not ok:
            bad.append(msg)
    assert not bad, "\n".join(bad[:10])
