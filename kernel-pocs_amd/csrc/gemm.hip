// Host launchers for the MFMA GEMM core: the generic forge_gemm entry point
// and the fused LoRA entry points (LoRA-MLP gate/up + SwiGLU / GeGLU, LoRA-MLP
// down-projection backward + SwiGLU / GeGLU backward, LoRA-QKV + RoPE).
#include "gemm_core.h"
#include "gemm_w4.h"

namespace fgemm {

// Tile configurations.
enum Cfg {
  CFG_BIG = 0,       // 256 x 256: 2 x 2 waves (128 x 128 per wave); 4 x 2 on the token-major LDS-DMA path
  CFG_SKINNY_N = 1,  // N <= 32-ish (rank-r outputs): 64 x 64 tiles (2 x 2 waves) for a K-contiguous
                     // A, else 256 x 32 (4 x 1 waves)
  CFG_SKINNY_M = 2,  // 32 x 256, 1 x 4 waves: M <= 32-ish (LoRA A gradients)
  CFG_SKINNY_N64 = 3,  // 32 < N <= 64: 64 x 64 tiles for a K-contiguous A, 256 x 64 for
                       // token-major operands, else 256 x 32
  CFG_NARROW_128 = 4,  // 64 < N <= 128, K-contiguous A: 64 x 128 tiles (2 x 2 waves)
  CFG_NARROW_256 = 5,  // 192 < N <= 256, K-contiguous A: 64 x 256 tiles (2 x 2 waves)
  CFG_NARROW_192 = 6,  // 128 < N <= 192, K-contiguous A: 96 x 192 tiles (3 x 2 waves, 32 x 96 per wave)
};

#ifndef SKINNY_NSTAGE
#define SKINNY_NSTAGE 2
#endif
#ifndef SKINNY_BKT
#define SKINNY_BKT 64
#endif
#ifndef SKINNY_WPE
#define SKINNY_WPE 2
#endif
// cache policy of a buffer load whose data is read once: nontemporal (the NT
// bit, 2, of the gfx950 buffer instruction's cache-policy field)
constexpr int CP_STREAM = 2;

// Column tiles of unequal K work (column-ranged segments of different
// lengths, e.g. [dQ B_q | dK B_k | dV B_v] with K = 4096, 1024, 1024) are
// dispatched heaviest first, so that the long tiles do not start in the last
// round; equal work keeps the default order.
static void order_columns(GemmArgs& a, int64_t out_bn, int64_t tn) {
  a.n_col_order = 0;
  if (tn < 2 || tn > MAX_COL_ORDER) return;
  int64_t work[MAX_COL_ORDER];
  int idx[MAX_COL_ORDER];
  bool uniform = true;
  for (int j = 0; j < tn; ++j) {
    const int64_t lo = j * out_bn, hi = lo + out_bn;
    work[j] = 0;
    for (int s = 0; s < a.n_segs; ++s)
      if (a.segs[s].n_hi > lo && a.segs[s].n_lo < hi) work[j] += a.segs[s].k;
    uniform = uniform && work[j] == work[0];
    idx[j] = j;
  }
  if (uniform) return;
  for (int i = 1; i < tn; ++i)  // stable insertion sort, heaviest first
    for (int j = i; j > 0 && work[idx[j]] > work[idx[j - 1]]; --j) {
      const int t = idx[j];
      idx[j] = idx[j - 1];
      idx[j - 1] = t;
    }
  a.n_col_order = (int)tn;
  for (int j = 0; j < tn; ++j) a.col_order[j] = (uint8_t)idx[j];
}

template <int BM, int BN, int WM, int WN, int AL, int BL, int BMODE, int EPI>
static int launch_cfg(GemmArgs a, hipStream_t s) {
  constexpr int OUT_BN = (BMODE == B_DUAL) ? BN / 2 : BN;
  const int64_t tm = (a.M + BM - 1) / BM;
  const int64_t tn = (a.N + OUT_BN - 1) / OUT_BN;
  if (tm * tn > 0x7fffffffLL) return forge_set_error(FORGE_ERR_INVALID, "gemm: too many tiles");
  order_columns(a, OUT_BN, tn);
  dim3 grid((unsigned)(tm * tn), 1, (unsigned)a.split_k);
  constexpr bool CAN_STAGE = staged_ok(BM, BN, WM, WN, EPI);
  const bool staged = CAN_STAGE && a.ep.vec_ok;
  if constexpr (BM == 256 && BN == 256 && AL == ROW && BL == COL) {
    // both operands K-contiguous: the 4-wave engine (128 x 128 per wave,
    // accumulators in AGPRs, a ring of five LDS half-slots fed by LDS-DMA)
    constexpr bool W4_STAGE = w4_staged_epi(EPI);
    const bool plain = a.ep.beta == 0.f && a.ep.act == ACT_NONE && a.ep.alpha_group == 0;
    if (W4_STAGE && a.ep.vec_ok && (EPI != EPI_STORE_BF16 || plain))
      gemm_w4_kernel<BMODE, EPI, W4_STAGE><<<grid, 256, 0, s>>>(a);
    else
      gemm_w4_kernel<BMODE, EPI, false><<<grid, 256, 0, s>>>(a);
  } else if constexpr (BM == 64 && (BN == 64 || BN == 128 || BN == 256) && AL == ROW &&
                       (BL == COL || BL == ROW) && BMODE == B_SINGLE) {
    // narrow outputs (N <= 256: X A^T, dY B) with A K-contiguous: 64-row
    // tiles as wide as the output (so X streams once) with 4 waves; a 3-stage
    // ring (48 / 72 KB of LDS: three / two workgroups per CU) or, at 64 x 256,
    // two stages in 80 KB (two per CU).  M/64 tiles fill the chip without a
    // split-K pass.  B may be [N][K] or, read with the transposing LDS loads,
    // [K][N] as stored.
    // (measured cold on MI355X: 4 or 5 stages at 64 x 64 were no faster)
    constexpr int NS = BN == 256 ? 2 : 3;
    constexpr int WPE_N = BN == 64 ? 3 : 2;
    // (nontemporal loads of A, read by one column of tiles, measured 0.2% slower)
    gemm_dma_kernel<BM, BN, WM, WN, BMODE, EPI, 64, NS, false, WPE_N, false, BL == ROW>
        <<<grid, WM * WN * 64, 0, s>>>(a);
  } else if constexpr (BM == 96 && BN == 192 && AL == ROW && BL == COL && BMODE == B_SINGLE) {
    // 129..192 output columns (the three stacked rank-64 LoRA-A products of
    // LoRA-QKV): 96-row tiles of 3 x 2 waves and a 3-stage ring (108 KB, one
    // workgroup per CU; 240 tiles at 22954 tokens, one round on 256 CUs),
    // with no padded columns.  Measured cold on MI355X against 64 x 192 tiles
    // with two stages (two workgroups per CU): [22954, 4096] x [4096, 192]
    // 116 -> 94 us, [4096, 4096] x [4096, 192] 78 -> 61 us, bitwise-equal
    // output; 4 stages no faster than 3; 64 x 64 or 64 x 128 tiles slower.
    gemm_dma_kernel<96, 192, 3, 2, BMODE, EPI, 64, 3, false, 2><<<grid, 384, 0, s>>>(a);
  } else if constexpr (AL == COL && BL == ROW && BMODE == B_SINGLE && BM == 256 && BN == 256) {
    // both operands token-major (A^T B reduced over tokens): the LDS-DMA
    // engine with transposing fragment reads, 8 waves as above
    constexpr int DWM = 4, DWN = 2;
    constexpr bool DMA_STAGE = staged_ok(BM, BN, DWM, DWN, EPI);
    if (DMA_STAGE && a.ep.vec_ok)
      gemm_dma_kernel<BM, BN, DWM, DWN, BMODE, EPI, 64, 2, DMA_STAGE, 2, true, true><<<grid, DWM * DWN * 64, 0, s>>>(a);
    else
      gemm_dma_kernel<BM, BN, DWM, DWN, BMODE, EPI, 64, 2, false, 2, true, true><<<grid, DWM * DWN * 64, 0, s>>>(a);
  } else if constexpr (AL == COL && BL == ROW && BMODE == B_SINGLE && ((BM == 256 && BN <= 64) || (BM == 32 && BN == 256))) {
    // skinny token reductions (LoRA weight gradients): as the skinny
    // K-contiguous case, with token-major operands
    // the wide operand (A of 256 x N tiles, B of 32 x 256) is read once, so
    // its loads are nontemporal and leave the caches to the narrow one
    // (LoRA-MLP step 0.35%, LoRA-QKV step 0.7% faster, same box)
    constexpr int CPA_T = BM == 256 ? CP_STREAM : 0, CPB_T = BM == 256 ? 0 : CP_STREAM;
    gemm_dma_kernel<BM, BN, WM, WN, BMODE, EPI, 64, SKINNY_NSTAGE, false, SKINNY_WPE, true, true, CPA_T, CPB_T>
        <<<grid, WM * WN * 64, 0, s>>>(a);
  } else if constexpr (BM == 256 && BN <= 64 && AL == ROW && BL == COL && BMODE == B_SINGLE) {
    // skinny output, K-contiguous operands (X A^T, dY B with B^T given): the
    // big operand streams through the LDS-DMA ring; ~72-80 KB of LDS lets two
    // workgroups share a CU, so two K tiles per CU are in flight
    gemm_dma_kernel<BM, BN, WM, WN, BMODE, EPI, SKINNY_BKT, SKINNY_NSTAGE, false, SKINNY_WPE><<<grid, WM * WN * 64, 0, s>>>(a);
  } else {
    if (staged)
      gemm_kernel<BM, BN, WM, WN, AL, BL, BMODE, EPI, CAN_STAGE><<<grid, WM * WN * 64, 0, s>>>(a);
    else
      gemm_kernel<BM, BN, WM, WN, AL, BL, BMODE, EPI, false><<<grid, WM * WN * 64, 0, s>>>(a);
  }
  FORGE_CHECK_LAUNCH();
  return FORGE_OK;
}

template <int AL, int BL, int BMODE, int EPI>
static int launch_layout(int cfg, const GemmArgs& a, hipStream_t s) {
  switch (cfg) {
    case CFG_BIG: return launch_cfg<256, 256, 2, 2, AL, BL, BMODE, EPI>(a, s);
    case CFG_SKINNY_N:
      if constexpr (BMODE == B_SINGLE) {
        if constexpr (AL == ROW) return launch_cfg<64, 64, 2, 2, AL, BL, BMODE, EPI>(a, s);
        return launch_cfg<256, 32, 4, 1, AL, BL, BMODE, EPI>(a, s);
      }
      break;
    case CFG_NARROW_128:
      if constexpr (BMODE == B_SINGLE && AL == ROW) return launch_cfg<64, 128, 2, 2, AL, BL, BMODE, EPI>(a, s);
      break;
    case CFG_NARROW_256:
      if constexpr (BMODE == B_SINGLE && AL == ROW) return launch_cfg<64, 256, 2, 2, AL, BL, BMODE, EPI>(a, s);
      break;
    case CFG_NARROW_192:  // B as [N][K] only (a 192-wide k-row is not a whole number of transposing reads)
      if constexpr (BMODE == B_SINGLE && AL == ROW && BL == COL) return launch_cfg<96, 192, 3, 2, AL, BL, BMODE, EPI>(a, s);
      break;
    case CFG_SKINNY_M:
      if constexpr (BMODE == B_SINGLE) return launch_cfg<32, 256, 1, 4, AL, BL, BMODE, EPI>(a, s);
      break;
    case CFG_SKINNY_N64:
      if constexpr (BMODE == B_SINGLE) {
        if constexpr (AL == ROW) return launch_cfg<64, 64, 2, 2, AL, BL, BMODE, EPI>(a, s);
        if constexpr (AL == COL && BL == ROW) return launch_cfg<256, 64, 4, 1, AL, BL, BMODE, EPI>(a, s);
        return launch_cfg<256, 32, 4, 1, AL, BL, BMODE, EPI>(a, s);
      }
      break;
  }
  return forge_set_error(FORGE_ERR_UNSUPPORTED, "gemm: tile config %d", cfg);
}

template <int EPI>
static int launch_epi(int cfg, int al, int bl, const GemmArgs& a, hipStream_t s) {
  if (al == ROW && bl == COL) return launch_layout<ROW, COL, B_SINGLE, EPI>(cfg, a, s);
  if (al == ROW && bl == ROW) return launch_layout<ROW, ROW, B_SINGLE, EPI>(cfg, a, s);
  if (al == COL && bl == ROW) return launch_layout<COL, ROW, B_SINGLE, EPI>(cfg, a, s);
  if (al == COL && bl == COL) return launch_layout<COL, COL, B_SINGLE, EPI>(cfg, a, s);
  return forge_set_error(FORGE_ERR_INVALID, "gemm: layout");
}

// GLU epilogues (SwiGLU / GeGLU, forward and backward) on 256 x 256 tiles:
// the forward reads the gate and up weights as one dual B (both [N][K]); the
// backward's W_down may be [K][N] or [N][K].
template <int EPI>
static int launch_glu(int al, int bl, const GemmArgs& a, hipStream_t s) {
  if constexpr (glu_fwd_epi(EPI)) {
    if (al == ROW && bl == COL) return launch_cfg<256, 256, 2, 2, ROW, COL, B_DUAL, EPI>(a, s);
  } else {
    if (al == ROW && bl == ROW) return launch_cfg<256, 256, 2, 2, ROW, ROW, B_SINGLE, EPI>(a, s);
    if (al == ROW && bl == COL) return launch_cfg<256, 256, 2, 2, ROW, COL, B_SINGLE, EPI>(a, s);
  }
  return forge_set_error(FORGE_ERR_UNSUPPORTED, "gemm: epilogue %d with layouts (%d, %d)", EPI, al, bl);
}

// Picks a tile shape from the output shape (a K-contiguous A takes the
// 64-row narrow tiles up to N = 256).
static int pick_cfg(int64_t M, int64_t N, int al, int bl) {
  if (al == ROW && (bl == COL || bl == ROW) && N <= 256 && M > N)
    return N <= 64 ? CFG_SKINNY_N64 : N <= 128 ? CFG_NARROW_128 : (N <= 192 && bl == COL) ? CFG_NARROW_192 : CFG_NARROW_256;
  if (N <= 32 && M > N) return CFG_SKINNY_N;
  if (N <= 64 && M > N) return CFG_SKINNY_N64;
  if (M <= 64 && N > M) return CFG_SKINNY_M;
  return CFG_BIG;
}

// Largest operand pitch (elements of 2 bytes): 256 rows of it span < 2^31 bytes.
constexpr int64_t kMaxLd = (int64_t(1) << 31) / (256 * 2) - 1;

static int check_segs(const GemmArgs& a, int al, int bl) {
  if (a.n_segs < 1 || a.n_segs > MAX_SEGS)
    return forge_set_error(FORGE_ERR_INVALID, "gemm: 1..%d segments", MAX_SEGS);
  for (int i = 0; i < a.n_segs; ++i) {
    const Seg& s = a.segs[i];
    // K-contiguous operands (A ROW, B COL) are fetched in 8-element chunks
    // along K; transposed operands check every k row individually.
    const bool kchunks = (al == ROW) || (bl == COL);
    if (s.k < 0 || (kchunks && s.k % 8 != 0))
      return forge_set_error(FORGE_ERR_INVALID, "gemm: segment %d K=%lld must be a multiple of 8", i,
                             (long long)s.k);
    if (!aligned16(s.a) || (s.b && !aligned16(s.b)) || (s.b2 && !aligned16(s.b2)))
      return forge_set_error(FORGE_ERR_INVALID, "gemm: segment %d operand not 16-byte aligned", i);
    if (s.lda % 8 != 0 || s.ldb % 8 != 0)
      return forge_set_error(FORGE_ERR_INVALID, "gemm: segment %d leading dims must be multiples of 8", i);
    // A lane's operand offset inside a tile is a 32-bit byte offset from the
    // tile's first row (buffer loads): up to 256 rows of the pitch must stay
    // below 2^31 bytes.
    if (s.lda > kMaxLd || s.ldb > kMaxLd)
      return forge_set_error(FORGE_ERR_INVALID, "gemm: segment %d leading dimension above %lld elements", i,
                             (long long)kMaxLd);
  }
  return FORGE_OK;
}

int run(int cfg, int al, int bl, int epi, const GemmArgs& args, hipStream_t s) {
  if (int e = check_segs(args, al, bl)) return e;
  // 16-byte vector epilogue when every buffer it touches allows it
  GemmArgs a = args;
  {
    const EpiArgs& ep = a.ep;
    bool ok = aligned16(ep.c) && ep.ldc % 8 == 0;
    if (ep.e || ep.g) ok = ok && aligned16(ep.e) && aligned16(ep.g) && ep.ld_eg % 8 == 0;
    if (ep.cos || ep.sin)
      ok = ok && aligned16(ep.cos) && aligned16(ep.sin) && ep.cs_ld % 8 == 0 && ep.head_dim % 16 == 0;
    a.ep.vec_ok = ok ? 1 : 0;
  }
  // transposed-operand tiles are fetched as 8-row blocks of 16-byte vectors
  if (al == COL && a.M % 8 != 0)
    return forge_set_error(FORGE_ERR_INVALID, "gemm: A^T layout needs M %% 8 == 0 (M=%lld)", (long long)a.M);
  if (bl == ROW && a.N % 8 != 0)
    return forge_set_error(FORGE_ERR_INVALID, "gemm: [K][N] B layout needs N %% 8 == 0 (N=%lld)", (long long)a.N);
  if (a.M == 0 || a.N == 0) return FORGE_OK;
  if (cfg < 0) cfg = pick_cfg(a.M, a.N, al, bl);
  switch (epi) {
    case EPI_STORE_BF16: return launch_epi<EPI_STORE_BF16>(cfg, al, bl, a, s);
    case EPI_STORE_F32: return launch_epi<EPI_STORE_F32>(cfg, al, bl, a, s);
    case EPI_ATOMIC_F32: return launch_epi<EPI_ATOMIC_F32>(cfg, al, bl, a, s);
    case EPI_SWIGLU_FWD: return launch_glu<EPI_SWIGLU_FWD>(al, bl, a, s);
    case EPI_SWIGLU_BWD: return launch_glu<EPI_SWIGLU_BWD>(al, bl, a, s);
    case EPI_GEGLU_TANH_FWD: return launch_glu<EPI_GEGLU_TANH_FWD>(al, bl, a, s);
    case EPI_GEGLU_TANH_BWD: return launch_glu<EPI_GEGLU_TANH_BWD>(al, bl, a, s);
    case EPI_GEGLU_ERF_FWD: return launch_glu<EPI_GEGLU_ERF_FWD>(al, bl, a, s);
    case EPI_GEGLU_ERF_BWD: return launch_glu<EPI_GEGLU_ERF_BWD>(al, bl, a, s);
    case EPI_ROPE:
      if (al == ROW && bl == COL) return launch_layout<ROW, COL, B_SINGLE, EPI_ROPE>(CFG_BIG, a, s);
      break;
  }
  return forge_set_error(FORGE_ERR_UNSUPPORTED, "gemm: epilogue %d with layouts (%d, %d)", epi, al, bl);
}

}  // namespace fgemm

using namespace fgemm;

extern "C" int forge_gemm(int64_t M, int64_t N, const forge_gemm_segment* segs, int n_segs,
                          int a_layout, int b_layout, void* c, int64_t ldc, int c_dtype,
                          float alpha, float beta, int epilogue, int split_k, void* stream) {
  if (M < 0 || N < 0) return forge_set_error(FORGE_ERR_INVALID, "gemm: negative shape");
  if (n_segs < 1 || n_segs > MAX_SEGS)
    return forge_set_error(FORGE_ERR_INVALID, "gemm: 1..%d segments", MAX_SEGS);
  if (split_k < 1) split_k = 1;
  GemmArgs a = {};
  a.M = M;
  a.N = N;
  a.n_segs = n_segs;
  bool ranged = false;
  int64_t width = 0;  // widest column range of a segment
  for (int i = 0; i < n_segs; ++i) {
    a.segs[i].a = (const __bf16*)segs[i].a;
    a.segs[i].lda = segs[i].lda;
    a.segs[i].b = (const __bf16*)segs[i].b;
    a.segs[i].b2 = nullptr;
    a.segs[i].ldb = segs[i].ldb;
    a.segs[i].k = segs[i].k;
    if (segs[i].n_lo == 0 && segs[i].n_hi == 0) {
      a.segs[i].n_lo = 0;
      a.segs[i].n_hi = N;
    } else {
      if (segs[i].n_lo < 0 || segs[i].n_hi <= segs[i].n_lo || segs[i].n_hi > N)
        return forge_set_error(FORGE_ERR_INVALID, "gemm: segment %d columns [%lld, %lld) outside [0, %lld)", i,
                               (long long)segs[i].n_lo, (long long)segs[i].n_hi, (long long)N);
      a.segs[i].n_lo = segs[i].n_lo;
      a.segs[i].n_hi = segs[i].n_hi;
      ranged = true;
    }
    if (a.segs[i].n_hi - a.segs[i].n_lo > width) width = a.segs[i].n_hi - a.segs[i].n_lo;
  }
  // column-ranged segments: tiles sized for the widest range, so that
  // independent products side by side get tiles of their own
  const int cfg = ranged ? pick_cfg(M, width, a_layout, b_layout) : -1;
  a.split_k = split_k;
  a.ep.c = c;
  a.ep.ldc = ldc;
  a.ep.alpha = alpha;
  a.ep.beta = beta;
  int epi;
  if (epilogue == FORGE_EPI_ATOMIC_F32) {
    if (c_dtype != FORGE_DTYPE_F32)
      return forge_set_error(FORGE_ERR_INVALID, "gemm: atomic epilogue needs an fp32 C");
    epi = EPI_ATOMIC_F32;
  } else if (epilogue == FORGE_EPI_STORE || epilogue == FORGE_EPI_SILU || epilogue == FORGE_EPI_RELU ||
             epilogue == FORGE_EPI_GELU) {
    a.ep.act = epilogue == FORGE_EPI_SILU ? ACT_SILU
             : epilogue == FORGE_EPI_RELU ? ACT_RELU
             : epilogue == FORGE_EPI_GELU ? ACT_GELU : ACT_NONE;
    if (a.ep.act != ACT_NONE && split_k != 1)
      return forge_set_error(FORGE_ERR_INVALID, "gemm: an activation epilogue needs split_k == 1");
    if (c_dtype == FORGE_DTYPE_BF16) {
      if (split_k != 1)
        return forge_set_error(FORGE_ERR_INVALID, "gemm: split_k needs an fp32 C (partials) or the atomic epilogue");
      epi = EPI_STORE_BF16;
    } else if (c_dtype == FORGE_DTYPE_F32) {
      epi = EPI_STORE_F32;
      if (split_k > 1) {  // partial sums: split z owns C[z] = c + z * M * ldc
        if (beta != 0.f) return forge_set_error(FORGE_ERR_INVALID, "gemm: split-K partials need beta == 0");
        a.ep.split_stride = M * ldc;
      }
    } else {
      return forge_set_error(FORGE_ERR_UNSUPPORTED, "gemm: C dtype %d", c_dtype);
    }
  } else {
    return forge_set_error(FORGE_ERR_INVALID, "gemm: epilogue %d", epilogue);
  }
  return run(cfg, a_layout, b_layout, epi, a, (hipStream_t)stream);
}
