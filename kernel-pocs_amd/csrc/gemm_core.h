// bf16 MFMA GEMM core for gfx950 (CDNA4), fp32 accumulation.
//
// C[M, N] = sum over K-segments s of A_s[M, K_s] @ B_s[K_s, N], with a fused
// epilogue.  Multi-segment K is how the LoRA terms ride along the base GEMM:
//     X W^T + s (X A^T) B^T  =  [X | s X A^T] @ [W | B]^T
// so the rank-r update costs one extra (zero-padded) K tile instead of a
// separate kernel and another pass over the output.
//
// Tiling: BM x BN x 64 block tile, WAVES_M x WAVES_N waves, each wave owns a
// (BM/WAVES_M) x (BN/WAVES_N) sub-tile computed with v_mfma_f32_32x32x16_bf16.
// Two main loops feed the same MFMA core:
//   * gemm_dma_kernel (256 x 256 tiles, both operands K-contiguous: X W^T and
//     its LoRA segments, the SwiGLU-dual and RoPE GEMMs): global -> LDS by
//     LDS-DMA (buffer_load ... lds, no VGPR staging, no ds_write), XOR-swizzled
//     unpadded LDS rows, a 2-stage ring (measured on MI355X: 918 -> 1018
//     TFLOP/s on the 8192 x 28672 x 4096 gate/up GEMM; a 4-stage ring of
//     32-deep tiles and an interleaved DMA issue were no faster).  It runs
//     8 waves (4 x 2, 64 x 128 per wave) so that each SIMD holds two waves
//     whose MFMA chains cover each other's LDS reads and barriers (measured:
//     the 8192 x 4096 x 14336 down-projection 1075 -> 1213 TFLOP/s);
//   * gemm_kernel (every layout): loads through registers into padded LDS
//     rows ([rows][64 + 8 pad] bf16, 144-byte pitch, conflict-free fragment
//     reads), double-buffered.  Operands whose K dimension is not contiguous
//     in memory (A^T, or a [K][N] B) are loaded as 8x8 blocks of 16-byte
//     vectors and transposed in registers (v_perm_b32) before the LDS store.
// Epilogues with bf16 outputs on 256 x 256 tiles are "staged": the fp32 tile
// goes through LDS so that side inputs and outputs move as 16-byte vectors
// (measured: the SwiGLU-backward GEMM of LoRA-MLP 1.93 -> ~1.2 ms).
//
// MFMA lane layouts (v_mfma_f32_32x32x16_bf16, 64 lanes):
//   A operand: lane l holds A[row = l % 32][k = 8 * (l / 32) + 0..7]
//   B operand: lane l holds B[k = 8 * (l / 32) + 0..7][col = l % 32]
//   (A and B use the same k assignment, so the contraction is exact whatever
//    order the hardware sums the 16 k values in)
//   D: acc[r] (r = 0..15) of lane l is D[8 * (r / 4) + 4 * (l / 32) + r % 4][l % 32]
#pragma once

#include <type_traits>

#include "common.h"
#include "gelu.h"

namespace fgemm {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int BK = 64;
constexpr int LDS_PITCH = BK + 8;  // bf16 elements per LDS row

enum Layout { ROW = 0, COL = 1 };

// Output-row mapping of B-tile rows in "dual" mode: the tile's B rows come
// alternately (in groups of 32) from two weights, so that a wave's N tiles
// t = 0,1,2,3 are (gate cols c..c+31, up cols c..c+31, gate c+32.., up c+32..)
// and the matching gate/up accumulators sit in the same lane and register.
enum BMode { B_SINGLE = 0, B_DUAL = 1 };

struct Seg {
  const __bf16* a;
  int64_t lda;
  const __bf16* b;   // B rows of the tile (or the "gate" rows in dual mode)
  const __bf16* b2;  // dual mode: the "up" rows (nullptr = zeros)
  int64_t ldb;
  int64_t k;         // K extent of the segment
  int64_t n_lo, n_hi;  // output columns this segment applies to (B row = n - n_lo)
  // dual mode only (the 4-wave engine): gate rows read k < k_split, up rows
  // read k >= k_split from column k - k_split of b2; 0 = both read every k.
  // Two rank-r LoRA-B products of a gate/up GEMM then share one K tile.
  int64_t k_split;
};

constexpr int MAX_SEGS = 6;

enum Epi {
  EPI_STORE_BF16 = 0,   // C = alpha*acc + beta*C
  EPI_STORE_F32 = 1,     // C = alpha*acc + beta*C; with split-K, one partial slice per split
  EPI_ATOMIC_F32 = 2,   // C += alpha*acc
  EPI_SWIGLU_FWD = 3,   // dual: e, g, h = silu(e) * g
  EPI_SWIGLU_BWD = 4,   // DW: (DW, e, g) -> (h, df, de) in place
  EPI_ROPE = 5,         // QKV: rotate columns < rope_cols per head, store bf16
  EPI_GEGLU_TANH_FWD = 6,  // dual: e, g, h = gelu_tanh(e) * g
  EPI_GEGLU_TANH_BWD = 7,  // DW: (DW, e, g) -> (h, dup, dgate) in place
  EPI_GEGLU_ERF_FWD = 8,   // as 6 with the exact (erf) GELU
  EPI_GEGLU_ERF_BWD = 9,   // as 7 with the exact (erf) GELU
};

// Gated-linear-unit epilogues: forward (dual-B gate/up GEMM) and backward
// (the DW = dY W_down GEMM, in place over the saved e / g).
constexpr bool glu_fwd_epi(int epi) {
  return epi == EPI_SWIGLU_FWD || epi == EPI_GEGLU_TANH_FWD || epi == EPI_GEGLU_ERF_FWD;
}
constexpr bool glu_bwd_epi(int epi) {
  return epi == EPI_SWIGLU_BWD || epi == EPI_GEGLU_TANH_BWD || epi == EPI_GEGLU_ERF_BWD;
}

struct EpiArgs {
  void* c;
  int64_t ldc;
  float alpha, beta;
  // per-column-group scale for the STORE/ATOMIC epilogues: columns
  // [g*alpha_group, (g+1)*alpha_group) use alphas[g] (alpha_group 0 = off)
  int64_t alpha_group;
  float alphas[4];
  __bf16* e;   // GLU forward: e buffer; GLU backward: e in / d(up) out
  __bf16* g;   // GLU forward: g buffer; GLU backward: g in / d(gate) out
  int64_t ld_eg;
  const __bf16* cos;
  const __bf16* sin;
  int64_t cs_ld;             // cos/sin row pitch (elements)
  int64_t cs_rows;           // cos/sin rows; a position outside [0, cs_rows) gives NaN (no read)
  const int64_t* positions;  // per output row (token); nullptr = row index
  int64_t rope_cols;         // columns [0, rope_cols) are rotated
  int head_dim;              // 64 or 128
  int vec_ok;                // every output / side buffer 16-byte aligned with pitches % 8 == 0
  int64_t split_stride;      // STORE_F32 with split-K: split z writes its partial sums at c + z * split_stride
  int act;                   // STORE epilogues: activation of the result (ACT_NONE / ACT_SILU / ACT_RELU / ACT_GELU)
  // Rank-r LoRA products formed by the gated-activation epilogues of the
  // 4-wave engine, as fp32 partial sums with one slice per column tile
  // (vpart == nullptr: off):
  //  * GLU backward: [df B_u | de B_g], vpart[(n0 / 256) * vpart_stride +
  //    m * 2 vr + j], j < vr from df B_u, vr <= j < 2 vr from de B_g;
  //    vbt = {B_u^T, B_g^T}, each [vr][N] with pitch vbt_ld;
  //  * GLU forward (dual B): h A_d^T, vpart[(n0 / 128) * vpart_stride +
  //    m * vr + j]; vbt[0] = A_d [vr][N] with pitch vbt_ld.
  float* vpart;
  int64_t vpart_stride;
  const __bf16* vbt[2];
  int64_t vbt_ld;
  int vr;
  // Token-reduction LoRA products of the GLU backward epilogue (wpart ==
  // nullptr: off), fp32 partial sums with one slice of two [N][vr] blocks per
  // 256-row tile: wpart[(m0 / 256) * wpart_stride + p * N * vr + n * vr + j]
  // = sum over the tile's rows m of df[m][n] xa_u[m][j] (p = 0), of
  // de[m][n] xa_g[m][j] (p = 1); wxt = {xa_u^T, xa_g^T}, each [vr][M] with
  // pitch wxt_ld.
  float* wpart;
  int64_t wpart_stride;
  const __bf16* wxt[2];
  int64_t wxt_ld;
};

// Activations of the STORE epilogues, applied to alpha * acc + beta * C.
enum EpiAct { ACT_NONE = 0, ACT_SILU = 1, ACT_RELU = 2, ACT_GELU = 3 };

constexpr int MAX_COL_ORDER = 8;
struct GemmArgs {
  int64_t M, N;  // N = output columns
  int n_segs;
  Seg segs[MAX_SEGS];
  int split_k;   // number of K partitions (grid z)
  EpiArgs ep;
  // Dispatch order of the column tiles when their K work differs (column-
  // ranged segments of different lengths): n_col_order = tiles_n (at most
  // MAX_COL_ORDER) and col_order[i] = the i-th column tile, heaviest first;
  // 0 = the default XCD-aware order.
  int n_col_order;
  uint8_t col_order[MAX_COL_ORDER];
};

__device__ __forceinline__ uint32_t perm_lo(uint32_t a, uint32_t b) {
  // (a.lo16, b.lo16) -> low half from a, high half from b
  return __builtin_amdgcn_perm(b, a, 0x05040100u);
}
__device__ __forceinline__ uint32_t perm_hi(uint32_t a, uint32_t b) {
  return __builtin_amdgcn_perm(b, a, 0x07060302u);
}

// In-register transpose of an 8x8 block of 16-bit values.
// in[i] holds row i (8 values, dword j = elements 2j, 2j+1).
// out[j] holds column j (8 values: in[0][j], ..., in[7][j]).
__device__ __forceinline__ void transpose8x8(const uint4 (&in)[8], uint4 (&out)[8]) {
  uint32_t r[8][4];
#pragma unroll
  for (int i = 0; i < 8; ++i) { r[i][0] = in[i].x; r[i][1] = in[i].y; r[i][2] = in[i].z; r[i][3] = in[i].w; }
  // column c = 2*j + h (h = 0 low half, 1 high half of dword j)
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    uint32_t lo[4], hi[4];
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      lo[p] = perm_lo(r[2 * p][j], r[2 * p + 1][j]);  // (row 2p, row 2p+1) of column 2j
      hi[p] = perm_hi(r[2 * p][j], r[2 * p + 1][j]);  // ... of column 2j+1
    }
    out[2 * j] = make_uint4(lo[0], lo[1], lo[2], lo[3]);
    out[2 * j + 1] = make_uint4(hi[0], hi[1], hi[2], hi[3]);
  }
}

// Tile loader: fetches a BROWS x BK operand tile from global memory into
// registers with raw buffer loads, then writes it k-contiguous into LDS.
//   KCONTIG: element (row, k) at base[row * ld + k]   (A ROW, B COL)
//   !KCONTIG: element (row, k) at base[k * ld + row]  (A COL, B ROW)
// Per segment, setup() precomputes each thread's byte offsets inside the
// tile's panel; rows outside the matrix / the segment's column range get an
// offset past the buffer's num_records, which the hardware returns as zeros,
// so the K loop has no branches.  Per K tile, load() rebases the buffer
// resource on k0 (scalar work) and masks k beyond the segment's end.
// DUAL (B only): vector i of a thread lies in 32-row group i % 4 of a 128-row
// wave slab; even groups read pointer 0 (gate), odd groups pointer 1 (up).
constexpr uint32_t OOB = 0x80000000u;       // offset >= num_records -> reads 0
constexpr int NUM_RECORDS = 0x7fffffff;

typedef int i32x4 __attribute__((ext_vector_type(4)));

// The base is wave-uniform by construction; readfirstlane makes that
// visible to the compiler so the descriptor lives in SGPRs (a descriptor it
// cannot prove uniform turns every buffer load into a waterfall loop).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base) {
  const uint64_t b = reinterpret_cast<uint64_t>(base);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)b);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(b >> 32));
  void* ub = reinterpret_cast<void*>(((uint64_t)hi << 32) | lo);
  return __builtin_amdgcn_make_buffer_rsrc(ub, (short)0, NUM_RECORDS, 0x00020000);
}

__device__ __forceinline__ uint4 buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  i32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0);
  return make_uint4((uint32_t)v.x, (uint32_t)v.y, (uint32_t)v.z, (uint32_t)v.w);
}

template <int BROWS, int NT, bool KCONTIG, bool DUAL>
struct TileLoader {
  static constexpr int NVEC = BROWS * BK / 8;                  // 16-byte vectors per tile
  static constexpr int NBLK = (BROWS / 8) * (BK / 8);          // 8x8 blocks per tile
  static constexpr int VPT = KCONTIG ? (NVEC + NT - 1) / NT : 8 * ((NBLK + NT - 1) / NT);
  static constexpr int BPT = VPT / 8;                          // 8x8 blocks per thread (!KCONTIG)
  static_assert(!DUAL || (KCONTIG && NT == 256 && BROWS == 256), "dual loader: 256x64 K-contiguous tile");

  struct Stage {  // one K tile in flight (registers)
    uint4 v[VPT];
  };
  uint32_t voff[KCONTIG ? VPT : BPT];  // byte offsets of the rows (OOB = zero-fill)
  const char* base[2];
  int64_t ld_bytes;

  // Panel p0/p1 + panel_off rows (KCONTIG) or columns (!KCONTIG);
  // row_src(q, sel) -> index of tile row q relative to that panel start
  // (-1 = no data: zero-fill).  Relative offsets keep every byte offset
  // inside one tile panel, far below 2^31.
  template <class RowSrc>
  __device__ __forceinline__ void setup(const void* p0, const void* p1, int64_t ld, int64_t panel_off,
                                        RowSrc row_src) {
    ld_bytes = ld * 2;
    const int64_t pan = KCONTIG ? panel_off * ld_bytes : panel_off * 2;
    base[0] = p0 ? (const char*)p0 + pan : nullptr;
    base[1] = DUAL ? (p1 ? (const char*)p1 + pan : nullptr) : base[0];
    const int tid = threadIdx.x;
    if constexpr (KCONTIG) {
#pragma unroll
      for (int i = 0; i < VPT; ++i) {
        const int v = tid + i * NT;
        const int q = v / (BK / 8);
        const int kc = (v % (BK / 8)) * 8;
        const int sel = DUAL ? (i % 2) : 0;
        const int64_t row = (v < NVEC && base[sel]) ? row_src(q, sel) : -1;
        voff[i] = row < 0 ? OOB : (uint32_t)(row * ld_bytes + kc * 2);
      }
    } else {
#pragma unroll
      for (int bi = 0; bi < BPT; ++bi) {
        const int blk = tid + bi * NT;
        const int kb = (blk % (BK / 8)) * 8;   // k-block fastest: the 8 lanes of a row
        const int qb = (blk / (BK / 8)) * 8;   // group write one 128-byte LDS row span
        const int64_t col = (blk < NBLK && base[0]) ? row_src(qb, 0) : -1;  // first of 8 contiguous rows
        voff[bi] = col < 0 ? OOB : (uint32_t)(kb * ld_bytes + col * 2);
      }
    }
  }

  __device__ __forceinline__ void load(int64_t k0, int64_t kvalid, Stage& st) {
    uint4* regs = st.v;
    const int tid = threadIdx.x;
    if constexpr (KCONTIG) {
      const __amdgpu_buffer_rsrc_t r0 = make_rsrc(base[0] + k0 * 2);
      const __amdgpu_buffer_rsrc_t r1 = make_rsrc(base[1] + k0 * 2);
      const int kc = (tid % (BK / 8)) * 8;  // same for every i (NT is a multiple of 8)
      const bool kin = kc < kvalid;
#pragma unroll
      for (int i = 0; i < VPT; ++i) {
        const uint32_t off = kin ? voff[i] : OOB;
        regs[i] = buf_load16((DUAL && (i % 2)) ? r1 : r0, off);
      }
    } else {
      const __amdgpu_buffer_rsrc_t r0 = make_rsrc(base[0] + k0 * ld_bytes);
#pragma unroll
      for (int bi = 0; bi < BPT; ++bi) {
        const int blk = tid + bi * NT;
        const int kb = (blk % (BK / 8)) * 8;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const bool ok = voff[bi] != OOB && kb + i < kvalid;
          regs[bi * 8 + i] = buf_load16(r0, ok ? voff[bi] + (uint32_t)(i * ld_bytes) : OOB);
        }
      }
    }
  }

  __device__ __forceinline__ void store(const Stage& st, __bf16* lds) {
    const uint4* regs = st.v;
    const int tid = threadIdx.x;
    if constexpr (KCONTIG) {
#pragma unroll
      for (int i = 0; i < VPT; ++i) {
        const int v = tid + i * NT;
        if (NVEC % NT == 0 || v < NVEC) {
          const int q = v / (BK / 8);
          const int kc = (v % (BK / 8)) * 8;
          *reinterpret_cast<uint4*>(lds + q * LDS_PITCH + kc) = regs[i];
        }
      }
    } else {
#pragma unroll
      for (int bi = 0; bi < BPT; ++bi) {
        const int blk = tid + bi * NT;
        if (NBLK % NT == 0 || blk < NBLK) {
          const int kb = (blk % (BK / 8)) * 8;
          const int qb = (blk / (BK / 8)) * 8;
          // transpose here, not in load(): the loads stay in flight during the MFMAs
          uint4 in[8], out[8];
#pragma unroll
          for (int i = 0; i < 8; ++i) in[i] = regs[bi * 8 + i];
          transpose8x8(in, out);
#pragma unroll
          for (int i = 0; i < 8; ++i)
            *reinterpret_cast<uint4*>(lds + (qb + i) * LDS_PITCH + kb) = out[i];
        }
      }
    }
  }
};

__device__ __forceinline__ float sigmoid_f(float x) { return __builtin_amdgcn_rcpf(1.0f + __expf(-x)); }
__device__ __forceinline__ float silu_f(float x) { return x * sigmoid_f(x); }
__device__ __forceinline__ float bf16r(float x) { return (float)(__bf16)x; }

// Activation of a STORE epilogue (act is uniform across the launch).
__device__ __forceinline__ float epi_act(int act, float v) {
  if (act == ACT_SILU) return silu_f(v);
  if (act == ACT_RELU) return v > 0.f ? v : 0.f;
  float a, d;  // ACT_GELU: tanh-approximate GELU
  fgelu::gelu_and_grad<true>(v, a, d);
  return a;
}

// h (before its bf16 rounding) of a GLU forward epilogue from the fp32
// accumulators e (gate) and g (up).
//  * SwiGLU: silu(e) g on the fp32 values (lora_mlp_kernel_v6.py:81-151);
//  * GeGLU: the GeGLU kernel's forward on the bf16 e and g that are stored
//    for the backward, round(gelu(e)) g (geglu.py:126-148), so h is what the
//    standalone GeGLU gives on those tensors.
template <int EPI>
__device__ __forceinline__ float glu_fwd_h(float e, float g) {
  if constexpr (EPI == EPI_SWIGLU_FWD) {
    return silu_f(e) * g;
  } else {
    float a, d;
    fgelu::gelu_and_grad<EPI == EPI_GEGLU_TANH_FWD>(bf16r(e), a, d);
    return bf16r(a) * bf16r(g);
  }
}

// GLU backward on one element: acc = DW (fp32), e / g the saved bf16 values;
// returns h (recomputed for the down-projection gradients), du = d(up) and
// dgt = d(gate), each before its bf16 rounding.
//  * SwiGLU, Unsloth-style (lora_mlp_kernel_v6.py:592-672):
//      f = round(silu(e)), h = f g, du = DW f, dgt = round(DW g) sig (1 + e (1 - sig));
//  * GeGLU, the GeGLU kernel's backward with dout = round(DW) (geglu.py:151-182):
//      a = round(gelu(e)), h = a g, du = DW a, dgt = DW g gelu'(e).
template <int EPI>
__device__ __forceinline__ void glu_bwd_vals(float acc, float e, float g, float& h, float& du, float& dgt) {
  const float dw = bf16r(acc);
  if constexpr (EPI == EPI_SWIGLU_BWD) {
    const float se = sigmoid_f(e);
    const float f = bf16r(se * e);
    h = f * g;
    du = dw * f;
    const float dg = bf16r(dw * g);
    dgt = dg * se * (1.0f + e * (1.0f - se));
  } else {
    float a, d;
    fgelu::gelu_and_grad<EPI == EPI_GEGLU_TANH_BWD>(e, a, d);
    const float ar = bf16r(a);
    h = ar * g;
    du = dw * ar;
    dgt = dw * g * d;
  }
}

// XCD-aware tile order: consecutive workgroup ids land on different XCDs
// (round-robin dispatch), so ids are regrouped so that each XCD walks a
// contiguous range of the tile order; within it, tiles go in groups of
// GROUP_M row-panels to share A and B panels in that XCD's L2.
// With a column order (column tiles of unequal K work), the tiles go column
// by column in that order instead, so the long tiles are dispatched first
// and the short ones fill in behind them.
__device__ __forceinline__ void tile_coords(int64_t tiles_m, int64_t tiles_n, int& tm, int& tn,
                                            const GemmArgs& args) {
  if (args.n_col_order > 0 && args.n_col_order == tiles_n) {
    const int64_t id = blockIdx.x;
    tm = (int)(id % tiles_m);
    tn = args.col_order[id / tiles_m];
    return;
  }
  constexpr int NXCD = 8;
  constexpr int GROUP_M = 8;
  const int64_t total = tiles_m * tiles_n;
  int64_t id = blockIdx.x;
  if (total % NXCD == 0) {
    const int64_t per = total / NXCD;
    id = (id % NXCD) * per + id / NXCD;
  }
  const int64_t group_span = (int64_t)GROUP_M * tiles_n;
  const int64_t g = id / group_span;
  const int64_t first_m = g * GROUP_M;
  const int64_t gm = (tiles_m - first_m) < GROUP_M ? (tiles_m - first_m) : GROUP_M;
  const int64_t in = id % group_span;
  tm = (int)(first_m + in % gm);
  tn = (int)(in / gm);
}

// Scheduling-group masks of __builtin_amdgcn_sched_group_barrier.
constexpr int SG_MFMA = 0x008;
constexpr int SG_DS_READ = 0x100;

// ---------------------------------------------------------------------------
// Staged epilogue (256 x 256 tiles, bf16 outputs): the accumulators go through
// LDS, half a tile (128 rows) at a time in fp32, so that every thread then
// owns contiguous 8-column chunks: side inputs (C for beta, e / g, cos / sin)
// are read and every output is written with 16-byte vector accesses instead
// of one 2-byte access per lane and element.  Values are rounded exactly as
// in the per-element epilogue (single rounding of the fp32 result).
// ---------------------------------------------------------------------------
constexpr int STAGED_PITCH = 256 + 4;                   // floats per LDS row (bank-shifted)
constexpr int STAGED_BYTES = 128 * STAGED_PITCH * 4;    // one 128-row half tile

__device__ __forceinline__ uint4 ld16(const void* p) { return *reinterpret_cast<const uint4*>(p); }
// Epilogue outputs are stored nontemporal: they are not read again by this
// GEMM, and keeping them out of the Infinity Cache leaves the next kernel of
// the step (the rank-r products that read h, df, de) no dirty lines to drain.
// Measured on MI355X, same box, alternating builds: LoRA-MLP step 5.61 ->
// 5.57 ms, LoRA-QKV step 2.60 -> 2.57 ms (the GEMMs themselves within noise).
__device__ __forceinline__ void st16(void* p, uint4 v) {
  const u32x4_t w = {v.x, v.y, v.z, v.w};
  __builtin_nontemporal_store(w, reinterpret_cast<u32x4_t*>(p));
}
__device__ __forceinline__ void unpack8(uint4 v, float (&f)[8]) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = __uint_as_float(w[i] << 16);
    f[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
  }
}
__device__ __forceinline__ uint4 pack8(const float (&f)[8]) {
  uint32_t w[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const __bf16 lo = (__bf16)f[2 * i], hi = (__bf16)f[2 * i + 1];
    w[i] = (uint32_t)__builtin_bit_cast(uint16_t, lo) | ((uint32_t)__builtin_bit_cast(uint16_t, hi) << 16);
  }
  return make_uint4(w[0], w[1], w[2], w[3]);
}

// Tiles and epilogues the staged epilogue serves.
constexpr bool staged_ok(int bm, int bn, int wm, int wn, int epi) {
  return bm == 256 && bn == 256 && (256 / wm) % 32 == 0 && (256 / wn) % 32 == 0 && 256 / wm <= 128 &&
         (epi == EPI_STORE_BF16 || epi == EPI_STORE_F32 || glu_fwd_epi(epi) || glu_bwd_epi(epi) ||
          epi == EPI_ROPE);
}

// Workgroup barrier that waits only for this wave's LDS accesses (lgkmcnt 0),
// not for its global stores: the epilogue's stores of one half tile stay in
// flight while the next half is staged (__syncthreads() would also wait for
// vmcnt 0, i.e. for every store to be acknowledged by memory; measured on
// the 8192 x 28672 x 4096 SwiGLU GEMM: 1791 -> 1683 us).
__device__ __forceinline__ void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xc07f);  // vmcnt 63, expcnt 7 (no wait), lgkmcnt 0
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

template <int WAVES_M, int WAVES_N, int BMODE, int EPI>
__device__ __forceinline__ void epilogue_staged(const GemmArgs& args,
                                                f32x16 (&acc)[256 / WAVES_M / 32][256 / WAVES_N / 32], int64_t m0,
                                                int64_t n0, int lane, int wm, int wn, float* lds) {
  constexpr int P = STAGED_PITCH;
  constexpr int NT = WAVES_M * WAVES_N * 64;
  constexpr int TM = 256 / WAVES_M, TN = 256 / WAVES_N;
  constexpr int FM = TM / 32, FN = TN / 32;
  const EpiArgs& ep = args.ep;
  const int64_t M = args.M, N = args.N;
  const int tid = threadIdx.x;
  lds_barrier();  // the main loop's LDS reads are done
#pragma unroll 1
  for (int pass = 0; pass < 2; ++pass) {
    if (pass) lds_barrier();  // pass 0's readers are done with the buffer
    if ((wm * TM) / 128 == pass) {  // this wave's rows lie in the half being staged
      const int row0 = wm * TM - pass * 128;
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
          for (int r = 0; r < 16; ++r)
            lds[(row0 + i * 32 + 8 * (r / 4) + 4 * (lane / 32) + r % 4) * P + wn * TN + j * 32 + lane % 32] =
                acc[i][j][r];
    }
    lds_barrier();
    const int64_t mrow0 = m0 + pass * 128;
    if constexpr (BMODE == B_DUAL) {
      // LDS column layout per wave wn: 32-col groups (gate jp=0, up jp=0, gate jp=1, up jp=1);
      // output column c (0..127) -> wave c/64, pair (c%64)/32
#pragma unroll 2
      for (int it = 0; it < 128 * 16 / NT; ++it) {
        const int id = it * NT + tid;
        const int rr = id / 16, c = (id % 16) * 8;
        const int64_t m = mrow0 + rr, n = n0 + c;
        if (m >= M || n >= N) continue;
        const int lc = (c / 64) * 128 + ((c % 64) / 32) * 64 + c % 32;
        const float* pg = lds + rr * P + lc;
        float e[8], g[8], h[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) { e[q] = pg[q]; g[q] = pg[32 + q]; h[q] = glu_fwd_h<EPI>(e[q], g[q]); }
        const int64_t off = m * ep.ld_eg + n;
        if (n + 8 <= N) {
          if (ep.e) {  // training saves e and g; inference (e = g = null) stores h only
            st16(ep.e + off, pack8(e));
            st16(ep.g + off, pack8(g));
          }
          st16((__bf16*)ep.c + m * ep.ldc + n, pack8(h));
        } else {
          for (int q = 0; q < 8 && n + q < N; ++q) {
            if (ep.e) {
              ep.e[off + q] = (__bf16)e[q];
              ep.g[off + q] = (__bf16)g[q];
            }
            ((__bf16*)ep.c)[m * ep.ldc + n + q] = (__bf16)h[q];
          }
        }
      }
    } else if constexpr (glu_bwd_epi(EPI)) {
      // As for RoPE below: a thread's chunks share one column chunk c, so the
      // saved e / g chunks of four rows are read before any of them is used
      // (one row at a time left the epilogue waiting on each load).
      static_assert(NT % 32 == 0, "rows of 32 chunk-threads");
      constexpr int IT = 128 * 32 / NT, RSTEP = NT / 32, GRP = IT >= 4 ? 4 : IT;
      const int c = (tid % 32) * 8;
      const int64_t n = n0 + c;
      const bool full = n + 8 <= N;
#pragma unroll
      for (int g0 = 0; g0 < IT; g0 += GRP) {
        uint4 ew[GRP], gw[GRP];
#pragma unroll
        for (int j = 0; j < GRP; ++j) {
          const int64_t m = mrow0 + (g0 + j) * RSTEP + tid / 32;
          if (m < M && full) {
            const int64_t off = m * ep.ld_eg + n;
            ew[j] = ld16(ep.e + off);
            gw[j] = ld16(ep.g + off);
          }
        }
#pragma unroll
        for (int j = 0; j < GRP; ++j) {
          const int rr = (g0 + j) * RSTEP + tid / 32;
          const int64_t m = mrow0 + rr;
          if (m >= M || n >= N) continue;
          const float* pv = lds + rr * P + c;
          const int64_t off = m * ep.ld_eg + n;
          float ev[8], gv[8], hv[8], dfv[8], dev[8];
          if (full) {
            unpack8(ew[j], ev);
            unpack8(gw[j], gv);
          } else {
            for (int q = 0; q < 8; ++q) {
              ev[q] = n + q < N ? (float)ep.e[off + q] : 0.f;
              gv[q] = n + q < N ? (float)ep.g[off + q] : 0.f;
            }
          }
#pragma unroll
          for (int q = 0; q < 8; ++q) glu_bwd_vals<EPI>(pv[q], ev[q], gv[q], hv[q], dfv[q], dev[q]);
          if (full) {
            st16((__bf16*)ep.c + m * ep.ldc + n, pack8(hv));
            st16(ep.e + off, pack8(dfv));
            st16(ep.g + off, pack8(dev));
          } else {
            for (int q = 0; q < 8 && n + q < N; ++q) {
              ((__bf16*)ep.c)[m * ep.ldc + n + q] = (__bf16)hv[q];
              ep.e[off + q] = (__bf16)dfv[q];
              ep.g[off + q] = (__bf16)dev[q];
            }
          }
        }
      }
    } else if constexpr (EPI == EPI_ROPE) {
      // A thread's chunks share one column chunk c (rows tid / 32 + 16 it), so
      // d and the lo / hi half are fixed: the positions of all its rows are
      // read first, then the cos / sin chunks of four rows at a time, then
      // those four rows are rotated and stored.  Issuing the table loads ahead
      // keeps several in flight (one row at a time left the epilogue waiting
      // on each load).
      static_assert(NT % 32 == 0, "rows of 32 chunk-threads");
      constexpr int IT = 128 * 32 / NT, RSTEP = NT / 32, GRP = IT >= 4 ? 4 : IT;
      const int c = (tid % 32) * 8;
      const int64_t n = n0 + c;
      const bool rot = n < N && n < ep.rope_cols;
      const int half = ep.head_dim / 2;
      const int in_head = (int)(n % ep.head_dim);
      const bool lo = in_head < half;
      const int d = in_head % half;
      int64_t posv[IT];
#pragma unroll
      for (int it = 0; it < IT; ++it) {
        const int64_t m = mrow0 + it * RSTEP + tid / 32;
        posv[it] = (rot && m < M) ? (ep.positions ? ep.positions[m] : m) : -1;
      }
#pragma unroll
      for (int g0 = 0; g0 < IT; g0 += GRP) {
        uint4 cv[GRP], sv[GRP];
#pragma unroll
        for (int j = 0; j < GRP; ++j) {
          const int64_t pos = posv[g0 + j];
          if (pos >= 0 && pos < ep.cs_rows) {
            cv[j] = ld16(ep.cos + pos * ep.cs_ld + d);
            sv[j] = ld16(ep.sin + pos * ep.cs_ld + d);
          }
        }
#pragma unroll
        for (int j = 0; j < GRP; ++j) {
          const int rr = (g0 + j) * RSTEP + tid / 32;
          const int64_t m = mrow0 + rr;
          if (m >= M || n >= N) continue;
          const float* pv = lds + rr * P + c;
          float v[8];
#pragma unroll
          for (int q = 0; q < 8; ++q) v[q] = pv[q];
          if (rot) {
            // the 128-column wave tile holds whole heads: partner half in LDS
            const float* pp = lds + rr * P + (lo ? c + half : c - half);
            const int64_t pos = posv[g0 + j];
            float cs[8], sn[8];
            if (pos >= 0 && pos < ep.cs_rows) {
              unpack8(cv[j], cs);
              unpack8(sv[j], sn);
            } else {
#pragma unroll
              for (int q = 0; q < 8; ++q) cs[q] = sn[q] = __builtin_nanf("");
            }
#pragma unroll
            for (int q = 0; q < 8; ++q) {
              const float x = bf16r(v[q]), xp = bf16r(pp[q]);
              v[q] = lo ? x * cs[q] - xp * sn[q] : x * cs[q] + xp * sn[q];
            }
          }
          __bf16* cp = (__bf16*)ep.c + m * ep.ldc + n;
          if (n + 8 <= N) st16(cp, pack8(v));
          else
            for (int q = 0; q < 8 && n + q < N; ++q) cp[q] = (__bf16)v[q];
        }
      }
    } else {
#pragma unroll 2
      for (int it = 0; it < 128 * 32 / NT; ++it) {
        const int id = it * NT + tid;
        const int rr = id / 32, c = (id % 32) * 8;
        const int64_t m = mrow0 + rr, n = n0 + c;
        if (m >= M || n >= N) continue;
        const float* pv = lds + rr * P + c;
        float v[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) v[q] = pv[q];
        const bool full = n + 8 <= N;
        if constexpr (EPI == EPI_STORE_F32) {
          // fp32 C (beta accumulation, or split z's partial slice): two
          // 16-byte accesses per 8-column chunk
#pragma unroll
          for (int q = 0; q < 8; ++q) {
            float a = ep.alpha;
            if (ep.alpha_group > 0) {
              const int64_t grp = (n + q) / ep.alpha_group;
              a = ep.alphas[grp < 4 ? grp : 3];
            }
            v[q] *= a;
          }
          float* cp = (float*)ep.c + blockIdx.z * ep.split_stride + m * ep.ldc + n;
          if (full) {
            float4* c4 = reinterpret_cast<float4*>(cp);
            if (ep.beta != 0.f) {
              const float4 c0 = c4[0], c1 = c4[1];
              v[0] += ep.beta * c0.x; v[1] += ep.beta * c0.y; v[2] += ep.beta * c0.z; v[3] += ep.beta * c0.w;
              v[4] += ep.beta * c1.x; v[5] += ep.beta * c1.y; v[6] += ep.beta * c1.z; v[7] += ep.beta * c1.w;
            }
            if (ep.act)
#pragma unroll
              for (int q = 0; q < 8; ++q) v[q] = epi_act(ep.act, v[q]);
            c4[0] = make_float4(v[0], v[1], v[2], v[3]);
            c4[1] = make_float4(v[4], v[5], v[6], v[7]);
          } else {
            for (int q = 0; q < 8 && n + q < N; ++q) {
              float o = ep.beta != 0.f ? v[q] + ep.beta * cp[q] : v[q];
              cp[q] = ep.act ? epi_act(ep.act, o) : o;
            }
          }
        } else if constexpr (EPI == EPI_STORE_BF16) {
#pragma unroll
          for (int q = 0; q < 8; ++q) {
            float a = ep.alpha;
            if (ep.alpha_group > 0) {
              const int64_t grp = (n + q) / ep.alpha_group;
              a = ep.alphas[grp < 4 ? grp : 3];
            }
            v[q] *= a;
          }
          __bf16* cp = (__bf16*)ep.c + m * ep.ldc + n;
          if (full) {
            if (ep.beta != 0.f) {
              float cv[8];
              unpack8(ld16(cp), cv);
#pragma unroll
              for (int q = 0; q < 8; ++q) v[q] += ep.beta * cv[q];
            }
            if (ep.act)
#pragma unroll
              for (int q = 0; q < 8; ++q) v[q] = epi_act(ep.act, v[q]);
            st16(cp, pack8(v));
          } else {
            for (int q = 0; q < 8 && n + q < N; ++q) {
              float o = v[q];
              if (ep.beta != 0.f) o += ep.beta * (float)cp[q];
              if (ep.act) o = epi_act(ep.act, o);
              cp[q] = (__bf16)o;
            }
          }
        }
      }
    }
  }
}

template <int BM, int BN, int WAVES_M, int WAVES_N, int BMODE, int EPI>
__device__ __forceinline__ void epilogue(const GemmArgs& args, f32x16 (&acc)[BM / WAVES_M / 32][BN / WAVES_N / 32],
                                         int64_t m0, int64_t n0, int lane, int wm, int wn) {
  constexpr int TM = BM / WAVES_M, TN = BN / WAVES_N;
  constexpr int FM = TM / 32, FN = TN / 32;
  const int64_t M = args.M;
  const EpiArgs& ep = args.ep;
  const int64_t row_base = m0 + wm * TM + 4 * (lane / 32);
  const int col_in = lane % 32;

  if constexpr (EPI == EPI_STORE_BF16 || EPI == EPI_STORE_F32 || EPI == EPI_ATOMIC_F32) {
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const int64_t n = n0 + wn * TN + j * 32 + col_in;
      if (n >= args.N) continue;
      float col_alpha = ep.alpha;
      if (ep.alpha_group > 0) {
        const int64_t grp = n / ep.alpha_group;
        col_alpha = ep.alphas[grp < 4 ? grp : 3];
      }
#pragma unroll
      for (int i = 0; i < FM; ++i) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int64_t m = row_base + i * 32 + 8 * (r / 4) + (r % 4);
          if (m >= M) continue;
          const float v = col_alpha * acc[i][j][r];
          if constexpr (EPI == EPI_STORE_BF16) {
            __bf16* cp = (__bf16*)ep.c + m * ep.ldc + n;
            float o = v;
            if (ep.beta != 0.f) o += ep.beta * (float)(*cp);
            if (ep.act) o = epi_act(ep.act, o);
            *cp = (__bf16)o;
          } else if constexpr (EPI == EPI_STORE_F32) {
            float* cp = (float*)ep.c + (int64_t)blockIdx.z * ep.split_stride + m * ep.ldc + n;
            float o = v;
            if (ep.beta != 0.f) o += ep.beta * (*cp);
            if (ep.act) o = epi_act(ep.act, o);
            *cp = o;
          } else {
            atomicAdd((float*)ep.c + m * ep.ldc + n, v);
          }
        }
      }
    }
  } else if constexpr (glu_fwd_epi(EPI)) {
    // wave tiles (0,1) and (2,3) are (gate, up) pairs for 32 output columns each
#pragma unroll
    for (int jp = 0; jp < FN / 2; ++jp) {
      const int64_t n = n0 + wn * 64 + jp * 32 + col_in;
      if (n >= args.N) continue;
#pragma unroll
      for (int i = 0; i < FM; ++i) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int64_t m = row_base + i * 32 + 8 * (r / 4) + (r % 4);
          if (m >= M) continue;
          const float e = acc[i][2 * jp][r];
          const float g = acc[i][2 * jp + 1][r];
          const int64_t off = m * ep.ld_eg + n;
          if (ep.e) {
            ep.e[off] = (__bf16)e;
            ep.g[off] = (__bf16)g;
          }
          ((__bf16*)ep.c)[m * ep.ldc + n] = (__bf16)glu_fwd_h<EPI>(e, g);
        }
      }
    }
  } else if constexpr (glu_bwd_epi(EPI)) {
    // in-place GLU backward on the DW = dY @ W_down tile (glu_bwd_vals)
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const int64_t n = n0 + wn * TN + j * 32 + col_in;
      if (n >= args.N) continue;
#pragma unroll
      for (int i = 0; i < FM; ++i) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int64_t m = row_base + i * 32 + 8 * (r / 4) + (r % 4);
          if (m >= M) continue;
          const int64_t off = m * ep.ld_eg + n;
          float h, df, de;
          glu_bwd_vals<EPI>(acc[i][j][r], (float)ep.e[off], (float)ep.g[off], h, df, de);
          ((__bf16*)ep.c)[m * ep.ldc + n] = (__bf16)h;
          ep.e[off] = (__bf16)df;
          ep.g[off] = (__bf16)de;
        }
      }
    }
  } else if constexpr (EPI == EPI_ROPE) {
    // Each wave covers TN = 128 output columns aligned to a head boundary
    // (head_dim 128: tiles 0,1 = lo half, 2,3 = hi half; head_dim 64: two
    // heads, tiles (0,1) and (2,3)).
    const int half_tiles = ep.head_dim / 64;  // partner distance in 32-col tiles
#pragma unroll
    for (int i = 0; i < FM; ++i) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t m = row_base + i * 32 + 8 * (r / 4) + (r % 4);
        if (m >= M) continue;
        const int64_t pos = ep.positions ? ep.positions[m] : m;
        const bool pos_ok = pos >= 0 && pos < ep.cs_rows;
#pragma unroll
        for (int j = 0; j < FN; ++j) {
          const int64_t n = n0 + wn * TN + j * 32 + col_in;
          if (n >= args.N) continue;
          float v = acc[i][j][r];
          if (n < ep.rope_cols) {
            const int jj = j % (2 * half_tiles);
            const bool lo = jj < half_tiles;
            const int partner = lo ? j + half_tiles : j - half_tiles;
            float pv = 0.f;
#pragma unroll
            for (int q = 0; q < FN; ++q)
              if (q == partner) pv = acc[i][q][r];
            const int d = (int)(n % ep.head_dim) % (ep.head_dim / 2);
            const float c = pos_ok ? (float)ep.cos[pos * ep.cs_ld + d] : __builtin_nanf("");
            const float s = pos_ok ? (float)ep.sin[pos * ep.cs_ld + d] : __builtin_nanf("");
            // round the projection to bf16 first: RoPE is applied to the
            // materialised Q/K in the unfused reference path
            const float x = bf16r(v), xp = bf16r(pv);
            v = lo ? x * c - xp * s : x * c + xp * s;
          }
          ((__bf16*)ep.c)[m * ep.ldc + n] = (__bf16)v;
        }
      }
    }
  }
}

template <int BM, int BN, int WAVES_M, int WAVES_N, int A_LAYOUT, int B_LAYOUT, int BMODE, int EPI, bool STAGED>
__global__ __launch_bounds__(WAVES_M * WAVES_N * 64) __attribute__((amdgpu_waves_per_eu(1, 1)))
void gemm_kernel(GemmArgs args) {
  constexpr int NT = WAVES_M * WAVES_N * 64;
  constexpr int TM = BM / WAVES_M, TN = BN / WAVES_N;  // wave sub-tile
  constexpr int FM = TM / 32, FN = TN / 32;            // 32x32 MFMA tiles per wave
  static_assert(TM % 32 == 0 && TN % 32 == 0, "wave tile must be a multiple of 32");
  static_assert(BMODE == B_SINGLE || TN == 128, "dual mode expects 128-row wave tiles");

  __shared__ __attribute__((aligned(16))) __bf16 smem[2 * (BM + BN) * LDS_PITCH];
  // stage b: A tile at smem + b*(BM+BN)*pitch, B tile right after it
  auto As = [&](int b) { return smem + b * (BM + BN) * LDS_PITCH; };
  auto Bs = [&](int b) { return smem + b * (BM + BN) * LDS_PITCH + BM * LDS_PITCH; };

  const int64_t M = args.M;
  // output columns covered by one tile (dual: BN B-rows -> BN/2 outputs)
  constexpr int OUT_BN = (BMODE == B_DUAL) ? BN / 2 : BN;
  const int64_t tiles_m = (M + BM - 1) / BM;
  const int64_t tiles_n = (args.N + OUT_BN - 1) / OUT_BN;
  int tmi, tni;
  tile_coords(tiles_m, tiles_n, tmi, tni, args);
  const int64_t m0 = (int64_t)tmi * BM;
  const int64_t n0 = (int64_t)tni * OUT_BN;

  const int lane = threadIdx.x % 64;
  const int wave = threadIdx.x / 64;
  const int wm = wave % WAVES_M;
  const int wn = wave / WAVES_M;

  // ---- K tiles of this workgroup (split-K partitions the flat tile list) ----
  int seg_tiles[MAX_SEGS];
  int total_tiles = 0;
  for (int s = 0; s < args.n_segs; ++s) {
    const Seg& sg = args.segs[s];
    const bool active = sg.n_hi > n0 && sg.n_lo < n0 + OUT_BN;
    seg_tiles[s] = active ? (int)((sg.k + BK - 1) / BK) : 0;
    total_tiles += seg_tiles[s];
  }
  const int per = (total_tiles + args.split_k - 1) / args.split_k;
  const int t_begin = blockIdx.z * per;
  const int t_end = min(total_tiles, t_begin + per);

  f32x16 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  TileLoader<BM, NT, A_LAYOUT == ROW, false> la;
  TileLoader<BN, NT, B_LAYOUT == COL, BMODE == B_DUAL> lb;

  // Points the loaders at segment s (this tile's panels of A and B).
  auto setup_seg = [&](int s) {
    const Seg& sg = args.segs[s];
    la.setup(sg.a, sg.a, sg.lda, m0, [&](int q, int) -> int64_t { return m0 + q < M ? q : -1; });
    if constexpr (BMODE == B_DUAL) {
      lb.setup(sg.b, sg.b2, sg.ldb, n0, [&](int q, int) -> int64_t {
        const int t4 = (q % 128) / 32;
        const int rel = (q / 128) * 64 + (t4 / 2) * 32 + q % 32;
        return n0 + rel < args.N ? rel : -1;
      });
    } else {
      const int64_t off = n0 - sg.n_lo;
      lb.setup(sg.b, sg.b, sg.ldb, off, [&](int q, int) -> int64_t {
        const int64_t n = n0 + q;
        return (n < args.N && n >= sg.n_lo && n < sg.n_hi) ? q : -1;
      });
    }
  };

  // cursor over (segment, k0) for the flat tile range [t_begin, t_end)
  int cur_s = 0, cur_t = t_begin;
  {
    int acc_t = 0;
    while (cur_s < args.n_segs && cur_t >= acc_t + seg_tiles[cur_s]) { acc_t += seg_tiles[cur_s]; ++cur_s; }
    cur_t -= acc_t;  // tile index inside segment cur_s
  }

  // Advances the (segment, tile) cursor to the next K tile of this workgroup;
  // a segment switch re-points the loaders (rare: once per segment).
  int64_t seg_k = 0;
  int cur_n = 0;
  auto next_tile = [&](bool first) {
    if (!first) {
      ++cur_t;
      if (cur_t >= cur_n) {
        do { ++cur_s; } while (seg_tiles[cur_s] == 0);
        cur_t = 0;
        cur_n = seg_tiles[cur_s];
        setup_seg(cur_s);
        seg_k = args.segs[cur_s].k;
      }
    } else {
      cur_n = seg_tiles[cur_s];
      setup_seg(cur_s);
      seg_k = args.segs[cur_s].k;
    }
  };
  typename decltype(la)::Stage sa[1];
  typename decltype(lb)::Stage sb[1];
  auto issue = [&](int set) {  // global loads of the cursor's tile into staging set `set`
    const int64_t k0 = (int64_t)cur_t * BK;
    la.load(k0, seg_k - k0, sa[set]);
    lb.load(k0, seg_k - k0, sb[set]);
  };

  // MFMAs of one K tile held in LDS stage `buf`.
  auto compute = [&](int buf) {
    const __bf16* a_s = As(buf) + (wm * TM + lane % 32) * LDS_PITCH + (lane / 32) * 8;
    const __bf16* b_s = Bs(buf) + (wn * TN + lane % 32) * LDS_PITCH + (lane / 32) * 8;
    // Two-slot fragment ring: the reads of k-steps 0 and 1 are issued first;
    // after the MFMAs of k-step ks consume slot ks&1, the reads of k-step
    // ks+2 refill it, so each k-step's operands arrive while the previous
    // k-step's MFMAs run.  (The sched_group_barriers pin this order.)
    bf16x8 af[2][FM], bfr[2][FN];
    auto read_frags = [&](int ks, int slot) {
#pragma unroll
      for (int i = 0; i < FM; ++i) af[slot][i] = *reinterpret_cast<const bf16x8*>(a_s + i * 32 * LDS_PITCH + ks * 16);
#pragma unroll
      for (int j = 0; j < FN; ++j) bfr[slot][j] = *reinterpret_cast<const bf16x8*>(b_s + j * 32 * LDS_PITCH + ks * 16);
    };
    read_frags(0, 0);
    read_frags(1, 1);
    __builtin_amdgcn_sched_group_barrier(SG_DS_READ, 2 * (FM + FN), 0);
#pragma unroll
    for (int ks = 0; ks < BK / 16; ++ks) {
      const int slot = ks & 1;
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[slot][i], bfr[slot][j], acc[i][j], 0, 0, 0);
      __builtin_amdgcn_sched_group_barrier(SG_MFMA, FM * FN, 0);
      if (ks + 2 < BK / 16) {
        read_frags(ks + 2, slot);
        __builtin_amdgcn_sched_group_barrier(SG_DS_READ, FM + FN, 0);
      }
    }
  };

  // Pipeline: global loads run one K tile ahead of the MFMAs (one register
  // staging set), LDS is double-buffered; one barrier per K tile.
  const int n_t = t_end - t_begin;
  if (n_t > 0) {
    next_tile(true);
    issue(0);
    la.store(sa[0], As(0));
    lb.store(sb[0], Bs(0));
    __syncthreads();
    int buf = 0;
    for (int t = 0; t < n_t; ++t) {
      const bool more = t + 1 < n_t;
      if (more) { next_tile(false); issue(0); }
      compute(buf);
      if (more) {
        la.store(sa[0], As(buf ^ 1));
        lb.store(sb[0], Bs(buf ^ 1));
      }
      __syncthreads();
      buf ^= 1;
    }
  }

  if constexpr (STAGED) {
    static_assert(staged_ok(BM, BN, WAVES_M, WAVES_N, EPI), "staged epilogue: 256 x 256 tile, wave tiles of <= 128 rows");
    epilogue_staged<WAVES_M, WAVES_N, BMODE, EPI>(args, acc, m0, n0, lane, wm, wn, reinterpret_cast<float*>(smem));
  } else {
    epilogue<BM, BN, WAVES_M, WAVES_N, BMODE, EPI>(args, acc, m0, n0, lane, wm, wn);
  }
}

// ===========================================================================
// LDS-DMA engine (both operands K-contiguous: A ROW, B COL).
//
// Global -> LDS without registers: each wave instruction (buffer_load ... lds)
// moves 64 lanes x 16 bytes into 1 KB of LDS at the wave-uniform M0 base, lane
// L at +16 L.  A tile stage is BROWS rows of BKT bf16 (RB = 2 BKT bytes per
// row, no padding); the lane -> (row, chunk) map applies an XOR swizzle to
// the 16-byte chunk positions, chunk' = chunk ^ swz(row), so that the MFMA
// fragment reads (32 rows, one chunk each) hit distinct banks.  NSTAGE stages
// form a ring: iteration t waits for its own tile, one barrier, issues the
// tile NSTAGE-1 ahead into the slot freed by iteration t-1, computes.
// ===========================================================================
template <int BKT>
__device__ __forceinline__ int swz(int row) {
  if constexpr (BKT == 64) return (row >> 1) & 7;  // 2 rows per 256 bytes
  else return (row >> 2) & 3;                      // BKT == 32: 4 rows per 256 bytes
}

template <int BROWS, int BKT, int NT, bool DUAL, int AUX = 0>
struct DmaLoader {
  static constexpr int RB = BKT * 2;          // LDS bytes per row
  static constexpr int CPR = RB / 16;         // 16-byte chunks per row
  static constexpr int RPI = 64 / CPR;        // rows per wave instruction
  static constexpr int NINST = BROWS / RPI;   // wave instructions per tile
  static constexpr int NW = NT / 64;
  static constexpr int IPW = NINST / NW;      // instructions per wave per tile
  static_assert(NINST % NW == 0 && IPW * RPI == BROWS / NW, "tile / wave split");
  static_assert(!DUAL || RPI <= 32, "dual: an instruction's rows inside one 32-row group");
  uint32_t voff[IPW];   // byte offset of this lane's chunk in the panel (OOB = zero-fill)
  const char* base[2];
  int64_t ld_bytes;

  template <class RowSrc>
  __device__ __forceinline__ void setup(const void* p0, const void* p1, int64_t ld, int64_t panel_off,
                                        RowSrc row_src) {
    ld_bytes = ld * 2;
    const int64_t pan = panel_off * ld_bytes;
    base[0] = p0 ? (const char*)p0 + pan : nullptr;
    base[1] = DUAL ? (p1 ? (const char*)p1 + pan : nullptr) : base[0];
    const int lane = threadIdx.x % 64, wave = threadIdx.x / 64;
#pragma unroll
    for (int j = 0; j < IPW; ++j) {
      const int q = (wave * IPW + j) * RPI + lane / CPR;   // tile row
      const int chunk = (lane % CPR) ^ swz<BKT>(q);        // source chunk of LDS slot lane % CPR
      const int sel = DUAL ? (((wave * IPW + j) * RPI) / 32) % 2 : 0;  // 32-row groups alternate gate / up
      const int64_t row = base[sel] ? row_src(q, sel) : -1;
      voff[j] = row < 0 ? OOB : (uint32_t)(row * ld_bytes + chunk * 16);
    }
  }

  // DMA of the K tile at k0 (kvalid valid k) into the LDS stage `dst`.
  __device__ __forceinline__ void load(int64_t k0, int64_t kvalid, char* dst) {
    const int lane = threadIdx.x % 64;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / 64);
    const __amdgpu_buffer_rsrc_t r0 = make_rsrc(base[0] + k0 * 2);
    const __amdgpu_buffer_rsrc_t r1 = make_rsrc(base[1] + k0 * 2);
#pragma unroll
    for (int j = 0; j < IPW; ++j) {
      uint32_t off = voff[j];
      if (kvalid < BKT) {  // segment tail: chunks past kvalid read zeros
        const int q = (wave * IPW + j) * RPI + lane / CPR;
        const int chunk = (lane % CPR) ^ swz<BKT>(q);
        if (chunk * 8 >= kvalid) off = OOB;
      }
      const int sel = DUAL ? (((wave * IPW + j) * RPI) / 32) % 2 : 0;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(sel ? r1 : r0,
                                               (__attribute__((address_space(3))) void*)(dst + (wave * IPW + j) * 1024),
                                               16, off, 0, 0, AUX);
    }
  }
};

// ---------------------------------------------------------------------------
// Token-major operands on the LDS-DMA engine.  A stored [K][M] (A_LAYOUT COL)
// or B stored [K][N] (B_LAYOUT ROW): the token-reduction products (LoRA A/B
// gradients, the fused-CE weight gradient), whose reduction dimension K is the
// slow one.  A stage holds BKT k-rows of BROWS elements (RB = 2 BROWS bytes
// per k-row, no padding), DMA'd as they lie in memory; the MFMA fragments are
// read with ds_read_b64_tr_b16, which transposes within each 16-lane group:
// lane L of a group supplies the 8 bytes at (k0 + L/4, r0 + 4 (L%4)), and
// result lane i receives (k0 + q, r0 + i) for q = 0..3, so two reads (k0 and
// k0 + 4) give the 8 consecutive k of row r0 + i that the 32x32x16 MFMA takes.
// The 16-byte chunks of k-row q are XOR-swizzled (chunk ^ swzT(q)) so that the
// four k-rows one half-wave reads (64 bytes each) fall in distinct 64-byte
// windows of the 256-byte bank cycle.
// ---------------------------------------------------------------------------
template <int CPR>
__device__ __forceinline__ int swzT(int q) {
  if constexpr (CPR >= 16) return 4 * (q & 3);       // k-rows of >= 256 bytes: all start at bank 0
  else if constexpr (CPR == 8) return 4 * ((q >> 1) & 1);  // 128-byte k-rows: two per bank cycle
  else return 0;                                     // 64-byte k-rows: four per bank cycle already
}

template <int BROWS, int BKT, int NT, int AUX = 0>
struct DmaLoaderT {
  static constexpr int RB = BROWS * 2;        // LDS bytes per k-row
  static constexpr int CPR = RB / 16;         // 16-byte chunks (8 rows) per k-row
  static constexpr int RPI = 64 / CPR;        // k-rows per wave instruction
  static constexpr int NINST = BKT / RPI;     // wave instructions per tile
  static constexpr int NW = NT / 64;
  static constexpr int IPW = NINST / NW;      // instructions per wave per tile
  static_assert(CPR >= 4 && CPR <= 64 && 64 % CPR == 0, "k-row of 4 .. 64 chunks");
  static_assert(NINST % NW == 0 && IPW >= 1, "tile / wave split");
  uint32_t voff[IPW];   // byte offset of this lane's chunk from the tile's first k-row (OOB = zero-fill)
  const char* base;
  int64_t ld_bytes;

  // p: operand base, ld: pitch between k-rows (elements), panel_off: first
  // row (element) of the tile, row_ok(r): row panel_off + r exists (rows come
  // in whole chunks of 8: the caller guarantees a multiple-of-8 extent).
  template <class RowOk>
  __device__ __forceinline__ void setup(const void* p, int64_t ld, int64_t panel_off, RowOk row_ok) {
    ld_bytes = ld * 2;
    base = p ? (const char*)p + panel_off * 2 : nullptr;
    const int lane = threadIdx.x % 64, wave = threadIdx.x / 64;
#pragma unroll
    for (int j = 0; j < IPW; ++j) {
      const int q = (wave * IPW + j) * RPI + lane / CPR;   // k-row in the tile
      const int chunk = (lane % CPR) ^ swzT<CPR>(q);       // source chunk of LDS slot lane % CPR
      voff[j] = (base && row_ok(chunk * 8)) ? (uint32_t)(q * ld_bytes + chunk * 16) : OOB;
    }
  }

  // DMA of the K tile at k0 (kvalid valid k-rows) into the LDS stage `dst`.
  __device__ __forceinline__ void load(int64_t k0, int64_t kvalid, char* dst) {
    const int lane = threadIdx.x % 64;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / 64);
    const __amdgpu_buffer_rsrc_t r = make_rsrc(base + k0 * ld_bytes);
#pragma unroll
    for (int j = 0; j < IPW; ++j) {
      uint32_t off = voff[j];
      if (kvalid < BKT && (wave * IPW + j) * RPI + lane / CPR >= kvalid) off = OOB;  // segment tail
      __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)(dst + (wave * IPW + j) * 1024),
                                               16, off, 0, 0, AUX);
    }
  }
};

// Byte offset, in a token-major stage, of the 8 bytes this lane supplies to
// ds_read_b64_tr_b16 for the fragment of rows r0 .. r0+31 at k 0..3 (or 8..11
// for lanes 32-63); add (k_base) * RB for other k.
template <int CPR>
__device__ __forceinline__ int tr_lane_offset(int r0, int lane) {
  constexpr int RB = CPR * 16;
  const int l = lane % 16, grp = lane / 16;
  const int q = 8 * (grp / 2) + l / 4;                  // k-row (mod 4 fixes the swizzle for every k step)
  const int r = r0 + 16 * (grp % 2) + 4 * (l % 4);      // first of the 4 rows this lane supplies
  return q * RB + (((r / 8) ^ swzT<CPR>(q)) * 16) + (r % 8) * 2;
}

typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef short i16x8 __attribute__((ext_vector_type(8)));

// one 32x32x16 operand fragment from a token-major stage: k 0..3 from p0 and
// k 4..7 from p1 = p0 + 4 RB (lanes 32-63: k 8..15)
__device__ __forceinline__ bf16x8 tr_frag(const char* p0, const char* p1) {
  const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) i16x4*)p0);
  const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) i16x4*)p1);
  const i16x8 v = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
  return __builtin_bit_cast(bf16x8, v);
}

// s_waitcnt with only vmcnt constrained (gfx9 encoding: vmcnt [3:0] + [15:14],
// expcnt [6:4] = 7 and lgkmcnt [11:8] = 15 mean "don't wait").
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// WPE = waves per SIMD the register budget is sized for (512 / WPE VGPRs per
// wave).  The 256 x 256 tiles hold one workgroup per CU (the ring plus the
// staged epilogue take ~130 KB of LDS): 8 waves -> WPE 2.  The skinny tiles
// (~72 KB of LDS) hold two workgroups of 4 waves per CU: WPE 2 as well.
// AT / BT: A stored [K][M] / B stored [K][N] (token-major, see DmaLoaderT).
// CPA / CPB: cache-policy bits of the A / B buffer loads (0 = default; 2 =
// nontemporal, for an operand that no other workgroup reads again).
template <int BM, int BN, int WAVES_M, int WAVES_N, int BMODE, int EPI, int BKT, int NSTAGE, bool STAGED, int WPE,
          bool AT = false, bool BT = false, int CPA = 0, int CPB = 0>
__global__ __launch_bounds__(WAVES_M * WAVES_N * 64) __attribute__((amdgpu_waves_per_eu(WPE, WPE)))
void gemm_dma_kernel(GemmArgs args) {
  constexpr int NT = WAVES_M * WAVES_N * 64;
  constexpr int TM = BM / WAVES_M, TN = BN / WAVES_N;
  constexpr int FM = TM / 32, FN = TN / 32;
  constexpr int RB = BKT * 2;
  constexpr int A_BYTES = BM * RB, B_BYTES = BN * RB, STAGE = A_BYTES + B_BYTES;
  static_assert(BMODE == B_SINGLE || TN == 128, "dual mode expects 128-row wave tiles");
  static_assert(!(BT && BMODE == B_DUAL), "dual B operands are K-contiguous");
  constexpr int STAGED_B = STAGED ? STAGED_BYTES : 0;
  constexpr int SMEM = NSTAGE * STAGE > STAGED_B ? NSTAGE * STAGE : STAGED_B;
  __shared__ __attribute__((aligned(1024))) char smem[SMEM];

  const int64_t M = args.M;
  constexpr int OUT_BN = (BMODE == B_DUAL) ? BN / 2 : BN;
  const int64_t tiles_m = (M + BM - 1) / BM;
  const int64_t tiles_n = (args.N + OUT_BN - 1) / OUT_BN;
  int tmi, tni;
  tile_coords(tiles_m, tiles_n, tmi, tni, args);
  const int64_t m0 = (int64_t)tmi * BM;
  const int64_t n0 = (int64_t)tni * OUT_BN;
  const int lane = threadIdx.x % 64;
  const int wave = threadIdx.x / 64;
  const int wm = wave % WAVES_M;
  const int wn = wave / WAVES_M;

  int seg_tiles[MAX_SEGS];
  int total_tiles = 0;
  for (int s = 0; s < args.n_segs; ++s) {
    const Seg& sg = args.segs[s];
    const bool active = sg.n_hi > n0 && sg.n_lo < n0 + OUT_BN;
    seg_tiles[s] = active ? (int)((sg.k + BKT - 1) / BKT) : 0;
    total_tiles += seg_tiles[s];
  }
  const int per = (total_tiles + args.split_k - 1) / args.split_k;
  const int t_begin = blockIdx.z * per;
  const int t_end = min(total_tiles, t_begin + per);

  f32x16 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  using LoaderA = std::conditional_t<AT, DmaLoaderT<BM, BKT, NT, CPA>, DmaLoader<BM, BKT, NT, false, CPA>>;
  using LoaderB = std::conditional_t<BT, DmaLoaderT<BN, BKT, NT, CPB>, DmaLoader<BN, BKT, NT, BMODE == B_DUAL, CPB>>;
  LoaderA la;
  LoaderB lb;
  auto setup_seg = [&](int s) {
    const Seg& sg = args.segs[s];
    if constexpr (AT) la.setup(sg.a, sg.lda, m0, [&](int r) { return m0 + r < M; });
    else la.setup(sg.a, sg.a, sg.lda, m0, [&](int q, int) -> int64_t { return m0 + q < M ? q : -1; });
    if constexpr (BT) {
      lb.setup(sg.b, sg.ldb, n0 - sg.n_lo, [&](int r) {
        const int64_t n = n0 + r;
        return n < args.N && n >= sg.n_lo && n < sg.n_hi;
      });
    } else if constexpr (BMODE == B_DUAL) {
      lb.setup(sg.b, sg.b2, sg.ldb, n0, [&](int q, int) -> int64_t {
        const int t4 = (q % 128) / 32;
        const int rel = (q / 128) * 64 + (t4 / 2) * 32 + q % 32;
        return n0 + rel < args.N ? rel : -1;
      });
    } else {
      const int64_t off = n0 - sg.n_lo;
      lb.setup(sg.b, sg.b, sg.ldb, off, [&](int q, int) -> int64_t {
        const int64_t n = n0 + q;
        return (n < args.N && n >= sg.n_lo && n < sg.n_hi) ? q : -1;
      });
    }
  };
  int cur_s = 0, cur_t = t_begin;
  {
    int acc_t = 0;
    while (cur_s < args.n_segs && cur_t >= acc_t + seg_tiles[cur_s]) { acc_t += seg_tiles[cur_s]; ++cur_s; }
    cur_t -= acc_t;
  }
  int64_t seg_k = 0;
  int cur_n = 0;
  auto next_tile = [&](bool first) {
    if (!first) {
      ++cur_t;
      if (cur_t >= cur_n) {
        do { ++cur_s; } while (seg_tiles[cur_s] == 0);
        cur_t = 0;
        cur_n = seg_tiles[cur_s];
        setup_seg(cur_s);
        seg_k = args.segs[cur_s].k;
      }
    } else {
      cur_n = seg_tiles[cur_s];
      setup_seg(cur_s);
      seg_k = args.segs[cur_s].k;
    }
  };
  auto issue = [&](int slot) {
    const int64_t k0 = (int64_t)cur_t * BKT;
    char* st = smem + slot * STAGE;
    la.load(k0, seg_k - k0, st);
    lb.load(k0, seg_k - k0, st + A_BYTES);
  };

  // per-lane fragment offsets: row (wave tile + lane % 32), chunk 2 ks + lane / 32, swizzled
  const int hi = lane / 32;
  const int g = swz<BKT>(lane % 32) ^ hi;          // chunk ^ swz = 2 ks ^ g
  const int a_row = (wm * TM + lane % 32) * RB;
  const int b_row = A_BYTES + (wn * TN + lane % 32) * RB;
  // token-major stages: k-row pitches and this lane's transposed-read offsets
  constexpr int RBA = BM * 2, RBB = BN * 2;
  int a_tr[FM], b_tr[FN];
#pragma unroll
  for (int i = 0; i < FM; ++i) a_tr[i] = AT ? tr_lane_offset<BM / 8>(wm * TM + 32 * i, lane) : 0;
#pragma unroll
  for (int j = 0; j < FN; ++j) b_tr[j] = BT ? A_BYTES + tr_lane_offset<BN / 8>(wn * TN + 32 * j, lane) : 0;
  constexpr int RD = (AT ? 2 : 1) * FM + (BT ? 2 : 1) * FN;  // LDS read instructions per k step
  auto compute = [&](int slot) {
    const char* st = smem + slot * STAGE;
    constexpr int KS = BKT / 16;
    bf16x8 af[2][FM], bfr[2][FN];
    auto read_frags = [&](int ks, int sl) {
      const int ko = ((2 * ks) ^ g) << 4;
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        if constexpr (AT) {
          const char* p = st + a_tr[i] + 16 * ks * RBA;
          af[sl][i] = tr_frag(p, p + 4 * RBA);
        } else {
          af[sl][i] = *reinterpret_cast<const bf16x8*>(st + a_row + i * 32 * RB + ko);
        }
      }
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        if constexpr (BT) {
          const char* p = st + b_tr[j] + 16 * ks * RBB;
          bfr[sl][j] = tr_frag(p, p + 4 * RBB);
        } else {
          bfr[sl][j] = *reinterpret_cast<const bf16x8*>(st + b_row + j * 32 * RB + ko);
        }
      }
    };
    read_frags(0, 0);
    if (KS > 1) read_frags(1, 1);
    __builtin_amdgcn_sched_group_barrier(SG_DS_READ, (KS > 1 ? 2 : 1) * RD, 0);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int sl = ks & 1;
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[sl][i], bfr[sl][j], acc[i][j], 0, 0, 0);
      __builtin_amdgcn_sched_group_barrier(SG_MFMA, FM * FN, 0);
      if (ks + 2 < KS) {
        read_frags(ks + 2, sl);
        __builtin_amdgcn_sched_group_barrier(SG_DS_READ, RD, 0);
      }
    }
  };

  constexpr int PER_TILE = LoaderA::IPW + LoaderB::IPW;
  const int n_t = t_end - t_begin;
  if (n_t > 0) {
    // prologue: tiles 0 .. NSTAGE-2 in flight
#pragma unroll
    for (int p = 0; p < NSTAGE - 1; ++p) {
      if (p < n_t) {
        next_tile(p == 0);
        issue(p);
      }
    }
    for (int t = 0; t < n_t; ++t) {
      // tile t landed when at most min(NSTAGE-2, n_t-1-t) later tiles are outstanding
      if (n_t - 1 - t >= NSTAGE - 2) wait_vmcnt<(NSTAGE - 2) * PER_TILE>();
      else wait_vmcnt<0>();
      // every wave has waited for its own part of tile t (vmcnt above), so
      // after the barrier the whole tile is in LDS and slot (t-1) % NSTAGE is
      // free.  A bare s_barrier: __syncthreads()'s release fence would make
      // the compiler drain every outstanding LDS-DMA (vmcnt(0)) here and
      // collapse the ring to one tile in flight.  The empty asm keeps LDS
      // accesses from moving across the barrier at compile time.
      asm volatile("" ::: "memory");
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
      if (t + NSTAGE - 1 < n_t) {
        next_tile(false);
        issue((t + NSTAGE - 1) % NSTAGE);
      }
      compute(t % NSTAGE);
    }
  }
  if constexpr (STAGED) {
    static_assert(staged_ok(BM, BN, WAVES_M, WAVES_N, EPI), "staged epilogue: 256 x 256 tile, wave tiles of <= 128 rows");
    epilogue_staged<WAVES_M, WAVES_N, BMODE, EPI>(args, acc, m0, n0, lane, wm, wn, reinterpret_cast<float*>(smem));
  } else {
    epilogue<BM, BN, WAVES_M, WAVES_N, BMODE, EPI>(args, acc, m0, n0, lane, wm, wn);
  }
}

// Launches one GEMM with tile config `cfg` (-1 = pick from the shape).
int run(int cfg, int a_layout, int b_layout, int epi, const GemmArgs& a, hipStream_t s);

}  // namespace fgemm
