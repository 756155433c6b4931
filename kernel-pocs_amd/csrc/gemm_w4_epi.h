// Epilogues of the 4-wave GEMM engine (gemm_w4.h).
//
// The engine issues its MFMAs with the operands swapped (each 32 x 32 block
// is computed as B_tile A_tile^T, i.e. C^T), so that a lane's accumulators
// hold runs of four consecutive output COLUMNS of one row:
//   acc[i][j][r] of lane l = C[m][n],  m = m0 + 128 wm + 32 i + l % 32,
//   n = colbase(j) + 8 (r / 4) + 4 (l / 32) + r % 4
// with colbase(j) = n0 + 128 wn + 32 j for a single B, and for the dual
// gate / up B (wave tile j = gate for even j, up for odd j) the output
// columns n0 + 64 wn + 32 (j / 2) + ...
// (With A and B in the usual order a lane holds four consecutive ROWS of one
// column, so staging a tile took 256 scattered 4-byte LDS writes per lane.)
//
// Staged epilogues (bf16 outputs; the hot path): the tile goes through LDS
// as bf16, 8 bytes per lane per write, all four waves at once, so that every
// thread then reads side inputs and writes outputs as 16-byte vectors.
// Staging in bf16 loses nothing: each of them rounds its GEMM result to bf16
// before any further arithmetic (STORE, RoPE, the GLU backward's DW) or
// computes its fp32 result in registers before staging (the GLU forward's h,
// the STORE activation and alpha).  Measured on MI355X, epilogue alone over a
// whole 8192 x 14336 output (K = 0 launches): fp32 staging of 128-row halves
// 16.2 us per round of 256 tiles.
//
// The direct epilogue (fp32 and atomic outputs, beta != 0, and buffers whose
// alignment rules out 16-byte vectors) works per element from registers.
#pragma once

#include "gemm_core.h"

namespace fgemm {

constexpr int W4_SP = 256 + 8;  // staged bf16 row, single B: 528 bytes (rows 4 banks apart)
constexpr int W4_DP = 128 + 8;  // staged bf16 row of one dual-B output (e, g or h)
constexpr int W4_STAGE_BYTES = 256 * W4_SP * 2;       // single B: the whole tile
constexpr int W4_DUAL_BYTES = 3 * 128 * W4_DP * 2;    // dual B: e, g, h of 128 rows

// Epilogues staged through LDS (with ep.vec_ok; STORE_BF16 only with a plain
// alpha: no beta, no activation, no per-column alpha groups).
constexpr bool w4_staged_epi(int epi) {
  return epi == EPI_STORE_BF16 || epi == EPI_ROPE || glu_fwd_epi(epi) || glu_bwd_epi(epi);
}

__device__ __forceinline__ uint2 pack4(const float (&f)[4]) {
  uint32_t w[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const __bf16 lo = (__bf16)f[2 * i], hi = (__bf16)f[2 * i + 1];
    w[i] = (uint32_t)__builtin_bit_cast(uint16_t, lo) | ((uint32_t)__builtin_bit_cast(uint16_t, hi) << 16);
  }
  return make_uint2(w[0], w[1]);
}

__device__ __forceinline__ float col_alpha(const EpiArgs& ep, int64_t n) {
  if (ep.alpha_group > 0) {
    const int64_t grp = n / ep.alpha_group;
    return ep.alphas[grp < 4 ? grp : 3];
  }
  return ep.alpha;
}

// ---------------------------------------------------------------------------
// Direct epilogue: every element from registers, bounds-checked.
// ---------------------------------------------------------------------------
template <int BMODE, int EPI>
__device__ __forceinline__ void w4_epilogue_direct(const GemmArgs& args, f32x16 (&acc)[4][4], int64_t m0, int64_t n0,
                                                   int lane, int wm, int wn) {
  const EpiArgs& ep = args.ep;
  const int64_t M = args.M, N = args.N;
  const int cl = 4 * (lane / 32);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t m = m0 + wm * 128 + i * 32 + lane % 32;
    if (m >= M) continue;
    if constexpr (glu_fwd_epi(EPI)) {
#pragma unroll
      for (int jp = 0; jp < 2; ++jp)
#pragma unroll
        for (int g = 0; g < 4; ++g)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int64_t n = n0 + wn * 64 + 32 * jp + 8 * g + cl + q;
            if (n >= N) continue;
            const float e = acc[i][2 * jp][4 * g + q], gg = acc[i][2 * jp + 1][4 * g + q];
            const int64_t off = m * ep.ld_eg + n;
            if (ep.e) {
              ep.e[off] = (__bf16)e;
              ep.g[off] = (__bf16)gg;
            }
            ((__bf16*)ep.c)[m * ep.ldc + n] = (__bf16)glu_fwd_h<EPI>(e, gg);
          }
    } else if constexpr (EPI == EPI_ROPE) {
      const int64_t pos = ep.positions ? ep.positions[m] : m;
      const bool pos_ok = pos >= 0 && pos < ep.cs_rows;
      const int half_tiles = ep.head_dim / 64;  // partner distance in 32-column tiles
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int g = 0; g < 4; ++g)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int64_t n = n0 + wn * 128 + 32 * j + 8 * g + cl + q;
            if (n >= N) continue;
            float v = acc[i][j][4 * g + q];
            if (n < ep.rope_cols) {
              const bool lo = (j % (2 * half_tiles)) < half_tiles;
              const int partner = lo ? j + half_tiles : j - half_tiles;
              float pv = 0.f;
#pragma unroll
              for (int t = 0; t < 4; ++t)
                if (t == partner) pv = acc[i][t][4 * g + q];
              const int d = (int)(n % ep.head_dim) % (ep.head_dim / 2);
              const float c = pos_ok ? (float)ep.cos[pos * ep.cs_ld + d] : __builtin_nanf("");
              const float s = pos_ok ? (float)ep.sin[pos * ep.cs_ld + d] : __builtin_nanf("");
              // the projection is rounded to bf16 first: RoPE is applied to the
              // materialised Q/K in the unfused reference path
              const float x = bf16r(v), xp = bf16r(pv);
              v = lo ? x * c - xp * s : x * c + xp * s;
            }
            ((__bf16*)ep.c)[m * ep.ldc + n] = (__bf16)v;
          }
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int64_t nb = n0 + wn * 128 + 32 * j + 8 * g + cl;
          if (nb >= N) continue;
          if constexpr (EPI == EPI_STORE_F32) {
            float* cp = (float*)ep.c + (int64_t)blockIdx.z * ep.split_stride + m * ep.ldc + nb;
            float v[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) v[q] = col_alpha(ep, nb + q) * acc[i][j][4 * g + q];
            if (ep.vec_ok && nb + 4 <= N) {  // 16-byte aligned: ldc % 8 == 0, nb % 4 == 0
              float4* c4 = reinterpret_cast<float4*>(cp);
              if (ep.beta != 0.f) {
                const float4 o = *c4;
                v[0] += ep.beta * o.x; v[1] += ep.beta * o.y; v[2] += ep.beta * o.z; v[3] += ep.beta * o.w;
              }
              if (ep.act)
#pragma unroll
                for (int q = 0; q < 4; ++q) v[q] = epi_act(ep.act, v[q]);
              *c4 = make_float4(v[0], v[1], v[2], v[3]);
            } else {
              for (int q = 0; q < 4 && nb + q < N; ++q) {
                float o = v[q];
                if (ep.beta != 0.f) o += ep.beta * cp[q];
                cp[q] = ep.act ? epi_act(ep.act, o) : o;
              }
            }
          } else if constexpr (EPI == EPI_ATOMIC_F32) {
            for (int q = 0; q < 4 && nb + q < N; ++q)
              atomicAdd((float*)ep.c + m * ep.ldc + nb + q, col_alpha(ep, nb + q) * acc[i][j][4 * g + q]);
          } else if constexpr (EPI == EPI_STORE_BF16) {
            __bf16* cp = (__bf16*)ep.c + m * ep.ldc + nb;
            for (int q = 0; q < 4 && nb + q < N; ++q) {
              float o = col_alpha(ep, nb + q) * acc[i][j][4 * g + q];
              if (ep.beta != 0.f) o += ep.beta * (float)cp[q];
              if (ep.act) o = epi_act(ep.act, o);
              cp[q] = (__bf16)o;
            }
          } else if constexpr (glu_bwd_epi(EPI)) {
            for (int q = 0; q < 4 && nb + q < N; ++q) {
              const int64_t off = m * ep.ld_eg + nb + q;
              float h, df, de;
              glu_bwd_vals<EPI>(acc[i][j][4 * g + q], (float)ep.e[off], (float)ep.g[off], h, df, de);
              ((__bf16*)ep.c)[m * ep.ldc + nb + q] = (__bf16)h;
              ep.e[off] = (__bf16)df;
              ep.g[off] = (__bf16)de;
            }
          }
        }
    }
  }
}

// ---------------------------------------------------------------------------
// RoPE over a staged Q/K tile (256 rows x 256 columns = 256 / HD whole heads):
// thread tid takes head-dimension chunk d = 8 (tid % DC) of the lo half and
// rows tid / DC + RS k.  One cos / sin load pair then serves the 2 * 256 / HD
// chunks of its row that share d (lo and hi of every head in the tile), and
// a thread's few rows are loaded at once, so the tables' latency is paid
// once per tile instead of once per group of rows (measured on MI355X at
// the LoRA-QKV BASELINE shape: a thread per 8-column chunk walking all 32
// of its rows, four rows' tables in flight, cost 125 us over a plain store).
// ---------------------------------------------------------------------------
template <int HD>
__device__ __forceinline__ void w4_rope_tile(const EpiArgs& ep, int64_t M, int64_t m0, int64_t n0,
                                             const __bf16* lds) {
  constexpr int HALF = HD / 2, DC = HALF / 8;  // 16-byte d-chunks per half
  constexpr int HPT = 256 / HD;                // heads per tile
  constexpr int RS = 256 / DC;                 // row sets
  constexpr int RPT = 256 / RS;                // rows per thread
  const int tid = threadIdx.x;
  const int d = (tid % DC) * 8;
  const int r0 = tid / DC;
  int pos[RPT];
#pragma unroll
  for (int k = 0; k < RPT; ++k) {
    const int64_t m = m0 + r0 + RS * k;
    const int64_t p = m < M ? (ep.positions ? ep.positions[m] : m) : -1;
    pos[k] = (p >= 0 && p < ep.cs_rows) ? (int)p : -1;
  }
  uint4 cv[RPT], sv[RPT];
#pragma unroll
  for (int k = 0; k < RPT; ++k)
    if (pos[k] >= 0) {
      cv[k] = ld16(ep.cos + (int64_t)pos[k] * ep.cs_ld + d);
      sv[k] = ld16(ep.sin + (int64_t)pos[k] * ep.cs_ld + d);
    }
#pragma unroll
  for (int k = 0; k < RPT; ++k) {
    const int rr = r0 + RS * k;
    const int64_t m = m0 + rr;
    if (m >= M) continue;
    float cs[8], sn[8];
    if (pos[k] >= 0) {
      unpack8(cv[k], cs);
      unpack8(sv[k], sn);
    } else {
#pragma unroll
      for (int t = 0; t < 8; ++t) cs[t] = sn[t] = __builtin_nanf("");
    }
    __bf16* crow = (__bf16*)ep.c + m * ep.ldc + n0;
#pragma unroll
    for (int h = 0; h < HPT; ++h) {
      const int cl = h * HD + d, ch = cl + HALF;
      float xl[8], xh[8], yl[8], yh[8];
      unpack8(*reinterpret_cast<const uint4*>(lds + rr * W4_SP + cl), xl);
      unpack8(*reinterpret_cast<const uint4*>(lds + rr * W4_SP + ch), xh);
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        yl[t] = xl[t] * cs[t] - xh[t] * sn[t];
        yh[t] = xh[t] * cs[t] + xl[t] * sn[t];
      }
      st16(crow + cl, pack8(yl));
      st16(crow + ch, pack8(yh));
    }
  }
}

// ---------------------------------------------------------------------------
// Rank-r partial product of a staged bf16 tile of ROWS x KCOLS (row pitch
// PITCH elements): vp[m][col0 + j] = sum over the tile's columns k of
// lds[m][k] bt[j][n0 + k] for j < r, with v_mfma_f32_16x16x32_bf16 (the
// ROWS / 16 row blocks split evenly over the 4 waves; each lane then holds
// four consecutive j of one row, stored as one 16-byte vector).  Columns at
// or past N read zeros from bt; rows at or past M are not stored.  Used for
// the LoRA rank-r products of the GEMMs' gated-activation epilogues: [df B_u |
// de B_g] in the backward (256 x 256 staged tiles), h A_d^T in the forward
// (128-row halves of 128 columns).
// ---------------------------------------------------------------------------
typedef float w4_f32x4 __attribute__((ext_vector_type(4)));

template <int RB, int ROWS, int KCOLS, int PITCH>
__device__ __forceinline__ void w4_rank_partial(const __bf16* lds, const __bf16* bt, int64_t ldbt, int r,
                                                int64_t N, int64_t n0, int64_t M, int64_t m0, float* vp,
                                                int64_t ldv, int col0) {
  constexpr int BPW = ROWS / 16 / 4;  // row blocks per wave
  constexpr int KS = KCOLS / 32;      // k-steps
  // bt fragments of KB k-steps are loaded before any of them is used, so the
  // L2 latency is paid once per batch, not once per k-step
  constexpr int KB = (KS * RB <= 8) ? KS : (8 / RB < 1 ? 1 : 8 / RB);
  static_assert(KS % KB == 0, "whole batches");
  const int lane = threadIdx.x % 64, wave = threadIdx.x / 64;
  w4_f32x4 acc[BPW][RB];
#pragma unroll
  for (int i = 0; i < BPW; ++i)
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) acc[i][rb] = w4_f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int kb = 0; kb < KS; kb += KB) {
    bf16x8 b[KB][RB];
#pragma unroll
    for (int u = 0; u < KB; ++u) {
      const int k = (kb + u) * 32 + (lane / 16) * 8;
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) {
        const int j = rb * 16 + lane % 16;
        if (j < r && n0 + k + 8 <= N) {
          b[u][rb] = *reinterpret_cast<const bf16x8*>(bt + (int64_t)j * ldbt + n0 + k);
        } else {
#pragma unroll
          for (int t = 0; t < 8; ++t) b[u][rb][t] = (__bf16)0.f;
        }
      }
    }
#pragma unroll
    for (int u = 0; u < KB; ++u) {
      const int k = (kb + u) * 32 + (lane / 16) * 8;
#pragma unroll
      for (int i = 0; i < BPW; ++i) {
        const int row = (wave * BPW + i) * 16 + lane % 16;
        const bf16x8 a = *reinterpret_cast<const bf16x8*>(lds + row * PITCH + k);
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
          acc[i][rb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(b[u][rb], a, acc[i][rb], 0, 0, 0);
      }
    }
  }
#pragma unroll
  for (int i = 0; i < BPW; ++i) {
    const int64_t m = m0 + (wave * BPW + i) * 16 + lane % 16;
    if (m >= M) continue;
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      const int j0 = rb * 16 + 4 * (lane / 16);
      if (j0 < r) *reinterpret_cast<w4_f32x4*>(vp + m * ldv + col0 + j0) = acc[i][rb];
    }
  }
}

// ---------------------------------------------------------------------------
// Token-reduction partial product of a staged bf16 tile of 256 rows (tokens)
// x 256 columns (row pitch PITCH elements):
//   wp[c * ldw + col0 + j] = sum over the tile's rows t of lds[t][c] xt[j][m0 + t]
// for j < r and the tile's columns c with n0 + c < N, with
// v_mfma_f32_16x16x32_bf16.  The column operand (8 consecutive rows of one
// column per lane) is read with ds_read_b64_tr_b16, which transposes within
// each 16-lane group: lane L of group g supplies the 8 bytes at row
// 32 ks + 8 g + L / 4 (+ 4 for the second read), columns 16 cb + 4 (L % 4),
// and result lane 16 g + i receives (row 32 ks + 8 g + q, column 16 cb + i).
// xt is token-contiguous ([r][tokens], pitch ldxt); tokens at or past M read
// zeros.  Each wave takes 4 of the 16 column blocks; each lane then holds four
// consecutive j of one column, stored as one 16-byte vector.  Used for the
// LoRA B gradients of the GLU backward epilogue: df^T xa_u and de^T xa_g.
// ---------------------------------------------------------------------------
template <int RB, int PITCH>
__device__ __forceinline__ void w4_token_partial(const __bf16* lds, const __bf16* xt, int64_t ldxt, int r,
                                                 int64_t N, int64_t n0, int64_t M, int64_t m0, float* wp,
                                                 int64_t ldw, int col0) {
  constexpr int BPW = 4;  // column blocks of 16 per wave
  constexpr int KS = 8;   // 32-row k-steps
  constexpr int KB = (RB == 1) ? 8 : (RB == 2 ? 4 : 2);  // xt fragments loaded per batch
  const int lane = threadIdx.x % 64, wave = threadIdx.x / 64;
  const int g = lane / 16, L = lane % 16;
  w4_f32x4 acc[BPW][RB];
#pragma unroll
  for (int i = 0; i < BPW; ++i)
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) acc[i][rb] = w4_f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int kb = 0; kb < KS; kb += KB) {
    bf16x8 b[KB][RB];
#pragma unroll
    for (int u = 0; u < KB; ++u) {
      const int64_t m = m0 + (kb + u) * 32 + 8 * g;
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) {
        const int j = rb * 16 + L;
        if (j < r && m + 8 <= M) {
          b[u][rb] = *reinterpret_cast<const bf16x8*>(xt + (int64_t)j * ldxt + m);
        } else {
#pragma unroll
          for (int t = 0; t < 8; ++t) b[u][rb][t] = (j < r && m + t < M) ? xt[(int64_t)j * ldxt + m + t] : (__bf16)0.f;
        }
      }
    }
#pragma unroll
    for (int u = 0; u < KB; ++u) {
      const int row = (kb + u) * 32 + 8 * g + L / 4;
#pragma unroll
      for (int i = 0; i < BPW; ++i) {
        const __bf16* p0 = lds + row * PITCH + (wave * BPW + i) * 16 + 4 * (L % 4);
        const bf16x8 a = tr_frag((const char*)p0, (const char*)(p0 + 4 * PITCH));
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
          acc[i][rb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(b[u][rb], a, acc[i][rb], 0, 0, 0);
      }
    }
  }
#pragma unroll
  for (int i = 0; i < BPW; ++i) {
    const int64_t n = n0 + (wave * BPW + i) * 16 + L;
    if (n >= N) continue;
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      const int j0 = rb * 16 + 4 * g;
      if (j0 < r) *reinterpret_cast<w4_f32x4*>(wp + (n - n0) * ldw + col0 + j0) = acc[i][rb];
    }
  }
}

template <int PITCH>
__device__ __forceinline__ void w4_token_partial_any(const __bf16* lds, const __bf16* xt, int64_t ldxt, int r,
                                                     int64_t N, int64_t n0, int64_t M, int64_t m0, float* wp,
                                                     int64_t ldw, int col0) {
  if (r <= 16) w4_token_partial<1, PITCH>(lds, xt, ldxt, r, N, n0, M, m0, wp, ldw, col0);
  else if (r <= 32) w4_token_partial<2, PITCH>(lds, xt, ldxt, r, N, n0, M, m0, wp, ldw, col0);
  else w4_token_partial<4, PITCH>(lds, xt, ldxt, r, N, n0, M, m0, wp, ldw, col0);
}

template <int ROWS, int KCOLS, int PITCH>
__device__ __forceinline__ void w4_rank_partial_any(const __bf16* lds, const __bf16* bt, int64_t ldbt, int r,
                                                    int64_t N, int64_t n0, int64_t M, int64_t m0, float* vp,
                                                    int64_t ldv, int col0) {
  if (r <= 16) w4_rank_partial<1, ROWS, KCOLS, PITCH>(lds, bt, ldbt, r, N, n0, M, m0, vp, ldv, col0);
  else if (r <= 32) w4_rank_partial<2, ROWS, KCOLS, PITCH>(lds, bt, ldbt, r, N, n0, M, m0, vp, ldv, col0);
  else w4_rank_partial<4, ROWS, KCOLS, PITCH>(lds, bt, ldbt, r, N, n0, M, m0, vp, ldv, col0);
}

// ---------------------------------------------------------------------------
// Staged epilogue, single B (STORE_BF16 at beta = 0, ROPE, GLU backward):
// the whole 256 x 256 tile in LDS as bf16, then each thread owns column chunk
// c = 8 (tid % 32) and walks rows tid / 32 + 8 it.
// ---------------------------------------------------------------------------
template <int EPI>
__device__ __forceinline__ void w4_epilogue_staged(const GemmArgs& args, f32x16 (&acc)[4][4], int64_t m0, int64_t n0,
                                                   int lane, int wm, int wn, __bf16* lds) {
  const EpiArgs& ep = args.ep;
  const int64_t M = args.M, N = args.N;
  const int tid = threadIdx.x;
  const int cl = 4 * (lane / 32);
  lds_barrier();  // the main loop's LDS reads are done (its DMAs drained before)
  // STORE_BF16 scales by alpha (the host launches per-column alpha groups,
  // activations and beta != 0 on the direct epilogue)
  const float alpha = EPI == EPI_STORE_BF16 ? ep.alpha : 1.f;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        float v[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) v[q] = alpha * acc[i][j][4 * g + q];
        *reinterpret_cast<uint2*>(lds + (wm * 128 + i * 32 + lane % 32) * W4_SP + wn * 128 + 32 * j + 8 * g + cl) =
            pack4(v);
      }
  lds_barrier();
  constexpr int IT = 256 / 8, GRP = 4;  // rows per thread; side inputs of 4 rows in flight
  const int c = (tid % 32) * 8;
  const int64_t n = n0 + c;
  const bool full = n + 8 <= N;
  if constexpr (EPI == EPI_STORE_BF16) {
#pragma unroll 4
    for (int it = 0; it < IT; ++it) {
      const int rr = it * 8 + tid / 32;
      const int64_t m = m0 + rr;
      if (m >= M || n >= N) continue;
      const uint4 v = *reinterpret_cast<const uint4*>(lds + rr * W4_SP + c);
      __bf16* cp = (__bf16*)ep.c + m * ep.ldc + n;
      if (full) {
        st16(cp, v);
      } else {
        const __bf16* pv = lds + rr * W4_SP + c;
        for (int q = 0; q < 8 && n + q < N; ++q) cp[q] = pv[q];
      }
    }
  } else if constexpr (glu_bwd_epi(EPI)) {
    // With ep.vpart the rank-r products [df B_u | de B_g] of this tile's
    // columns (and with ep.wpart the token products df^T xa_u, de^T xa_g of
    // its rows) are formed here from df and de as they are produced, instead
    // of by later passes that stream both [M, I] tensors again: df goes into
    // the staged tile in place of DW (each thread overwrites only the chunk it
    // read), de stays in registers until the df product is done and then
    // replaces df.
    const bool vp = ep.vpart != nullptr;
    uint4 de_keep[IT];
    // the saved e / g chunks of four rows are read before any of them is used
#pragma unroll
    for (int g0 = 0; g0 < IT; g0 += GRP) {
      uint4 ew[GRP], gw[GRP];
#pragma unroll
      for (int q = 0; q < GRP; ++q) {
        const int64_t m = m0 + (g0 + q) * 8 + tid / 32;
        if (m < M && full) {
          const int64_t off = m * ep.ld_eg + n;
          ew[q] = ld16(ep.e + off);
          gw[q] = ld16(ep.g + off);
        }
      }
#pragma unroll
      for (int q = 0; q < GRP; ++q) {
        const int rr = (g0 + q) * 8 + tid / 32;
        const int64_t m = m0 + rr;
        if (m >= M || n >= N) continue;
        const int64_t off = m * ep.ld_eg + n;
        float dw[8], ev[8], gv[8], hv[8], dfv[8], dev[8];
        unpack8(*reinterpret_cast<const uint4*>(lds + rr * W4_SP + c), dw);
        if (full) {
          unpack8(ew[q], ev);
          unpack8(gw[q], gv);
        } else {
          for (int t = 0; t < 8; ++t) {
            ev[t] = n + t < N ? (float)ep.e[off + t] : 0.f;
            gv[t] = n + t < N ? (float)ep.g[off + t] : 0.f;
          }
        }
#pragma unroll
        for (int t = 0; t < 8; ++t) glu_bwd_vals<EPI>(dw[t], ev[t], gv[t], hv[t], dfv[t], dev[t]);
        const uint4 dfp = pack8(dfv), dep = pack8(dev);
        if (full) {
          st16((__bf16*)ep.c + m * ep.ldc + n, pack8(hv));
          st16(ep.e + off, dfp);
          st16(ep.g + off, dep);
        } else {
          for (int t = 0; t < 8 && n + t < N; ++t) {
            ((__bf16*)ep.c)[m * ep.ldc + n + t] = (__bf16)hv[t];
            ep.e[off + t] = (__bf16)dfv[t];
            ep.g[off + t] = (__bf16)dev[t];
          }
        }
        if (vp) {
          *reinterpret_cast<uint4*>(lds + rr * W4_SP + c) = dfp;
          de_keep[g0 + q] = dep;
        }
      }
    }
    if (vp) {
      // (rows and columns outside the output hold the staged zeros of DW:
      // their operand rows and columns were read as zeros)
      float* part = ep.vpart + (n0 / 256) * ep.vpart_stride;
      const int r = ep.vr;
      lds_barrier();  // df of the whole tile staged
      w4_rank_partial_any<256, 256, W4_SP>(lds, ep.vbt[0], ep.vbt_ld, r, N, n0, M, m0, part, 2 * r, 0);
      float* wpart = ep.wpart ? ep.wpart + (m0 / 256) * ep.wpart_stride + n0 * r : nullptr;
      if (wpart) w4_token_partial_any<W4_SP>(lds, ep.wxt[0], ep.wxt_ld, r, N, n0, M, m0, wpart, r, 0);
      lds_barrier();  // every wave is done reading df
#pragma unroll
      for (int it = 0; it < IT; ++it) {
        const int rr = it * 8 + tid / 32;
        if (m0 + rr < M && n < N) *reinterpret_cast<uint4*>(lds + rr * W4_SP + c) = de_keep[it];
      }
      lds_barrier();
      w4_rank_partial_any<256, 256, W4_SP>(lds, ep.vbt[1], ep.vbt_ld, r, N, n0, M, m0, part, 2 * r, r);
      if (wpart) w4_token_partial_any<W4_SP>(lds, ep.wxt[1], ep.wxt_ld, r, N, n0, M, m0, wpart + N * r, r, 0);
    }
  } else {  // EPI_ROPE
    // Q / K tiles (the host launches the RoPE epilogue only when Q and K are
    // whole 256-column tiles and head_dim is 64 or 128)
    if (n0 < ep.rope_cols && n0 + 256 <= N) {
      if (ep.head_dim == 128) w4_rope_tile<128>(ep, M, m0, n0, lds);
      else w4_rope_tile<64>(ep, M, m0, n0, lds);
      return;
    }
    // V tiles (and any other shape): a thread per 8-column chunk
    const bool rot = n < N && n < ep.rope_cols;
    const int half = ep.head_dim / 2;
    const int in_head = (int)(n % ep.head_dim);
    const bool lo = in_head < half;
    const int d = in_head % half;
    const int pc = lo ? c + half : c - half;  // partner chunk (the 256-column tile holds whole heads)
    int64_t posv[IT];
#pragma unroll
    for (int it = 0; it < IT; ++it) {
      const int64_t m = m0 + it * 8 + tid / 32;
      posv[it] = (rot && m < M) ? (ep.positions ? ep.positions[m] : m) : -1;
    }
#pragma unroll
    for (int g0 = 0; g0 < IT; g0 += GRP) {
      uint4 cv[GRP], sv[GRP];
#pragma unroll
      for (int q = 0; q < GRP; ++q) {
        const int64_t pos = posv[g0 + q];
        if (pos >= 0 && pos < ep.cs_rows) {
          cv[q] = ld16(ep.cos + pos * ep.cs_ld + d);
          sv[q] = ld16(ep.sin + pos * ep.cs_ld + d);
        }
      }
#pragma unroll
      for (int q = 0; q < GRP; ++q) {
        const int rr = (g0 + q) * 8 + tid / 32;
        const int64_t m = m0 + rr;
        if (m >= M || n >= N) continue;
        float v[8];
        unpack8(*reinterpret_cast<const uint4*>(lds + rr * W4_SP + c), v);
        if (rot) {
          float pv[8], cs[8], sn[8];
          unpack8(*reinterpret_cast<const uint4*>(lds + rr * W4_SP + pc), pv);
          const int64_t pos = posv[g0 + q];
          if (pos >= 0 && pos < ep.cs_rows) {
            unpack8(cv[q], cs);
            unpack8(sv[q], sn);
          } else {
#pragma unroll
            for (int t = 0; t < 8; ++t) cs[t] = sn[t] = __builtin_nanf("");
          }
#pragma unroll
          for (int t = 0; t < 8; ++t) v[t] = lo ? v[t] * cs[t] - pv[t] * sn[t] : v[t] * cs[t] + pv[t] * sn[t];
        }
        __bf16* cp = (__bf16*)ep.c + m * ep.ldc + n;
        if (full) st16(cp, pack8(v));
        else
          for (int t = 0; t < 8 && n + t < N; ++t) cp[t] = (__bf16)v[t];
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Staged epilogue, dual B (GLU forward): e, g and h = glu(e, g) of one
// 128-row half at a time (three [128][128] bf16 buffers); h is formed in
// registers from the fp32 accumulators before anything is rounded.
// ---------------------------------------------------------------------------
template <int EPI>
__device__ __forceinline__ void w4_epilogue_staged_dual(const GemmArgs& args, f32x16 (&acc)[4][4], int64_t m0,
                                                        int64_t n0, int lane, int wm, int wn, __bf16* lds) {
  const EpiArgs& ep = args.ep;
  const int64_t M = args.M, N = args.N;
  const int tid = threadIdx.x;
  const int cl = 4 * (lane / 32);
  __bf16* le = lds;
  __bf16* lg = lds + 128 * W4_DP;
  __bf16* lh = lds + 2 * 128 * W4_DP;
  lds_barrier();  // the main loop's LDS reads are done
#pragma unroll 1
  for (int pass = 0; pass < 2; ++pass) {
    if (pass) lds_barrier();  // pass 0's readers are done with the buffers
    if (wm == pass) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = i * 32 + lane % 32;
#pragma unroll
        for (int jp = 0; jp < 2; ++jp)
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const int col = wn * 64 + 32 * jp + 8 * g + cl;
            float e[4], gg[4], h[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              e[q] = acc[i][2 * jp][4 * g + q];
              gg[q] = acc[i][2 * jp + 1][4 * g + q];
              h[q] = glu_fwd_h<EPI>(e[q], gg[q]);
            }
            *reinterpret_cast<uint2*>(le + row * W4_DP + col) = pack4(e);
            *reinterpret_cast<uint2*>(lg + row * W4_DP + col) = pack4(gg);
            *reinterpret_cast<uint2*>(lh + row * W4_DP + col) = pack4(h);
          }
      }
    }
    lds_barrier();
    const int64_t mrow0 = m0 + pass * 128;
    // forward LoRA: this half's partial of h A_d^T over the tile's 128 h
    // columns (one slice per column tile), read from the staged h
    if (ep.vpart)
      w4_rank_partial_any<128, 128, W4_DP>(lh, ep.vbt[0], ep.vbt_ld, ep.vr, N, n0, M, mrow0,
                                           ep.vpart + (n0 / 128) * ep.vpart_stride, ep.vr, 0);
#pragma unroll 2
    for (int it = 0; it < 128 * 16 / 256; ++it) {
      const int id = it * 256 + tid;
      const int rr = id / 16, c = (id % 16) * 8;
      const int64_t m = mrow0 + rr, n = n0 + c;
      if (m >= M || n >= N) continue;
      const int o = rr * W4_DP + c;
      const int64_t off = m * ep.ld_eg + n;
      __bf16* hp = (__bf16*)ep.c + m * ep.ldc + n;
      if (n + 8 <= N) {
        if (ep.e) {  // training saves e and g; inference (e = g = null) stores h only
          st16(ep.e + off, *reinterpret_cast<const uint4*>(le + o));
          st16(ep.g + off, *reinterpret_cast<const uint4*>(lg + o));
        }
        st16(hp, *reinterpret_cast<const uint4*>(lh + o));
      } else {
        for (int q = 0; q < 8 && n + q < N; ++q) {
          if (ep.e) {
            ep.e[off + q] = le[o + q];
            ep.g[off + q] = lg[o + q];
          }
          hp[q] = lh[o + q];
        }
      }
    }
  }
}

}  // namespace fgemm
