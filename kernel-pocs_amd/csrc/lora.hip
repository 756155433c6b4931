// Fused LoRA entry points built on the MFMA GEMM core.
//
// LoRA-MLP (reference: kernels/lora_mlp/experiments/v6/lora_mlp_kernel_v6.py
// :335-451 forward, :592-672 backward; math of
// kernels/lora_mlp/reference/lora_mlp_pytorch.py:111-225):
//   forward  e = X Wg^T + sg (X Ag^T) Bg^T,  g = X Wu^T + su (X Au^T) Bu^T,
//            h = silu(e) * g                      -> forge_lora_mlp_gate_up
//   backward DW = dY Wd + sd (dY Bd) Ad, then the in-place SwiGLU backward
//            (DW, e, g) -> (h, df, de)            -> forge_lora_mlp_down_bwd
// The same two entry points take the GeGLU activation (tanh or exact GELU)
// for Gemma MLPs, replacing the reference's layered path there (PEFT
// projections + the GeGLU kernel, forge/forge/patching/kernels/lora.py:170-188).
// LoRA-QKV (reference: kernels/lora_qkv/experiments/v2/lora_qkv_kernel_v2_3.py
// :177-267 + the caller's RoPE, forge/forge/patching/kernels/lora.py:250-264):
//   [Q | K | V] = X [Wq; Wk; Wv]^T + per-projection LoRA, RoPE on Q and K
//                                                  -> forge_lora_qkv_rope
// The LoRA-A products (X A^T, dY B, ...) arrive pre-scaled by s from the
// caller (computed with forge_gemm); the LoRA-B product rides along the base
// GEMM as one more K segment.
#include <mutex>

#include "gemm_core.h"

using namespace fgemm;

namespace {

// FORGE_ACT_* -> the forward / backward GLU epilogue (-1: unknown)
int glu_epi(int activation, bool backward) {
  switch (activation) {
    case FORGE_ACT_SILU: return backward ? EPI_SWIGLU_BWD : EPI_SWIGLU_FWD;
    case FORGE_ACT_GELU_TANH: return backward ? EPI_GEGLU_TANH_BWD : EPI_GEGLU_TANH_FWD;
    case FORGE_ACT_GELU_ERF: return backward ? EPI_GEGLU_ERF_BWD : EPI_GEGLU_ERF_FWD;
  }
  return -1;
}

constexpr int kGluBlock = 256;
constexpr int kGluMaxBlocks = 256 * 64;

// The gated-activation backward of the down-projection epilogue as a kernel
// of its own: (D, e, g) -> (h, df, de), df and de over e and g, with the
// epilogue's per-element formula (glu_bwd_vals; its rounding of D to bf16 is
// exact on a bf16 input, so the results equal the fused epilogue's for equal
// D).  For SiLU this is Unsloth's in-place `_DWf_DW_dfg_kernel`
// (kernels/lora_mlp/reference/unsloth_baseline.py:118-168) on a D that the
// caller computed.
template <int EPI>
__global__ __launch_bounds__(kGluBlock) void lora_glu_bwd_kernel(const __bf16* d, int64_t ld_d, __bf16* e, __bf16* g,
                                                                 int64_t ld_eg, __bf16* h, int64_t ld_h, int64_t rows,
                                                                 int64_t cols) {
  const int64_t cpr = cols / 8, n = rows * cpr;
  for (int64_t i = (int64_t)blockIdx.x * kGluBlock + threadIdx.x; i < n; i += (int64_t)gridDim.x * kGluBlock) {
    const int64_t r = i / cpr, c = (i - r * cpr) * 8;
    const Vec16<__bf16> dv = load16(d + r * ld_d + c), ev = load16(e + r * ld_eg + c), gv = load16(g + r * ld_eg + c);
    Vec16<__bf16> hv, dfv, dev;
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      float hh, du, dg;
      glu_bwd_vals<EPI>((float)dv.v[q], (float)ev.v[q], (float)gv.v[q], hh, du, dg);
      hv.v[q] = (__bf16)hh;
      dfv.v[q] = (__bf16)du;
      dev.v[q] = (__bf16)dg;
    }
    store16(h + r * ld_h + c, hv);
    store16(e + r * ld_eg + c, dfv);
    store16(g + r * ld_eg + c, dev);
  }
}

}  // namespace

static int gate_up(int64_t M, int64_t H, int64_t I, int64_t r, const void* x, int64_t ldx, const void* w_gate,
                   const void* w_up, int64_t ldw, const void* xa, int64_t ld_xa, const void* b_gate, const void* b_up,
                   int64_t ldb, void* e, void* g, void* h, int64_t ld_out, int activation, const void* a_down,
                   int64_t ld_ad, int64_t rd, float* v_part, void* stream) {
  if (M < 0 || H < 0 || I < 0 || r < 0) return forge_set_error(FORGE_ERR_INVALID, "lora_mlp_gate_up: shape");
  const int epi = glu_epi(activation, false);
  if (epi < 0) return forge_set_error(FORGE_ERR_INVALID, "lora_mlp_gate_up: activation %d", activation);
  if ((e == nullptr) != (g == nullptr))
    return forge_set_error(FORGE_ERR_INVALID, "lora_mlp_gate_up: e and g are both given or both NULL");
  GemmArgs a = {};
  a.M = M;
  a.N = I;
  a.split_k = 1;
  int ns = 0;
  a.segs[ns++] = Seg{(const __bf16*)x, ldx, (const __bf16*)w_gate, (const __bf16*)w_up, ldw, H, 0, I};
  if (r > 0 && xa) {
    // one K segment of 2r: gate rows take xa[:, :r] Bg^T, up rows xa[:, r:2r]
    // Bu^T (k_split = r), so both rank-r products share one K tile of the
    // 4-wave engine (which every dual-B launch runs on) instead of two
    a.segs[ns++] = Seg{(const __bf16*)xa, ld_xa, (const __bf16*)b_gate, (const __bf16*)b_up, ldb, 2 * r, 0, I, r};
  }
  a.n_segs = ns;
  a.ep.c = h;
  a.ep.ldc = ld_out;
  a.ep.alpha = 1.f;
  a.ep.e = (__bf16*)e;
  a.ep.g = (__bf16*)g;
  a.ep.ld_eg = ld_out;
  if (r > 0 && xa && (ld_xa % 8 != 0 || r % 8 != 0))
    return forge_set_error(FORGE_ERR_INVALID, "lora_mlp_gate_up: rank and ld_xa must be multiples of 8");
  if (v_part) {
    // formed by the staged dual epilogue: 16-byte vectors everywhere
    if (!e || rd <= 0 || rd > 64 || rd % 8 != 0 || I % 8 != 0 || ld_ad % 8 != 0 || ld_ad < I)
      return forge_set_error(FORGE_ERR_INVALID, "lora_mlp_gate_up_v: e, g given, rank %lld (8..64, a multiple of 8), "
                             "I %lld, ld_ad %lld", (long long)rd, (long long)I, (long long)ld_ad);
    if (!a_down || !aligned16(a_down) || !aligned16(v_part) || !aligned16(e) || !aligned16(g) || !aligned16(h) ||
        ld_out % 8 != 0)
      return forge_set_error(FORGE_ERR_INVALID, "lora_mlp_gate_up_v: operands must be 16-byte aligned, ld %% 8 == 0");
    a.ep.vpart = v_part;
    a.ep.vpart_stride = M * rd;
    a.ep.vbt[0] = (const __bf16*)a_down;
    a.ep.vbt_ld = ld_ad;
    a.ep.vr = (int)rd;
  }
  return run(-1, ROW, COL, epi, a, (hipStream_t)stream);
}

extern "C" int forge_lora_mlp_gate_up(int64_t M, int64_t H, int64_t I, int64_t r,
                                      const void* x, int64_t ldx,
                                      const void* w_gate, const void* w_up, int64_t ldw,
                                      const void* xa, int64_t ld_xa,
                                      const void* b_gate, const void* b_up, int64_t ldb,
                                      void* e, void* g, void* h, int64_t ld_out, int activation, void* stream) {
  return gate_up(M, H, I, r, x, ldx, w_gate, w_up, ldw, xa, ld_xa, b_gate, b_up, ldb, e, g, h, ld_out, activation,
                 nullptr, 0, 0, nullptr, stream);
}

extern "C" int forge_lora_mlp_gate_up_v(int64_t M, int64_t H, int64_t I, int64_t r,
                                        const void* x, int64_t ldx,
                                        const void* w_gate, const void* w_up, int64_t ldw,
                                        const void* xa, int64_t ld_xa,
                                        const void* b_gate, const void* b_up, int64_t ldb,
                                        void* e, void* g, void* h, int64_t ld_out, int activation,
                                        const void* a_down, int64_t ld_ad, int64_t rd, float* v_part, void* stream) {
  if (!v_part) return forge_set_error(FORGE_ERR_INVALID, "lora_mlp_gate_up_v: v_part is NULL");
  return gate_up(M, H, I, r, x, ldx, w_gate, w_up, ldw, xa, ld_xa, b_gate, b_up, ldb, e, g, h, ld_out, activation,
                 a_down, ld_ad, rd, v_part, stream);
}

static int down_bwd(int64_t M, int64_t H, int64_t I, int64_t r, const void* dy, int64_t lddy, const void* w_down,
                    int64_t ldwd, const void* t_d, int64_t ld_t, const void* a_down, int64_t ld_ad, int w_layout,
                    void* h_out, void* e_df, void* g_de, int64_t ld, int activation, const void* bu_t,
                    const void* bg_t, int64_t ld_bt, int64_t rv, float* v_part, const void* xat_up,
                    const void* xat_gate, int64_t ld_xat, float* w_part, void* stream) {
  if (M < 0 || H < 0 || I < 0 || r < 0) return forge_set_error(FORGE_ERR_INVALID, "lora_mlp_down_bwd: shape");
  const int epi = glu_epi(activation, true);
  if (epi < 0) return forge_set_error(FORGE_ERR_INVALID, "lora_mlp_down_bwd: activation %d", activation);
  if (w_layout != ROW && w_layout != COL) return forge_set_error(FORGE_ERR_INVALID, "lora_mlp_down_bwd: w_layout");
  GemmArgs a = {};
  a.M = M;
  a.N = I;
  a.split_k = 1;
  int ns = 0;
  // DW[m, i] = sum_h dY[m, h] Wd[h, i]  (+ sum_j T[m, j] Ad[j, i]).
  // ROW: w_down = Wd [H][I], a_down = Ad [r][I] (B as [K][N]);
  // COL: w_down = Wd^T [I][H], a_down = Ad^T [I][r] (B K-contiguous: the LDS-DMA engine)
  a.segs[ns++] = Seg{(const __bf16*)dy, lddy, (const __bf16*)w_down, nullptr, ldwd, H, 0, I};
  if (r > 0 && t_d) a.segs[ns++] = Seg{(const __bf16*)t_d, ld_t, (const __bf16*)a_down, nullptr, ld_ad, r, 0, I};
  a.n_segs = ns;
  a.ep.c = h_out;
  a.ep.ldc = ld;
  a.ep.alpha = 1.f;
  a.ep.e = (__bf16*)e_df;
  a.ep.g = (__bf16*)g_de;
  a.ep.ld_eg = ld;
  if (v_part) {
    // the rank-r partials are formed by the staged epilogue of the 4-wave
    // engine: K-contiguous W (COL) and 16-byte vectors everywhere
    if (w_layout != COL)
      return forge_set_error(FORGE_ERR_UNSUPPORTED, "lora_mlp_down_bwd_v: W_down must be given as W^T (layout COL)");
    if (rv <= 0 || rv > 64 || rv % 8 != 0 || I % 8 != 0 || ld_bt % 8 != 0 || ld_bt < I)
      return forge_set_error(FORGE_ERR_INVALID, "lora_mlp_down_bwd_v: rank %lld (8..64, a multiple of 8), I %lld, "
                             "ld_bt %lld", (long long)rv, (long long)I, (long long)ld_bt);
    if (!bu_t || !bg_t || !aligned16(bu_t) || !aligned16(bg_t) || !aligned16(v_part) || !aligned16(h_out) ||
        !aligned16(e_df) || !aligned16(g_de) || ld % 8 != 0)
      return forge_set_error(FORGE_ERR_INVALID, "lora_mlp_down_bwd_v: operands must be 16-byte aligned, ld %% 8 == 0");
    a.ep.vpart = v_part;
    a.ep.vpart_stride = M * 2 * rv;
    a.ep.vbt[0] = (const __bf16*)bu_t;
    a.ep.vbt[1] = (const __bf16*)bg_t;
    a.ep.vbt_ld = ld_bt;
    a.ep.vr = (int)rv;
    if (w_part) {
      if (!xat_up || !xat_gate || !aligned16(xat_up) || !aligned16(xat_gate) || !aligned16(w_part) ||
          ld_xat % 8 != 0 || ld_xat < M)
        return forge_set_error(FORGE_ERR_INVALID, "lora_mlp_down_bwd_v: xa^T operands must be 16-byte aligned "
                               "with ld_xat (%lld) >= M and a multiple of 8", (long long)ld_xat);
      a.ep.wpart = w_part;
      a.ep.wpart_stride = 2 * I * rv;
      a.ep.wxt[0] = (const __bf16*)xat_up;
      a.ep.wxt[1] = (const __bf16*)xat_gate;
      a.ep.wxt_ld = ld_xat;
    }
  }
  return run(-1, ROW, w_layout, epi, a, (hipStream_t)stream);
}

extern "C" int forge_lora_mlp_down_bwd(int64_t M, int64_t H, int64_t I, int64_t r,
                                       const void* dy, int64_t lddy,
                                       const void* w_down, int64_t ldwd,
                                       const void* t_d, int64_t ld_t,
                                       const void* a_down, int64_t ld_ad, int w_layout,
                                       void* h_out, void* e_df, void* g_de, int64_t ld, int activation,
                                       void* stream) {
  return down_bwd(M, H, I, r, dy, lddy, w_down, ldwd, t_d, ld_t, a_down, ld_ad, w_layout, h_out, e_df, g_de, ld,
                  activation, nullptr, nullptr, 0, 0, nullptr, nullptr, nullptr, 0, nullptr, stream);
}

extern "C" int forge_lora_mlp_down_bwd_v(int64_t M, int64_t H, int64_t I, int64_t r,
                                         const void* dy, int64_t lddy,
                                         const void* w_down_t, int64_t ldwd,
                                         const void* t_d, int64_t ld_t,
                                         const void* a_down_t, int64_t ld_ad,
                                         void* h_out, void* e_df, void* g_de, int64_t ld, int activation,
                                         const void* b_up_t, const void* b_gate_t, int64_t ld_bt, int64_t rv,
                                         float* v_part, const void* xa_t_up, const void* xa_t_gate,
                                         int64_t ld_xat, float* w_part, void* stream) {
  if (!v_part) return forge_set_error(FORGE_ERR_INVALID, "lora_mlp_down_bwd_v: v_part is NULL");
  return down_bwd(M, H, I, r, dy, lddy, w_down_t, ldwd, t_d, ld_t, a_down_t, ld_ad, COL, h_out, e_df, g_de, ld,
                  activation, b_up_t, b_gate_t, ld_bt, rv, v_part, xa_t_up, xa_t_gate, ld_xat, w_part, stream);
}

extern "C" int forge_lora_mlp_glu_bwd(int64_t M, int64_t I, const void* d, int64_t ld_d, void* e_df, void* g_de,
                                      int64_t ld_eg, void* h, int64_t ld_h, int activation, void* stream) {
  if (M < 0 || I < 0) return forge_set_error(FORGE_ERR_INVALID, "lora_mlp_glu_bwd: shape");
  if (M == 0 || I == 0) return FORGE_OK;
  if (!d || !e_df || !g_de || !h) return forge_set_error(FORGE_ERR_INVALID, "lora_mlp_glu_bwd: null pointer");
  if (I % 8 || ld_d % 8 || ld_eg % 8 || ld_h % 8 || ld_d < I || ld_eg < I || ld_h < I || !aligned16(d) ||
      !aligned16(e_df) || !aligned16(g_de) || !aligned16(h))
    return forge_set_error(FORGE_ERR_UNSUPPORTED,
                           "lora_mlp_glu_bwd: I and the pitches must be multiples of 8, pointers 16-byte aligned");
  const int grid = grid_for(M * (I / 8), kGluBlock, kGluMaxBlocks);
  hipStream_t s = (hipStream_t)stream;
  const __bf16* dp = (const __bf16*)d;
  __bf16 *ep = (__bf16*)e_df, *gp = (__bf16*)g_de, *hp = (__bf16*)h;
  switch (glu_epi(activation, true)) {
    case EPI_SWIGLU_BWD:
      lora_glu_bwd_kernel<EPI_SWIGLU_BWD><<<grid, kGluBlock, 0, s>>>(dp, ld_d, ep, gp, ld_eg, hp, ld_h, M, I);
      break;
    case EPI_GEGLU_TANH_BWD:
      lora_glu_bwd_kernel<EPI_GEGLU_TANH_BWD><<<grid, kGluBlock, 0, s>>>(dp, ld_d, ep, gp, ld_eg, hp, ld_h, M, I);
      break;
    case EPI_GEGLU_ERF_BWD:
      lora_glu_bwd_kernel<EPI_GEGLU_ERF_BWD><<<grid, kGluBlock, 0, s>>>(dp, ld_d, ep, gp, ld_eg, hp, ld_h, M, I);
      break;
    default: return forge_set_error(FORGE_ERR_INVALID, "lora_mlp_glu_bwd: activation %d", activation);
  }
  FORGE_CHECK_LAUNCH();
  return FORGE_OK;
}

extern "C" int forge_lora_qkv_rope(int64_t M, int64_t K, int64_t hq, int64_t hkv, int64_t r,
                                   const void* x, int64_t ldx,
                                   const void* w_q, const void* w_k, const void* w_v, int64_t ldw,
                                   const void* xa, int64_t ld_xa,
                                   const void* b_q, const void* b_k, const void* b_v, int64_t ldb,
                                   void* out, int64_t ld_out,
                                   const void* cos, const void* sin, int64_t cs_ld,
                                   int64_t cs_rows, const int64_t* positions, int64_t head_dim,
                                   int apply_rope, void* stream) {
  if (M < 0 || K < 0 || hq < 0 || hkv < 0 || r < 0)
    return forge_set_error(FORGE_ERR_INVALID, "lora_qkv_rope: shape");
  if (apply_rope && !(head_dim == 64 || head_dim == 128))
    return forge_set_error(FORGE_ERR_UNSUPPORTED, "lora_qkv_rope: head_dim %lld (64 or 128 fused)",
                           (long long)head_dim);
  if (apply_rope && (hq % 256 != 0 || hkv % 256 != 0))
    return forge_set_error(FORGE_ERR_UNSUPPORTED,
                           "lora_qkv_rope: projection widths must be multiples of 256 (got %lld, %lld)",
                           (long long)hq, (long long)hkv);
  if (apply_rope && !positions && cs_rows < M)
    return forge_set_error(FORGE_ERR_INVALID, "lora_qkv_rope: cos/sin have %lld rows for %lld tokens",
                           (long long)cs_rows, (long long)M);
  GemmArgs a = {};
  a.M = M;
  a.N = hq + 2 * hkv;
  a.split_k = 1;
  int ns = 0;
  const int64_t q1 = hq, k1 = hq + hkv, v1 = hq + 2 * hkv;
  a.segs[ns++] = Seg{(const __bf16*)x, ldx, (const __bf16*)w_q, nullptr, ldw, K, 0, q1};
  a.segs[ns++] = Seg{(const __bf16*)x, ldx, (const __bf16*)w_k, nullptr, ldw, K, q1, k1};
  a.segs[ns++] = Seg{(const __bf16*)x, ldx, (const __bf16*)w_v, nullptr, ldw, K, k1, v1};
  if (r > 0 && xa) {
    a.segs[ns++] = Seg{(const __bf16*)xa, ld_xa, (const __bf16*)b_q, nullptr, ldb, r, 0, q1};
    a.segs[ns++] = Seg{(const __bf16*)xa + r, ld_xa, (const __bf16*)b_k, nullptr, ldb, r, q1, k1};
    a.segs[ns++] = Seg{(const __bf16*)xa + 2 * r, ld_xa, (const __bf16*)b_v, nullptr, ldb, r, k1, v1};
  }
  a.n_segs = ns;
  a.ep.c = out;
  a.ep.ldc = ld_out;
  a.ep.alpha = 1.f;
  a.ep.cos = (const __bf16*)cos;
  a.ep.sin = (const __bf16*)sin;
  a.ep.cs_ld = cs_ld;
  a.ep.cs_rows = cs_rows;
  a.ep.positions = positions;
  a.ep.rope_cols = apply_rope ? k1 : 0;
  a.ep.head_dim = (int)(head_dim > 0 ? head_dim : 128);
  if (!apply_rope) return run(-1, ROW, COL, EPI_STORE_BF16, a, (hipStream_t)stream);
  return run(-1, ROW, COL, EPI_ROPE, a, (hipStream_t)stream);
}

extern "C" int forge_lora_a(int64_t M, int64_t K, int64_t r, int n_proj, const void* x, int64_t ldx,
                            const void* const* a_mats, int64_t lda, const float* scales, void* out,
                            int64_t ld_out, float* work, int split_k, void* stream) {
  if (M < 0 || K < 0 || r <= 0 || n_proj < 1 || n_proj > 4)
    return forge_set_error(FORGE_ERR_INVALID, "lora_a: shape (r > 0, 1 <= n_proj <= 4)");
  if (split_k > 1 && !work) return forge_set_error(FORGE_ERR_INVALID, "lora_a: split_k > 1 needs a workspace");
  const int64_t N = r * n_proj;
  hipStream_t s = (hipStream_t)stream;
  GemmArgs a = {};
  a.M = M;
  a.N = N;
  a.split_k = split_k > 1 ? split_k : 1;
  // Matrices that are consecutive rows of one [n_proj * r][K] buffer (a
  // stacked A) form a single K segment: X streams once per column tile.
  // Otherwise each projection is a segment of its own, applied to its r
  // output columns.
  bool stacked = true;
  for (int p = 1; p < n_proj; ++p)
    stacked = stacked && (const char*)a_mats[p] == (const char*)a_mats[0] + (int64_t)p * r * lda * 2;
  if (stacked) {
    a.n_segs = 1;
    a.segs[0] = Seg{(const __bf16*)x, ldx, (const __bf16*)a_mats[0], nullptr, lda, K, 0, N};
  } else {
    a.n_segs = n_proj;
    for (int p = 0; p < n_proj; ++p)
      a.segs[p] = Seg{(const __bf16*)x, ldx, (const __bf16*)a_mats[p], nullptr, lda, K, p * r, (p + 1) * r};
  }
  a.ep.alpha = 1.f;
  a.ep.alpha_group = r;
  for (int p = 0; p < 4; ++p) a.ep.alphas[p] = p < n_proj ? scales[p] : 1.f;
  // 64-row tiles as wide as the output (64, 128, 192 or 256 columns: X A^T
  // is K-contiguous, on the LDS-DMA ring).  With split_k the K range is
  // spread over split_k workgroups per tile (when M / 64 tiles alone do not
  // fill the chip): split z writes fp32 partial sums to work[z]
  // ([split_k][M][N]), which one reduction pass sums in a fixed order
  // (deterministic) and rounds to bf16.
  const int cfg = -1;  // the narrow K-contiguous tiles (64 x N, N up to 256) picked from the shape
  if (split_k <= 1) {
    a.ep.c = out;
    a.ep.ldc = ld_out;
    return run(cfg, ROW, COL, EPI_STORE_BF16, a, s);
  }
  a.ep.c = work;
  a.ep.ldc = N;
  a.ep.split_stride = M * N;
  if (int e = run(cfg, ROW, COL, EPI_STORE_F32, a, s)) return e;
  return forge_splitk_reduce(work, M * N, split_k, M, N, N, out, ld_out, FORGE_DTYPE_BF16, 1.0f, stream);
}

// ---------------------------------------------------------------------------
// forge_lora_a without a caller workspace: the split-K partial sums go to a
// file-scope device array (one per GPU, resident until the process ends).
// Every split writes its whole [M, N] slice before the reduction reads it, so
// the array needs no clearing between calls; calls that overlap on one GPU
// (two streams) share it and race.
// ---------------------------------------------------------------------------
namespace {

constexpr int64_t kScratchFloats = FORGE_LORA_A_SCRATCH_BYTES / 4;
static __device__ __align__(256) float scratch[kScratchFloats];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
float* g_scratch_ptr[kMaxDevices] = {};

// Device address of this GPU's `scratch`, looked up once per device with that
// device current (host code must never pass the symbol itself to a kernel).
int scratch_for_current_device(float** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return forge_set_error(FORGE_ERR_HIP, "lora_a_noalloc: no current device (or device index >= %d)", kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return forge_set_error(FORGE_ERR_HIP, "lora_a_noalloc: hipGetSymbolAddress(scratch) failed on device %d: %s",
                             dev, hipGetErrorString(e));
    g_scratch_ptr[dev] = static_cast<float*>(p);
  }
  *out = g_scratch_ptr[dev];
  return FORGE_OK;
}

}  // namespace

extern "C" int forge_lora_a_noalloc(int64_t M, int64_t K, int64_t r, int n_proj, const void* x, int64_t ldx,
                                    const void* const* a_mats, int64_t lda, const float* scales, void* out,
                                    int64_t ld_out, int split_k, void* stream) {
  if (M < 0 || K < 0 || r <= 0 || n_proj < 1 || n_proj > 4)
    return forge_set_error(FORGE_ERR_INVALID, "lora_a_noalloc: shape (r > 0, 1 <= n_proj <= 4)");
  if (split_k <= 1)
    return forge_lora_a(M, K, r, n_proj, x, ldx, a_mats, lda, scales, out, ld_out, nullptr, 1, stream);
  const int64_t need = (int64_t)split_k * M * r * n_proj;
  if (need > kScratchFloats)
    return forge_set_error(FORGE_ERR_INVALID,
                           "lora_a_noalloc: split_k * M * n_proj * r = %lld fp32 partials exceed the %lld-byte scratch "
                           "(use forge_lora_a with a workspace, or a smaller split_k)",
                           (long long)need, (long long)FORGE_LORA_A_SCRATCH_BYTES);
  float* work = nullptr;
  if (int e = scratch_for_current_device(&work)) return e;
  return forge_lora_a(M, K, r, n_proj, x, ldx, a_mats, lda, scales, out, ld_out, work, split_k, stream);
}
