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
#include <type_traits>

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

// LoRA-QKV backward through RoPE with the LoRA-B products of its outputs, in
// one pass over the gradients: dQ and dK rotated back by -theta per token
// (forge_rope's backward: the same per-element formula and rounding) into
// dq_out / dk_out, and
//   t[m] = alpha [dQu[m] B_q | dKu[m] B_k | dV[m] B_v]     (bf16, one rounding)
// from the rotated rows while they are on chip, instead of a second pass
// that reads dQu, dKu and dV again.  A workgroup takes 32 tokens and walks
// every head, Q, then K, then V (head_dim 128): thread (row, c) owns token
// row m0 + row and the 8-column chunks 8c.. and 64 + 8c.. of each head; the
// rotated head goes to a double-buffered LDS slab, and the four waves
// multiply it by the head's slice of B^T ([r][width], read from L2) with
// v_mfma_f32_16x16x32_bf16: wave w takes the 16-wide j block w (r <= 64) for
// all 32 tokens.  Each head's
// chunks are loaded four heads ahead, its B^T fragments one head ahead.
constexpr int kQrTok = 32, kQrD = 128, kQrP = kQrD + 8;

struct QkvRopeBwdArgs {
  int64_t M;
  int nq, nkv, r;
  const __bf16* src[3];   // dQ, dK, dV
  int64_t ld_src[3];
  __bf16* dst[2];         // dQu, dKu
  int64_t ld_dst[2];
  const __bf16* cos;
  const __bf16* sin;
  int64_t cs_ld, cs_rows;
  const int64_t* positions;
  const __bf16* bt[3];    // B_q^T, B_k^T, B_v^T
  int64_t ld_bt[3];
  __bf16* t;
  int64_t ld_t;
  float alpha;
};

typedef float qr_f32x4 __attribute__((ext_vector_type(4)));

// Barrier that leaves global loads in flight: this wave's LDS writes are
// done (lgkmcnt 0) before it, vmcnt is not waited on.
__device__ __forceinline__ void qr_barrier() {
  __builtin_amdgcn_s_waitcnt(15 | (7 << 4) | (3 << 14));
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

template <int NQ, int NKV>
__global__ __launch_bounds__(256) void qkv_rope_bwd_rank_kernel(QkvRopeBwdArgs a) {
  __shared__ __attribute__((aligned(16))) __bf16 slab[2][kQrTok * kQrP];
  const int tid = threadIdx.x, lane = tid % 64, w = tid / 64;
  const int row = tid / 8, c = tid % 8;
  const int64_t m0 = (int64_t)blockIdx.x * kQrTok, m = m0 + row;
  const bool mok = m < a.M;
  constexpr int nh = NQ + 2 * NKV;
  // cos / sin of this token's position at dims 8c .. 8c+7; the backward
  // rotates by -theta (sin scaled by -1, as forge_rope's backward does)
  float cs[8], sn[8];
  {
    const int64_t pos = mok ? (a.positions ? a.positions[m] : m) : 0;
    if (mok && pos >= 0 && pos < a.cs_rows) {
      const Vec16<__bf16> cv = load16(a.cos + pos * a.cs_ld + 8 * c);
      const Vec16<__bf16> sv = load16(a.sin + pos * a.cs_ld + 8 * c);
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        cs[q] = 1.0f * (float)cv.v[q];
        sn[q] = -1.0f * (float)sv.v[q];
      }
    } else {
#pragma unroll
      for (int q = 0; q < 8; ++q) cs[q] = sn[q] = __builtin_nanf("");
    }
  }
  // Loads and stores go through buffer instructions with out-of-range offsets
  // for rows past M (zeros read, writes dropped): no branch around them, so
  // the compiler counts the loads in flight exactly.
  auto load_head = [&](int h, uint4& lo, uint4& hi) {
    if (h >= nh) return;  // (h is a compile-time index)
    const int p = h < NQ ? 0 : (h < NQ + NKV ? 1 : 2);
    const int hh = p == 0 ? h : (p == 1 ? h - NQ : h - NQ - NKV);
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(a.src[p] + m0 * a.ld_src[p] + (int64_t)hh * kQrD);
    const uint32_t off = mok ? (uint32_t)((row * a.ld_src[p] + 8 * c) * 2) : OOB;
    // (nontemporal: each gradient chunk is read once; the B^T slices that every
    // workgroup reads stay in L2)
    lo = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rs, (int)off, 0, 2));
    hi = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rs, (int)(mok ? off + kQrD : OOB), 0, 2));
  };
  constexpr int PD = 4;  // heads whose chunks are in flight ahead of the one in use
  uint4 nlo[PD] = {}, nhi[PD] = {};
#pragma unroll
  for (int i = 0; i < PD; ++i) load_head(i, nlo[i], nhi[i]);
  const int r = a.r;
  // the B^T fragments of head h (this wave's j block w, 4 k-steps of 32)
  auto load_b = [&](int h, bf16x8 (&dst)[4]) {
    if (h >= nh) return;  // (h is a compile-time index)
    const int p = h < NQ ? 0 : (h < NQ + NKV ? 1 : 2);
    const int hh = p == 0 ? h : (p == 1 ? h - NQ : h - NQ - NKV);
    const __amdgpu_buffer_rsrc_t rb = make_rsrc(a.bt[p] + (int64_t)hh * kQrD);
    const int j = 16 * w + lane % 16;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const uint32_t off = j < r ? (uint32_t)((j * a.ld_bt[p] + 32 * ks + 8 * (lane / 16)) * 2) : OOB;
      dst[ks] = __builtin_bit_cast(bf16x8, buf_load16(rb, off));
    }
  };
  bf16x8 bslot[2][4];  // head h's fragments in slot h % 2, loaded one head ahead
  load_b(0, bslot[0]);
  qr_f32x4 acc[3][2];
#pragma unroll
  for (int p = 0; p < 3; ++p)
#pragma unroll
    for (int u = 0; u < 2; ++u) acc[p][u] = qr_f32x4{0.f, 0.f, 0.f, 0.f};

  // head h (projection P, register slot S = h % 2)
  // (every head loop is unrolled, so h, and with it every slot index below, is
  // a compile-time constant)
  auto head = [&](int h, auto pc) {
    constexpr int P = decltype(pc)::value;
    const int S = h % 2, SD = h % PD;
    const int hh = P == 0 ? h : (P == 1 ? h - NQ : h - NQ - NKV);
    // the next head's B^T fragments (this head's were loaded one head ago)
    load_b(h + 1, bslot[1 - S]);
    uint4 lo = nlo[SD], hi = nhi[SD];
    load_head(h + PD, nlo[SD], nhi[SD]);
    if constexpr (P < 2) {
      Vec16<__bf16> l, u, ol, oh;
      l.raw = lo;
      u.raw = hi;
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const float x0 = (float)l.v[q], x1 = (float)u.v[q];
        ol.v[q] = (__bf16)(x0 * cs[q] - x1 * sn[q]);
        oh.v[q] = (__bf16)(x1 * cs[q] + x0 * sn[q]);
      }
      {
        const __amdgpu_buffer_rsrc_t rd = make_rsrc(a.dst[P] + m0 * a.ld_dst[P] + (int64_t)hh * kQrD);
        const uint32_t off = mok ? (uint32_t)((row * a.ld_dst[P] + 8 * c) * 2) : OOB;
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i32x4, ol.raw), rd, (int)off, 0, 2);
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i32x4, oh.raw), rd, (int)(mok ? off + kQrD : OOB), 0,
                                               2);
      }
      lo = ol.raw;
      hi = oh.raw;
    }
    __bf16* sb = slab[h & 1];
    *reinterpret_cast<uint4*>(sb + row * kQrP + 8 * c) = lo;
    *reinterpret_cast<uint4*>(sb + row * kQrP + kQrD / 2 + 8 * c) = hi;
    qr_barrier();  // the slab is whole; the slab of head h - 1 is no longer read
    if (16 * w < r) {
#pragma unroll
      for (int ks = 0; ks < 4; ++ks)
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const bf16x8 af =
              *reinterpret_cast<const bf16x8*>(sb + (16 * u + lane % 16) * kQrP + 32 * ks + 8 * (lane / 16));
          acc[P][u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bslot[S][ks], af, acc[P][u], 0, 0, 0);
        }
    }
  };
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;
  // every head unrolled: the compiler then counts the loads in flight
  // exactly (across a loop's back edge it waited for all of them, the
  // prefetch included)
#pragma unroll
  for (int h = 0; h < NQ; ++h) head(h, I0{});
#pragma unroll
  for (int h = NQ; h < NQ + NKV; ++h) head(h, I1{});
#pragma unroll
  for (int h = NQ + NKV; h < nh; ++h) head(h, I2{});
  // acc[p][u][q] = sum for j = 16 w + 4 (lane / 16) + q, token 16 u + lane % 16
  const int j0 = 16 * w + 4 * (lane / 16);
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int64_t tok = m0 + 16 * u + lane % 16;
    if (tok >= a.M || j0 >= r) continue;
#pragma unroll
    for (int p = 0; p < 3; ++p) {
      const uint32_t w0 = (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)(a.alpha * acc[p][u][0])) |
                          ((uint32_t)__builtin_bit_cast(uint16_t, (__bf16)(a.alpha * acc[p][u][1])) << 16);
      const uint32_t w1 = (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)(a.alpha * acc[p][u][2])) |
                          ((uint32_t)__builtin_bit_cast(uint16_t, (__bf16)(a.alpha * acc[p][u][3])) << 16);
      *reinterpret_cast<uint2*>(a.t + tok * a.ld_t + p * r + j0) = make_uint2(w0, w1);
    }
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


extern "C" int forge_lora_qkv_rope_bwd(int64_t M, int64_t hq, int64_t hkv, int64_t r, int64_t head_dim,
                                       const void* dq, int64_t ld_dq, const void* dk, int64_t ld_dk,
                                       const void* dv, int64_t ld_dv,
                                       const void* cos, const void* sin, int64_t cs_ld, int64_t cs_rows,
                                       const int64_t* positions,
                                       void* dq_out, int64_t ld_qo, void* dk_out, int64_t ld_ko,
                                       const void* bq_t, const void* bk_t, const void* bv_t,
                                       int64_t ld_bq, int64_t ld_bk, int64_t ld_bv,
                                       void* t, int64_t ld_t, float alpha, void* stream) {
  if (M < 0 || hq < 0 || hkv < 0) return forge_set_error(FORGE_ERR_INVALID, "lora_qkv_rope_bwd: shape");
  if (head_dim != kQrD || hq % (2 * kQrD) != 0 || hkv % (2 * kQrD) != 0 || hkv == 0)
    return forge_set_error(FORGE_ERR_UNSUPPORTED,
                           "lora_qkv_rope_bwd: head_dim 128 and even head counts (hq %lld, hkv %lld, head_dim %lld)",
                           (long long)hq, (long long)hkv, (long long)head_dim);
  if (r <= 0 || r > 64 || r % 16 != 0)
    return forge_set_error(FORGE_ERR_UNSUPPORTED, "lora_qkv_rope_bwd: rank %lld (16, 32, 48 or 64)", (long long)r);
  if (M == 0) return FORGE_OK;
  const void* ptrs[] = {dq, dk, dv, cos, sin, dq_out, dk_out, bq_t, bk_t, bv_t, t};
  for (const void* p : ptrs)
    if (!p || !aligned16(p)) return forge_set_error(FORGE_ERR_INVALID, "lora_qkv_rope_bwd: null or unaligned operand");
  if (ld_dq < hq || ld_dk < hkv || ld_dv < hkv || ld_qo < hq || ld_ko < hkv || ld_bq < hq || ld_bk < hkv ||
      ld_bv < hkv || ld_t < 3 * r || cs_ld < head_dim)
    return forge_set_error(FORGE_ERR_INVALID, "lora_qkv_rope_bwd: pitch below the row width");
  if (ld_dq % 8 || ld_dk % 8 || ld_dv % 8 || ld_qo % 8 || ld_ko % 8 || ld_bq % 8 || ld_bk % 8 || ld_bv % 8 ||
      ld_t % 4 || cs_ld % 8)
    return forge_set_error(FORGE_ERR_INVALID, "lora_qkv_rope_bwd: pitches must be multiples of 8 (ld_t of 4)");
  if (!positions && cs_rows < M)
    return forge_set_error(FORGE_ERR_INVALID, "lora_qkv_rope_bwd: cos/sin have %lld rows for %lld tokens",
                           (long long)cs_rows, (long long)M);
  QkvRopeBwdArgs a = {};
  a.M = M;
  a.nq = (int)(hq / kQrD);
  a.nkv = (int)(hkv / kQrD);
  a.r = (int)r;
  a.src[0] = (const __bf16*)dq;
  a.src[1] = (const __bf16*)dk;
  a.src[2] = (const __bf16*)dv;
  a.ld_src[0] = ld_dq;
  a.ld_src[1] = ld_dk;
  a.ld_src[2] = ld_dv;
  a.dst[0] = (__bf16*)dq_out;
  a.dst[1] = (__bf16*)dk_out;
  a.ld_dst[0] = ld_qo;
  a.ld_dst[1] = ld_ko;
  a.cos = (const __bf16*)cos;
  a.sin = (const __bf16*)sin;
  a.cs_ld = cs_ld;
  a.cs_rows = cs_rows;
  a.positions = positions;
  a.bt[0] = (const __bf16*)bq_t;
  a.bt[1] = (const __bf16*)bk_t;
  a.bt[2] = (const __bf16*)bv_t;
  a.ld_bt[0] = ld_bq;
  a.ld_bt[1] = ld_bk;
  a.ld_bt[2] = ld_bv;
  a.t = (__bf16*)t;
  a.ld_t = ld_t;
  a.alpha = alpha;
  const int64_t grid = (M + kQrTok - 1) / kQrTok;
  if (grid > 0x7fffffffLL) return forge_set_error(FORGE_ERR_INVALID, "lora_qkv_rope_bwd: too many tokens");
  hipStream_t s = (hipStream_t)stream;
  if (a.nq == 32 && a.nkv == 8) qkv_rope_bwd_rank_kernel<32, 8><<<(unsigned)grid, 256, 0, s>>>(a);
  else if (a.nq == 32 && a.nkv == 32) qkv_rope_bwd_rank_kernel<32, 32><<<(unsigned)grid, 256, 0, s>>>(a);
  else if (a.nq == 64 && a.nkv == 8) qkv_rope_bwd_rank_kernel<64, 8><<<(unsigned)grid, 256, 0, s>>>(a);
  else if (a.nq == 16 && a.nkv == 8) qkv_rope_bwd_rank_kernel<16, 8><<<(unsigned)grid, 256, 0, s>>>(a);
  else if (a.nq == 8 && a.nkv == 2) qkv_rope_bwd_rank_kernel<8, 2><<<(unsigned)grid, 256, 0, s>>>(a);
  else if (a.nq == 4 && a.nkv == 2) qkv_rope_bwd_rank_kernel<4, 2><<<(unsigned)grid, 256, 0, s>>>(a);
  else
    return forge_set_error(FORGE_ERR_UNSUPPORTED, "lora_qkv_rope_bwd: %d Q / %d KV heads not instantiated", a.nq,
                           a.nkv);
  FORGE_CHECK_LAUNCH();
  return FORGE_OK;
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
