// Generic GEMM: C[M, N] = act(alpha * sum_k A(m, k) B(k, n) + beta * C + bias[n]).
//
// Any strides (so every layout: X W^T, dY W, dY^T X), fp32 / fp16 / bf16
// operands, fp32 accumulation with one fmaf per k in increasing k order
// (deterministic, and exact to fp32 rounding).  It is the path for what the
// bf16 MFMA core does not take: fp32 and fp16 models, and K or row pitches
// that are not multiples of 8.  The fused linear + cross-entropy path uses it
// for those shapes; bf16 shapes with aligned pitches go to the MFMA core.
//
// Tiling: 64 x 64 output tiles, 16-deep K tiles staged in LDS as fp32,
// 256 threads with 4 x 4 outputs each.  Operand loads are coalesced along
// whichever of the two strides is unit (checked once per launch).
#include "common.h"
#include "gelu.h"

namespace {

struct GenArgs {
  int64_t M, N, K;
  const void* a;
  int64_t a_sm, a_sk;
  const void* b;
  int64_t b_sk, b_sn;
  void* c;
  int64_t ldc;
  const void* bias;
  float alpha, beta;
  int act;  // FORGE_GEMM_ACT_*: activation applied to the result
};

__device__ __forceinline__ float gen_act(int act, float v) {
  if (act == FORGE_GEMM_ACT_SILU) return v * __builtin_amdgcn_rcpf(1.0f + __expf(-v));
  if (act == FORGE_GEMM_ACT_RELU) return v > 0.f ? v : 0.f;
  if (act == FORGE_GEMM_ACT_GELU) {  // tanh form, as the MFMA core's GELU epilogue
    float a, d;
    fgelu::gelu_and_grad<true>(v, a, d);
    return a;
  }
  return v;
}

constexpr int GBM = 64, GBN = 64, GBK = 16;

template <class T, class TC>
__global__ __launch_bounds__(256) void generic_gemm_kernel(GenArgs g, int64_t tiles_n) {
  __shared__ float As[GBK][GBM + 4];
  __shared__ float Bs[GBK][GBN + 4];
  const int64_t tile = blockIdx.x;
  const int64_t m0 = (tile / tiles_n) * GBM, n0 = (tile % tiles_n) * GBN;
  const int tid = threadIdx.x, tx = tid % 16, ty = tid / 16;
  const T* A = static_cast<const T*>(g.a);
  const T* B = static_cast<const T*>(g.b);
  const bool a_kfast = g.a_sk == 1;  // row-major A: neighbouring threads walk k
  const bool b_nfast = g.b_sn == 1;  // row-major B ([K][N]): neighbouring threads walk n
  float acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = 0.f;

  for (int64_t k0 = 0; k0 < g.K; k0 += GBK) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = tid + 256 * i;  // 1024 elements per operand tile
      int r, ka;
      if (a_kfast) { r = e / GBK; ka = e % GBK; } else { ka = e / GBM; r = e % GBM; }
      const int64_t m = m0 + r, k = k0 + ka;
      As[ka][r] = (m < g.M && k < g.K) ? to_f32<T>(A[m * g.a_sm + k * g.a_sk]) : 0.f;
      int cn, kb;
      if (b_nfast) { kb = e / GBN; cn = e % GBN; } else { cn = e / GBK; kb = e % GBK; }
      const int64_t n = n0 + cn, k2 = k0 + kb;
      Bs[kb][cn] = (n < g.N && k2 < g.K) ? to_f32<T>(B[k2 * g.b_sk + n * g.b_sn]) : 0.f;
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < GBK; ++kk) {
      float av[4], bv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) av[i] = As[kk][ty * 4 + i];
#pragma unroll
      for (int j = 0; j < 4; ++j) bv[j] = Bs[kk][tx * 4 + j];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(av[i], bv[j], acc[i][j]);
    }
    __syncthreads();
  }

  TC* C = static_cast<TC*>(g.c);
  const T* bias = static_cast<const T*>(g.bias);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t m = m0 + ty * 4 + i;
    if (m >= g.M) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t n = n0 + tx * 4 + j;
      if (n >= g.N) continue;
      float v = g.alpha * acc[i][j];
      if (g.beta != 0.f) v += g.beta * to_f32<TC>(C[m * g.ldc + n]);
      if (bias) v += to_f32<T>(bias[n]);
      if (g.act) v = gen_act(g.act, v);
      C[m * g.ldc + n] = from_f32<TC>(v);
    }
  }
}

template <class T>
int launch_generic(const GenArgs& g, int c_dtype, hipStream_t s) {
  const int64_t tm = (g.M + GBM - 1) / GBM, tn = (g.N + GBN - 1) / GBN;
  if (tm * tn > 0x7fffffffLL) return forge_set_error(FORGE_ERR_INVALID, "gemm_generic: too many tiles");
  const dim3 grid((unsigned)(tm * tn));
  if (c_dtype == FORGE_DTYPE_F32)
    generic_gemm_kernel<T, float><<<grid, 256, 0, s>>>(g, tn);
  else
    generic_gemm_kernel<T, T><<<grid, 256, 0, s>>>(g, tn);
  FORGE_CHECK_LAUNCH();
  return FORGE_OK;
}

}  // namespace

extern "C" int forge_gemm_generic(int64_t M, int64_t N, int64_t K, int dtype, const void* a, int64_t a_sm,
                                  int64_t a_sk, const void* b, int64_t b_sk, int64_t b_sn, void* c, int64_t ldc,
                                  int c_dtype, float alpha, float beta, const void* bias, int act,
                                  void* stream) {
  if (M < 0 || N < 0 || K < 0) return forge_set_error(FORGE_ERR_INVALID, "gemm_generic: negative shape");
  if (dtype != FORGE_DTYPE_F32 && dtype != FORGE_DTYPE_F16 && dtype != FORGE_DTYPE_BF16)
    return forge_set_error(FORGE_ERR_UNSUPPORTED, "gemm_generic: dtype %d", dtype);
  if (c_dtype != FORGE_DTYPE_F32 && c_dtype != dtype)
    return forge_set_error(FORGE_ERR_UNSUPPORTED, "gemm_generic: C dtype %d with operands %d", c_dtype, dtype);
  if (act != FORGE_GEMM_ACT_NONE && act != FORGE_GEMM_ACT_SILU && act != FORGE_GEMM_ACT_RELU &&
      act != FORGE_GEMM_ACT_GELU)
    return forge_set_error(FORGE_ERR_UNSUPPORTED, "gemm_generic: activation %d", act);
  if (M == 0 || N == 0) return FORGE_OK;
  if (!c || (K > 0 && (!a || !b))) return forge_set_error(FORGE_ERR_INVALID, "gemm_generic: null operand");
  GenArgs g{M, N, K, a, a_sm, a_sk, b, b_sk, b_sn, c, ldc, bias, alpha, beta, act};
  hipStream_t s = (hipStream_t)stream;
  switch (dtype) {
    case FORGE_DTYPE_F32: return launch_generic<float>(g, c_dtype, s);
    case FORGE_DTYPE_F16: return launch_generic<fp16_t>(g, c_dtype, s);
    default: return launch_generic<bf16_t>(g, c_dtype, s);
  }
}
