// GeGLU forward/backward for gfx950 (the gated-linear-unit engine of
// glu_engine.h with the GELU policy below), tanh-approximate or exact (erf).
//
// Reference semantics (kernels/geglu/geglu.py:90-183, the Triton kernels; the
// PyTorch path torch_geglu_reference, :255-263, computes the same forward):
//     a   = gelu(gate.float())           (fp32)
//     out = a.to(dtype) * up             (product rounded to dtype)
//     dup   = dout * a.to(dtype)          (fp32, then rounded)
//     dgate = dout * up * gelu'(gate)     (fp32, then rounded)
// GELU, tanh form:  0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3)))
//       exact form: x Phi(x) = 0.5 x (1 + erf(x / sqrt 2)),
//                   d/dx = Phi(x) + x exp(-x^2 / 2) / sqrt(2 pi).
// (tanh and erf evaluation: see gelu_and_grad.)
#include "glu_engine.h"

namespace {

constexpr float kSqrt2OverPi = 0.7978845608028654f;
constexpr float kGeluCubic = 0.044715f;
constexpr float kInvSqrt2 = 0.7071067811865476f;
constexpr float kInvSqrt2Pi = 0.3989422804014327f;

constexpr float kLog2e = 1.4426950408889634f;

// The elementwise GeGLU kernels are close to ALU-bound with the library's
// tanhf / erff (tens of instructions per element), so both forms are
// evaluated with the hardware base-2 exponential and reciprocal, in forms
// with no cancellation (the GELU derivative crosses zero near x = -0.75, and
// 1 + t, 1 - t^2 vanish as t -> -1 / +-1):
//  * tanh form: with e = e^{2u} and s = 1 / (1 + e), tanh u = 1 - 2 s, so
//      (1 + t) / 2 = e s   (= 1 - s once e > 1)   and   1 - t^2 = 4 (e s) s;
//  * exact form: erf(z), z >= 0, by Abramowitz & Stegun 7.1.26,
//      erf(z) = 1 - t (a1 + t (a2 + t (a3 + t (a4 + t a5)))) e^{-z^2},
//      t = 1 / (1 + p z)                        (|error| <= 1.5e-7),
//    so Phi(x) = (1 + erf(x / sqrt 2)) / 2 is 1 - h for x >= 0 and h for
//    x < 0, h = poly e^{-x^2/2} / 2; that e^{-x^2/2} is also the derivative's.
// fp32 errors against float64: activation <= 3e-6 absolute (<= 3e-7
// relative), derivative <= 3e-7 absolute.
template <bool TANH>
__device__ __forceinline__ void gelu_and_grad(float x, float& act, float& grad) {
  if constexpr (TANH) {
    const float x2 = x * x;
    const float u = kSqrt2OverPi * x * (1.0f + kGeluCubic * x2);
    const float e = __builtin_amdgcn_exp2f(2.0f * kLog2e * u);
    const float sr = __builtin_amdgcn_rcpf(1.0f + e);
    const float es = e > 1.0f ? 1.0f - sr : e * sr;  // (1 + tanh u) / 2
    act = x * es;
    grad = es + 2.0f * x * es * sr * kSqrt2OverPi * (1.0f + 3.0f * kGeluCubic * x2);
  } else {
    const float ez = __builtin_amdgcn_exp2f(-0.5f * kLog2e * x * x);  // e^{-x^2/2}
    const float t = __builtin_amdgcn_rcpf(1.0f + 0.3275911f * kInvSqrt2 * fabsf(x));
    const float poly =
        t * (0.254829592f + t * (-0.284496736f + t * (1.421413741f + t * (-1.453152027f + t * 1.061405429f))));
    const float h = 0.5f * poly * ez;
    const float cdf = x >= 0.0f ? 1.0f - h : h;
    act = x * cdf;
    grad = cdf + kInvSqrt2Pi * x * ez;
  }
}

template <bool TANH>
struct GeluAct {
  template <class T>
  __device__ __forceinline__ float fwd(float gate, float up) const {
    float a, g;
    gelu_and_grad<TANH>(gate, a, g);
    return round_to<T>(a) * up;
  }
  template <class T>
  __device__ __forceinline__ void bwd(float dout, float gate, float up, float& dgate, float& dup) const {
    float a, g;
    gelu_and_grad<TANH>(gate, a, g);
    dup = dout * round_to<T>(a);
    dgate = dout * up * g;
  }
};

template <class T>
int fwd_t(const void* gate, const void* up, int64_t ld_in, void* out, int64_t ld_out, int64_t rows, int64_t cols,
          int approximate_tanh, hipStream_t s) {
  if (approximate_tanh) return glu::launch_fwd<T>(gate, up, ld_in, out, ld_out, rows, cols, GeluAct<true>{}, s);
  return glu::launch_fwd<T>(gate, up, ld_in, out, ld_out, rows, cols, GeluAct<false>{}, s);
}

template <class T>
int bwd_t(const void* dout, int64_t ld_dout, const void* gate, const void* up, int64_t ld_in, void* dgate, void* dup,
          int64_t ld_dg, int64_t rows, int64_t cols, int approximate_tanh, hipStream_t s) {
  if (approximate_tanh)
    return glu::launch_bwd<T>(dout, ld_dout, gate, up, ld_in, dgate, dup, ld_dg, rows, cols, GeluAct<true>{}, s);
  return glu::launch_bwd<T>(dout, ld_dout, gate, up, ld_in, dgate, dup, ld_dg, rows, cols, GeluAct<false>{}, s);
}

}  // namespace

extern "C" int forge_geglu_fwd(int dtype, const void* gate, const void* up, int64_t ld_in, void* out,
                               int64_t ld_out, int64_t rows, int64_t cols, int approximate_tanh, void* stream) {
  if (rows < 0 || cols < 0) return forge_set_error(FORGE_ERR_INVALID, "geglu_fwd: negative shape");
  if (rows == 0 || cols == 0) return FORGE_OK;
  if (ld_in < cols || ld_out < cols)
    return forge_set_error(FORGE_ERR_INVALID, "geglu_fwd: leading dimension smaller than cols");
  hipStream_t s = (hipStream_t)stream;
  switch (dtype) {
    case FORGE_DTYPE_F32: return fwd_t<float>(gate, up, ld_in, out, ld_out, rows, cols, approximate_tanh, s);
    case FORGE_DTYPE_BF16: return fwd_t<bf16_t>(gate, up, ld_in, out, ld_out, rows, cols, approximate_tanh, s);
    case FORGE_DTYPE_F16: return fwd_t<fp16_t>(gate, up, ld_in, out, ld_out, rows, cols, approximate_tanh, s);
    default: return forge_set_error(FORGE_ERR_UNSUPPORTED, "geglu_fwd: dtype %d", dtype);
  }
}

extern "C" int forge_geglu_bwd(int dtype, const void* dout, int64_t ld_dout, const void* gate, const void* up,
                               int64_t ld_in, void* dgate, void* dup, int64_t ld_dg, int64_t rows, int64_t cols,
                               int approximate_tanh, void* stream) {
  if (rows < 0 || cols < 0) return forge_set_error(FORGE_ERR_INVALID, "geglu_bwd: negative shape");
  if (rows == 0 || cols == 0) return FORGE_OK;
  if (ld_in < cols || ld_dout < cols || ld_dg < cols)
    return forge_set_error(FORGE_ERR_INVALID, "geglu_bwd: leading dimension smaller than cols");
  hipStream_t s = (hipStream_t)stream;
  switch (dtype) {
    case FORGE_DTYPE_F32:
      return bwd_t<float>(dout, ld_dout, gate, up, ld_in, dgate, dup, ld_dg, rows, cols, approximate_tanh, s);
    case FORGE_DTYPE_BF16:
      return bwd_t<bf16_t>(dout, ld_dout, gate, up, ld_in, dgate, dup, ld_dg, rows, cols, approximate_tanh, s);
    case FORGE_DTYPE_F16:
      return bwd_t<fp16_t>(dout, ld_dout, gate, up, ld_in, dgate, dup, ld_dg, rows, cols, approximate_tanh, s);
    default: return forge_set_error(FORGE_ERR_UNSUPPORTED, "geglu_bwd: dtype %d", dtype);
  }
}
