// GELU and its derivative in fp32 for gfx950, shared by the elementwise
// GeGLU kernels and the GeGLU epilogues of the MFMA GEMM (one evaluation, so
// the fused LoRA-GeGLU MLP and the standalone GeGLU agree bit for bit on the
// same bf16 inputs).
//   tanh form:  0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3)))
//   exact form: x Phi(x) = 0.5 x (1 + erf(x / sqrt 2)),
//               d/dx = Phi(x) + x exp(-x^2 / 2) / sqrt(2 pi).
#pragma once

#include <hip/hip_runtime.h>

namespace fgelu {

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

}  // namespace fgelu
