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
// (tanh and erf evaluation: gelu_and_grad in gelu.h.)
#include "gelu.h"
#include "glu_engine.h"

namespace {

using fgelu::gelu_and_grad;

template <bool TANH>
struct GeluAct {
  static constexpr int kUnroll = 1;
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
