// SwiGLU forward/backward for gfx950 (the gated-linear-unit engine of
// glu_engine.h with the SiLU policy below).
//
// Reference semantics (kernels/swiglu/swiglu.py:179-188, the PyTorch path the
// Triton kernels are tested against):
//     s   = silu(gate.float() * gm).to(dtype)
//     out = (s * up) * dm                      (each product materialised in dtype)
// and its autograd backward.  Every intermediate stays in fp32 registers and
// is rounded to the storage type exactly where the PyTorch graph materialises
// a tensor, so fp32 results match to an ulp and bf16/fp16 results match to a
// rounding step.
#include "glu_engine.h"

namespace {

__device__ __forceinline__ float silu_f32(float x) { return x / (1.0f + expf(-x)); }
__device__ __forceinline__ float sigmoid_f32(float x) { return 1.0f / (1.0f + expf(-x)); }

struct SiluAct {
  static constexpr int kUnroll = 2;
  float gm, dm;
  template <class T>
  __device__ __forceinline__ float fwd(float gate, float up) const {
    float s = round_to<T>(silu_f32(gate * gm));
    float p = round_to<T>(s * up);
    return p * dm;
  }
  // Backward of the graph above: (dgate, dup) in fp32 before the final rounding to T.
  template <class T>
  __device__ __forceinline__ void bwd(float dout, float gate, float up, float& dgate, float& dup) const {
    float g = gate * gm;
    float sig = sigmoid_f32(g);
    float s = round_to<T>(silu_f32(g));
    float dp = round_to<T>(dout * dm);
    dup = dp * s;
    float ds = round_to<T>(dp * up);
    dgate = (ds * (sig * (1.0f + g * (1.0f - sig)))) * gm;
  }
};

int check_common(int64_t rows, int64_t cols) {
  if (rows < 0 || cols < 0) return forge_set_error(FORGE_ERR_INVALID, "swiglu: negative shape");
  return FORGE_OK;
}

}  // namespace


extern "C" int forge_swiglu_fwd(int dtype, const void* gate, const void* up, int64_t ld_in,
                                void* out, int64_t ld_out, int64_t rows, int64_t cols,
                                float gm, float dm, void* stream) {
  if (int e = check_common(rows, cols)) return e;
  if (rows == 0 || cols == 0) return FORGE_OK;
  if (ld_in < cols || ld_out < cols)
    return forge_set_error(FORGE_ERR_INVALID, "swiglu_fwd: leading dimension smaller than cols");
  hipStream_t s = (hipStream_t)stream;
  switch (dtype) {
    case FORGE_DTYPE_F32: return glu::launch_fwd<float>(gate, up, ld_in, out, ld_out, rows, cols, SiluAct{gm, dm}, s);
    case FORGE_DTYPE_BF16: return glu::launch_fwd<bf16_t>(gate, up, ld_in, out, ld_out, rows, cols, SiluAct{gm, dm}, s);
    case FORGE_DTYPE_F16: return glu::launch_fwd<fp16_t>(gate, up, ld_in, out, ld_out, rows, cols, SiluAct{gm, dm}, s);
    default: return forge_set_error(FORGE_ERR_UNSUPPORTED, "swiglu_fwd: dtype %d", dtype);
  }
}

extern "C" int forge_swiglu_bwd(int dtype, const void* dout, int64_t ld_dout, const void* gate,
                                const void* up, int64_t ld_in, void* dgate, void* dup,
                                int64_t ld_dg, int64_t rows, int64_t cols, float gm, float dm,
                                void* stream) {
  if (int e = check_common(rows, cols)) return e;
  if (rows == 0 || cols == 0) return FORGE_OK;
  if (ld_in < cols || ld_dout < cols || ld_dg < cols)
    return forge_set_error(FORGE_ERR_INVALID, "swiglu_bwd: leading dimension smaller than cols");
  hipStream_t s = (hipStream_t)stream;
  switch (dtype) {
    case FORGE_DTYPE_F32:
      return glu::launch_bwd<float>(dout, ld_dout, gate, up, ld_in, dgate, dup, ld_dg, rows, cols, SiluAct{gm, dm}, s);
    case FORGE_DTYPE_BF16:
      return glu::launch_bwd<bf16_t>(dout, ld_dout, gate, up, ld_in, dgate, dup, ld_dg, rows, cols, SiluAct{gm, dm}, s);
    case FORGE_DTYPE_F16:
      return glu::launch_bwd<fp16_t>(dout, ld_dout, gate, up, ld_in, dgate, dup, ld_dg, rows, cols, SiluAct{gm, dm}, s);
    default: return forge_set_error(FORGE_ERR_UNSUPPORTED, "swiglu_bwd: dtype %d", dtype);
  }
}
