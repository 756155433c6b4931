// Small utility kernels used by the split-K paths: zero fill of an fp32
// workspace (a kernel, not hipMemsetAsync, so the sequence stays valid under
// stream capture) and the fp32 -> bf16 cast of the reduced result.
#include "common.h"

namespace {

__global__ __launch_bounds__(256) void zero_kernel(uint4* p, int64_t n16, uint8_t* tail, int64_t ntail) {
  const int64_t stride = (int64_t)gridDim.x * 256;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n16; i += stride) p[i] = make_uint4(0, 0, 0, 0);
  if (blockIdx.x == 0 && threadIdx.x < ntail) tail[threadIdx.x] = 0;
}

__global__ __launch_bounds__(256) void cast_f32_bf16_kernel(const float* src, int64_t lds, bf16_t* dst,
                                                            int64_t ldd, int64_t rows, int64_t cols) {
  const int64_t n = rows * cols;
  const int64_t stride = (int64_t)gridDim.x * 256;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += stride) {
    const int64_t r = i / cols, c = i - r * cols;
    dst[r * ldd + c] = (bf16_t)src[r * lds + c];
  }
}

}  // namespace

extern "C" int forge_zero(void* ptr, int64_t bytes, void* stream) {
  if (bytes <= 0) return FORGE_OK;
  if (!aligned16(ptr)) return forge_set_error(FORGE_ERR_INVALID, "zero: pointer not 16-byte aligned");
  const int64_t n16 = bytes / 16;
  zero_kernel<<<grid_for(n16 > 0 ? n16 : 1, 256, 2048), 256, 0, (hipStream_t)stream>>>(
      (uint4*)ptr, n16, (uint8_t*)ptr + n16 * 16, bytes - n16 * 16);
  FORGE_CHECK_LAUNCH();
  return FORGE_OK;
}

extern "C" int forge_cast_f32_bf16(const float* src, int64_t ld_src, void* dst, int64_t ld_dst, int64_t rows,
                                   int64_t cols, void* stream) {
  if (rows <= 0 || cols <= 0) return FORGE_OK;
  cast_f32_bf16_kernel<<<grid_for(rows * cols, 256, 4096), 256, 0, (hipStream_t)stream>>>(
      src, ld_src, (bf16_t*)dst, ld_dst, rows, cols);
  FORGE_CHECK_LAUNCH();
  return FORGE_OK;
}
