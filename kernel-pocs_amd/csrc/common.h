// Shared device helpers for the gfx950 (CDNA4) kernel library.
//
// Every kernel in this library is written for 64-lane wavefronts and the
// MI355X memory system: 16-byte global accesses, fp32 math on bf16/fp16/fp32
// storage, and hardware bf16 rounding (v_cvt_pk_bf16_f32, round-to-nearest-even).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/forge_hip.h"

typedef __bf16 bf16_t;
typedef _Float16 fp16_t;

// ---------------------------------------------------------------------------
// scalar conversions (fp32 is the compute type everywhere)
// ---------------------------------------------------------------------------
template <class T> __device__ __forceinline__ float to_f32(T v);
template <> __device__ __forceinline__ float to_f32<float>(float v) { return v; }
template <> __device__ __forceinline__ float to_f32<double>(double v) { return (float)v; }
template <> __device__ __forceinline__ float to_f32<bf16_t>(bf16_t v) { return (float)v; }
template <> __device__ __forceinline__ float to_f32<fp16_t>(fp16_t v) { return (float)v; }

template <class T> __device__ __forceinline__ T from_f32(float v);
template <> __device__ __forceinline__ float from_f32<float>(float v) { return v; }
template <> __device__ __forceinline__ double from_f32<double>(float v) { return (double)v; }
template <> __device__ __forceinline__ bf16_t from_f32<bf16_t>(float v) { return (bf16_t)v; }
template <> __device__ __forceinline__ fp16_t from_f32<fp16_t>(float v) { return (fp16_t)v; }

// Round-trip through the storage type: models a tensor op whose result is
// materialised in dtype T (what PyTorch does between two ops).
template <class T> __device__ __forceinline__ float round_to(float v) {
  return to_f32<T>(from_f32<T>(v));
}

// ---------------------------------------------------------------------------
// 16-byte vectors of storage elements
// ---------------------------------------------------------------------------
template <class T> struct Vec16 {
  static constexpr int N = 16 / sizeof(T);
  union {
    uint4 raw;
    T v[16 / sizeof(T)];
  };
};

template <class T> __device__ __forceinline__ Vec16<T> load16(const T* p) {
  Vec16<T> r;
  r.raw = *reinterpret_cast<const uint4*>(p);
  return r;
}

// Streaming load: the data is touched once, keep it out of the way in L2.
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

template <class T> __device__ __forceinline__ Vec16<T> load16_nt(const T* p) {
  Vec16<T> r;
  u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
  r.raw = make_uint4(v.x, v.y, v.z, v.w);
  return r;
}

template <class T> __device__ __forceinline__ void store16(T* p, const Vec16<T>& v) {
  *reinterpret_cast<uint4*>(p) = v.raw;
}

template <class T> __device__ __forceinline__ void store16_nt(T* p, const Vec16<T>& v) {
  u32x4_t w = {v.raw.x, v.raw.y, v.raw.z, v.raw.w};
  __builtin_nontemporal_store(w, reinterpret_cast<u32x4_t*>(p));
}

// ---------------------------------------------------------------------------
// wavefront reductions (wave64)
// ---------------------------------------------------------------------------
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// dtype helpers shared by the C entry points
static inline size_t dtype_size(int dtype) {
  switch (dtype) {
    case FORGE_DTYPE_F32: return 4;
    case FORGE_DTYPE_F16: return 2;
    case FORGE_DTYPE_BF16: return 2;
    case FORGE_DTYPE_F64: return 8;
    default: return 0;
  }
}

static inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// Grid sizing: enough workgroups to cover 256 CUs several times over.
static inline int grid_for(int64_t work_items, int block, int max_blocks = 256 * 32) {
  int64_t g = (work_items + block - 1) / block;
  if (g < 1) g = 1;
  if (g > max_blocks) g = max_blocks;
  return (int)g;
}

// Records the error string for forge_last_error() and returns the status.
int forge_set_error(int status, const char* fmt, ...);

#define FORGE_CHECK_LAUNCH()                                                         \
  do {                                                                               \
    hipError_t _e = hipGetLastError();                                               \
    if (_e != hipSuccess)                                                            \
      return forge_set_error(FORGE_ERR_HIP, "%s: launch failed: %s", __func__,       \
                             hipGetErrorString(_e));                                 \
  } while (0)
