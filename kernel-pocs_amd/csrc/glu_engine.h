// Elementwise gated-linear-unit engine for gfx950: out = f(gate, up) and its
// backward, for every activation policy (SiLU for SwiGLU, GELU for GeGLU).
//
// Layout: rows of `cols` elements, `ld` elements apart.  The packed variant
// (gate_up = [.., 2H]) is the same kernel with up = gate + H and ld = 2H.
// One thread owns one 16-byte vector of each operand; Act::kUnroll vectors
// are in flight per thread, and the grid covers the tensor in one pass up to
// kMaxBlocks workgroups (many resident workgroups keep the bytes outstanding
// that HBM needs).  Measured fwd+bwd steps on MI355X: SwiGLU fp32
// [2048, 11008] 5.65 -> 5.82 TB/s with 2 vectors per thread and no grid cap
// (was 4 vectors, 8192 workgroups); GeGLU bf16 [4096, 24576] 4.9 -> 5.65
// TB/s with 1 vector (its GELU math holds more registers per vector).
// Loads and stores are nontemporal: every operand is touched once per
// launch.  In a training step the backward runs long after the forward, so
// nothing it reads is still cached; measured on MI355X over rotating buffer
// sets (nothing cached, as in training) at SwiGLU [2048, 11008] fp32,
// nontemporal loads take the backward from 84.9 to 73.0 us (5.31 -> 6.18
// TB/s) and the forward from 47.4 to 43.0 us.
//
// An activation policy Act provides, in fp32 registers with rounding to the
// storage type T exactly where its reference materialises a tensor:
//   template <class T> float fwd(float gate, float up) const;
//   template <class T> void bwd(float dout, float gate, float up, float& dgate, float& dup) const;
//   static constexpr int kUnroll;  // 16-byte vectors per thread per operand
#pragma once

#include "common.h"

namespace glu {


constexpr int kBlock = 256;
// Grid cap: 256 workgroups per CU; larger tensors loop (grid-stride).
constexpr int kMaxBlocks = 256 * 256;

// Index math: the flat chunk id i maps to (row, col) = (i / cpr, (i % cpr) * VEC).
// TWO_D=false is the contiguous case (one row), which skips the division.
template <bool TWO_D>
__device__ __forceinline__ void chunk_rc(int64_t i, int64_t cpr, int vec, int64_t& r, int64_t& c) {
  if (TWO_D) {
    r = i / cpr;
    c = (i - r * cpr) * vec;
  } else {
    r = 0;
    c = i * vec;
  }
}

template <class T, int VEC, bool TWO_D, class Act>
__global__ __launch_bounds__(kBlock) void glu_fwd_kernel(
    const T* __restrict__ gate, const T* __restrict__ up, int64_t ld_in, T* __restrict__ out,
    int64_t ld_out, int64_t n_chunks, int64_t cpr, Act act) {
  constexpr int kUnroll = Act::kUnroll;
  const int64_t stride = (int64_t)gridDim.x * kBlock;
  for (int64_t base = (int64_t)blockIdx.x * kBlock + threadIdx.x; base < n_chunks;
       base += stride * kUnroll) {
    T gv[kUnroll][VEC], uv[kUnroll][VEC];
    int64_t ri[kUnroll], ci[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      int64_t i = base + u * stride;
      chunk_rc<TWO_D>(i, cpr, VEC, ri[u], ci[u]);
      if (i < n_chunks) {
        const T* gp = gate + ri[u] * ld_in + ci[u];
        const T* up_ = up + ri[u] * ld_in + ci[u];
        if constexpr (VEC * sizeof(T) == 16) {
          Vec16<T> a = load16_nt(gp), b = load16_nt(up_);
#pragma unroll
          for (int j = 0; j < VEC; ++j) { gv[u][j] = a.v[j]; uv[u][j] = b.v[j]; }
        } else {
#pragma unroll
          for (int j = 0; j < VEC; ++j) { gv[u][j] = gp[j]; uv[u][j] = up_[j]; }
        }
      }
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      int64_t i = base + u * stride;
      if (i < n_chunks) {
        T* op = out + ri[u] * ld_out + ci[u];
        if constexpr (VEC * sizeof(T) == 16) {
          Vec16<T> o;
#pragma unroll
          for (int j = 0; j < VEC; ++j)
            o.v[j] = from_f32<T>(act.template fwd<T>(to_f32(gv[u][j]), to_f32(uv[u][j])));
          store16_nt(op, o);
        } else {
#pragma unroll
          for (int j = 0; j < VEC; ++j)
            op[j] = from_f32<T>(act.template fwd<T>(to_f32(gv[u][j]), to_f32(uv[u][j])));
        }
      }
    }
  }
}

template <class T, int VEC, bool TWO_D, class Act>
__global__ __launch_bounds__(kBlock) void glu_bwd_kernel(
    const T* dout, int64_t ld_dout, const T* gate, const T* up, int64_t ld_in, T* dgate,
    T* dup, int64_t ld_dg, int64_t n_chunks, int64_t cpr, Act act) {
  // No __restrict__: dgate/dup alias gate/up in the default in-place mode.
  // Each element is read before it is overwritten by the same thread.
  constexpr int kUnroll = Act::kUnroll;
  const int64_t stride = (int64_t)gridDim.x * kBlock;
  for (int64_t base = (int64_t)blockIdx.x * kBlock + threadIdx.x; base < n_chunks;
       base += stride * kUnroll) {
    T dv[kUnroll][VEC], gv[kUnroll][VEC], uv[kUnroll][VEC];
    int64_t ri[kUnroll], ci[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      int64_t i = base + u * stride;
      chunk_rc<TWO_D>(i, cpr, VEC, ri[u], ci[u]);
      if (i < n_chunks) {
        const T* dp = dout + ri[u] * ld_dout + ci[u];
        const T* gp = gate + ri[u] * ld_in + ci[u];
        const T* up_ = up + ri[u] * ld_in + ci[u];
        if constexpr (VEC * sizeof(T) == 16) {
          Vec16<T> a = load16_nt(dp), b = load16_nt(gp), c = load16_nt(up_);
#pragma unroll
          for (int j = 0; j < VEC; ++j) { dv[u][j] = a.v[j]; gv[u][j] = b.v[j]; uv[u][j] = c.v[j]; }
        } else {
#pragma unroll
          for (int j = 0; j < VEC; ++j) { dv[u][j] = dp[j]; gv[u][j] = gp[j]; uv[u][j] = up_[j]; }
        }
      }
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      int64_t i = base + u * stride;
      if (i < n_chunks) {
        T* dgp = dgate + ri[u] * ld_dg + ci[u];
        T* dup_ = dup + ri[u] * ld_dg + ci[u];
        if constexpr (VEC * sizeof(T) == 16) {
          Vec16<T> og, ou;
#pragma unroll
          for (int j = 0; j < VEC; ++j) {
            float a, b;
            act.template bwd<T>(to_f32(dv[u][j]), to_f32(gv[u][j]), to_f32(uv[u][j]), a, b);
            og.v[j] = from_f32<T>(a);
            ou.v[j] = from_f32<T>(b);
          }
          store16_nt(dgp, og);
          store16_nt(dup_, ou);
        } else {
#pragma unroll
          for (int j = 0; j < VEC; ++j) {
            float a, b;
            act.template bwd<T>(to_f32(dv[u][j]), to_f32(gv[u][j]), to_f32(uv[u][j]), a, b);
            dgp[j] = from_f32<T>(a);
            dup_[j] = from_f32<T>(b);
          }
        }
      }
    }
  }
}

// Chooses the vector width and index mode for a (rows, cols, ld...) problem.
struct Plan {
  bool contiguous;  // all operands dense with ld == cols: one flat row
  bool vec;         // 16-byte vectors usable
};

template <class T>
Plan make_plan(int64_t rows, int64_t cols, std::initializer_list<int64_t> lds,
               std::initializer_list<const void*> ptrs) {
  constexpr int V = 16 / sizeof(T);
  Plan p;
  p.contiguous = true;
  for (int64_t ld : lds) p.contiguous = p.contiguous && (ld == cols || rows == 1);
  bool al = true;
  for (const void* q : ptrs) al = al && aligned16(q);
  if (p.contiguous) {
    p.vec = al && ((rows * cols) % V == 0);
  } else {
    bool ldok = true;
    for (int64_t ld : lds) ldok = ldok && (ld % V == 0);
    p.vec = al && ldok && (cols % V == 0);
  }
  return p;
}

template <class T, class Act>
int launch_fwd(const void* gate, const void* up, int64_t ld_in, void* out, int64_t ld_out,
               int64_t rows, int64_t cols, Act act, hipStream_t s) {
  constexpr int V = 16 / sizeof(T);
  Plan p = make_plan<T>(rows, cols, {ld_in, ld_out}, {gate, up, out});
  const T* g = (const T*)gate;
  const T* u = (const T*)up;
  T* o = (T*)out;
  int vec = p.vec ? V : 1;
  int64_t n_chunks = rows * cols / vec;
  int64_t cpr = cols / vec;
  int grid = grid_for((n_chunks + Act::kUnroll - 1) / Act::kUnroll, kBlock, kMaxBlocks);
  if (p.contiguous) {
    if (p.vec)
      glu_fwd_kernel<T, V, false, Act><<<grid, kBlock, 0, s>>>(g, u, ld_in, o, ld_out, n_chunks, cpr, act);
    else
      glu_fwd_kernel<T, 1, false, Act><<<grid, kBlock, 0, s>>>(g, u, ld_in, o, ld_out, n_chunks, cpr, act);
  } else {
    if (p.vec)
      glu_fwd_kernel<T, V, true, Act><<<grid, kBlock, 0, s>>>(g, u, ld_in, o, ld_out, n_chunks, cpr, act);
    else
      glu_fwd_kernel<T, 1, true, Act><<<grid, kBlock, 0, s>>>(g, u, ld_in, o, ld_out, n_chunks, cpr, act);
  }
  FORGE_CHECK_LAUNCH();
  return FORGE_OK;
}

template <class T, class Act>
int launch_bwd(const void* dout, int64_t ld_dout, const void* gate, const void* up, int64_t ld_in,
               void* dgate, void* dup, int64_t ld_dg, int64_t rows, int64_t cols, Act act, hipStream_t s) {
  constexpr int V = 16 / sizeof(T);
  Plan p = make_plan<T>(rows, cols, {ld_dout, ld_in, ld_dg}, {dout, gate, up, dgate, dup});
  int vec = p.vec ? V : 1;
  int64_t n_chunks = rows * cols / vec;
  int64_t cpr = cols / vec;
  int grid = grid_for((n_chunks + Act::kUnroll - 1) / Act::kUnroll, kBlock, kMaxBlocks);
  const T* d = (const T*)dout;
  const T* g = (const T*)gate;
  const T* u = (const T*)up;
  T* dg = (T*)dgate;
  T* du = (T*)dup;
  if (p.contiguous) {
    if (p.vec)
      glu_bwd_kernel<T, V, false, Act><<<grid, kBlock, 0, s>>>(d, ld_dout, g, u, ld_in, dg, du, ld_dg, n_chunks, cpr, act);
    else
      glu_bwd_kernel<T, 1, false, Act><<<grid, kBlock, 0, s>>>(d, ld_dout, g, u, ld_in, dg, du, ld_dg, n_chunks, cpr, act);
  } else {
    if (p.vec)
      glu_bwd_kernel<T, V, true, Act><<<grid, kBlock, 0, s>>>(d, ld_dout, g, u, ld_in, dg, du, ld_dg, n_chunks, cpr, act);
    else
      glu_bwd_kernel<T, 1, true, Act><<<grid, kBlock, 0, s>>>(d, ld_dout, g, u, ld_in, dg, du, ld_dg, n_chunks, cpr, act);
  }
  FORGE_CHECK_LAUNCH();
  return FORGE_OK;
}


}  // namespace glu
