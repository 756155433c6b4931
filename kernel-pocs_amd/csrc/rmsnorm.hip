// RMSNorm forward/backward for gfx950.
//
// Reference semantics (kernels/rmsnorm/forge_rmsnorm_v4.py:73-184, the same
// kernels as v2/v3; v1 in forge_rmsnorm_v1.py:32-106):
//   forward   rstd = rsqrt(mean(x^2) + eps)        (fp32; fp64 for fp64 input)
//             llama: y = (x rstd).to(dtype) * (w + offset)
//             gemma: y = (x rstd) * (float(w) + offset)           (fp32, one rounding)
//             none:  y = (x * rstd.to(dtype)) * (w + offset)       (dtype products)
//   backward  s = dy (w + offset); dot = sum(s x)
//             dx = rstd (s - x rstd^2 dot / H);  dw = sum over rows of dy x rstd
//             (v1: s = (dy w) rounded to dtype, dw terms dy * (x rstd).to(dtype)
//             rounded to dtype)
//
// Layout: rows of H elements (row pitches ld*); every row is read from HBM
// once.  Two engines, chosen by the row's width in 16-byte vectors:
//  * workgroup per row block (256 .. 2048 vectors, aligned rows): the 256
//    threads of a workgroup span the row, NVT vectors each, with R rows per
//    chunk (fwd_rows / bwd_rows below); a row sum is a wave shuffle
//    reduction plus a fixed-order sum of the four wave totals in LDS (one
//    barrier per chunk).  Each thread owns the same columns for the whole
//    launch: it loads their weights once, and the backward writes its
//    per-workgroup dw partial row straight from registers.  Both directions
//    run persistent grids (the backward's is capped at one dw partial row
//    per workgroup), so each workgroup loops over chunks; up to NVT = 4 it
//    loads the next chunk's rows while it reduces and writes the current
//    one (two register sets).  This is the engine of Llama-class hidden
//    sizes (2048 .. 16384 bf16).
//  * wave per row (narrower or unaligned rows): one 64-lane wave per row,
//    four rows per workgroup, reductions by shuffles only.  A lane's share
//    is held in registers up to NV = 8 vectors; wider rows take a two-pass
//    loop whose second pass hits the caches, and their dw comes from a
//    separate column-tiled pass.  The backward combines the four waves' dw
//    accumulators in LDS in a fixed order into one partial row per
//    workgroup.
// dw = a fixed-order column sum of the partial rows (one launch), rounded
// once to the weight dtype: deterministic, no atomics.  dx may alias dy (in
// place): every thread reads its dy elements before it writes the dx
// elements at the same addresses.  The 16-byte row loads and stores are
// nontemporal (each row is touched once per launch): backward bf16
// [8192, 4096] over rotating buffers (nothing cached) 46.0 -> 43.3 us on
// MI355X.
#include <type_traits>

#include "common.h"

namespace {

constexpr int kWaves = 4;
enum { MODE_LLAMA = 0, MODE_GEMMA = 1, MODE_NONE = 2 };

template <class T> struct Acc { typedef float type; };
template <> struct Acc<double> { typedef double type; };

template <class A> __device__ __forceinline__ A wave_sum_a(A v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}
__device__ __forceinline__ float rsqrt_a(float v) { return rsqrtf(v); }
__device__ __forceinline__ double rsqrt_a(double v) { return 1.0 / sqrt(v); }

// conversions between a storage type and the accumulation type
template <class A, class T> __device__ __forceinline__ A cv(T v) { return (A)to_f32<T>(v); }
template <> __device__ __forceinline__ double cv<double, double>(double v) { return v; }
template <class T, class A> __device__ __forceinline__ T st(A v) { return from_f32<T>((float)v); }
template <> __device__ __forceinline__ double st<double, double>(double v) { return v; }
template <class T, class A> __device__ __forceinline__ A rnd(A v) { return cv<A, T>(st<T, A>(v)); }

// VEC consecutive elements at p (16-byte vector when VEC > 1)
template <class T, int VEC, class A>
__device__ __forceinline__ void load_vec(const T* p, A (&o)[VEC]) {
  if constexpr (VEC > 1) {
    const Vec16<T> v = load16(p);
#pragma unroll
    for (int q = 0; q < VEC; ++q) o[q] = cv<A, T>(v.v[q]);
  } else {
    o[0] = cv<A, T>(p[0]);
  }
}
// VEC raw storage elements (kept packed in registers, converted on use)
template <class T, int VEC>
__device__ __forceinline__ void load_raw(const T* p, T (&o)[VEC]) {
  if constexpr (VEC > 1) {
    const Vec16<T> v = load16(p);
#pragma unroll
    for (int q = 0; q < VEC; ++q) o[q] = v.v[q];
  } else {
    o[0] = p[0];
  }
}
template <class T, int VEC, class A>
__device__ __forceinline__ void store_vec(T* p, const A (&o)[VEC]) {
  if constexpr (VEC > 1) {
    Vec16<T> v;
#pragma unroll
    for (int q = 0; q < VEC; ++q) v.v[q] = st<T, A>(o[q]);
    store16_nt(p, v);
  } else {
    p[0] = st<T, A>(o[0]);
  }
}
// weight elements (their own dtype TW; vector loads only when TW == T)
template <class TW, int VEC, class A>
__device__ __forceinline__ void load_w(const TW* w, int64_t c, A (&o)[VEC], bool wvec) {
  if constexpr (VEC * sizeof(TW) == 16) {
    if (wvec) {
      load_vec<TW, VEC, A>(w + c, o);
      return;
    }
  }
#pragma unroll
  for (int q = 0; q < VEC; ++q) o[q] = cv<A, TW>(w[c + q]);
}

struct RmsArgs {
  const void* x; int64_t ldx;
  const void* w;
  void* y; int64_t ldy;        // forward output
  const void* dy; int64_t lddy;
  void* dx; int64_t lddx;      // backward output (may alias dy)
  void* rstd;                  // [rows] of the accumulation type
  void* part;                  // dw partials [n_part][H] (accumulation type), or null
  int64_t rows, H;
  double eps, offset;
  int mode, variant, wvec;
};

// y for one element: x and rstd in A, w as loaded (A), per casting mode
template <class T, class TW, class TY, class A>
__device__ __forceinline__ A fwd_elem(A x, A rstd, A w, A off, int mode) {
  if (mode == MODE_GEMMA) return (x * rstd) * (w + off);
  const A wo = rnd<TW, A>(w + off);
  if (mode == MODE_LLAMA) return rnd<T, A>(x * rstd) * wo;
  return rnd<T, A>(x * rnd<T, A>(rstd)) * wo;  // MODE_NONE
}

template <class T, class TW, class TY, int VEC, int NV>
__global__ __launch_bounds__(256) void rms_fwd_kernel(RmsArgs a) {
  using A = typename Acc<T>::type;
  const int lane = threadIdx.x % 64;
  const int64_t H = a.H;
  const A eps = (A)a.eps, off = (A)a.offset;
  const TW* w = (const TW*)a.w;
  for (int64_t row = (int64_t)blockIdx.x * kWaves + threadIdx.x / 64; row < a.rows;
       row += (int64_t)gridDim.x * kWaves) {
    const T* xr = (const T*)a.x + row * a.ldx;
    TY* yr = (TY*)a.y + row * a.ldy;
    A ss = 0;
    if constexpr (NV > 0) {
      T xv[NV][VEC];
#pragma unroll
      for (int j = 0; j < NV; ++j) {
        const int64_t c = (int64_t)(lane + 64 * j) * VEC;
        if (c < H) {
          load_raw<T, VEC>(xr + c, xv[j]);
#pragma unroll
          for (int q = 0; q < VEC; ++q) ss += cv<A, T>(xv[j][q]) * cv<A, T>(xv[j][q]);
        }
      }
      ss = wave_sum_a(ss);
      const A rstd = rsqrt_a(ss / (A)H + eps);
      if (lane == 0) ((A*)a.rstd)[row] = rstd;
#pragma unroll
      for (int j = 0; j < NV; ++j) {
        const int64_t c = (int64_t)(lane + 64 * j) * VEC;
        if (c < H) {
          A wv[VEC], o[VEC];
          load_w<TW, VEC, A>(w, c, wv, a.wvec);
#pragma unroll
          for (int q = 0; q < VEC; ++q) o[q] = fwd_elem<T, TW, TY, A>(cv<A, T>(xv[j][q]), rstd, wv[q], off, a.mode);
          if constexpr (sizeof(TY) == sizeof(T)) {
            store_vec<TY, VEC, A>(yr + c, o);
          } else {
#pragma unroll
            for (int q = 0; q < VEC; ++q) yr[c + q] = st<TY, A>(o[q]);
          }
        }
      }
    } else {
      for (int64_t c = (int64_t)lane * VEC; c < H; c += 64 * VEC) {
        A xv[VEC];
        load_vec<T, VEC, A>(xr + c, xv);
#pragma unroll
        for (int q = 0; q < VEC; ++q) ss += xv[q] * xv[q];
      }
      ss = wave_sum_a(ss);
      const A rstd = rsqrt_a(ss / (A)H + eps);
      if (lane == 0) ((A*)a.rstd)[row] = rstd;
      for (int64_t c = (int64_t)lane * VEC; c < H; c += 64 * VEC) {
        A xv[VEC], wv[VEC], o[VEC];
        load_vec<T, VEC, A>(xr + c, xv);
        load_w<TW, VEC, A>(w, c, wv, a.wvec);
#pragma unroll
        for (int q = 0; q < VEC; ++q) o[q] = fwd_elem<T, TW, TY, A>(xv[q], rstd, wv[q], off, a.mode);
#pragma unroll
        for (int q = 0; q < VEC; ++q) yr[c + q] = st<TY, A>(o[q]);
      }
    }
  }
}

// s = dy * (w + offset): fp32 (v2-v4) or rounded to the product dtype (v1)
template <class T, class TW, class A>
__device__ __forceinline__ A scaled_dy(A dy, A w, A off, int variant) {
  if (variant == 1) return sizeof(TW) > sizeof(T) ? dy * w : rnd<T, A>(dy * w);
  return dy * (w + off);
}

// one row's contribution to dw[c]: dy * x rstd (v2-v4, fp32); v1 rounds the
// normalised x and the product to the storage dtype (its bf16 dy * normed)
template <class T, class A>
__device__ __forceinline__ A dw_term(A dy, A x, A rstd, int variant) {
  if (variant == 1) return rnd<T, A>(dy * rnd<T, A>(x * rstd));
  return dy * (x * rstd);
}

// Backward, NV > 0: rows in registers, dw accumulated per lane and reduced per
// workgroup into part[blockIdx.x].  NV == 0: two passes per row, no dw (the
// separate column pass computes it).
template <class T, class TW, int VEC, int NV>
__global__ __launch_bounds__(256) void rms_bwd_kernel(RmsArgs a) {
  using A = typename Acc<T>::type;
  constexpr int COLS = NV > 0 ? 64 * NV * VEC : 1;
  __shared__ A red[NV > 0 ? kWaves : 1][COLS];
  const int lane = threadIdx.x % 64, wave = threadIdx.x / 64;
  const int64_t H = a.H;
  const A off = (A)a.offset;
  const A inv_h = (A)1 / (A)H;
  const TW* w = (const TW*)a.w;
  const bool want_dw = a.part != nullptr;
  A dwacc[NV > 0 ? NV : 1][VEC];
#pragma unroll
  for (int j = 0; j < (NV > 0 ? NV : 1); ++j)
#pragma unroll
    for (int q = 0; q < VEC; ++q) dwacc[j][q] = 0;

  for (int64_t row = (int64_t)blockIdx.x * kWaves + wave; row < a.rows; row += (int64_t)gridDim.x * kWaves) {
    const T* xr = (const T*)a.x + row * a.ldx;
    const T* dyr = (const T*)a.dy + row * a.lddy;
    T* dxr = (T*)a.dx + row * a.lddx;
    const A rstd = ((const A*)a.rstd)[row];
    A dot = 0;
    if constexpr (NV > 0) {
      // x and dy stay packed in registers; s = dy (w + offset) is recomputed
      // in the second pass from the (cached) weight
      T xv[NV][VEC], dv[NV][VEC];
#pragma unroll
      for (int j = 0; j < NV; ++j) {
        const int64_t c = (int64_t)(lane + 64 * j) * VEC;
        if (c < H) {
          A wv[VEC];
          load_raw<T, VEC>(xr + c, xv[j]);
          load_raw<T, VEC>(dyr + c, dv[j]);
          load_w<TW, VEC, A>(w, c, wv, a.wvec);
#pragma unroll
          for (int q = 0; q < VEC; ++q)
            dot += scaled_dy<T, TW, A>(cv<A, T>(dv[j][q]), wv[q], off, a.variant) * cv<A, T>(xv[j][q]);
        }
      }
      dot = wave_sum_a(dot);
      const A k = rstd * rstd * dot * inv_h;
#pragma unroll
      for (int j = 0; j < NV; ++j) {
        const int64_t c = (int64_t)(lane + 64 * j) * VEC;
        if (c < H) {
          A wv[VEC], o[VEC];
          load_w<TW, VEC, A>(w, c, wv, a.wvec);
#pragma unroll
          for (int q = 0; q < VEC; ++q) {
            const A x = cv<A, T>(xv[j][q]), d = cv<A, T>(dv[j][q]);
            o[q] = rstd * (scaled_dy<T, TW, A>(d, wv[q], off, a.variant) - x * k);
            dwacc[j][q] += dw_term<T, A>(d, x, rstd, a.variant);
          }
          store_vec<T, VEC, A>(dxr + c, o);
        }
      }
    } else {
      for (int64_t c = (int64_t)lane * VEC; c < H; c += 64 * VEC) {
        A xv[VEC], dv[VEC], wv[VEC];
        load_vec<T, VEC, A>(xr + c, xv);
        load_vec<T, VEC, A>(dyr + c, dv);
        load_w<TW, VEC, A>(w, c, wv, a.wvec);
#pragma unroll
        for (int q = 0; q < VEC; ++q) dot += scaled_dy<T, TW, A>(dv[q], wv[q], off, a.variant) * xv[q];
      }
      dot = wave_sum_a(dot);
      const A k = rstd * rstd * dot * inv_h;
      for (int64_t c = (int64_t)lane * VEC; c < H; c += 64 * VEC) {
        A xv[VEC], dv[VEC], wv[VEC], o[VEC];
        load_vec<T, VEC, A>(xr + c, xv);
        load_vec<T, VEC, A>(dyr + c, dv);
        load_w<TW, VEC, A>(w, c, wv, a.wvec);
#pragma unroll
        for (int q = 0; q < VEC; ++q) o[q] = rstd * (scaled_dy<T, TW, A>(dv[q], wv[q], off, a.variant) - xv[q] * k);
        store_vec<T, VEC, A>(dxr + c, o);
      }
    }
  }

  if constexpr (NV > 0) {
    if (!want_dw) return;
    // the four waves' accumulators -> one partial row, summed in wave order
#pragma unroll
    for (int j = 0; j < NV; ++j)
#pragma unroll
      for (int q = 0; q < VEC; ++q) red[wave][(lane + 64 * j) * VEC + q] = dwacc[j][q];
    __syncthreads();
    A* part = (A*)a.part + (int64_t)blockIdx.x * H;
    for (int64_t c = threadIdx.x; c < H; c += 256) {
      A s = red[0][c];
#pragma unroll
      for (int v = 1; v < kWaves; ++v) s += red[v][c];
      part[c] = s;
    }
  }
}

// ---------------------------------------------------------------------------
// Workgroup-per-row-block engine (rows of 256*VEC .. 2048*VEC elements).
// The 256 threads of a workgroup span a row: thread t owns the NVT vectors
// at columns (t + 256 j) VEC, and a chunk of R rows is in flight at once
// (R * NVT = 8 vectors of x and of dy per thread).  A row's sum is a wave
// shuffle reduction plus a fixed-order sum of the four wave totals through
// LDS (double-buffered: one barrier per chunk).  In the backward each thread
// owns its dw columns outright, so a workgroup's dw partial row is written
// straight from registers.
// ---------------------------------------------------------------------------
template <class TW, int VEC>
__device__ __forceinline__ void load_w_raw(const TW* w, int64_t c, TW (&o)[VEC], bool wvec) {
  constexpr int PER = 16 / sizeof(TW);
  if constexpr (VEC >= PER && VEC % PER == 0) {
    if (wvec) {
#pragma unroll
      for (int k = 0; k < VEC / PER; ++k) {
        const Vec16<TW> v = load16(w + c + k * PER);
#pragma unroll
        for (int q = 0; q < PER; ++q) o[k * PER + q] = v.v[q];
      }
      return;
    }
  }
#pragma unroll
  for (int q = 0; q < VEC; ++q) o[q] = w[c + q];
}
// VEC values stored as TY: 16-byte stores when VEC*sizeof(TY) is a multiple
// of 16 (vec > 1 guarantees the alignment), else element stores
template <class TY, int VEC, class A>
__device__ __forceinline__ void store_n(TY* p, const A (&o)[VEC]) {
  constexpr int PER = 16 / sizeof(TY);
  if constexpr (VEC >= PER && VEC % PER == 0) {
#pragma unroll
    for (int k = 0; k < VEC / PER; ++k) {
      Vec16<TY> v;
#pragma unroll
      for (int q = 0; q < PER; ++q) v.v[q] = st<TY, A>(o[k * PER + q]);
      store16_nt(p + k * PER, v);
    }
  } else {
#pragma unroll
    for (int q = 0; q < VEC; ++q) p[q] = st<TY, A>(o[q]);
  }
}

// VEC storage elements held as 32-bit words (a 16-bit element in a scalar
// register would take a whole VGPR): 16-byte vectors load as four words,
// elements widen on use (bf16 by a shift or mask, fp16 by a convert).
template <class T, int VEC>
struct Pk {
  static constexpr int NW = (VEC * (int)sizeof(T) + 3) / 4;
  uint32_t w[NW];
};
template <class T, int VEC>
__device__ __forceinline__ void pk_load(const T* p, Pk<T, VEC>& o) {
  if constexpr (VEC * sizeof(T) == 16) {
    const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
    o.w[0] = v.x; o.w[1] = v.y; o.w[2] = v.z; o.w[3] = v.w;
  } else if constexpr (sizeof(T) == 2) {
    o.w[0] = *reinterpret_cast<const uint16_t*>(p);
  } else {
    __builtin_memcpy(o.w, p, sizeof(T));
  }
}
template <class A, class T, int VEC>
__device__ __forceinline__ A pk_get(const Pk<T, VEC>& o, int q) {
  if constexpr (std::is_same<T, bf16_t>::value) {
    const uint32_t u = o.w[q / 2];
    return (A)__uint_as_float((q & 1) ? (u & 0xffff0000u) : (u << 16));
  } else if constexpr (std::is_same<T, fp16_t>::value) {
    const uint32_t u = o.w[q / 2];
    return (A)(float)__builtin_bit_cast(fp16_t, (uint16_t)((q & 1) ? (u >> 16) : (u & 0xffffu)));
  } else if constexpr (std::is_same<T, float>::value) {
    return (A)__uint_as_float(o.w[q]);
  } else {
    double d;
    __builtin_memcpy(&d, &o.w[2 * q], 8);
    return (A)d;
  }
}
// Makes the words opaque to the optimiser (an empty asm that "modifies"
// them), so values widened before this point are not kept alive after it:
// the second pass widens the words again (a shift per element) instead of
// holding twice the registers across the barrier.
template <class T, int VEC>
__device__ __forceinline__ void keep_packed(Pk<T, VEC>& o) {
#pragma unroll
  for (int k = 0; k < Pk<T, VEC>::NW; ++k) asm volatile("" : "+v"(o.w[k]));
}

// sum over the workgroup of one value per row: wave shuffles, then the four
// wave totals in wave order (every thread gets the same bits)
template <class A, int R>
__device__ __forceinline__ void block_row_sums(A (&v)[R], A (*buf)[R], int lane, int wave) {
#pragma unroll
  for (int r = 0; r < R; ++r) v[r] = wave_sum_a(v[r]);
  if (lane == 0) {
#pragma unroll
    for (int r = 0; r < R; ++r) buf[wave][r] = v[r];
  }
  __syncthreads();
#pragma unroll
  for (int r = 0; r < R; ++r) {
    A s = buf[0][r];
#pragma unroll
    for (int k = 1; k < kWaves; ++k) s += buf[k][r];
    v[r] = s;
  }
}

// One chunk (R rows) of the workgroup forward: load() queues the rows' x
// loads into one register set; process() sums the squares, reduces them
// across the workgroup and writes y and rstd.
template <class T, class TW, class TY, int VEC, int NVT, int R, int MODE>
struct FwdChunk {
  using A = typename Acc<T>::type;
  using P = Pk<T, VEC>;

  __device__ __forceinline__ static void load(const RmsArgs& a, int tid, int64_t ch, P (&xv)[R][NVT]) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int64_t row = ch * R + r;
#pragma unroll
      for (int j = 0; j < NVT; ++j) {
        const uint32_t c = (uint32_t)(tid + 256 * j) * VEC;
        if (row < a.rows && (int64_t)c < a.H) pk_load<T, VEC>((const T*)a.x + row * a.ldx + c, xv[r][j]);
      }
    }
  }

  __device__ __forceinline__ static void process(const RmsArgs& a, int tid, int lane, int wave, int64_t ch,
                                                 P (&xv)[R][NVT], const TW (&wr)[NVT][VEC], A (*sbuf)[R]) {
    const int64_t H = a.H;
    const A eps = (A)a.eps, off = (A)a.offset;
    A ss[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      ss[r] = 0;
      const int64_t row = ch * R + r;
#pragma unroll
      for (int j = 0; j < NVT; ++j) {
        const uint32_t c = (uint32_t)(tid + 256 * j) * VEC;
        if (row < a.rows && (int64_t)c < H) {
#pragma unroll
          for (int q = 0; q < VEC; ++q) {
            const A x = pk_get<A>(xv[r][j], q);
            ss[r] += x * x;
          }
        }
      }
    }
    block_row_sums<A, R>(ss, sbuf, lane, wave);
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int j = 0; j < NVT; ++j) keep_packed(xv[r][j]);
#pragma unroll
    for (int j = 0; j < NVT; ++j) {
      const uint32_t c = (uint32_t)(tid + 256 * j) * VEC;
      if ((int64_t)c >= H) continue;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int64_t row = ch * R + r;
        if (row >= a.rows) continue;
        const A rstd = rsqrt_a(ss[r] / (A)H + eps);
        A o[VEC];
#pragma unroll
        for (int q = 0; q < VEC; ++q)
          o[q] = fwd_elem<T, TW, TY, A>(pk_get<A>(xv[r][j], q), rstd, cv<A, TW>(wr[j][q]), off, MODE);
        store_n<TY, VEC, A>((TY*)a.y + row * a.ldy + c, o);
      }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int64_t row = ch * R + r;
      if (tid == r && row < a.rows) ((A*)a.rstd)[row] = rsqrt_a(ss[r] / (A)H + eps);
    }
  }
};

// A persistent grid (fwd_grid below) over chunks blockIdx.x + i gridDim.x:
// each workgroup loads its weights once and, up to NVT = 4, queues the next
// chunk's x loads before it processes the current one (two register sets,
// as the backward).  One row per workgroup on 8192 workgroups had read the
// whole weight vector from L2 once per row.
template <class T, class TW, class TY, int VEC, int NVT, int R, int MODE>
__global__ __launch_bounds__(256) void rms_fwd_wg_kernel(RmsArgs a) {
  using K = FwdChunk<T, TW, TY, VEC, NVT, R, MODE>;
  using A = typename K::A;
  using P = typename K::P;
  __shared__ A sums[2][kWaves][R];
  const int tid = threadIdx.x, lane = tid % 64, wave = tid / 64;
  const TW* w = (const TW*)a.w;
  TW wr[NVT][VEC];  // this thread's weights, loaded once before the first row
#pragma unroll
  for (int j = 0; j < NVT; ++j) {
    const uint32_t c = (uint32_t)(tid + 256 * j) * VEC;
    if ((int64_t)c < a.H) load_w_raw<TW, VEC>(w, c, wr[j], a.wvec);
  }
  const int64_t n_chunks = (a.rows + R - 1) / R;
  const int64_t G = gridDim.x;
  if constexpr (NVT <= 4) {
    P xa[R][NVT], xb[R][NVT];
    int64_t ch = blockIdx.x;
    if (ch < n_chunks) K::load(a, tid, ch, xa);
    for (; ch < n_chunks; ch += 2 * G) {
      if (ch + G < n_chunks) K::load(a, tid, ch + G, xb);
      K::process(a, tid, lane, wave, ch, xa, wr, sums[0]);
      if (ch + G >= n_chunks) break;
      if (ch + 2 * G < n_chunks) K::load(a, tid, ch + 2 * G, xa);
      K::process(a, tid, lane, wave, ch + G, xb, wr, sums[1]);
    }
  } else {
    int buf = 0;
    for (int64_t ch = blockIdx.x; ch < n_chunks; ch += G, buf ^= 1) {
      P xv[R][NVT];
      K::load(a, tid, ch, xv);
      K::process(a, tid, lane, wave, ch, xv, wr, sums[buf]);
    }
  }
}

// One chunk (R rows) of the workgroup backward: load() queues the chunk's x,
// dy and rstd loads into one register set; process() reduces the row dots,
// writes dx and adds the dw terms.  Splitting the two lets the kernel queue
// chunk i+1's loads before it processes chunk i.
template <class T, class TW, int VEC, int NVT, int R, int VARIANT>
struct BwdChunk {
  using A = typename Acc<T>::type;
  using P = Pk<T, VEC>;

  __device__ __forceinline__ static void load(const RmsArgs& a, int tid, int64_t ch, P (&xv)[R][NVT],
                                              P (&dv)[R][NVT], A (&rs)[R]) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int64_t row = ch * R + r;
      rs[r] = row < a.rows ? ((const A*)a.rstd)[row] : (A)0;
#pragma unroll
      for (int j = 0; j < NVT; ++j) {
        const uint32_t c = (uint32_t)(tid + 256 * j) * VEC;
        if (row < a.rows && (int64_t)c < a.H) {
          pk_load<T, VEC>((const T*)a.x + row * a.ldx + c, xv[r][j]);
          pk_load<T, VEC>((const T*)a.dy + row * a.lddy + c, dv[r][j]);
        }
      }
    }
  }

  __device__ __forceinline__ static void process(const RmsArgs& a, int tid, int lane, int wave, int64_t ch,
                                                 P (&xv)[R][NVT], P (&dv)[R][NVT], const A (&rs)[R],
                                                 const TW (&wr)[NVT][VEC], A (&dwacc)[NVT][VEC],
                                                 A (*dbuf)[R]) {
    const int64_t H = a.H;
    const A off = (A)a.offset;
    const A inv_h = (A)1 / (A)H;
    A dot[R];
#pragma unroll
    for (int r = 0; r < R; ++r) dot[r] = 0;
#pragma unroll
    for (int j = 0; j < NVT; ++j) {
      const uint32_t c = (uint32_t)(tid + 256 * j) * VEC;
      if ((int64_t)c >= H) continue;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        if (ch * R + r >= a.rows) continue;
#pragma unroll
        for (int q = 0; q < VEC; ++q)
          dot[r] += scaled_dy<T, TW, A>(pk_get<A>(dv[r][j], q), cv<A, TW>(wr[j][q]), off, VARIANT) *
                    pk_get<A>(xv[r][j], q);
      }
    }
    block_row_sums<A, R>(dot, dbuf, lane, wave);
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int j = 0; j < NVT; ++j) {
        keep_packed(xv[r][j]);
        keep_packed(dv[r][j]);
      }
#pragma unroll
    for (int j = 0; j < NVT; ++j) {
      const uint32_t c = (uint32_t)(tid + 256 * j) * VEC;
      if ((int64_t)c >= H) continue;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int64_t row = ch * R + r;
        if (row >= a.rows) continue;
        const A k = rs[r] * rs[r] * dot[r] * inv_h;
        A o[VEC];
#pragma unroll
        for (int q = 0; q < VEC; ++q) {
          const A x = pk_get<A>(xv[r][j], q), d = pk_get<A>(dv[r][j], q);
          o[q] = rs[r] * (scaled_dy<T, TW, A>(d, cv<A, TW>(wr[j][q]), off, VARIANT) - x * k);
          dwacc[j][q] += dw_term<T, A>(d, x, rs[r], VARIANT);
        }
        store_vec<T, VEC, A>((T*)a.dx + row * a.lddx + c, o);
      }
    }
  }
};

// Chunks ch = blockIdx.x + i * gridDim.x in order.  With PF (NVT <= 4) two
// register sets alternate: the loads of the next chunk are queued before the
// current chunk's reduction, so a workgroup keeps HBM reads in flight across
// its barrier and its dx stores (measured on MI355X, bf16 [8192, 4096]:
// backward 52 -> 44 us cold).  At NVT = 8 the second set would take the
// kernel to 256 VGPRs and one wave per SIMD, so it runs one set.  dx may
// alias dy: the prefetched chunk's rows are never the rows being written.
template <class T, class TW, int VEC, int NVT, int R, int VARIANT>
__global__ __launch_bounds__(256) void rms_bwd_wg_kernel(RmsArgs a) {
  using K = BwdChunk<T, TW, VEC, NVT, R, VARIANT>;
  using A = typename K::A;
  using P = typename K::P;
  constexpr bool PF = NVT <= 4;
  __shared__ A dots[2][kWaves][R];
  const int tid = threadIdx.x, lane = tid % 64, wave = tid / 64;
  const int64_t H = a.H;
  const TW* w = (const TW*)a.w;
  TW wr[NVT][VEC];  // this thread's weights, loaded once
#pragma unroll
  for (int j = 0; j < NVT; ++j) {
    const uint32_t c = (uint32_t)(tid + 256 * j) * VEC;
    if ((int64_t)c < H) load_w_raw<TW, VEC>(w, c, wr[j], a.wvec);
  }
  A dwacc[NVT][VEC];
#pragma unroll
  for (int j = 0; j < NVT; ++j)
#pragma unroll
    for (int q = 0; q < VEC; ++q) dwacc[j][q] = 0;
  const int64_t n_chunks = (a.rows + R - 1) / R;
  const int64_t G = gridDim.x;
  if constexpr (PF) {
    P xa[R][NVT], da[R][NVT], xb[R][NVT], db[R][NVT];
    A ra[R], rb[R];
    int64_t ch = blockIdx.x;
    if (ch < n_chunks) K::load(a, tid, ch, xa, da, ra);
    for (; ch < n_chunks; ch += 2 * G) {
      if (ch + G < n_chunks) K::load(a, tid, ch + G, xb, db, rb);
      K::process(a, tid, lane, wave, ch, xa, da, ra, wr, dwacc, dots[0]);
      if (ch + G >= n_chunks) break;
      if (ch + 2 * G < n_chunks) K::load(a, tid, ch + 2 * G, xa, da, ra);
      K::process(a, tid, lane, wave, ch + G, xb, db, rb, wr, dwacc, dots[1]);
    }
  } else {
    int buf = 0;
    for (int64_t ch = blockIdx.x; ch < n_chunks; ch += G, buf ^= 1) {
      P xv[R][NVT], dv[R][NVT];
      A rs[R];
      K::load(a, tid, ch, xv, dv, rs);
      K::process(a, tid, lane, wave, ch, xv, dv, rs, wr, dwacc, dots[buf]);
    }
  }
  if (a.part == nullptr) return;
  A* part = (A*)a.part + (int64_t)blockIdx.x * H;
#pragma unroll
  for (int j = 0; j < NVT; ++j) {
    const uint32_t c = (uint32_t)(tid + 256 * j) * VEC;
    if ((int64_t)c < H) store_n<A, VEC, A>(part + c, dwacc[j]);
  }
}

// Column-tiled dw partials for rows too wide for register accumulators:
// part[split, c] = sum over the split's rows of dy * xhat.  Runs before the
// row kernel, which may overwrite dy with dx.
template <class T, int VEC>
__global__ __launch_bounds__(256) void rms_dw_kernel(RmsArgs a, int64_t rows_per_split) {
  using A = typename Acc<T>::type;
  const int64_t c = ((int64_t)blockIdx.x * 256 + threadIdx.x) * VEC;
  if (c >= a.H) return;
  const int64_t r0 = (int64_t)blockIdx.y * rows_per_split;
  const int64_t r1 = r0 + rows_per_split < a.rows ? r0 + rows_per_split : a.rows;
  A acc[VEC];
#pragma unroll
  for (int q = 0; q < VEC; ++q) acc[q] = 0;
  for (int64_t r = r0; r < r1; ++r) {
    const A rstd = ((const A*)a.rstd)[r];
    A xv[VEC], dv[VEC];
    load_vec<T, VEC, A>((const T*)a.x + r * a.ldx + c, xv);
    load_vec<T, VEC, A>((const T*)a.dy + r * a.lddy + c, dv);
#pragma unroll
    for (int q = 0; q < VEC; ++q) acc[q] += dw_term<T, A>(dv[q], xv[q], rstd, a.variant);
  }
  A* part = (A*)a.part + (int64_t)blockIdx.y * a.H + c;
#pragma unroll
  for (int q = 0; q < VEC; ++q) part[q] = acc[q];
}

// The column sum of the n partial rows in one launch: 64 columns per
// workgroup (one per lane); wave w of the 16 takes the consecutive block of
// ceil(n/16) partial rows starting at w ceil(n/16), loads them NB at a time
// (all in flight together) and adds them in row order; wave 0 then adds the
// 16 wave totals in wave order and rounds once to the weight dtype.  Fixed
// order throughout: deterministic.  (Replaced a two-launch version, a group
// sum of 16 rows and then a sum of the groups: 8.8 -> 4.6 us for 512
// partial rows of 4096 columns on MI355X.)
constexpr int kColsumWaves = 16;

template <class A, class TO>
__global__ __launch_bounds__(64 * kColsumWaves) void colsum_kernel(const A* part, int64_t n, int64_t H, TO* out) {
  constexpr int NB = sizeof(A) == 8 ? 16 : 32;  // rows in flight per lane (no spills at 1024 threads)
  __shared__ A red[kColsumWaves][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t c = (int64_t)blockIdx.x * 64 + lane;
  const int64_t per = (n + kColsumWaves - 1) / kColsumWaves;
  const int64_t p0 = wave * per, p1 = p0 + per < n ? p0 + per : n;
  A s = 0;
  if (c < H) {
    for (int64_t p = p0; p < p1; p += NB) {
      A v[NB];
#pragma unroll
      for (int k = 0; k < NB; ++k) v[k] = p + k < p1 ? part[(p + k) * H + c] : (A)0;
#pragma unroll
      for (int k = 0; k < NB; ++k) s += v[k];
    }
  }
  red[wave][lane] = s;
  __syncthreads();
  if (wave == 0 && c < H) {
    A t = red[0][lane];
#pragma unroll
    for (int k = 1; k < kColsumWaves; ++k) t += red[k][lane];
    out[c] = st<TO, A>(t);
  }
}

// fp32 partials, H a multiple of 16 with 16-byte aligned rows: 16 columns
// per workgroup, so a 4096-column sum spreads over 256 workgroups (one per
// CU) instead of 64.  Thread (ty, tx) (64 row groups x 4 float4 columns)
// adds the consecutive partial rows ty ceil(n/64) .. in row order, 8 loads
// in flight; the 64 group totals are then added in group order.  Fixed
// order: deterministic.
template <class TO>
__global__ __launch_bounds__(256) void colsum16_kernel(const float* part, int64_t n, int64_t H, TO* out) {
  __shared__ float red[64][17];
  const int tx = threadIdx.x & 3, ty = threadIdx.x >> 2;
  const int64_t c = (int64_t)blockIdx.x * 16 + tx * 4;
  const int64_t per = (n + 63) / 64;
  const int64_t p0 = ty * per, p1 = p0 + per < n ? p0 + per : n;
  float4 s = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int64_t p = p0; p < p1; p += 8) {
    float4 v[8];
#pragma unroll
    for (int k = 0; k < 8; ++k)
      v[k] = p + k < p1 ? *reinterpret_cast<const float4*>(part + (p + k) * H + c) : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      s.x += v[k].x;
      s.y += v[k].y;
      s.z += v[k].z;
      s.w += v[k].w;
    }
  }
  red[ty][tx * 4 + 0] = s.x;
  red[ty][tx * 4 + 1] = s.y;
  red[ty][tx * 4 + 2] = s.z;
  red[ty][tx * 4 + 3] = s.w;
  __syncthreads();
  if (threadIdx.x < 16) {
    float t = red[0][threadIdx.x];
    for (int k = 1; k < 64; ++k) t += red[k][threadIdx.x];
    out[(int64_t)blockIdx.x * 16 + threadIdx.x] = st<TO, float>(t);
  }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
constexpr int kMaxNV = 8;
#ifndef RMS_BWD_WG
#define RMS_BWD_WG 512
#endif
constexpr int kBwdMaxWG = RMS_BWD_WG;  // most dw partial rows (one per workgroup)

// dw partial rows for a backward over `rows` rows (the workspace's row count)
inline int64_t n_part_max(int64_t rows) {
  const int64_t wgs = (rows + kWaves - 1) / kWaves;
  return wgs < kBwdMaxWG ? wgs : kBwdMaxWG;
}

template <class T>
int vec_width(const RmsArgs& a, bool bwd) {
  constexpr int V = 16 / sizeof(T);
  bool ok = a.H % V == 0 && aligned16(a.x) && a.ldx % V == 0;
  if (bwd)
    ok = ok && aligned16(a.dy) && aligned16(a.dx) && a.lddy % V == 0 && a.lddx % V == 0 &&
         (a.part == nullptr || aligned16(a.part));
  else
    ok = ok && aligned16(a.y) && a.ldy % V == 0;
  return ok ? V : 1;
}

// NV (vectors per lane) for the wave-per-row engine: smallest power of two
// that covers the row, 0 (two-pass) beyond kMaxNV
inline int pick_nv(int64_t H, int vec) {
  const int64_t per_lane = (H + 64 * vec - 1) / (64 * vec);
  for (int nv = 1; nv <= kMaxNV; nv *= 2)
    if (per_lane <= nv) return nv;
  return 0;
}

// NVT (vectors per thread) for the workgroup engine: 0 when the row has
// fewer than 256 vectors (the wave-per-row engine wastes fewer lanes) or
// more than 8 per thread
inline int pick_nvt(int64_t H, int vec) {
  const int64_t nvec = (H + vec - 1) / vec;
  if (nvec < 256) return 0;
  const int64_t per = (nvec + 255) / 256;
  for (int n = 1; n <= 8; n *= 2)
    if (per <= n) return n;
  return 0;
}

template <class T, class TW, class TY, int VEC, int NVT, int R>
void fwd_wg(const RmsArgs& a, int grid, hipStream_t s) {
  switch (a.mode) {
    case MODE_LLAMA: rms_fwd_wg_kernel<T, TW, TY, VEC, NVT, R, MODE_LLAMA><<<grid, 256, 0, s>>>(a); break;
    case MODE_GEMMA: rms_fwd_wg_kernel<T, TW, TY, VEC, NVT, R, MODE_GEMMA><<<grid, 256, 0, s>>>(a); break;
    default: rms_fwd_wg_kernel<T, TW, TY, VEC, NVT, R, MODE_NONE><<<grid, 256, 0, s>>>(a); break;
  }
}

// Rows per chunk and forward grid of the workgroup engine, by vectors per
// thread (NVT 1, 2, 4, 8), from sweeps of cold fwd+bwd steps on MI355X over
// bf16 widths 2048 .. 16384 at 2^25 elements:
//  * forward: 2 / 1 / 1 / 1 rows per chunk (fewer VGPRs than 8 / 4 / 2 / 1,
//    whose 89 VGPRs at NVT = 2 left 1280 of 2048 workgroups resident) on a
//    persistent grid of 2048 workgroups up to NVT = 2 and 1024 beyond
//    (against 8192: forward 30.2 -> 27.0 us at H 2048, 29.1 -> 27.1 at
//    4096, 30.8 -> 27.7 at 8192, 35.5 -> 31.5 at 16384; 512 was slower at
//    the two narrow widths);
//  * backward: 4 / 2 / 1 / 1 rows per chunk behind its 512-workgroup cap.
// Steps against the previous kernels (8 / 4 / 2 / 1 rows both ways, one
// chunk per forward workgroup): 76.8 -> 66.2 us (H 2048), 80.6 -> 67.7
// (4096), 87.0 -> 70.4 (8192), 96.2 -> 79.8 (16384).
constexpr int fwd_rows(int nvt) { return nvt == 1 ? 2 : 1; }
constexpr int fwd_grid(int nvt) { return nvt <= 2 ? 2048 : 1024; }
constexpr int bwd_rows_per_chunk(int nvt) { return nvt == 1 ? 4 : nvt == 2 ? 2 : 1; }

template <class T, class TW, class TY, int VEC>
int fwd_v(const RmsArgs& a, hipStream_t s) {
  const int nvt = VEC > 1 ? pick_nvt(a.H, VEC) : 0;
  if constexpr (VEC > 1) {
    if (nvt) {
      const int r = fwd_rows(nvt);
      const int grid = grid_for((a.rows + r - 1) / r, 1, fwd_grid(nvt));
      switch (nvt) {
        case 1: fwd_wg<T, TW, TY, VEC, 1, fwd_rows(1)>(a, grid, s); break;
        case 2: fwd_wg<T, TW, TY, VEC, 2, fwd_rows(2)>(a, grid, s); break;
        case 4: fwd_wg<T, TW, TY, VEC, 4, fwd_rows(4)>(a, grid, s); break;
        default: fwd_wg<T, TW, TY, VEC, 8, fwd_rows(8)>(a, grid, s); break;
      }
      FORGE_CHECK_LAUNCH();
      return FORGE_OK;
    }
  }
  const int grid = grid_for((a.rows + kWaves - 1) / kWaves, 1, 256 * 8);
  switch (pick_nv(a.H, VEC)) {
    case 1: rms_fwd_kernel<T, TW, TY, VEC, 1><<<grid, 256, 0, s>>>(a); break;
    case 2: rms_fwd_kernel<T, TW, TY, VEC, 2><<<grid, 256, 0, s>>>(a); break;
    case 4: rms_fwd_kernel<T, TW, TY, VEC, 4><<<grid, 256, 0, s>>>(a); break;
    case 8: rms_fwd_kernel<T, TW, TY, VEC, 8><<<grid, 256, 0, s>>>(a); break;
    default: rms_fwd_kernel<T, TW, TY, VEC, 0><<<grid, 256, 0, s>>>(a); break;
  }
  FORGE_CHECK_LAUNCH();
  return FORGE_OK;
}

template <class T, class TW, class TY>
int fwd_t(RmsArgs a, hipStream_t s) {
  constexpr int V = 16 / sizeof(T);
  const int vec = vec_width<T>(a, false);
  a.wvec = vec > 1 && aligned16(a.w);
  if (vec == V) return fwd_v<T, TW, TY, V>(a, s);
  return fwd_v<T, TW, TY, 1>(a, s);
}

template <class T, class TW, int VEC, int NVT, int R>
void bwd_wg(const RmsArgs& a, int grid, hipStream_t s) {
  if (a.variant == 1) rms_bwd_wg_kernel<T, TW, VEC, NVT, R, 1><<<grid, 256, 0, s>>>(a);
  else rms_bwd_wg_kernel<T, TW, VEC, NVT, R, 0><<<grid, 256, 0, s>>>(a);
}

// the row kernels of the backward; returns the number of dw partial rows
// they wrote (0 when a.part is null)
template <class T, class TW, int VEC>
int64_t bwd_rows(RmsArgs a, hipStream_t s) {
  const int64_t npm = n_part_max(a.rows);
  const int nvt = VEC > 1 ? pick_nvt(a.H, VEC) : 0;
  if constexpr (VEC > 1) {
    if (nvt) {
      const int br = bwd_rows_per_chunk(nvt);
      const int64_t chunks = (a.rows + br - 1) / br;
      const int grid = (int)(chunks < npm ? chunks : npm);
      switch (nvt) {
        case 1: bwd_wg<T, TW, VEC, 1, bwd_rows_per_chunk(1)>(a, grid, s); break;
        case 2: bwd_wg<T, TW, VEC, 2, bwd_rows_per_chunk(2)>(a, grid, s); break;
        case 4: bwd_wg<T, TW, VEC, 4, bwd_rows_per_chunk(4)>(a, grid, s); break;
        default: bwd_wg<T, TW, VEC, 8, bwd_rows_per_chunk(8)>(a, grid, s); break;
      }
      return a.part ? grid : 0;
    }
  }
  const int nv = pick_nv(a.H, VEC);
  int64_t np = 0;
  if (nv == 0 && a.part) {  // column pass first (the row pass may overwrite dy)
    const int64_t per = (a.rows + npm - 1) / npm;
    np = (a.rows + per - 1) / per;
    const dim3 g2((unsigned)((a.H / VEC + 255) / 256), (unsigned)np);
    rms_dw_kernel<T, VEC><<<g2, 256, 0, s>>>(a, per);
    a.part = nullptr;
  } else if (a.part) {
    np = npm;
  }
  switch (nv) {
    case 1: rms_bwd_kernel<T, TW, VEC, 1><<<(int)npm, 256, 0, s>>>(a); break;
    case 2: rms_bwd_kernel<T, TW, VEC, 2><<<(int)npm, 256, 0, s>>>(a); break;
    case 4: rms_bwd_kernel<T, TW, VEC, 4><<<(int)npm, 256, 0, s>>>(a); break;
    case 8: rms_bwd_kernel<T, TW, VEC, 8><<<(int)npm, 256, 0, s>>>(a); break;
    default: rms_bwd_kernel<T, TW, VEC, 0><<<(int)npm, 256, 0, s>>>(a); break;
  }
  return np;
}

template <class A, class TO>
void colsum(const A* part, int64_t np, int64_t H, TO* dw, hipStream_t s) {
  if constexpr (std::is_same<A, float>::value) {
    if (H % 16 == 0 && aligned16(part)) {
      colsum16_kernel<TO><<<(unsigned)(H / 16), 256, 0, s>>>(part, np, H, dw);
      return;
    }
  }
  colsum_kernel<A, TO><<<(unsigned)((H + 63) / 64), 64 * kColsumWaves, 0, s>>>(part, np, H, dw);
}

template <class T, class TW>
int bwd_launch(RmsArgs a, void* dw, int w_dtype, hipStream_t s) {
  using A = typename Acc<T>::type;
  constexpr int V = 16 / sizeof(T);
  const int vec = vec_width<T>(a, true);
  a.wvec = vec > 1 && aligned16(a.w);
  const int64_t np = vec == V ? bwd_rows<T, TW, V>(a, s) : bwd_rows<T, TW, 1>(a, s);
  FORGE_CHECK_LAUNCH();
  if (np && dw) {
    A* part = (A*)a.part;
    switch (w_dtype) {
      case FORGE_DTYPE_F32: colsum<A, float>(part, np, a.H, (float*)dw, s); break;
      case FORGE_DTYPE_BF16: colsum<A, bf16_t>(part, np, a.H, (bf16_t*)dw, s); break;
      case FORGE_DTYPE_F16: colsum<A, fp16_t>(part, np, a.H, (fp16_t*)dw, s); break;
      case FORGE_DTYPE_F64: colsum<A, double>(part, np, a.H, (double*)dw, s); break;
      default: return forge_set_error(FORGE_ERR_UNSUPPORTED, "rmsnorm_bwd: weight dtype %d", w_dtype);
    }
    FORGE_CHECK_LAUNCH();
  }
  return FORGE_OK;
}

int64_t acc_size(int dtype) { return dtype == FORGE_DTYPE_F64 ? 8 : 4; }

}  // namespace

extern "C" int64_t forge_rmsnorm_bwd_workspace(int dtype, int64_t rows, int64_t cols) {
  if (rows <= 0 || cols <= 0) return 0;
  return n_part_max(rows) * cols * acc_size(dtype);
}

extern "C" int forge_rmsnorm_fwd(int dtype, int w_dtype, int y_dtype, const void* x, int64_t ldx, const void* w,
                                 void* y, int64_t ldy, void* rstd, int64_t rows, int64_t cols, double eps,
                                 double offset, int casting_mode, void* stream) {
  if (rows < 0 || cols < 0) return forge_set_error(FORGE_ERR_INVALID, "rmsnorm_fwd: negative shape");
  if (rows == 0 || cols == 0) return FORGE_OK;
  if (ldx < cols || ldy < cols) return forge_set_error(FORGE_ERR_INVALID, "rmsnorm_fwd: row pitch < cols");
  if (casting_mode < MODE_LLAMA || casting_mode > MODE_NONE)
    return forge_set_error(FORGE_ERR_INVALID, "rmsnorm_fwd: casting mode %d", casting_mode);
  RmsArgs a = {};
  a.x = x; a.ldx = ldx; a.w = w; a.y = y; a.ldy = ldy; a.rstd = rstd;
  a.rows = rows; a.H = cols; a.eps = eps; a.offset = offset; a.mode = casting_mode;
  hipStream_t s = (hipStream_t)stream;
  const bool same_w = w_dtype == dtype, fw = w_dtype == FORGE_DTYPE_F32;
  const bool same_y = y_dtype == dtype, fy = y_dtype == FORGE_DTYPE_F32;
  switch (dtype) {
    case FORGE_DTYPE_F32:
      if (same_w && same_y) return fwd_t<float, float, float>(a, s);
      break;
    case FORGE_DTYPE_F64:
      if (same_w && same_y) return fwd_t<double, double, double>(a, s);
      break;
    case FORGE_DTYPE_BF16:
      if (same_w && same_y) return fwd_t<bf16_t, bf16_t, bf16_t>(a, s);
      if (fw && same_y) return fwd_t<bf16_t, float, bf16_t>(a, s);
      if (fw && fy) return fwd_t<bf16_t, float, float>(a, s);
      break;
    case FORGE_DTYPE_F16:
      if (same_w && same_y) return fwd_t<fp16_t, fp16_t, fp16_t>(a, s);
      if (fw && same_y) return fwd_t<fp16_t, float, fp16_t>(a, s);
      if (fw && fy) return fwd_t<fp16_t, float, float>(a, s);
      break;
  }
  return forge_set_error(FORGE_ERR_UNSUPPORTED, "rmsnorm_fwd: dtypes x %d, weight %d, y %d", dtype, w_dtype, y_dtype);
}

extern "C" int forge_rmsnorm_bwd(int dtype, int w_dtype, const void* dy, int64_t lddy, const void* x, int64_t ldx,
                                 const void* w, const void* rstd, void* dx, int64_t lddx, void* dw, void* work,
                                 int64_t rows, int64_t cols, double offset, int variant, void* stream) {
  if (rows < 0 || cols < 0) return forge_set_error(FORGE_ERR_INVALID, "rmsnorm_bwd: negative shape");
  if (rows == 0 || cols == 0) return FORGE_OK;
  if (ldx < cols || lddy < cols || lddx < cols)
    return forge_set_error(FORGE_ERR_INVALID, "rmsnorm_bwd: row pitch < cols");
  if (variant != 0 && variant != 1) return forge_set_error(FORGE_ERR_INVALID, "rmsnorm_bwd: variant %d", variant);
  if (dw && !work) return forge_set_error(FORGE_ERR_INVALID, "rmsnorm_bwd: dw needs the partial-sum workspace");
  RmsArgs a = {};
  a.x = x; a.ldx = ldx; a.w = w; a.dy = dy; a.lddy = lddy; a.dx = dx; a.lddx = lddx; a.rstd = const_cast<void*>(rstd);
  a.part = dw ? work : nullptr;
  a.rows = rows; a.H = cols; a.offset = offset; a.variant = variant;
  hipStream_t s = (hipStream_t)stream;
  const bool same_w = w_dtype == dtype, fw = w_dtype == FORGE_DTYPE_F32;
  switch (dtype) {
    case FORGE_DTYPE_F32:
      if (same_w) return bwd_launch<float, float>(a, dw, w_dtype, s);
      break;
    case FORGE_DTYPE_F64:
      if (same_w) return bwd_launch<double, double>(a, dw, w_dtype, s);
      break;
    case FORGE_DTYPE_BF16:
      if (same_w) return bwd_launch<bf16_t, bf16_t>(a, dw, w_dtype, s);
      if (fw) return bwd_launch<bf16_t, float>(a, dw, w_dtype, s);
      break;
    case FORGE_DTYPE_F16:
      if (same_w) return bwd_launch<fp16_t, fp16_t>(a, dw, w_dtype, s);
      if (fw) return bwd_launch<fp16_t, float>(a, dw, w_dtype, s);
      break;
  }
  return forge_set_error(FORGE_ERR_UNSUPPORTED, "rmsnorm_bwd: dtypes x %d, weight %d", dtype, w_dtype);
}
