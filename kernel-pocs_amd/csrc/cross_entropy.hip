// Cross-entropy forward (+ in-place dlogits) for gfx950.
//
// Reference: forge_cross_entropy_kernel,
// kernels/cross_entropy/experiments/v2/cross_entropy_kernel_v2.py:65-338.
// Per row of logits:
//   * target == ignore_index: the row is zero-filled (always, as in the
//     reference, :139-151), accuracy 0, predicted -1, loss 0.
//   * otherwise an online max/sum over the row gives lse = m + log d (:167-218);
//     with gradients the row is overwritten by dloss/dlogits (:234-285); the
//     loss is lse - x_y with label smoothing, class weights, z-loss and the
//     reduction scaling of :298-330.
//
// Two row engines:
//   * ce_resident_kernel: the whole row is held in registers (one 1024-thread
//     workgroup per row), so the logits are read from HBM once and written once.
//     Pass A finds the exact row max, pass B sums exp(x - m) and keeps
//     p = exp(x - m) as fp16 in place of the input, pass C writes p/d.
//     Used for the common case (no class weights / softcap / argmax) when the
//     row fits in 1024 * 8 * NV elements.
//   * ce_stream_kernel: any row length and every feature; the row is streamed
//     twice (online max/sum, then gradient), the second read largely served by
//     the L2 / Infinity Cache.
// exp is evaluated as exp2 on log2e-prescaled values (one FMA + v_exp_f32).
#include "common.h"

namespace {

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

struct CeArgs {
  void* x;
  int64_t ld;
  int64_t n_rows, n_cols;
  const int64_t* target;
  int64_t target_stride;
  const float* weight;
  float* loss;
  float* z_loss;
  float* acc;
  int64_t* pred;
  int64_t ignore_index;
  float n_non_ignore, sum_non_ignore_weight, weight_sum, lse_square_scale, label_smoothing, softcap;
  int flags;
};

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Merges two (max, sum) pairs of an online softmax in the log2 domain.
__device__ __forceinline__ void lse_merge(float& m, float& d, float m2, float d2) {
  float mn = fmaxf(m, m2);
  if (mn == -INFINITY) return;  // both empty
  d = d * fast_exp2(m - mn) + d2 * fast_exp2(m2 - mn);
  m = mn;
}

// Block-wide reductions through LDS.  `red` holds one slot per wave.
template <int NW>
__device__ __forceinline__ float block_max(float v, float* red) {
  v = wave_max(v);
  const int w = threadIdx.x / 64, l = threadIdx.x % 64;
  __syncthreads();
  if (l == 0) red[w] = v;
  __syncthreads();
  float r = red[0];
#pragma unroll
  for (int i = 1; i < NW; ++i) r = fmaxf(r, red[i]);
  return r;
}

template <int NW>
__device__ __forceinline__ float block_sum(float v, float* red) {
  v = wave_sum(v);
  const int w = threadIdx.x / 64, l = threadIdx.x % 64;
  __syncthreads();
  if (l == 0) red[w] = v;
  __syncthreads();
  float r = 0.f;
#pragma unroll
  for (int i = 0; i < NW; ++i) r += red[i];
  return r;
}

template <int NW>
__device__ __forceinline__ void block_lse(float& m, float& d, float* red) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    float m2 = __shfl_xor(m, off, 64), d2 = __shfl_xor(d, off, 64);
    lse_merge(m, d, m2, d2);
  }
  const int w = threadIdx.x / 64, l = threadIdx.x % 64;
  __syncthreads();
  if (l == 0) { red[2 * w] = m; red[2 * w + 1] = d; }
  __syncthreads();
  m = red[0];
  d = red[1];
#pragma unroll
  for (int i = 1; i < NW; ++i) lse_merge(m, d, red[2 * i], red[2 * i + 1]);
}

// (max value, first index) reduction for argmax.
template <int NW>
__device__ __forceinline__ int64_t block_argmax(float v, int64_t idx, float* redf, int64_t* redi) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    float v2 = __shfl_xor(v, off, 64);
    int64_t i2 = __shfl_xor(idx, off, 64);
    if (v2 > v || (v2 == v && i2 < idx)) { v = v2; idx = i2; }
  }
  const int w = threadIdx.x / 64, l = threadIdx.x % 64;
  __syncthreads();
  if (l == 0) { redf[w] = v; redi[w] = idx; }
  __syncthreads();
  v = redf[0];
  idx = redi[0];
#pragma unroll
  for (int i = 1; i < NW; ++i)
    if (redf[i] > v || (redf[i] == v && redi[i] < idx)) { v = redf[i]; idx = redi[i]; }
  return idx;
}

template <class T>
__device__ __forceinline__ void zero_row(T* row, int64_t n, bool vec) {
  if (vec) {
    constexpr int V = 16 / sizeof(T);
    Vec16<T> z;
    z.raw = make_uint4(0, 0, 0, 0);
    for (int64_t c = (int64_t)threadIdx.x * V; c < n; c += (int64_t)blockDim.x * V) store16(row + c, z);
  } else {
    for (int64_t c = threadIdx.x; c < n; c += blockDim.x) row[c] = from_f32<T>(0.f);
  }
}

// Loss bookkeeping shared by both engines (thread 0 only).
__device__ __forceinline__ void write_row_outputs(const CeArgs& a, int64_t row, int64_t y, float lse,
                                                  float xy, float wy, float scaled_x_sum,
                                                  int64_t argmax) {
  const bool has_w = a.flags & FORGE_CE_HAS_WEIGHT;
  const bool mean = a.flags & FORGE_CE_REDUCTION_MEAN;
  float loss = lse - xy;
  if (has_w) loss = wy * loss;
  if (a.label_smoothing > 0.f) {
    const float eps = a.label_smoothing / (float)a.n_cols;
    float smooth = has_w ? scaled_x_sum + eps * lse * a.weight_sum : scaled_x_sum + a.label_smoothing * lse;
    loss = loss * (1.f - a.label_smoothing) + smooth;
  }
  float z = a.lse_square_scale * lse * lse;
  if (mean) {
    loss = loss / (has_w ? a.sum_non_ignore_weight : a.n_non_ignore);
    z = z / a.n_non_ignore;
  }
  loss += z;
  a.loss[row] = loss;
  if (a.flags & FORGE_CE_RETURN_Z_LOSS) a.z_loss[row] = z;
  if (a.flags & FORGE_CE_RETURN_ACCURACY) a.acc[row] = (argmax == y) ? 1.f : 0.f;
  if (a.flags & FORGE_CE_RETURN_PREDICTED) a.pred[row] = argmax;
}

__device__ __forceinline__ void write_ignored_outputs(const CeArgs& a, int64_t row) {
  a.loss[row] = 0.f;
  if (a.flags & FORGE_CE_RETURN_Z_LOSS) a.z_loss[row] = 0.f;
  if (a.flags & FORGE_CE_RETURN_ACCURACY) a.acc[row] = 0.f;
  if (a.flags & FORGE_CE_RETURN_PREDICTED) a.pred[row] = -1;
}

// ---------------------------------------------------------------------------
// Streaming engine (every feature, any row length)
// ---------------------------------------------------------------------------
constexpr int kStreamBlock = 512;
constexpr int kStreamWaves = kStreamBlock / 64;

template <class T, int VEC>
__global__ __launch_bounds__(kStreamBlock) void ce_stream_kernel(CeArgs a) {
  __shared__ float redf[2 * kStreamWaves];
  __shared__ int64_t redi[kStreamWaves];
  const int64_t row = blockIdx.x;
  const int64_t y = a.target[row * a.target_stride];
  T* xr = (T*)a.x + row * a.ld;
  const int64_t V = a.n_cols;
  const bool vec = VEC > 1;

  if (y == a.ignore_index) {
    zero_row<T>(xr, V, vec);
    if (threadIdx.x == 0) write_ignored_outputs(a, row);
    return;
  }

  const bool has_w = a.flags & FORGE_CE_HAS_WEIGHT;
  const bool has_sc = a.flags & FORGE_CE_HAS_SOFTCAP;
  const bool need_arg = a.flags & (FORGE_CE_RETURN_ACCURACY | FORGE_CE_RETURN_PREDICTED);
  const bool grads = a.flags & FORGE_CE_HAS_GRADIENTS;
  const float sc = a.softcap;
  const float ls = a.label_smoothing;
  const float eps = ls / (float)V;
  const float wy = has_w ? a.weight[y] : 1.f;
  float xy = to_f32(xr[y]);
  if (has_sc) xy = sc * tanhf(xy / sc);

  // ---- pass 1: online max / sum (log2 domain), argmax, smoothing sum ----
  float m = -INFINITY, d = 0.f, sxs = 0.f, amax_v = -INFINITY;
  int64_t amax_i = V;
  for (int64_t c0 = (int64_t)threadIdx.x * VEC; c0 < V; c0 += (int64_t)kStreamBlock * VEC) {
    float v[VEC];
    if constexpr (VEC > 1) {
      Vec16<T> raw = load16(xr + c0);
#pragma unroll
      for (int j = 0; j < VEC; ++j) v[j] = to_f32(raw.v[j]);
    } else {
      v[0] = to_f32(xr[c0]);
    }
    float vm = -INFINITY;
#pragma unroll
    for (int j = 0; j < VEC; ++j) {
      if (has_sc) v[j] = sc * tanhf(v[j] / sc);
      if (need_arg && v[j] > amax_v) { amax_v = v[j]; amax_i = c0 + j; }
      if (ls > 0.f) sxs += has_w ? -eps * v[j] * a.weight[c0 + j] : -eps * v[j];
      v[j] *= kLog2e;
      vm = fmaxf(vm, v[j]);
    }
    if (vm > m) {
      d = (m == -INFINITY) ? 0.f : d * fast_exp2(m - vm);
      m = vm;
    }
    if (m != -INFINITY) {
#pragma unroll
      for (int j = 0; j < VEC; ++j) d += fast_exp2(v[j] - m);
    }
  }
  block_lse<kStreamWaves>(m, d, redf);
  float sxs_tot = 0.f;
  if (ls > 0.f) sxs_tot = block_sum<kStreamWaves>(sxs, redf);
  int64_t amax = 0;
  if (need_arg) amax = block_argmax<kStreamWaves>(amax_v, amax_i, redf, redi);
  // natural-log lse: m is log2-scaled
  const float lse = (m + __log2f(d)) * kLn2;

  // ---- pass 2: gradient in place ----
  if (grads) {
    const bool mean = a.flags & FORGE_CE_REDUCTION_MEAN;
    const float lss = a.lse_square_scale;
    const float m2 = m + __log2f(d);  // exp2(v*log2e - m2) = softmax
    const float inv_n = 1.f / a.n_non_ignore;
    const float inv_snw = 1.f / a.sum_non_ignore_weight;
    for (int64_t c0 = (int64_t)threadIdx.x * VEC; c0 < V; c0 += (int64_t)kStreamBlock * VEC) {
      float v[VEC], th[VEC];
      if constexpr (VEC > 1) {
        Vec16<T> raw = load16(xr + c0);
#pragma unroll
        for (int j = 0; j < VEC; ++j) v[j] = to_f32(raw.v[j]);
      } else {
        v[0] = to_f32(xr[c0]);
      }
      float g[VEC];
#pragma unroll
      for (int j = 0; j < VEC; ++j) {
        if (has_sc) { th[j] = tanhf(v[j] / sc); v[j] = sc * th[j]; }
        const float p = fast_exp2(fmaf(v[j], kLog2e, -m2));
        const bool is_y = (c0 + j) == y;
        if (!has_w) {
          float t = p + 2.f * lss * lse * p;
          t += -eps;
          if (is_y) t -= (1.f - ls);
          if (mean) t = t / a.n_non_ignore;
          g[j] = t;
        } else {
          float ori = (1.f - ls) * p;
          if (is_y) ori -= (1.f - ls);
          ori *= wy;
          float smooth = eps * (-a.weight[c0 + j] + p * a.weight_sum);
          float dz = 2.f * lss * lse * p;
          if (mean) { ori *= inv_snw; smooth *= inv_snw; dz *= inv_n; }
          g[j] = ori + smooth + dz;
        }
        if (has_sc) g[j] *= (1.f - th[j] * th[j]);
      }
      if constexpr (VEC > 1) {
        Vec16<T> o;
#pragma unroll
        for (int j = 0; j < VEC; ++j) o.v[j] = from_f32<T>(g[j]);
        store16(xr + c0, o);
      } else {
        xr[c0] = from_f32<T>(g[0]);
      }
    }
  }
  if (threadIdx.x == 0) write_row_outputs(a, row, y, lse, xy, wy, sxs_tot, amax);
}

// ---------------------------------------------------------------------------
// Register-resident engine (plain CE with optional smoothing / z-loss)
// ---------------------------------------------------------------------------
constexpr int kResBlock = 1024;
constexpr int kResWaves = kResBlock / 64;

typedef __fp16 half2_t __attribute__((ext_vector_type(2)));

template <class T, int NV>
__global__ __launch_bounds__(kResBlock) void ce_resident_kernel(CeArgs a) {
  constexpr int VEC = 16 / sizeof(T);
  __shared__ float redf[2 * kResWaves];
  const int64_t row = blockIdx.x;
  const int64_t y = a.target[row * a.target_stride];
  T* xr = (T*)a.x + row * a.ld;
  const int64_t V = a.n_cols;

  if (y == a.ignore_index) {
    zero_row<T>(xr, V, true);
    if (threadIdx.x == 0) write_ignored_outputs(a, row);
    return;
  }
  const float xy = to_f32(xr[y]);
  const float ls = a.label_smoothing;

  // Column of vector i of this thread: (i * kResBlock + tid) * VEC.
  Vec16<T> buf[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int64_t c0 = ((int64_t)i * kResBlock + threadIdx.x) * VEC;
    if (c0 < V) buf[i] = load16_nt(xr + c0);
  }

  // pass A: exact max (and the smoothing sum)
  float m = -INFINITY, sx = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int64_t c0 = ((int64_t)i * kResBlock + threadIdx.x) * VEC;
    if (c0 < V) {
#pragma unroll
      for (int j = 0; j < VEC; ++j) {
        float v = to_f32(buf[i].v[j]);
        m = fmaxf(m, v);
        if (ls > 0.f) sx += v;
      }
    }
  }
  m = block_max<kResWaves>(m, redf);
  const float ml2 = m * kLog2e;

  // pass B: sum of exp(x - m); keep p = exp(x - m) as fp16 in the buffer
  float d = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int64_t c0 = ((int64_t)i * kResBlock + threadIdx.x) * VEC;
    if (c0 < V) {
      Vec16<T> pv;
      half2_t* ph = reinterpret_cast<half2_t*>(&pv.raw);
#pragma unroll
      for (int j = 0; j < VEC; j += 2) {
        float p0 = fast_exp2(fmaf(to_f32(buf[i].v[j]), kLog2e, -ml2));
        float p1 = fast_exp2(fmaf(to_f32(buf[i].v[j + 1]), kLog2e, -ml2));
        d += p0 + p1;
        if constexpr (sizeof(T) == 2) ph[j / 2] = __builtin_amdgcn_cvt_pkrtz(p0, p1);
        else { buf[i].v[j] = from_f32<T>(p0); buf[i].v[j + 1] = from_f32<T>(p1); }
      }
      if constexpr (sizeof(T) == 2) buf[i].raw = pv.raw;
    }
  }
  d = block_sum<kResWaves>(d, redf);
  float sx_tot = 0.f;
  if (ls > 0.f) sx_tot = block_sum<kResWaves>(sx, redf);
  const float lse = m + __logf(d);

  if (a.flags & FORGE_CE_HAS_GRADIENTS) {
    const bool mean = a.flags & FORGE_CE_REDUCTION_MEAN;
    const float eps = ls / (float)V;
    // g = p * scale - shift   (+ the target adjustment below)
    float scale = (1.f + 2.f * a.lse_square_scale * lse) / d;
    float shift = eps;
    float ydelta = (1.f - ls);
    if (mean) {
      scale /= a.n_non_ignore;
      shift /= a.n_non_ignore;
      ydelta /= a.n_non_ignore;
    }
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int64_t c0 = ((int64_t)i * kResBlock + threadIdx.x) * VEC;
      if (c0 < V) {
        Vec16<T> o;
        const half2_t* ph = reinterpret_cast<const half2_t*>(&buf[i].raw);
#pragma unroll
        for (int j = 0; j < VEC; j += 2) {
          float p0, p1;
          if constexpr (sizeof(T) == 2) { p0 = (float)ph[j / 2].x; p1 = (float)ph[j / 2].y; }
          else { p0 = to_f32(buf[i].v[j]); p1 = to_f32(buf[i].v[j + 1]); }
          o.v[j] = from_f32<T>(fmaf(p0, scale, -shift));
          o.v[j + 1] = from_f32<T>(fmaf(p1, scale, -shift));
        }
        if (y >= c0 && y < c0 + VEC) {
          // exact value for the target column (recomputed from x_y in fp32)
          const float py = fast_exp2(fmaf(xy, kLog2e, -ml2));
          o.v[y - c0] = from_f32<T>(fmaf(py, scale, -shift) - ydelta);
        }
        store16_nt(xr + c0, o);
      }
    }
  }
  if (threadIdx.x == 0) {
    const float sxs = -(ls / (float)V) * sx_tot;
    write_row_outputs(a, row, y, lse, xy, 1.f, sxs, 0);
  }
}

template <class T>
int launch_ce(CeArgs a, hipStream_t s) {
  constexpr int V = 16 / sizeof(T);
  const bool vec = aligned16(a.x) && (a.ld % V == 0) && (a.n_cols % V == 0);
  const bool plain = !(a.flags & (FORGE_CE_HAS_WEIGHT | FORGE_CE_HAS_SOFTCAP |
                                  FORGE_CE_RETURN_ACCURACY | FORGE_CE_RETURN_PREDICTED));
  const int64_t nvec = (a.n_cols + (int64_t)kResBlock * V - 1) / ((int64_t)kResBlock * V);
  dim3 grid((unsigned)a.n_rows);
  if (vec && plain && sizeof(T) == 2 && nvec <= 16) {
    if (nvec <= 4)
      ce_resident_kernel<T, 4><<<grid, kResBlock, 0, s>>>(a);
    else if (nvec <= 8)
      ce_resident_kernel<T, 8><<<grid, kResBlock, 0, s>>>(a);
    else
      ce_resident_kernel<T, 16><<<grid, kResBlock, 0, s>>>(a);
  } else if (vec) {
    ce_stream_kernel<T, V><<<grid, kStreamBlock, 0, s>>>(a);
  } else {
    ce_stream_kernel<T, 1><<<grid, kStreamBlock, 0, s>>>(a);
  }
  FORGE_CHECK_LAUNCH();
  return FORGE_OK;
}

// ---------------------------------------------------------------------------
// grad_output scaling and the fp32 loss sum
// ---------------------------------------------------------------------------
template <class T, int VEC>
__global__ __launch_bounds__(256) void ce_scale_kernel(T* x, int64_t ld, int64_t rows, int64_t cols,
                                                       const float* g) {
  const float s = *g;
  const int64_t cpr = cols / VEC;
  const int64_t n = rows * cpr;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    const int64_t r = i / cpr, c = (i - r * cpr) * VEC;
    T* p = x + r * ld + c;
    if constexpr (VEC > 1) {
      Vec16<T> v = load16(p);
#pragma unroll
      for (int j = 0; j < VEC; ++j) v.v[j] = from_f32<T>(to_f32(v.v[j]) * s);
      store16(p, v);
    } else {
      p[0] = from_f32<T>(to_f32(p[0]) * s);
    }
  }
}

template <class T>
int launch_scale(void* x, int64_t ld, int64_t rows, int64_t cols, const float* g, hipStream_t s) {
  constexpr int V = 16 / sizeof(T);
  const bool vec = aligned16(x) && ld % V == 0 && cols % V == 0;
  if (vec) {
    int grid = grid_for(rows * cols / V, 256);
    ce_scale_kernel<T, V><<<grid, 256, 0, s>>>((T*)x, ld, rows, cols, g);
  } else {
    int grid = grid_for(rows * cols, 256);
    ce_scale_kernel<T, 1><<<grid, 256, 0, s>>>((T*)x, ld, rows, cols, g);
  }
  FORGE_CHECK_LAUNCH();
  return FORGE_OK;
}

// Single-workgroup deterministic sum (the vector is one value per row).
__global__ __launch_bounds__(1024) void sum_f32_kernel(const float* x, int64_t n, float* out) {
  __shared__ float red[16];
  float acc = 0.f;
  for (int64_t i = threadIdx.x; i < n; i += 1024) acc += x[i];
  acc = block_sum<16>(acc, red);
  if (threadIdx.x == 0) out[0] = acc;
}

}  // namespace

extern "C" int forge_ce_fwd(int dtype, void* logits, int64_t ld, int64_t n_rows, int64_t n_cols,
                            const int64_t* target, int64_t target_stride, const float* weight,
                            float* loss, float* z_loss, float* token_accuracy,
                            int64_t* predicted_tokens, int64_t ignore_index, float n_non_ignore,
                            float sum_non_ignore_weight, float weight_sum, float lse_square_scale,
                            float label_smoothing, float softcap, int flags, void* stream) {
  if (n_rows < 0 || n_cols < 0) return forge_set_error(FORGE_ERR_INVALID, "ce_fwd: negative shape");
  if (n_rows == 0) return FORGE_OK;
  if (n_rows > 0x7fffffff) return forge_set_error(FORGE_ERR_INVALID, "ce_fwd: too many rows");
  if (ld < n_cols) return forge_set_error(FORGE_ERR_INVALID, "ce_fwd: ld < n_cols");
  if ((flags & FORGE_CE_HAS_WEIGHT) && !weight)
    return forge_set_error(FORGE_ERR_INVALID, "ce_fwd: weight flag without weight");
  if (!loss) return forge_set_error(FORGE_ERR_INVALID, "ce_fwd: loss buffer required");
  if ((flags & FORGE_CE_RETURN_Z_LOSS) && !z_loss)
    return forge_set_error(FORGE_ERR_INVALID, "ce_fwd: z_loss buffer required");
  if ((flags & FORGE_CE_RETURN_ACCURACY) && !token_accuracy)
    return forge_set_error(FORGE_ERR_INVALID, "ce_fwd: accuracy buffer required");
  if ((flags & FORGE_CE_RETURN_PREDICTED) && !predicted_tokens)
    return forge_set_error(FORGE_ERR_INVALID, "ce_fwd: predicted buffer required");
  CeArgs a;
  a.x = logits; a.ld = ld; a.n_rows = n_rows; a.n_cols = n_cols;
  a.target = target; a.target_stride = target_stride; a.weight = weight;
  a.loss = loss; a.z_loss = z_loss; a.acc = token_accuracy; a.pred = predicted_tokens;
  a.ignore_index = ignore_index; a.n_non_ignore = n_non_ignore;
  a.sum_non_ignore_weight = sum_non_ignore_weight; a.weight_sum = weight_sum;
  a.lse_square_scale = lse_square_scale; a.label_smoothing = label_smoothing; a.softcap = softcap;
  a.flags = flags;
  hipStream_t s = (hipStream_t)stream;
  switch (dtype) {
    case FORGE_DTYPE_F32: return launch_ce<float>(a, s);
    case FORGE_DTYPE_BF16: return launch_ce<bf16_t>(a, s);
    case FORGE_DTYPE_F16: return launch_ce<fp16_t>(a, s);
    default: return forge_set_error(FORGE_ERR_UNSUPPORTED, "ce_fwd: dtype %d", dtype);
  }
}

extern "C" int forge_ce_scale(int dtype, void* x, int64_t ld, int64_t n_rows, int64_t n_cols,
                              const float* grad_output, void* stream) {
  if (n_rows <= 0 || n_cols <= 0) return FORGE_OK;
  hipStream_t s = (hipStream_t)stream;
  switch (dtype) {
    case FORGE_DTYPE_F32: return launch_scale<float>(x, ld, n_rows, n_cols, grad_output, s);
    case FORGE_DTYPE_BF16: return launch_scale<bf16_t>(x, ld, n_rows, n_cols, grad_output, s);
    case FORGE_DTYPE_F16: return launch_scale<fp16_t>(x, ld, n_rows, n_cols, grad_output, s);
    default: return forge_set_error(FORGE_ERR_UNSUPPORTED, "ce_scale: dtype %d", dtype);
  }
}

extern "C" int forge_sum_f32(const float* x, int64_t n, float* out, void* stream) {
  if (n < 0) return forge_set_error(FORGE_ERR_INVALID, "sum_f32: negative length");
  sum_f32_kernel<<<1, 1024, 0, (hipStream_t)stream>>>(x, n, out);
  FORGE_CHECK_LAUNCH();
  return FORGE_OK;
}
