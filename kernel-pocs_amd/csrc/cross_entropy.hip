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
//   * ce_resident_kernel: the whole row is held on chip (LDS + registers of
//     one 512-thread workgroup, two rows per CU), so the logits are read from
//     HBM once and written once.  Pass A finds the exact row max, pass B sums
//     exp(x - m) and keeps p = exp(x - m) as fp16 in place of the input, pass
//     C writes p/d.  Used for the common case (2-byte logits, no class
//     weights / softcap / argmax) when the row fits in 512 * 32 * 8 elements.
//   * ce_stream_kernel: any row length and every feature; the row is streamed
//     twice (online max/sum, then gradient), the second read largely served by
//     the L2 / Infinity Cache.
// exp is evaluated as exp2 on log2e-prescaled values (one FMA + v_exp_f32).
#include <atomic>
#include <mutex>
#include <sched.h>
#include <string.h>
#include <time.h>

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
  const int64_t* stats;  // optional device [n_valid, min, max, in_range] from forge_ce_target_stats
  // In-launch statistics and loss reduction (forge_ce_fwd_reduce); word ==
  // nullptr for forge_ce_fwd.
  struct {
    uint64_t* word;    // device: [epoch:32 | in_range:1 | n_valid:31]
    uint64_t* stage;   // device [n_rows][2]: (epoch << 32 | loss bits), (epoch << 32 | z-loss bits)
    int64_t* host;     // pinned host slot, device-visible: ticket, n_valid, min, max, in_range
    uint64_t ticket;   // epoch = low 32 bits
    float* loss_sum;   // nullptr: per-row losses only
    float* z_sum;
    void* loss_cast;
    void* z_cast;
    int cast_dtype;
  } il;
};

// Row preamble shared by both engines.  With device-side target stats the
// non-ignored count comes from them (no host round trip), and a launch whose
// targets failed the range check touches nothing: the host raises the
// reference's AssertionError once it reads the same stats.  A row whose own
// target is out of range is left untouched too (a direct C-ABI caller that
// skipped the check must not make the kernel read outside the row).
// Returns false when the row must be skipped.
__device__ __forceinline__ bool ce_prologue(CeArgs& a, int64_t y) {
  if (a.stats) {
    if (a.stats[3] == 0) return false;
    a.n_non_ignore = (float)a.stats[0];
    if (!(a.flags & FORGE_CE_HAS_WEIGHT)) a.sum_non_ignore_weight = a.n_non_ignore;
  }
  return y == a.ignore_index || (y >= 0 && y < a.n_cols);
}

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

// n_valid and min / max of target * (target != ignore) over n targets
// (ignored rows count as 0, as the reference's masked max / min do,
// cross_entropy_kernel_v2.py:374-387), by one workgroup of NT threads; every
// thread gets the result.  Thread i takes i, i + NT, ... with kBatch loads in
// flight (one memory latency per NT * kBatch targets).
constexpr int kBatch = 8;

template <int NT>
__device__ void block_target_stats(const int64_t* t, int64_t stride, int64_t n, int64_t ignore, int64_t& cnt,
                                   int64_t& mn, int64_t& mx) {
  constexpr int NW = NT / 64;
  __shared__ int64_t red[3][NW];
  cnt = 0;
  mn = INT64_MAX;
  mx = INT64_MIN;
  for (int64_t i0 = threadIdx.x; i0 < n; i0 += (int64_t)NT * kBatch) {
    int64_t v[kBatch];
#pragma unroll
    for (int k = 0; k < kBatch; ++k) v[k] = i0 + k * NT < n ? t[(i0 + k * NT) * stride] : ignore;
#pragma unroll
    for (int k = 0; k < kBatch; ++k) {
      const bool valid = v[k] != ignore;
      const int64_t m = valid ? v[k] : 0;
      cnt += valid;
      if (i0 + k * NT < n) {  // a row past the end counts as nothing, not as an ignored 0
        mn = m < mn ? m : mn;
        mx = m > mx ? m : mx;
      }
    }
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    cnt += __shfl_xor(cnt, off, 64);
    const int64_t a = __shfl_xor(mn, off, 64), b = __shfl_xor(mx, off, 64);
    mn = a < mn ? a : mn;
    mx = b > mx ? b : mx;
  }
  const int w = threadIdx.x >> 6;
  __syncthreads();  // red may still be read by an earlier call
  if ((threadIdx.x & 63) == 0) { red[0][w] = cnt; red[1][w] = mn; red[2][w] = mx; }
  __syncthreads();
  cnt = red[0][0];
  mn = red[1][0];
  mx = red[2][0];
#pragma unroll
  for (int i = 1; i < NW; ++i) {
    cnt += red[0][i];
    mn = red[1][i] < mn ? red[1][i] : mn;
    mx = red[2][i] > mx ? red[2][i] : mx;
  }
}

// ---- in-launch statistics and loss reduction (forge_ce_fwd_reduce) ----
// The reference reads the target count and range on the host before its
// launch and sums the row losses with torch.sum after it
// (cross_entropy_kernel_v2.py:374-387, 451).  Here both happen inside the
// row kernel's one launch:
//   * workgroup 0 computes the statistics first thing and publishes them to a
//     device word (epoch-tagged, so a word left by an earlier launch never
//     matches) and to the caller's pinned host slot;
//   * a workgroup that needs them (before its first write) reads the word,
//     and if workgroup 0 has not stored it yet computes the same values
//     itself: no workgroup ever waits for another;
//   * each row stages its loss in a per-call array as one 64-bit atomic
//     store of (epoch, value); the last row's workgroup sums the staged
//     values in a fixed order once each carries the call's epoch.
// No fences and no returning atomics: an agent-scope fence writes back the
// whole L2 and costs about 55 ns per workgroup here (450 us over 8192 rows),
// and a per-row atomic whose result the workgroup waited for cost 27-40 us
// over the launch.
__device__ __forceinline__ uint64_t il_pack(uint32_t epoch, bool ok, int64_t cnt) {
  return ((uint64_t)epoch << 32) | (ok ? 0x80000000ull : 0ull) | (uint64_t)(cnt & 0x7fffffff);
}

// n_valid if every non-ignored target is in [0, n_cols) (the statistics'
// in_range), else -n_valid - 1; every thread gets the result.
template <int NT>
__device__ int block_count_in_range(const CeArgs& a) {
  constexpr int NW = NT / 64;
  __shared__ int red[2][NW];
  int c = 0, bad = 0;
  for (int i = threadIdx.x; i < (int)a.n_rows; i += NT) {
    const int64_t v = a.target[(int64_t)i * a.target_stride];
    const bool valid = v != a.ignore_index;
    c += valid;
    bad |= valid && (v < 0 || v >= a.n_cols);
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    c += __shfl_xor(c, off, 64);
    bad |= __shfl_xor(bad, off, 64);
  }
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) { red[0][w] = c; red[1][w] = bad; }
  __syncthreads();
  c = 0;
  bad = 0;
#pragma unroll
  for (int i = 0; i < NW; ++i) { c += red[0][i]; bad |= red[1][i]; }
  return bad ? -c - 1 : c;
}

template <int NT>
__device__ void il_publish(const CeArgs& a) {
  int64_t cnt, mn, mx;
  block_target_stats<NT>(a.target, a.target_stride, a.n_rows, a.ignore_index, cnt, mn, mx);
  if (threadIdx.x == 0) {
    const bool ok = mn >= 0 && mx < a.n_cols;
    __hip_atomic_store(a.il.word, il_pack((uint32_t)a.il.ticket, ok, cnt), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
    int64_t* h = a.il.host;
    __hip_atomic_store(h + 1, cnt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    __hip_atomic_store(h + 2, mn, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    __hip_atomic_store(h + 3, mx, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    __hip_atomic_store(h + 4, (int64_t)ok, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    // the ticket last, with release order: a host that reads it reads the rest
    __hip_atomic_store(h, (int64_t)a.il.ticket, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
  }
}

// Sets n_non_ignore (and sum_non_ignore_weight, no class weights here) from
// the statistics and returns in_range.  Called by every thread of the
// workgroup (the result is workgroup-uniform).
template <int NT>
__device__ bool il_stats(CeArgs& a) {
  __shared__ uint64_t s_word;
  if (threadIdx.x == 0) s_word = __hip_atomic_load(a.il.word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __syncthreads();
  uint64_t w = s_word;
  const uint32_t epoch = (uint32_t)a.il.ticket;
  if ((uint32_t)(w >> 32) != epoch) {
    // rare (workgroup 0 has not published yet): count and range only, one
    // load in flight, so a caller holding its row in registers does not spill
    const int cnt = block_count_in_range<NT>(a);
    w = il_pack(epoch, cnt >= 0, cnt >= 0 ? cnt : -cnt - 1);
    if (threadIdx.x == 0) __hip_atomic_store(a.il.word, w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  a.n_non_ignore = (float)(int64_t)(w & 0x7fffffffull);
  a.sum_non_ignore_weight = a.n_non_ignore;
  return (w >> 31) & 1;
}

__device__ __forceinline__ void store_cast(void* p, int dtype, float v) {
  if (dtype == FORGE_DTYPE_BF16) *(bf16_t*)p = (bf16_t)v;
  else if (dtype == FORGE_DTYPE_F16) *(fp16_t*)p = (fp16_t)v;
  else *(float*)p = v;
}

// Thread 0, once per row: the row's loss (and z-loss) in the call's staging
// array, each with the call's epoch in the same 64-bit atomic store (so a
// reader that sees the epoch sees the value; nothing waits for the store).
__device__ __forceinline__ void il_row_store(const CeArgs& a, int64_t row, float loss, float z) {
  const uint64_t tag = (uint64_t)(uint32_t)a.il.ticket << 32;
  __hip_atomic_store(a.il.stage + 2 * row, tag | __float_as_uint(loss), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (a.flags & FORGE_CE_RETURN_Z_LOSS)
    __hip_atomic_store(a.il.stage + 2 * row + 1, tag | __float_as_uint(z), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}

// Staged value k of `row` once it carries this call's epoch (bounded wait:
// about 4 s, then NaN).
__device__ __forceinline__ float il_wait_value(const CeArgs& a, int64_t row, int k) {
  const uint32_t epoch = (uint32_t)a.il.ticket;
  for (int it = 0; it < (1 << 20); ++it) {
    const uint64_t w = __hip_atomic_load(a.il.stage + 2 * row + k, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if ((uint32_t)(w >> 32) == epoch) return __uint_as_float((uint32_t)w);
    __builtin_amdgcn_s_sleep(127);
  }
  return __builtin_nanf("");
}

// Sum of staged value k over all rows: thread i adds rows i, i + NT, ... in
// order (kBatch loads in flight), then the workgroup tree: a fixed order.
template <int NW>
__device__ float il_sum(const CeArgs& a, int k, float* red) {
  constexpr int NT = NW * 64;
  const uint32_t epoch = (uint32_t)a.il.ticket;
  float s = 0.f;
  for (int64_t i0 = threadIdx.x; i0 < a.n_rows; i0 += (int64_t)NT * kBatch) {
    uint64_t w[kBatch];
#pragma unroll
    for (int j = 0; j < kBatch; ++j)
      w[j] = i0 + j * NT < a.n_rows
                 ? __hip_atomic_load(a.il.stage + 2 * (i0 + j * NT) + k, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                 : 0;
#pragma unroll
    for (int j = 0; j < kBatch; ++j) {
      if (i0 + j * NT >= a.n_rows) continue;
      s += (uint32_t)(w[j] >> 32) == epoch ? __uint_as_float((uint32_t)w[j]) : il_wait_value(a, i0 + j * NT, k);
    }
  }
  return block_sum<NW>(s, red);
}

// Every thread, at the end of the workgroup.  The last row's workgroup (the
// last one dispatched) sums loss (and z-loss) over all rows once every row's
// staged value carries this call's epoch; no other workgroup waits for
// anything, so the rows it waits for finish whichever order they run in.
template <int NW>
__device__ void il_last_sum(const CeArgs& a, int64_t row, float* red) {
  if (row != a.n_rows - 1) return;
  const bool z = a.flags & FORGE_CE_RETURN_Z_LOSS;
  const float s = il_sum<NW>(a, 0, red);
  const float zs = z ? il_sum<NW>(a, 1, red) : 0.f;
  if (threadIdx.x == 0) {
    *a.il.loss_sum = s;
    if (a.il.loss_cast) store_cast(a.il.loss_cast, a.il.cast_dtype, s);
    if (z) {
      if (a.il.z_sum) *a.il.z_sum = zs;
      if (a.il.z_cast) store_cast(a.il.z_cast, a.il.cast_dtype, zs);
    }
  }
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

// Thread 0: a row's outputs.  With the in-launch reduction the loss and
// z-loss are also staged (for every row, so the summing workgroup never waits
// for a row that writes nothing else).  ok == false (the launch's targets are
// out of range): nothing but the staged zeros is written.
__device__ __forceinline__ void store_row_outputs(const CeArgs& a, int64_t row, float loss, float z, float acc,
                                                      int64_t pred, bool ok) {
  if (a.il.loss_sum) il_row_store(a, row, ok ? loss : 0.f, ok ? z : 0.f);
  if (ok) {
    if (a.flags & FORGE_CE_RETURN_ACCURACY) a.acc[row] = acc;
    if (a.flags & FORGE_CE_RETURN_PREDICTED) a.pred[row] = pred;
    a.loss[row] = loss;
    if (a.flags & FORGE_CE_RETURN_Z_LOSS) a.z_loss[row] = z;
  }
}

// Loss bookkeeping shared by both engines (thread 0 only).
__device__ __forceinline__ void write_row_outputs(const CeArgs& a, int64_t row, int64_t y, float lse,
                                                      float xy, float wy, float scaled_x_sum, int64_t argmax,
                                                      bool ok = true) {
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
  store_row_outputs(a, row, loss, z, (argmax == y) ? 1.f : 0.f, argmax, ok);
}

__device__ __forceinline__ void write_ignored_outputs(const CeArgs& a, int64_t row, bool ok = true) {
  store_row_outputs(a, row, 0.f, 0.f, 0.f, -1, ok);
}

// Start of a row in either engine (all threads).  Handles the rows that do no
// softmax work (ignored targets; a target out of range) and returns true for
// them.  forge_ce_fwd: as ce_prologue.  forge_ce_fwd_reduce: workgroup 0
// publishes the statistics; an ignored row is zero-filled once they say the
// targets are in range; every such row is still counted for the reduction.
template <class T, int NT>
__device__ __forceinline__ bool ce_row_head(CeArgs& a, int64_t row, int64_t y, T* xr, bool vec, float* redf) {
  if (!a.il.word) {
    if (!ce_prologue(a, y)) return true;
    if (y != a.ignore_index) return false;
    zero_row<T>(xr, a.n_cols, vec);
    if (threadIdx.x == 0) write_ignored_outputs(a, row);
    return true;
  }
  if (row == 0) il_publish<NT>(a);
  if (y != a.ignore_index && y >= 0 && y < a.n_cols) return false;
  // ignored, or out of range (then in_range is 0 and only the count is written)
  const bool ok = il_stats<NT>(a) && y == a.ignore_index;
  if (threadIdx.x == 0) write_ignored_outputs(a, row, ok);
  if (ok) zero_row<T>(xr, a.n_cols, vec);
  if (a.il.loss_sum) il_last_sum<NT / 64>(a, row, redf);
  return true;
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
  if (ce_row_head<T, kStreamBlock>(a, row, y, xr, vec, redf)) return;

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
  const bool ok = a.il.word ? il_stats<kStreamBlock>(a) : true;
  if (threadIdx.x == 0) write_row_outputs(a, row, y, lse, xy, wy, sxs_tot, amax, ok);

  // ---- pass 2: gradient in place ----
  if (grads && ok) {
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
  if (a.il.loss_sum) il_last_sum<kStreamWaves>(a, row, redf);
}

// ---------------------------------------------------------------------------
// Resident engine (plain CE with optional label smoothing / z-loss)
//
// One 512-thread workgroup per row, two workgroups per CU.  The row is read
// from HBM once and written once: thread t owns the 16-byte vectors
// t + 512 i; vectors i < NL live in LDS (filled by LDS-DMA loads, no
// registers involved), vectors NL <= i < NL + NR in registers (up to 8 + 24
// vectors = 131072 bf16 values per row, within the 128-VGPR budget of 4
// waves per SIMD, with no spills).  With two rows per CU, one row's exp /
// reduction work overlaps the other row's memory traffic.  Every global
// access carries the nontemporal policy (the row is touched once): measured
// on MI355X at [8192, 128256] bf16, 811 -> 765 us.
//   pass A: row max via packed 16-bit integer max on the raw bf16/fp16 bits
//           (order-preserving for non-negative values; a row whose max is
//           negative takes a float max pass instead)
//   pass B: p = exp(x - m) in fp32, row sum, p kept as fp16 in place of x
//   pass C: dlogits = p * scale - shift (target column corrected), stored
// ---------------------------------------------------------------------------
constexpr int kResBlock = 512;
constexpr int kResWaves = kResBlock / 64;
constexpr int kResNL = 8;      // vectors per thread in LDS (64 KB per workgroup)
constexpr int kResNRMax = 24;  // vectors per thread in registers (96 VGPRs)
constexpr int kNT = 2;         // buffer-instruction cache policy: nontemporal

typedef __fp16 half2_t __attribute__((ext_vector_type(2)));
typedef short short2_t __attribute__((ext_vector_type(2)));
typedef int i32x4_t __attribute__((ext_vector_type(4)));

#define LDS_AS __attribute__((address_space(3)))

__device__ __forceinline__ __amdgpu_buffer_rsrc_t row_rsrc(const void* base, uint32_t bytes) {
  const uint64_t b = reinterpret_cast<uint64_t>(base);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)b);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(b >> 32));
  return __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>(((uint64_t)hi << 32) | lo), (short)0,
                                           (int)bytes, 0x00020000);
}

__device__ __forceinline__ short2_t as_s2(uint32_t w) { return __builtin_bit_cast(short2_t, w); }

template <class T, int NR>
__global__ __launch_bounds__(kResBlock) __attribute__((amdgpu_waves_per_eu(4, 4)))
void ce_resident_kernel(CeArgs a) {
  constexpr int VEC = 16 / sizeof(T);
  constexpr int NL = kResNL;
  constexpr int VSTRIDE = kResBlock * 16;  // bytes between a thread's vectors i and i+1
  __shared__ __attribute__((aligned(16))) uint4 lds_row[NL * kResBlock];
  __shared__ float redf[2 * kResWaves];
  const int64_t row = blockIdx.x;
  const int64_t y = a.target[row * a.target_stride];
  T* xr = (T*)a.x + row * a.ld;
  const int64_t V = a.n_cols;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  if (ce_row_head<T, kResBlock>(a, row, y, xr, true, redf)) return;
  const float xy = to_f32(xr[y]);
  const float ls = a.label_smoothing;
  // vector i of this thread is valid iff tid < lim(i) (lim is wave-uniform)
  const int nvec = (int)(V / VEC);
  auto valid = [&](int i) { return tid < nvec - i * kResBlock; };
  const uint32_t voff = (uint32_t)tid * 16u;

  // ---- loads: LDS part by DMA (1 KB per wave instruction, lane-ordered),
  //      register part by buffer loads ----
  const __amdgpu_buffer_rsrc_t rs = row_rsrc(xr, (uint32_t)(V * sizeof(T)));
#pragma unroll
  for (int i = 0; i < NL; ++i) {
    if (valid(i)) {
      LDS_AS void* dst = (LDS_AS void*)((LDS_AS char*)lds_row + (i * kResWaves + wave) * 1024);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, dst, 16, voff, i * VSTRIDE, 0, kNT);
    }
  }
  uint4 reg[NR];
#pragma unroll
  for (int i = 0; i < NR; ++i) {
    reg[i] = make_uint4(0, 0, 0, 0);
    if (valid(NL + i)) {
      i32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(rs, (int)voff, (NL + i) * VSTRIDE, kNT);
      reg[i] = make_uint4((uint32_t)v.x, (uint32_t)v.y, (uint32_t)v.z, (uint32_t)v.w);
    }
  }
  __builtin_amdgcn_s_waitcnt(0);  // our DMA writes have landed
  __syncthreads();                // ... and everyone else's
  uint4* my_lds = lds_row + tid;  // slot of vector i: my_lds[i * kResBlock]

  // ---- pass A: row max ----
  short2_t mi = {(short)0x8000, (short)0x8000};
  auto max_vec = [&](const uint4& v) {
    mi = __builtin_elementwise_max(mi, as_s2(v.x));
    mi = __builtin_elementwise_max(mi, as_s2(v.y));
    mi = __builtin_elementwise_max(mi, as_s2(v.z));
    mi = __builtin_elementwise_max(mi, as_s2(v.w));
  };
#pragma unroll 1
  for (int i = 0; i < NL; ++i)
    if (valid(i)) max_vec(my_lds[i * kResBlock]);
#pragma unroll
  for (int i = 0; i < NR; ++i)
    if (valid(NL + i)) max_vec(reg[i]);
  auto bits_to_f = [](short h) -> float {
    return __is_same(T, bf16_t) ? __uint_as_float(((uint32_t)(uint16_t)h) << 16)
                                : (float)__builtin_bit_cast(fp16_t, h);
  };
  const short hmax = mi.x > mi.y ? mi.x : mi.y;
  // int16 order matches float order for non-negative values (both types)
  float m = block_max<kResWaves>(hmax >= 0 ? bits_to_f(hmax) : -INFINITY, redf);
  if (m == -INFINITY) {  // every value negative (or -inf): float max pass
    float fm = -INFINITY;
    auto fmax_vec = [&](const uint4& v) {
      Vec16<T> t;
      t.raw = v;
#pragma unroll
      for (int j = 0; j < VEC; ++j) fm = fmaxf(fm, to_f32(t.v[j]));
    };
#pragma unroll 1
    for (int i = 0; i < NL; ++i)
      if (valid(i)) fmax_vec(my_lds[i * kResBlock]);
#pragma unroll
    for (int i = 0; i < NR; ++i)
      if (valid(NL + i)) fmax_vec(reg[i]);
    m = block_max<kResWaves>(fm, redf);
  }
  // p is kept as fp16 scaled by 2^kPShift (max 2^15 < 65504), which moves
  // fp16's flush-to-zero point from ~6e-8 down to ~2e-12 of the row max;
  // d carries the same factor, so p / d is unchanged
  constexpr float kPShift = 15.f;
  const float ml2 = m * kLog2e - kPShift;

  // ---- pass B: p = exp(x - m) * 2^kPShift, sum; p overwrites x as fp16 pairs ----
  float d = 0.f, sx = 0.f;
  auto exp_vec = [&](uint4& v) {
    Vec16<T> t;
    t.raw = v;
    uint32_t w[4];
#pragma unroll
    for (int j = 0; j < VEC; j += 2) {
      const float x0 = to_f32(t.v[j]), x1 = to_f32(t.v[j + 1]);
      if (ls > 0.f) sx += x0 + x1;
      const float p0 = fast_exp2(fmaf(x0, kLog2e, -ml2));
      const float p1 = fast_exp2(fmaf(x1, kLog2e, -ml2));
      d += p0 + p1;
      // round to nearest (not toward zero): the stored p carries no bias
      const half2_t ph = {(__fp16)p0, (__fp16)p1};
      w[j / 2] = __builtin_bit_cast(uint32_t, ph);
    }
    v = make_uint4(w[0], w[1], w[2], w[3]);
  };
#pragma unroll 1
  for (int i = 0; i < NL; ++i)
    if (valid(i)) {
      uint4 v = my_lds[i * kResBlock];
      exp_vec(v);
      my_lds[i * kResBlock] = v;
    }
#pragma unroll
  for (int i = 0; i < NR; ++i)
    if (valid(NL + i)) exp_vec(reg[i]);
  d = block_sum<kResWaves>(d, redf);
  float sx_tot = 0.f;
  if (ls > 0.f) sx_tot = block_sum<kResWaves>(sx, redf);
  const float lse = m + __logf(d) - kPShift * kLn2;
  const bool ok = a.il.word ? il_stats<kResBlock>(a) : true;
  if (tid == 0) write_row_outputs(a, row, y, lse, xy, 1.f, -(ls / (float)V) * sx_tot, 0, ok);

  // ---- pass C: gradient ----
  if ((a.flags & FORGE_CE_HAS_GRADIENTS) && ok) {
    const bool mean = a.flags & FORGE_CE_REDUCTION_MEAN;
    const float eps = ls / (float)V;
    float scale = (1.f + 2.f * a.lse_square_scale * lse) / d;
    float shift = eps;
    float ydelta = 1.f - ls;
    if (mean) {
      scale /= a.n_non_ignore;
      shift /= a.n_non_ignore;
      ydelta /= a.n_non_ignore;
    }
    const int yv = (int)(y / VEC);            // vector holding the target column
    const int yi = yv / kResBlock, yt = yv % kResBlock;  // (i, thread) of that vector
    auto grad_vec = [&](const uint4& v, int i) -> uint4 {
      const uint32_t w[4] = {v.x, v.y, v.z, v.w};
      Vec16<T> o;
#pragma unroll
      for (int j = 0; j < VEC; j += 2) {
        const half2_t ph = __builtin_bit_cast(half2_t, w[j / 2]);
        o.v[j] = from_f32<T>(fmaf((float)ph.x, scale, -shift));
        o.v[j + 1] = from_f32<T>(fmaf((float)ph.y, scale, -shift));
      }
      if (i == yi && tid == yt) {
        const float py = fast_exp2(fmaf(xy, kLog2e, -ml2));
        const T gy = from_f32<T>(fmaf(py, scale, -shift) - ydelta);
        const int yj = (int)(y % VEC);
#pragma unroll
        for (int j = 0; j < VEC; ++j)
          if (j == yj) o.v[j] = gy;  // static indices: no scratch array
      }
      return o.raw;
    };
    auto store = [&](const uint4& o, int i) {
      const i32x4_t ov = {(int)o.x, (int)o.y, (int)o.z, (int)o.w};
      __builtin_amdgcn_raw_buffer_store_b128(ov, rs, (int)voff, i * VSTRIDE, kNT);
    };
    // the register part first, in place, then every store
#pragma unroll
    for (int i = 0; i < NR; ++i)
      if (valid(NL + i)) reg[i] = grad_vec(reg[i], NL + i);
#pragma unroll 1
    for (int i = 0; i < NL; ++i)
      if (valid(i)) store(grad_vec(my_lds[i * kResBlock], i), i);
#pragma unroll
    for (int i = 0; i < NR; ++i)
      if (valid(NL + i)) store(reg[i], NL + i);
  }
  if (a.il.loss_sum) il_last_sum<kResWaves>(a, row, redf);
}

template <class T>
int launch_ce(CeArgs a, hipStream_t s) {
  constexpr int V = 16 / sizeof(T);
  const bool vec = aligned16(a.x) && (a.ld % V == 0) && (a.n_cols % V == 0);
  const bool plain = !(a.flags & (FORGE_CE_HAS_WEIGHT | FORGE_CE_HAS_SOFTCAP |
                                  FORGE_CE_RETURN_ACCURACY | FORGE_CE_RETURN_PREDICTED));
  // vectors per thread of the resident engine
  const int64_t nvec = (a.n_cols / V + kResBlock - 1) / kResBlock;
  dim3 grid((unsigned)a.n_rows);
  bool resident = false;
  if constexpr (sizeof(T) == 2) {  // 2-byte logits only: no fp32 instances
    if (vec && plain && nvec <= kResNL + kResNRMax && a.n_cols * (int64_t)sizeof(T) < 0x7fffffff) {
      resident = true;
      const int64_t nr = nvec > kResNL ? nvec - kResNL : 0;
      if (nr <= 8)
        ce_resident_kernel<T, 8><<<grid, kResBlock, 0, s>>>(a);
      else if (nr <= 16)
        ce_resident_kernel<T, 16><<<grid, kResBlock, 0, s>>>(a);
      else
        ce_resident_kernel<T, kResNRMax><<<grid, kResBlock, 0, s>>>(a);
    }
  }
  if (resident) {
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
                                                       const void* g, int g_dtype) {
  const float s = g_dtype == FORGE_DTYPE_BF16 ? (float)*(const bf16_t*)g
                  : g_dtype == FORGE_DTYPE_F16 ? (float)*(const fp16_t*)g
                                               : *(const float*)g;
  if (s == 1.0f) return;  // the reference skips grad_output == 1 (torch.equal), here without a host sync
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
int launch_scale(void* x, int64_t ld, int64_t rows, int64_t cols, const void* g, int g_dtype, hipStream_t s) {
  constexpr int V = 16 / sizeof(T);
  const bool vec = aligned16(x) && ld % V == 0 && cols % V == 0;
  // 8 workgroups per CU, grid-stride: full bandwidth when scaling, and a
  // cheap launch when grad_output == 1 makes every workgroup exit at once
  if (vec) {
    int grid = grid_for(rows * cols / V, 256, 2048);
    ce_scale_kernel<T, V><<<grid, 256, 0, s>>>((T*)x, ld, rows, cols, g, g_dtype);
  } else {
    int grid = grid_for(rows * cols, 256, 2048);
    ce_scale_kernel<T, 1><<<grid, 256, 0, s>>>((T*)x, ld, rows, cols, g, g_dtype);
  }
  FORGE_CHECK_LAUNCH();
  return FORGE_OK;
}

// Target statistics for forge_ce_fwd: n_valid, min / max of the masked
// targets and whether that range is inside [0, n_cols), by one workgroup
// (labels are a few thousand to a few million).
__global__ __launch_bounds__(1024) void ce_target_stats_kernel(const int64_t* t, int64_t stride, int64_t n,
                                                               int64_t ignore, int64_t n_cols, int64_t* out) {
  int64_t cnt, mn, mx;
  block_target_stats<1024>(t, stride, n, ignore, cnt, mn, mx);
  if (threadIdx.x == 0) {
    out[0] = cnt;
    out[1] = mn;
    out[2] = mx;
    out[3] = (mn >= 0 && mx < n_cols) ? 1 : 0;
  }
}

// Single-workgroup deterministic sum (the vector is one value per row):
// thread i adds i, i + 1024, ... in order, kBatch loads in flight.
__global__ __launch_bounds__(1024) void sum_f32_kernel(const float* x, int64_t n, float* out, void* out_cast,
                                                       int cast_dtype) {
  __shared__ float red[16];
  float acc = 0.f;
  for (int64_t i0 = threadIdx.x; i0 < n; i0 += 1024 * kBatch) {
    float v[kBatch];
#pragma unroll
    for (int k = 0; k < kBatch; ++k) v[k] = i0 + k * 1024 < n ? x[i0 + k * 1024] : 0.f;
#pragma unroll
    for (int k = 0; k < kBatch; ++k)
      if (i0 + k * 1024 < n) acc += v[k];
  }
  acc = block_sum<16>(acc, red);
  if (threadIdx.x == 0) {
    out[0] = acc;
    if (out_cast) {
      if (cast_dtype == FORGE_DTYPE_BF16) *(bf16_t*)out_cast = (bf16_t)acc;
      else if (cast_dtype == FORGE_DTYPE_F16) *(fp16_t*)out_cast = (fp16_t)acc;
      else *(float*)out_cast = acc;
    }
  }
}

// Token scaling of the fused linear + cross-entropy path: the probability of
// the target class under softmax(softcap(x)) of each row, detached from the
// graph.  The softcapped logits are rounded to the logits dtype and p is
// rounded to it too, as the reference builds both as tensors of that dtype;
// ignored rows get 0.  One 256-thread workgroup per row.
template <class T>
__global__ __launch_bounds__(256) void ce_target_prob_kernel(const T* x, int64_t ld, int64_t V, const int64_t* target,
                                                             int64_t tstride, int64_t ignore_index, float softcap,
                                                             float* prob) {
  __shared__ float red[8];
  const int64_t row = blockIdx.x;
  const int64_t y = target[row * tstride];
  if (y == ignore_index || y < 0 || y >= V) {
    if (threadIdx.x == 0) prob[row] = 0.f;
    return;
  }
  const T* xr = x + row * ld;
  auto capped = [&](float v) { return softcap > 0.f ? round_to<T>(softcap * tanhf(v / softcap)) : v; };
  float m = -INFINITY, d = 0.f;
  for (int64_t c = threadIdx.x; c < V; c += 256) {
    const float v = capped(to_f32(xr[c])) * kLog2e;
    if (v > m) {
      d = (m == -INFINITY) ? 0.f : d * fast_exp2(m - v);
      m = v;
    }
    d += fast_exp2(v - m);
  }
  block_lse<4>(m, d, red);
  if (threadIdx.x == 0) prob[row] = round_to<T>(fast_exp2(capped(to_f32(xr[y])) * kLog2e - m) / d);
}

// x[r, c] *= s[r], rounded to x's dtype (the per-row token scale).
template <class T>
__global__ __launch_bounds__(256) void row_scale_kernel(T* x, int64_t ld, int64_t rows, int64_t cols, const float* s) {
  const int64_t n = rows * cols;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    const int64_t r = i / cols, c = i - r * cols;
    T* p = x + r * ld + c;
    *p = from_f32<T>(to_f32(*p) * s[r]);
  }
}

}  // namespace

extern "C" int forge_ce_fwd(int dtype, void* logits, int64_t ld, int64_t n_rows, int64_t n_cols,
                            const int64_t* target, int64_t target_stride, const float* weight,
                            float* loss, float* z_loss, float* token_accuracy,
                            int64_t* predicted_tokens, int64_t ignore_index, float n_non_ignore,
                            float sum_non_ignore_weight, float weight_sum, float lse_square_scale,
                            float label_smoothing, float softcap, int flags, const int64_t* stats,
                            void* stream) {
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
  a.stats = stats;
  a.il = {};
  hipStream_t s = (hipStream_t)stream;
  switch (dtype) {
    case FORGE_DTYPE_F32: return launch_ce<float>(a, s);
    case FORGE_DTYPE_BF16: return launch_ce<bf16_t>(a, s);
    case FORGE_DTYPE_F16: return launch_ce<fp16_t>(a, s);
    default: return forge_set_error(FORGE_ERR_UNSUPPORTED, "ce_fwd: dtype %d", dtype);
  }
}

// ---------------------------------------------------------------------------
// forge_ce_fwd_reduce: per device, kIlSlots slots, one per call in turn (call
// t uses slot t % kIlSlots): a 64-byte device slot (statistics word), a
// 64-byte pinned host slot (ticket, n_valid, min, max, in_range) and, for
// calls that reduce, a staging array of 16 bytes per row (grown when a call
// has more rows than it holds).  Allocated on first use and kept until the
// process ends.  Everything a launch writes there is tagged with its call's
// epoch (the ticket's low 32 bits), so nothing needs clearing between calls.
// ---------------------------------------------------------------------------
namespace {

constexpr int kIlSlots = 64;
constexpr int kIlMaxDevices = 64;
constexpr int kIlSlotBytes = 64;

struct IlDevice {
  char* dev = nullptr;       // kIlSlots device slots
  int64_t* host = nullptr;   // kIlSlots host slots (8 int64 each)
  int64_t* host_dev = nullptr;
  uint64_t* stage[kIlSlots] = {};
  int64_t stage_rows[kIlSlots] = {};
  std::atomic<uint64_t> next{0};
};
IlDevice g_il[kIlMaxDevices];
std::mutex g_il_mu;

int il_device_of(hipStream_t s, int* dev_out) {
  int dev = -1;
  const hipError_t e = hipStreamGetDevice(s, &dev);
  if (e != hipSuccess || dev < 0 || dev >= kIlMaxDevices)
    return forge_set_error(FORGE_ERR_HIP, "ce_fwd_reduce: stream device: %s", hipGetErrorString(e));
  *dev_out = dev;
  return FORGE_OK;
}

int il_init(int dev) {
  std::lock_guard<std::mutex> lock(g_il_mu);
  IlDevice& d = g_il[dev];
  if (d.dev) return FORGE_OK;
  int prev = 0;
  if (hipGetDevice(&prev) != hipSuccess) return forge_set_error(FORGE_ERR_HIP, "ce_fwd_reduce: hipGetDevice");
  if (hipSetDevice(dev) != hipSuccess) return forge_set_error(FORGE_ERR_HIP, "ce_fwd_reduce: hipSetDevice(%d)", dev);
  void *dp = nullptr, *hp = nullptr, *hdp = nullptr;
  hipError_t e = hipMalloc(&dp, kIlSlots * kIlSlotBytes);
  if (e == hipSuccess) e = hipMemset(dp, 0, kIlSlots * kIlSlotBytes);
  if (e == hipSuccess) e = hipHostMalloc(&hp, kIlSlots * kIlSlotBytes, hipHostMallocMapped | hipHostMallocCoherent);
  if (e == hipSuccess) {
    memset(hp, 0, kIlSlots * kIlSlotBytes);
    e = hipHostGetDevicePointer(&hdp, hp, 0);
  }
  (void)hipSetDevice(prev);
  if (e != hipSuccess) {
    if (dp) (void)hipFree(dp);
    if (hp) (void)hipHostFree(hp);
    return forge_set_error(FORGE_ERR_HIP, "ce_fwd_reduce: slot allocation on device %d: %s", dev, hipGetErrorString(e));
  }
  d.host = static_cast<int64_t*>(hp);
  d.host_dev = static_cast<int64_t*>(hdp);
  d.dev = static_cast<char*>(dp);  // last: a non-null dev marks the device ready
  return FORGE_OK;
}

}  // namespace

extern "C" int forge_ce_fwd_reduce(int dtype, void* logits, int64_t ld, int64_t n_rows, int64_t n_cols,
                                   const int64_t* target, int64_t target_stride, float* loss, float* z_loss,
                                   float* token_accuracy, int64_t* predicted_tokens, int64_t ignore_index,
                                   float lse_square_scale, float label_smoothing, float softcap, int flags,
                                   float* loss_sum, float* z_sum, void* loss_cast, void* z_cast, int cast_dtype,
                                   uint64_t* ticket, void* stream) {
  if (n_rows <= 0 || n_cols <= 0) return forge_set_error(FORGE_ERR_INVALID, "ce_fwd_reduce: empty shape");
  if (n_rows > 0x7fffffff) return forge_set_error(FORGE_ERR_INVALID, "ce_fwd_reduce: too many rows");
  if (ld < n_cols) return forge_set_error(FORGE_ERR_INVALID, "ce_fwd_reduce: ld < n_cols");
  if (!logits || !target || !loss || !ticket) return forge_set_error(FORGE_ERR_INVALID, "ce_fwd_reduce: null pointer");
  if (flags & FORGE_CE_HAS_WEIGHT)
    return forge_set_error(FORGE_ERR_INVALID, "ce_fwd_reduce: class weights need host-side sums (use forge_ce_fwd)");
  if ((flags & FORGE_CE_RETURN_Z_LOSS) && !z_loss)
    return forge_set_error(FORGE_ERR_INVALID, "ce_fwd_reduce: z_loss buffer required");
  if ((flags & FORGE_CE_RETURN_ACCURACY) && !token_accuracy)
    return forge_set_error(FORGE_ERR_INVALID, "ce_fwd_reduce: accuracy buffer required");
  if ((flags & FORGE_CE_RETURN_PREDICTED) && !predicted_tokens)
    return forge_set_error(FORGE_ERR_INVALID, "ce_fwd_reduce: predicted buffer required");
  if ((loss_cast || z_cast) && cast_dtype != FORGE_DTYPE_F32 && cast_dtype != FORGE_DTYPE_BF16 &&
      cast_dtype != FORGE_DTYPE_F16)
    return forge_set_error(FORGE_ERR_UNSUPPORTED, "ce_fwd_reduce: cast dtype %d", cast_dtype);
  hipStream_t s = (hipStream_t)stream;
  int dev = 0;
  if (int rc = il_device_of(s, &dev)) return rc;
  if (int rc = il_init(dev)) return rc;
  IlDevice& d = g_il[dev];
  uint64_t t = d.next.fetch_add(1) + 1;
  if ((uint32_t)t == 0) t = d.next.fetch_add(1) + 1;  // epoch 0 is a fresh slot's word
  const int slot = (int)(t % kIlSlots);
  CeArgs a;
  a.x = logits; a.ld = ld; a.n_rows = n_rows; a.n_cols = n_cols;
  a.target = target; a.target_stride = target_stride; a.weight = nullptr;
  a.loss = loss; a.z_loss = z_loss; a.acc = token_accuracy; a.pred = predicted_tokens;
  a.ignore_index = ignore_index; a.n_non_ignore = 0.f;
  a.sum_non_ignore_weight = 0.f; a.weight_sum = 0.f;
  a.lse_square_scale = lse_square_scale; a.label_smoothing = label_smoothing; a.softcap = softcap;
  a.flags = flags;
  a.stats = nullptr;
  char* ds = d.dev + slot * kIlSlotBytes;
  a.il.word = reinterpret_cast<uint64_t*>(ds);
  a.il.stage = nullptr;
  if (loss_sum) {
    std::lock_guard<std::mutex> lock(g_il_mu);
    if (d.stage_rows[slot] < n_rows) {
      // the slot's previous staging array (if any) was last used 64 calls
      // ago; hipFree waits for the device before releasing it
      int prev = 0;
      (void)hipGetDevice(&prev);
      (void)hipSetDevice(dev);
      if (d.stage[slot]) (void)hipFree(d.stage[slot]);
      d.stage[slot] = nullptr;
      d.stage_rows[slot] = 0;
      void* p = nullptr;
      hipError_t e = hipMalloc(&p, (size_t)n_rows * 16);
      if (e == hipSuccess) e = hipMemset(p, 0, (size_t)n_rows * 16);  // epoch 0: never a call's
      (void)hipSetDevice(prev);
      if (e != hipSuccess)
        return forge_set_error(FORGE_ERR_HIP, "ce_fwd_reduce: staging array of %lld rows: %s", (long long)n_rows,
                               hipGetErrorString(e));
      d.stage[slot] = static_cast<uint64_t*>(p);
      d.stage_rows[slot] = n_rows;
    }
    a.il.stage = d.stage[slot];
  }
  a.il.host = d.host_dev + slot * (kIlSlotBytes / 8);
  a.il.ticket = t;
  a.il.loss_sum = loss_sum;
  a.il.z_sum = z_sum;
  a.il.loss_cast = loss_cast;
  a.il.z_cast = z_cast;
  a.il.cast_dtype = cast_dtype;
  if (!loss_sum && (z_sum || loss_cast || z_cast))
    return forge_set_error(FORGE_ERR_INVALID, "ce_fwd_reduce: reduced outputs need loss_sum");
  int rc;
  switch (dtype) {
    case FORGE_DTYPE_F32: rc = launch_ce<float>(a, s); break;
    case FORGE_DTYPE_BF16: rc = launch_ce<bf16_t>(a, s); break;
    case FORGE_DTYPE_F16: rc = launch_ce<fp16_t>(a, s); break;
    default: return forge_set_error(FORGE_ERR_UNSUPPORTED, "ce_fwd_reduce: dtype %d", dtype);
  }
  if (rc == FORGE_OK) *ticket = t;
  return rc;
}

extern "C" int forge_ce_stats_wait(uint64_t ticket, int64_t* stats, void* stream) {
  if (!stats || ticket == 0) return forge_set_error(FORGE_ERR_INVALID, "ce_stats_wait: bad arguments");
  hipStream_t s = (hipStream_t)stream;
  int dev = 0;
  if (int rc = il_device_of(s, &dev)) return rc;
  IlDevice& d = g_il[dev];
  if (!d.host) return forge_set_error(FORGE_ERR_INVALID, "ce_stats_wait: no forge_ce_fwd_reduce call on this device");
  int64_t* h = d.host + (ticket % kIlSlots) * (kIlSlotBytes / 8);
  // spin briefly, then poll with short sleeps; a stream that has finished all
  // its work without the ticket appearing means the launch never wrote it
  for (long it = 0;; ++it) {
    const int64_t tag = __atomic_load_n(h, __ATOMIC_ACQUIRE);
    if ((uint64_t)tag == ticket) break;
    if ((uint64_t)tag > ticket)
      return forge_set_error(FORGE_ERR_INVALID, "ce_stats_wait: slot reused by a later call (more than %d calls in flight)",
                             kIlSlots);
    if (it < 2000) {
      sched_yield();
      continue;
    }
    if (it % 64 == 0 && hipStreamQuery(s) == hipSuccess &&
        (uint64_t)__atomic_load_n(h, __ATOMIC_ACQUIRE) != ticket)
      return forge_set_error(FORGE_ERR_HIP, "ce_stats_wait: the launch of ticket %llu wrote no statistics",
                             (unsigned long long)ticket);
    const timespec ts{0, 20000};
    nanosleep(&ts, nullptr);
  }
  for (int i = 0; i < 4; ++i) stats[i] = __atomic_load_n(h + 1 + i, __ATOMIC_RELAXED);
  return FORGE_OK;
}

extern "C" int forge_ce_scale(int dtype, void* x, int64_t ld, int64_t n_rows, int64_t n_cols,
                              const void* grad_output, int grad_dtype, void* stream) {
  if (n_rows <= 0 || n_cols <= 0) return FORGE_OK;
  if (grad_dtype != FORGE_DTYPE_F32 && grad_dtype != FORGE_DTYPE_BF16 && grad_dtype != FORGE_DTYPE_F16)
    return forge_set_error(FORGE_ERR_UNSUPPORTED, "ce_scale: grad_output dtype %d", grad_dtype);
  hipStream_t s = (hipStream_t)stream;
  switch (dtype) {
    case FORGE_DTYPE_F32: return launch_scale<float>(x, ld, n_rows, n_cols, grad_output, grad_dtype, s);
    case FORGE_DTYPE_BF16: return launch_scale<bf16_t>(x, ld, n_rows, n_cols, grad_output, grad_dtype, s);
    case FORGE_DTYPE_F16: return launch_scale<fp16_t>(x, ld, n_rows, n_cols, grad_output, grad_dtype, s);
    default: return forge_set_error(FORGE_ERR_UNSUPPORTED, "ce_scale: dtype %d", dtype);
  }
}

extern "C" int forge_ce_target_stats(const int64_t* target, int64_t target_stride, int64_t n_rows,
                                     int64_t ignore_index, int64_t n_cols, int64_t* stats, void* stream) {
  if (n_rows <= 0) return forge_set_error(FORGE_ERR_INVALID, "ce_target_stats: n_rows must be positive");
  if (!target || !stats) return forge_set_error(FORGE_ERR_INVALID, "ce_target_stats: null pointer");
  ce_target_stats_kernel<<<1, 1024, 0, (hipStream_t)stream>>>(target, target_stride, n_rows, ignore_index, n_cols,
                                                              stats);
  FORGE_CHECK_LAUNCH();
  return FORGE_OK;
}

extern "C" int forge_sum_f32(const float* x, int64_t n, float* out, void* out_cast, int cast_dtype, void* stream) {
  if (n < 0) return forge_set_error(FORGE_ERR_INVALID, "sum_f32: negative length");
  if (out_cast && cast_dtype != FORGE_DTYPE_F32 && cast_dtype != FORGE_DTYPE_BF16 && cast_dtype != FORGE_DTYPE_F16)
    return forge_set_error(FORGE_ERR_UNSUPPORTED, "sum_f32: cast dtype %d", cast_dtype);
  sum_f32_kernel<<<1, 1024, 0, (hipStream_t)stream>>>(x, n, out, out_cast, cast_dtype);
  FORGE_CHECK_LAUNCH();
  return FORGE_OK;
}

extern "C" int forge_ce_target_prob(int dtype, const void* logits, int64_t ld, int64_t n_rows, int64_t n_cols,
                                    const int64_t* target, int64_t target_stride, int64_t ignore_index, float softcap,
                                    float* prob, void* stream) {
  if (n_rows < 0 || n_cols <= 0) return forge_set_error(FORGE_ERR_INVALID, "ce_target_prob: shape");
  if (n_rows == 0) return FORGE_OK;
  if (n_rows > 0x7fffffff) return forge_set_error(FORGE_ERR_INVALID, "ce_target_prob: too many rows");
  if (!logits || !target || !prob) return forge_set_error(FORGE_ERR_INVALID, "ce_target_prob: null pointer");
  hipStream_t s = (hipStream_t)stream;
  const dim3 grid((unsigned)n_rows);
  switch (dtype) {
    case FORGE_DTYPE_F32:
      ce_target_prob_kernel<float><<<grid, 256, 0, s>>>((const float*)logits, ld, n_cols, target, target_stride,
                                                        ignore_index, softcap, prob);
      break;
    case FORGE_DTYPE_BF16:
      ce_target_prob_kernel<bf16_t><<<grid, 256, 0, s>>>((const bf16_t*)logits, ld, n_cols, target, target_stride,
                                                         ignore_index, softcap, prob);
      break;
    case FORGE_DTYPE_F16:
      ce_target_prob_kernel<fp16_t><<<grid, 256, 0, s>>>((const fp16_t*)logits, ld, n_cols, target, target_stride,
                                                         ignore_index, softcap, prob);
      break;
    default: return forge_set_error(FORGE_ERR_UNSUPPORTED, "ce_target_prob: dtype %d", dtype);
  }
  FORGE_CHECK_LAUNCH();
  return FORGE_OK;
}

extern "C" int forge_row_scale(int dtype, void* x, int64_t ld, int64_t n_rows, int64_t n_cols, const float* scale,
                               void* stream) {
  if (n_rows < 0 || n_cols < 0) return forge_set_error(FORGE_ERR_INVALID, "row_scale: shape");
  if (n_rows == 0 || n_cols == 0) return FORGE_OK;
  if (!x || !scale) return forge_set_error(FORGE_ERR_INVALID, "row_scale: null pointer");
  hipStream_t s = (hipStream_t)stream;
  const int grid = grid_for(n_rows * n_cols, 256, 4096);
  switch (dtype) {
    case FORGE_DTYPE_F32: row_scale_kernel<float><<<grid, 256, 0, s>>>((float*)x, ld, n_rows, n_cols, scale); break;
    case FORGE_DTYPE_BF16: row_scale_kernel<bf16_t><<<grid, 256, 0, s>>>((bf16_t*)x, ld, n_rows, n_cols, scale); break;
    case FORGE_DTYPE_F16: row_scale_kernel<fp16_t><<<grid, 256, 0, s>>>((fp16_t*)x, ld, n_rows, n_cols, scale); break;
    default: return forge_set_error(FORGE_ERR_UNSUPPORTED, "row_scale: dtype %d", dtype);
  }
  FORGE_CHECK_LAUNCH();
  return FORGE_OK;
}
