// Small utility kernels: the deterministic reduction of per-split fp32
// partial sums, zero fill of an fp32 workspace (a kernel, not
// hipMemsetAsync, so the sequence stays valid under stream capture), the
// fp32 -> bf16 cast, and a 2-byte transpose (K-contiguous operands for the
// LDS-DMA GEMM).
#include "common.h"

namespace {

__global__ __launch_bounds__(256) void zero_kernel(uint4* p, int64_t n16, uint8_t* tail, int64_t ntail) {
  const int64_t stride = (int64_t)gridDim.x * 256;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n16; i += stride) p[i] = make_uint4(0, 0, 0, 0);
  if (blockIdx.x == 0 && threadIdx.x < ntail) tail[threadIdx.x] = 0;
}

// Plain device copy: 16-byte nontemporal loads and stores, VPT vectors in
// flight per thread (the access pattern of this library's streaming kernels);
// the last bytes % 16 bytes are copied by workgroup 0.  Measured sustained on
// MI355X (rotating buffers): one vector per thread streams 6.3-6.4 TB/s for
// copies of 0.3-0.5 GB, two 6.2; at 2 GB two vectors are best (6.2 against
// 6.0).
template <int VPT>
__global__ __launch_bounds__(256) void copy_kernel(const uint4* src, uint4* dst, int64_t n16, const uint8_t* src_tail,
                                                   uint8_t* dst_tail, int64_t ntail) {
  const int64_t stride = (int64_t)gridDim.x * 256 * VPT;
  for (int64_t i = (int64_t)blockIdx.x * 256 * VPT + threadIdx.x; i < n16; i += stride) {
    u32x4_t v[VPT];
#pragma unroll
    for (int j = 0; j < VPT; ++j)
      if (i + j * 256 < n16) v[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(src + i + j * 256));
#pragma unroll
    for (int j = 0; j < VPT; ++j)
      if (i + j * 256 < n16) __builtin_nontemporal_store(v[j], reinterpret_cast<u32x4_t*>(dst + i + j * 256));
  }
  if (blockIdx.x == 0 && threadIdx.x < ntail) dst_tail[threadIdx.x] = src_tail[threadIdx.x];
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

// out[m, n] = alpha * sum_z parts[z * stride + m * ldp + n], z = 0 .. n_split-1
// in that order (deterministic), rounded once to the output type.
template <class T, int VEC>
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float* parts, int64_t stride, int n_split,
                                                            int64_t rows, int64_t cols, int64_t ldp, T* out,
                                                            int64_t ldo, float alpha) {
  const int64_t cpr = cols / VEC;
  const int64_t n = rows * cpr;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    const int64_t r = i / cpr, c = (i - r * cpr) * VEC;
    float acc[VEC];
#pragma unroll
    for (int q = 0; q < VEC; ++q) acc[q] = 0.f;
    const float* p = parts + r * ldp + c;
    // 8 slices' loads in flight, then their adds in z order (the sum order,
    // and so the result, is that of the plain loop)
    constexpr int U = 8;
    int z = 0;
    for (; z + U <= n_split; z += U, p += U * stride) {
      float v[U][VEC];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if constexpr (VEC == 4) {
          const float4 w = *reinterpret_cast<const float4*>(p + u * stride);
          v[u][0] = w.x; v[u][1] = w.y; v[u][2] = w.z; v[u][3] = w.w;
        } else {
          v[u][0] = p[u * stride];
        }
      }
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int q = 0; q < VEC; ++q) acc[q] += v[u][q];
    }
    for (; z < n_split; ++z, p += stride) {
      if constexpr (VEC == 4) {
        const float4 v = *reinterpret_cast<const float4*>(p);
        acc[0] += v.x; acc[1] += v.y; acc[2] += v.z; acc[3] += v.w;
      } else {
        acc[0] += p[0];
      }
    }
#pragma unroll
    for (int q = 0; q < VEC; ++q) out[r * ldo + c + q] = from_f32<T>(alpha * acc[q]);
  }
}

template <class T>
int launch_reduce(const float* parts, int64_t stride, int n_split, int64_t rows, int64_t cols, int64_t ldp, void* out,
                  int64_t ldo, float alpha, hipStream_t s) {
  const bool vec = cols % 4 == 0 && ldp % 4 == 0 && stride % 4 == 0 && ((uintptr_t)parts % 16) == 0;
  if (vec)
    splitk_reduce_kernel<T, 4><<<grid_for(rows * cols / 4, 256, 4096), 256, 0, s>>>(parts, stride, n_split, rows, cols,
                                                                                   ldp, (T*)out, ldo, alpha);
  else
    splitk_reduce_kernel<T, 1><<<grid_for(rows * cols, 256, 4096), 256, 0, s>>>(parts, stride, n_split, rows, cols, ldp,
                                                                               (T*)out, ldo, alpha);
  FORGE_CHECK_LAUNCH();
  return FORGE_OK;
}

// out[c, r] = in[r, c] for 2-byte elements (bf16 / fp16), one 64 x 64 tile
// (index `tidx`) through LDS (row pitch 66 elements against bank conflicts on
// the column reads), 16-byte loads and stores when pitches and bases allow.
__device__ __forceinline__ void transpose_tile(const uint16_t* in, int64_t ld_in, int64_t rows, int64_t cols,
                                               uint16_t* out, int64_t ld_out, int64_t tiles_c, int vec,
                                               int64_t tidx, uint16_t (&tile)[64][66]) {
  const int64_t r0 = (tidx / tiles_c) * 64, c0 = (tidx % tiles_c) * 64;
  const int t = threadIdx.x;
#pragma unroll
  for (int it = 0; it < 2; ++it) {
    const int v = t + 256 * it, rr = v / 8, cc = (v % 8) * 8;
    const int64_t r = r0 + rr, c = c0 + cc;
    if (vec && r < rows && c + 8 <= cols) {
      const uint4 q = *reinterpret_cast<const uint4*>(in + r * ld_in + c);
      const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        tile[rr][cc + 2 * j] = (uint16_t)(w[j] & 0xffff);
        tile[rr][cc + 2 * j + 1] = (uint16_t)(w[j] >> 16);
      }
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) tile[rr][cc + j] = (r < rows && c + j < cols) ? in[r * ld_in + c + j] : 0;
    }
  }
  __syncthreads();
#pragma unroll
  for (int it = 0; it < 2; ++it) {
    const int v = t + 256 * it, oc = v / 8, orr = (v % 8) * 8;  // output row = input column
    const int64_t c = c0 + oc, r = r0 + orr;
    if (c >= cols) continue;
    uint16_t e[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) e[j] = tile[orr + j][oc];
    if (vec && r + 8 <= rows) {
      uint4 q;
      q.x = e[0] | ((uint32_t)e[1] << 16);
      q.y = e[2] | ((uint32_t)e[3] << 16);
      q.z = e[4] | ((uint32_t)e[5] << 16);
      q.w = e[6] | ((uint32_t)e[7] << 16);
      *reinterpret_cast<uint4*>(out + c * ld_out + r) = q;
    } else {
      for (int j = 0; j < 8 && r + j < rows; ++j) out[c * ld_out + r + j] = e[j];
    }
  }
}

__global__ __launch_bounds__(256) void transpose2_kernel(const uint16_t* in, int64_t ld_in, int64_t rows, int64_t cols,
                                                         uint16_t* out, int64_t ld_out, int64_t tiles_c, int vec) {
  __shared__ uint16_t tile[64][66];
  transpose_tile(in, ld_in, rows, cols, out, ld_out, tiles_c, vec, blockIdx.x, tile);
}

// out[c, r] = in[r, c] for larger 2-byte matrices with 16-byte aligned bases
// and pitches that are multiples of 8: 64 x 256 tiles, so that each input row
// segment read is 512 bytes and each output row segment written 128 bytes,
// eight 16-byte loads per thread in flight before the tile goes to LDS, and
// the columns read back with ds_read_b64_tr_b16, which transposes within each
// 16-lane group: lane L supplies the 8 bytes at tile row k0 + L / 4, columns
// cb + 4 (L % 4), and receives rows k0 .. k0+3 of column cb + L; two reads
// (k0, k0 + 4) give a lane the 8 consecutive input rows of one output row
// chunk.  Partial tiles are zero-filled in LDS and their stores bounds-checked.
constexpr int TW_R = 64, TW_C = 256, TW_P = TW_C + 8;  // pitch: rows 16 bytes apart in the bank cycle
typedef short tw_i16x4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(256) void transpose2_wide_kernel(const uint16_t* in, int64_t ld_in, int64_t rows,
                                                              int64_t cols, uint16_t* out, int64_t ld_out,
                                                              int64_t tiles_c) {
  __shared__ __attribute__((aligned(16))) uint16_t tile[TW_R * TW_P];
  const int64_t r0 = ((int64_t)blockIdx.x / tiles_c) * TW_R, c0 = ((int64_t)blockIdx.x % tiles_c) * TW_C;
  const int t = threadIdx.x;
  uint4 q[8];
#pragma unroll
  for (int it = 0; it < 8; ++it) {
    const int row = t / 32 + 8 * it, cc = (t % 32) * 8;
    const int64_t r = r0 + row, c = c0 + cc;
    if (r < rows && c + 8 <= cols) {
      q[it] = *reinterpret_cast<const uint4*>(in + r * ld_in + c);
    } else {
      uint16_t e[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) e[j] = (r < rows && c + j < cols) ? in[r * ld_in + c + j] : 0;
      q[it] = make_uint4(e[0] | ((uint32_t)e[1] << 16), e[2] | ((uint32_t)e[3] << 16), e[4] | ((uint32_t)e[5] << 16),
                         e[6] | ((uint32_t)e[7] << 16));
    }
  }
#pragma unroll
  for (int it = 0; it < 8; ++it)
    *reinterpret_cast<uint4*>(tile + (t / 32 + 8 * it) * TW_P + (t % 32) * 8) = q[it];
  __syncthreads();
  const int lane = t % 64, w = t / 64, g = lane / 16, L = lane % 16;
#pragma unroll
  for (int it = 0; it < 8; ++it) {
    // (column block, row chunk) of this 16-lane group: the four groups of a
    // wave take four consecutive row chunks of one column block
    const int pidx = it * 16 + w * 4 + g, cb = (pidx / 8) * 16, rc = (pidx % 8) * 8;
    const uint16_t* a0 = tile + (rc + L / 4) * TW_P + cb + 4 * (L % 4);
    const tw_i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) tw_i16x4*)a0);
    const tw_i16x4 hi =
        __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) tw_i16x4*)(a0 + 4 * TW_P));
    const int64_t oc = c0 + cb + L, r = r0 + rc;
    if (oc >= cols || r >= rows) continue;
    const uint16_t e[8] = {(uint16_t)lo[0], (uint16_t)lo[1], (uint16_t)lo[2], (uint16_t)lo[3],
                           (uint16_t)hi[0], (uint16_t)hi[1], (uint16_t)hi[2], (uint16_t)hi[3]};
    if (r + 8 <= rows) {
      *reinterpret_cast<uint4*>(out + oc * ld_out + r) =
          make_uint4(e[0] | ((uint32_t)e[1] << 16), e[2] | ((uint32_t)e[3] << 16), e[4] | ((uint32_t)e[5] << 16),
                     e[6] | ((uint32_t)e[7] << 16));
    } else {
      for (int j = 0; j < 8 && r + j < rows; ++j) out[oc * ld_out + r + j] = e[j];
    }
  }
}

// Up to FORGE_TRANSPOSE_BATCH_MAX transposes in one launch: workgroup b takes
// tile b - first[i] of matrix i, first[i] <= b < first[i + 1].
struct TransposeBatch {
  int n;
  const uint16_t* in[FORGE_TRANSPOSE_BATCH_MAX];
  uint16_t* out[FORGE_TRANSPOSE_BATCH_MAX];
  int64_t ld_in[FORGE_TRANSPOSE_BATCH_MAX], ld_out[FORGE_TRANSPOSE_BATCH_MAX];
  int64_t rows[FORGE_TRANSPOSE_BATCH_MAX], cols[FORGE_TRANSPOSE_BATCH_MAX];
  int64_t tiles_c[FORGE_TRANSPOSE_BATCH_MAX];
  int64_t first[FORGE_TRANSPOSE_BATCH_MAX + 1];
  int vec[FORGE_TRANSPOSE_BATCH_MAX];
};

__global__ __launch_bounds__(256) void transpose2_batch_kernel(TransposeBatch b) {
  __shared__ uint16_t tile[64][66];
  const int64_t blk = blockIdx.x;
  int i = 0;
  while (i + 1 < b.n && blk >= b.first[i + 1]) ++i;
  transpose_tile(b.in[i], b.ld_in[i], b.rows[i], b.cols[i], b.out[i], b.ld_out[i], b.tiles_c[i], b.vec[i],
                 blk - b.first[i], tile);
}

}  // namespace

extern "C" int forge_transpose_2b(const void* src, int64_t ld_src, int64_t rows, int64_t cols, void* dst,
                                  int64_t ld_dst, void* stream) {
  if (rows < 0 || cols < 0 || ld_src < cols || ld_dst < rows)
    return forge_set_error(FORGE_ERR_INVALID, "transpose_2b: shape / pitch");
  if (rows == 0 || cols == 0) return FORGE_OK;
  if (!src || !dst) return forge_set_error(FORGE_ERR_INVALID, "transpose_2b: null pointer");
  const int64_t tr = (rows + 63) / 64, tc = (cols + 63) / 64;
  if (tr * tc > 0x7fffffffLL) return forge_set_error(FORGE_ERR_INVALID, "transpose_2b: too many tiles");
  const int vec = aligned16(src) && aligned16(dst) && ld_src % 8 == 0 && ld_dst % 8 == 0;
  if (vec && rows * cols >= (int64_t(1) << 16)) {
    // (measured on MI355X, bf16 [8192, 128256]: 64 x 64 tiles 864 us, these
    // 843 us; 64 to 256 rows x 128 or 256 columns 847-904 us: about 5 TB/s
    // whatever the tile shape)
    const int64_t wr = (rows + TW_R - 1) / TW_R, wc = (cols + TW_C - 1) / TW_C;
    transpose2_wide_kernel<<<(unsigned)(wr * wc), 256, 0, (hipStream_t)stream>>>(
        (const uint16_t*)src, ld_src, rows, cols, (uint16_t*)dst, ld_dst, wc);
  } else {
    transpose2_kernel<<<(unsigned)(tr * tc), 256, 0, (hipStream_t)stream>>>(
        (const uint16_t*)src, ld_src, rows, cols, (uint16_t*)dst, ld_dst, tc, vec);
  }
  FORGE_CHECK_LAUNCH();
  return FORGE_OK;
}

extern "C" int forge_transpose_2b_batch(int n, const void* const* src, const int64_t* ld_src, const int64_t* rows,
                                        const int64_t* cols, void* const* dst, const int64_t* ld_dst, void* stream) {
  if (n < 0 || n > FORGE_TRANSPOSE_BATCH_MAX)
    return forge_set_error(FORGE_ERR_INVALID, "transpose_2b_batch: 0..%d matrices", FORGE_TRANSPOSE_BATCH_MAX);
  TransposeBatch b = {};
  b.n = n;
  int64_t tiles = 0;
  for (int i = 0; i < n; ++i) {
    if (rows[i] < 0 || cols[i] < 0 || ld_src[i] < cols[i] || ld_dst[i] < rows[i])
      return forge_set_error(FORGE_ERR_INVALID, "transpose_2b_batch: shape / pitch of matrix %d", i);
    if (rows[i] > 0 && cols[i] > 0 && (!src[i] || !dst[i]))
      return forge_set_error(FORGE_ERR_INVALID, "transpose_2b_batch: null pointer (matrix %d)", i);
    b.in[i] = (const uint16_t*)src[i];
    b.out[i] = (uint16_t*)dst[i];
    b.ld_in[i] = ld_src[i];
    b.ld_out[i] = ld_dst[i];
    b.rows[i] = rows[i];
    b.cols[i] = cols[i];
    b.tiles_c[i] = (cols[i] + 63) / 64;
    b.vec[i] = aligned16(src[i]) && aligned16(dst[i]) && ld_src[i] % 8 == 0 && ld_dst[i] % 8 == 0;
    b.first[i] = tiles;
    tiles += (rows[i] > 0 && cols[i] > 0) ? ((rows[i] + 63) / 64) * b.tiles_c[i] : 0;
  }
  b.first[n] = tiles;
  if (tiles == 0) return FORGE_OK;
  if (tiles > 0x7fffffffLL) return forge_set_error(FORGE_ERR_INVALID, "transpose_2b_batch: too many tiles");
  transpose2_batch_kernel<<<(unsigned)tiles, 256, 0, (hipStream_t)stream>>>(b);
  FORGE_CHECK_LAUNCH();
  return FORGE_OK;
}

extern "C" int forge_splitk_reduce(const float* parts, int64_t split_stride, int n_split, int64_t rows, int64_t cols,
                                   int64_t ld_parts, void* out, int64_t ld_out, int out_dtype, float alpha,
                                   void* stream) {
  if (rows < 0 || cols < 0 || n_split < 1) return forge_set_error(FORGE_ERR_INVALID, "splitk_reduce: shape");
  if (rows == 0 || cols == 0) return FORGE_OK;
  hipStream_t s = (hipStream_t)stream;
  switch (out_dtype) {
    case FORGE_DTYPE_F32: return launch_reduce<float>(parts, split_stride, n_split, rows, cols, ld_parts, out, ld_out, alpha, s);
    case FORGE_DTYPE_BF16: return launch_reduce<bf16_t>(parts, split_stride, n_split, rows, cols, ld_parts, out, ld_out, alpha, s);
    case FORGE_DTYPE_F16: return launch_reduce<fp16_t>(parts, split_stride, n_split, rows, cols, ld_parts, out, ld_out, alpha, s);
    default: return forge_set_error(FORGE_ERR_UNSUPPORTED, "splitk_reduce: dtype %d", out_dtype);
  }
}

extern "C" int forge_zero(void* ptr, int64_t bytes, void* stream) {
  if (bytes <= 0) return FORGE_OK;
  if (!aligned16(ptr)) return forge_set_error(FORGE_ERR_INVALID, "zero: pointer not 16-byte aligned");
  const int64_t n16 = bytes / 16;
  zero_kernel<<<grid_for(n16 > 0 ? n16 : 1, 256, 2048), 256, 0, (hipStream_t)stream>>>(
      (uint4*)ptr, n16, (uint8_t*)ptr + n16 * 16, bytes - n16 * 16);
  FORGE_CHECK_LAUNCH();
  return FORGE_OK;
}

extern "C" int forge_copy(void* dst, const void* src, int64_t bytes, void* stream) {
  if (bytes <= 0) return FORGE_OK;
  if (!dst || !src) return forge_set_error(FORGE_ERR_INVALID, "copy: null pointer");
  if (!aligned16(dst) || !aligned16(src)) return forge_set_error(FORGE_ERR_INVALID, "copy: pointers not 16-byte aligned");
  const uintptr_t d = (uintptr_t)dst, s = (uintptr_t)src;
  if (d < s + (uintptr_t)bytes && s < d + (uintptr_t)bytes)
    return forge_set_error(FORGE_ERR_INVALID, "copy: source and destination overlap");
  const int64_t n16 = bytes / 16;
  const bool one = n16 <= (64LL << 20);  // up to 1 GiB: one vector per thread
  const int vpt = one ? 1 : 2;
  int64_t blocks = (n16 + 256 * vpt - 1) / (256 * vpt);
  if (blocks < 1) blocks = 1;
  if (blocks > 65536) blocks = 65536;
  const uint8_t* st = (const uint8_t*)src + n16 * 16;
  uint8_t* dt = (uint8_t*)dst + n16 * 16;
  if (one)
    copy_kernel<1><<<(unsigned)blocks, 256, 0, (hipStream_t)stream>>>((const uint4*)src, (uint4*)dst, n16, st, dt,
                                                                      bytes - n16 * 16);
  else
    copy_kernel<2><<<(unsigned)blocks, 256, 0, (hipStream_t)stream>>>((const uint4*)src, (uint4*)dst, n16, st, dt,
                                                                      bytes - n16 * 16);
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
