// Rotary position embedding (half-split / rotate_half convention) for gfx950.
//
// Reference: kernels/rope/forge_rope_v3.py:32-96 (kernel) and :99-132
// (launcher); the HF formula it is tested against is
// kernels/rope/tests/test_v1.py:49-61:
//     out = x * cos + rotate_half(x) * sin,   rotate_half(x) = cat(-x_hi, x_lo)
// i.e. for j < D/2:  out_lo = lo*cos_j - hi*sin_j,  out_hi = hi*cos_j + lo*sin_j
// (only the first D/2 cos/sin columns are read, as in the reference kernel).
// Backward is the same rotation with -sin.
//
// Work decomposition: one work item = (token t, 16-byte column chunk c of the
// lo half, group of HPT heads, HPT = 1).  The item loads its cos/sin chunk
// (L2-resident: the table is a few MB) and rotates that chunk of its head
// (Q heads first, then K heads); the lanes that share (t, head) cover the
// head's half rows, so for head_dim 128 every load and store instruction
// consumes whole 128-byte lines.  Measured on MI355X, cold, on the BASELINE
// shape: one head per item with up to 64 workgroups per CU streams 5.8-5.96
// TB/s, against 5.4-5.6 with 4 heads per item and 8 workgroups per CU, 5.9
// with 2 heads and 32-64 per CU, 5.1 with 8 heads (more items in flight beat
// fewer cos/sin reads).  Any element
// strides for (batch, head, seq) are accepted, so the HF `transpose(1, 2)`
// view of a [B, S, H, D] projection is rotated in place of memory order, with
// no copy.  Index math runs in 32 bits whenever every offset fits (the usual
// case); x is touched once, so its 16-byte loads and stores are nontemporal.
// The grid is capped at 64 workgroups per CU and strides over the items
// beyond that.
#include "common.h"

namespace {

constexpr int kBlock = 256;
constexpr int kHPT = 1;            // heads per work item
constexpr int kMaxBlocks = 16384;  // 64 workgroups per CU

struct RopeArgs {
  const void* q; int64_t q_sb, q_sh, q_ss;
  const void* k; int64_t k_sb, k_sh, k_ss;
  void* qo; int64_t qo_sb, qo_sh, qo_ss;
  void* ko; int64_t ko_sb, ko_sh, ko_ss;
  const void* cos; int64_t cos_sb, cos_ss;
  const void* sin; int64_t sin_sb, sin_ss;
  const int64_t* positions;
  int64_t table_rows;  // rows of cos/sin along the position axis
  int64_t seq_len, n_q, n_heads, half, chunks, n_hgroups, n_items;
  float sign;  // +1 forward, -1 backward
};

// VEC table values of type TC, as fp32 (times `scale`).  With kVec the
// VEC * sizeof(TC) bytes are 16-byte aligned and read as 16-byte vectors.
template <class TC, int VEC, bool kVec>
__device__ __forceinline__ void load_table(const TC* p, float scale, float (&out)[VEC]) {
  constexpr int BYTES = VEC * (int)sizeof(TC);
  if constexpr (kVec && BYTES % 16 == 0) {
    constexpr int PER = 16 / (int)sizeof(TC);
#pragma unroll
    for (int k = 0; k < BYTES / 16; ++k) {
      Vec16<TC> v = load16(p + k * PER);
#pragma unroll
      for (int j = 0; j < PER; ++j) out[k * PER + j] = scale * to_f32(v.v[j]);
    }
  } else {
#pragma unroll
    for (int j = 0; j < VEC; ++j) out[j] = scale * to_f32(p[j]);
  }
}

// T: q/k storage type; TC: cos/sin storage type (T, or fp32 tables with
// narrower q/k: the table is read as stored and the math is fp32, as in the
// reference kernel).  I: index type of the item / x offset math (int32_t
// when every offset fits).
template <class T, class TC, int VEC, class I>
__global__ __launch_bounds__(kBlock) void rope_kernel(RopeArgs a) {
  constexpr bool kVec16 = VEC * sizeof(T) == 16;
  const I stride = (I)gridDim.x * kBlock;
  const I n_items = (I)a.n_items, chunks = (I)a.chunks, n_hgroups = (I)a.n_hgroups;
  const I seq_len = (I)a.seq_len, n_q = (I)a.n_q, n_heads = (I)a.n_heads, half = (I)a.half;
  for (I i = (I)blockIdx.x * kBlock + threadIdx.x; i < n_items; i += stride) {
    const I c = i % chunks;
    const I rest = i / chunks;
    const I hg = rest % n_hgroups;
    const I t = rest / n_hgroups;
    const I b = t / seq_len;
    const I s = t - b * seq_len;
    const I col = c * VEC;
    // table offsets stay 64-bit: positions are caller data
    const int64_t pos = a.positions ? a.positions[t] : (int64_t)s;
    const int64_t cso = (int64_t)b * a.cos_sb + pos * a.cos_ss + col;
    const int64_t sno = (int64_t)b * a.sin_sb + pos * a.sin_ss + col;

    float cs[VEC], sn[VEC];
    if (pos >= 0 && pos < a.table_rows) {
      load_table<TC, VEC, kVec16>((const TC*)a.cos + cso, 1.0f, cs);
      load_table<TC, VEC, kVec16>((const TC*)a.sin + sno, a.sign, sn);
    } else {
      // a position outside the table: no table read, the token's outputs
      // are NaN (the host wrappers reject such positions before launching)
#pragma unroll
      for (int j = 0; j < VEC; ++j) { cs[j] = __builtin_nanf(""); sn[j] = cs[j]; }
    }

    const I h0 = hg * kHPT;
    T lo[kHPT][VEC], hi[kHPT][VEC];
#pragma unroll
    for (int u = 0; u < kHPT; ++u) {
      const I h = h0 + u;
      if (h < n_heads) {
        const T* src = h < n_q ? (const T*)a.q + (b * (I)a.q_sb + h * (I)a.q_sh + s * (I)a.q_ss + col)
                               : (const T*)a.k + (b * (I)a.k_sb + (h - n_q) * (I)a.k_sh + s * (I)a.k_ss + col);
        if constexpr (kVec16) {
          Vec16<T> l = load16_nt(src), r = load16_nt(src + half);
#pragma unroll
          for (int j = 0; j < VEC; ++j) { lo[u][j] = l.v[j]; hi[u][j] = r.v[j]; }
        } else {
#pragma unroll
          for (int j = 0; j < VEC; ++j) { lo[u][j] = src[j]; hi[u][j] = src[half + j]; }
        }
      }
    }
#pragma unroll
    for (int u = 0; u < kHPT; ++u) {
      const I h = h0 + u;
      if (h < n_heads) {
        T* dst = h < n_q ? (T*)a.qo + (b * (I)a.qo_sb + h * (I)a.qo_sh + s * (I)a.qo_ss + col)
                         : (T*)a.ko + (b * (I)a.ko_sb + (h - n_q) * (I)a.ko_sh + s * (I)a.ko_ss + col);
        if constexpr (kVec16) {
          Vec16<T> ol, oh;
#pragma unroll
          for (int j = 0; j < VEC; ++j) {
            float x0 = to_f32(lo[u][j]), x1 = to_f32(hi[u][j]);
            ol.v[j] = from_f32<T>(x0 * cs[j] - x1 * sn[j]);
            oh.v[j] = from_f32<T>(x1 * cs[j] + x0 * sn[j]);
          }
          store16_nt(dst, ol);
          store16_nt(dst + half, oh);
        } else {
#pragma unroll
          for (int j = 0; j < VEC; ++j) {
            float x0 = to_f32(lo[u][j]), x1 = to_f32(hi[u][j]);
            dst[j] = from_f32<T>(x0 * cs[j] - x1 * sn[j]);
            dst[half + j] = from_f32<T>(x1 * cs[j] + x0 * sn[j]);
          }
        }
      }
    }
  }
}

// Largest |element offset| any (b, h, s, d < D) address of a tensor reaches.
int64_t max_offset(int64_t sb, int64_t sh, int64_t ss, int64_t nb, int64_t nh, int64_t ns, int64_t d) {
  auto ext = [](int64_t st, int64_t n) { return n > 0 ? (st < 0 ? -st : st) * (n - 1) : 0; };
  return ext(sb, nb) + ext(sh, nh) + ext(ss, ns) + d;
}

template <class T, class TC>
int launch(RopeArgs a, bool all_aligned, bool offsets_fit32, hipStream_t s) {
  constexpr int V = 16 / sizeof(T);
  const bool vec = all_aligned && (a.half % V == 0);
  const int vw = vec ? V : 1;
  a.chunks = a.half / vw;
  a.n_hgroups = (a.n_heads + kHPT - 1) / kHPT;
  a.n_items = a.n_items * a.chunks * a.n_hgroups;  // n_items held the token count
  int64_t blocks = (a.n_items + kBlock - 1) / kBlock;
  if (blocks > kMaxBlocks) blocks = kMaxBlocks;
  // the loop index runs up to n_items + one grid stride
  const bool i32 = offsets_fit32 && a.n_items + (int64_t)kMaxBlocks * kBlock < 0x7fffffffLL;
  const dim3 grid((unsigned)blocks);
  if (vec) {
    if (i32) rope_kernel<T, TC, V, int32_t><<<grid, kBlock, 0, s>>>(a);
    else rope_kernel<T, TC, V, int64_t><<<grid, kBlock, 0, s>>>(a);
  } else {
    if (i32) rope_kernel<T, TC, 1, int32_t><<<grid, kBlock, 0, s>>>(a);
    else rope_kernel<T, TC, 1, int64_t><<<grid, kBlock, 0, s>>>(a);
  }
  FORGE_CHECK_LAUNCH();
  return FORGE_OK;
}

}  // namespace

extern "C" int forge_rope(int dtype, const void* q, int64_t q_sb, int64_t q_sh, int64_t q_ss,
                          const void* k, int64_t k_sb, int64_t k_sh, int64_t k_ss, void* q_out,
                          int64_t qo_sb, int64_t qo_sh, int64_t qo_ss, void* k_out, int64_t ko_sb,
                          int64_t ko_sh, int64_t ko_ss, const void* cos, int64_t cos_sb,
                          int64_t cos_ss, const void* sin, int64_t sin_sb, int64_t sin_ss,
                          int table_dtype, int64_t table_rows, const int64_t* positions,
                          int64_t batch, int64_t n_q, int64_t n_kv, int64_t seq_len,
                          int64_t head_dim, int backward, void* stream) {
  if (batch < 0 || n_q < 0 || n_kv < 0 || seq_len < 0 || head_dim < 0)
    return forge_set_error(FORGE_ERR_INVALID, "rope: negative shape");
  if (head_dim % 2 != 0) return forge_set_error(FORGE_ERR_INVALID, "rope: head_dim must be even");
  if (table_dtype != dtype && table_dtype != FORGE_DTYPE_F32)
    return forge_set_error(FORGE_ERR_UNSUPPORTED,
                           "rope: cos/sin dtype %d with q dtype %d (tables are q's dtype or fp32)",
                           table_dtype, dtype);
  if (table_rows < 0) return forge_set_error(FORGE_ERR_INVALID, "rope: negative table_rows");
  if (!positions && table_rows < seq_len)
    return forge_set_error(FORGE_ERR_INVALID, "rope: cos/sin have %lld rows for seq_len %lld",
                           (long long)table_rows, (long long)seq_len);
  if (batch == 0 || seq_len == 0 || head_dim == 0 || (n_q + n_kv) == 0) return FORGE_OK;

  RopeArgs a;
  a.q = q; a.q_sb = q_sb; a.q_sh = q_sh; a.q_ss = q_ss;
  a.k = k; a.k_sb = k_sb; a.k_sh = k_sh; a.k_ss = k_ss;
  a.qo = q_out; a.qo_sb = qo_sb; a.qo_sh = qo_sh; a.qo_ss = qo_ss;
  a.ko = k_out; a.ko_sb = ko_sb; a.ko_sh = ko_sh; a.ko_ss = ko_ss;
  a.cos = cos; a.cos_sb = cos_sb; a.cos_ss = cos_ss;
  a.sin = sin; a.sin_sb = sin_sb; a.sin_ss = sin_ss;
  a.positions = positions;
  a.table_rows = table_rows;
  a.seq_len = seq_len;
  a.n_q = n_q;
  a.n_heads = n_q + n_kv;
  a.half = head_dim / 2;
  a.n_items = batch * seq_len;
  a.sign = backward ? -1.0f : 1.0f;

  // 16-byte vectors need every base pointer and every non-unit stride aligned.
  const size_t es = dtype_size(dtype), ets = dtype_size(table_dtype);
  const int64_t V = es ? (int64_t)(16 / es) : 1;
  const int64_t Vt = ets ? (int64_t)(16 / ets) : 1;
  bool al = aligned16(q) && aligned16(k) && aligned16(q_out) && aligned16(k_out) &&
            aligned16(cos) && aligned16(sin);
  for (int64_t st : {q_sb, q_sh, q_ss, k_sb, k_sh, k_ss, qo_sb, qo_sh, qo_ss, ko_sb, ko_sh, ko_ss})
    al = al && (st % V == 0);
  for (int64_t st : {cos_sb, cos_ss, sin_sb, sin_ss}) al = al && (st % Vt == 0);

  // 32-bit x offsets when every Q / K / output address fits
  const int64_t lim = 0x7fffffffLL;
  const bool fit32 = max_offset(q_sb, q_sh, q_ss, batch, n_q, seq_len, head_dim) < lim &&
                     max_offset(qo_sb, qo_sh, qo_ss, batch, n_q, seq_len, head_dim) < lim &&
                     max_offset(k_sb, k_sh, k_ss, batch, n_kv, seq_len, head_dim) < lim &&
                     max_offset(ko_sb, ko_sh, ko_ss, batch, n_kv, seq_len, head_dim) < lim &&
                     batch * seq_len < lim;

  hipStream_t s = (hipStream_t)stream;
  const bool f32_table = table_dtype != dtype;
  switch (dtype) {
    case FORGE_DTYPE_F32: return launch<float, float>(a, al, fit32, s);
    case FORGE_DTYPE_BF16:
      return f32_table ? launch<bf16_t, float>(a, al, fit32, s) : launch<bf16_t, bf16_t>(a, al, fit32, s);
    case FORGE_DTYPE_F16:
      return f32_table ? launch<fp16_t, float>(a, al, fit32, s) : launch<fp16_t, fp16_t>(a, al, fit32, s);
    case FORGE_DTYPE_F64:
      return f32_table ? launch<double, float>(a, al, fit32, s) : launch<double, double>(a, al, fit32, s);
    default: return forge_set_error(FORGE_ERR_UNSUPPORTED, "rope: dtype %d", dtype);
  }
}
