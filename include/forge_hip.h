/*
 * forge_hip.h — C ABI of libforge_hip.so, the MI355X (gfx950) kernel library
 * behind the drop-in `kernels.{swiglu,rope,cross_entropy,lora_mlp,lora_qkv}`
 * Python modules.
 *
 * Conventions (all entry points):
 *   - Plain device pointers, element counts and element strides; no framework
 *     types.  The caller (PyTorch's caching allocator on the Python side) owns
 *     every buffer; the library retains no caller pointer past the call.  Its
 *     own memory: forge_ce_fwd_reduce's call slots (device memory and pinned
 *     host memory, allocated on a device's first call and kept until the
 *     process ends) and forge_lora_a_noalloc's static scratch array.
 *   - Every launch is asynchronous on the caller's `stream` (a hipStream_t
 *     passed as void*; NULL = the legacy default stream).  No host syncs.
 *   - Return value: FORGE_OK (0) or a FORGE_ERR_* code; forge_last_error()
 *     returns a message for the last failure on the calling thread.
 *   - dtype codes: FORGE_DTYPE_*.
 *
 * Each declaration names the reference interface it replaces
 * (paths relative to the Forge-researchlab/kernel-POCs root).
 */
#ifndef FORGE_HIP_H
#define FORGE_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  FORGE_DTYPE_F32 = 0,
  FORGE_DTYPE_F16 = 1,
  FORGE_DTYPE_BF16 = 2,
  FORGE_DTYPE_F64 = 3,
};

enum {
  FORGE_OK = 0,
  FORGE_ERR_INVALID = 1,     /* bad argument (shape, stride, alignment, dtype) */
  FORGE_ERR_UNSUPPORTED = 2, /* valid request this build does not implement */
  FORGE_ERR_HIP = 3,         /* HIP runtime error */
};

/* Library identity / diagnostics. */
const char* forge_version(void);
const char* forge_last_error(void);
/* 1 when the current HIP device is a gfx950 (hipDeviceProp_t.gcnArchName)
 * and this library's gfx950 code object loads on it (the attributes of a
 * probe kernel resolve); 0 otherwise, including when no device is visible. */
int forge_arch_ok(void);

/* ------------------------------------------------------------------------
 * SwiGLU
 * ------------------------------------------------------------------------ */

/* out[r, c] = (silu(gate[r, c] * gm) -> dtype) * up[r, c] * dm
 * gate/up rows are `ld_in` elements apart (gate and up may be two halves of
 * one packed [rows, 2*cols] row: up = gate + cols, ld_in = 2*cols).
 * Replaces `_swiglu_forward_kernel` / `_swiglu_packed_forward_kernel`
 * (kernels/swiglu/swiglu.py:60-82, 119-142) launched by `swiglu_forward` /
 * `swiglu_packed_forward` (kernels/swiglu/swiglu.py:201-229, 265-292). */
int forge_swiglu_fwd(int dtype, const void* gate, const void* up, int64_t ld_in,
                     void* out, int64_t ld_out, int64_t rows, int64_t cols,
                     float gate_multiplier, float down_multiplier, void* stream);

/* dup = dout*dm*silu(gate*gm); dgate = dout*dm*up*dsilu(gate*gm)*gm.
 * dgate/dup may alias gate/up (the reference's in-place default).
 * Replaces `_swiglu_backward_kernel` / `_swiglu_packed_backward_kernel`
 * (kernels/swiglu/swiglu.py:85-116, 145-176) launched by `swiglu_backward` /
 * `swiglu_packed_backward` (kernels/swiglu/swiglu.py:232-262, 295-323). */
int forge_swiglu_bwd(int dtype, const void* dout, int64_t ld_dout,
                     const void* gate, const void* up, int64_t ld_in,
                     void* dgate, void* dup, int64_t ld_dgrad,
                     int64_t rows, int64_t cols,
                     float gate_multiplier, float down_multiplier, void* stream);

/* GeGLU: out = gelu(gate).to(dtype) * up, GELU in its tanh form
 * (approximate_tanh != 0) or exact (erf); same layout contract as SwiGLU
 * (rows of `cols` elements, pitches ld_*, packed gate_up via up = gate + H and
 * ld = 2H).  Replaces `_geglu_forward_kernel` / `_geglu_packed_forward_kernel`
 * (kernels/geglu/geglu.py:126-148, 185-213) launched by `geglu_forward` /
 * `geglu_packed_forward` (:380-406, 440-467). */
int forge_geglu_fwd(int dtype, const void* gate, const void* up, int64_t ld_in,
                    void* out, int64_t ld_out, int64_t rows, int64_t cols,
                    int approximate_tanh, void* stream);

/* GeGLU backward: dup = dout * gelu(gate).to(dtype), dgate = dout * up *
 * gelu'(gate) (fp32, rounded once); dgate/dup may alias gate/up (in place).
 * Replaces `_geglu_backward_kernel` / `_geglu_packed_backward_kernel`
 * (kernels/geglu/geglu.py:151-182, 216-252) launched by `geglu_backward` /
 * `geglu_packed_backward` (:409-437, 470-498). */
int forge_geglu_bwd(int dtype, const void* dout, int64_t ld_dout,
                    const void* gate, const void* up, int64_t ld_in,
                    void* dgate, void* dup, int64_t ld_dgrad,
                    int64_t rows, int64_t cols, int approximate_tanh, void* stream);

/* ------------------------------------------------------------------------
 * RoPE (half-split rotation; any n_q, n_kv)
 * ------------------------------------------------------------------------ */

/* Rotates Q [B, n_q, S, D] and K [B, n_kv, S, D] given by element strides
 * (batch, head, seq; the D stride must be 1) into q_out/k_out (same
 * convention).  cos/sin rows are [D] with the given batch/seq strides
 * (batch stride 0 = broadcast); only the first D/2 entries of each row are
 * read.  cos/sin are stored in `table_dtype`: q's dtype, or fp32 for any q
 * (read as stored, math in fp32, as the reference kernel loads the table).
 * `table_rows` is the table's extent along the position axis.  If
 * `positions` (int64, [B*S]) is non-NULL the cos/sin row of token (b, s) is
 * positions[b*S + s] instead of s; a position outside [0, table_rows) reads
 * no table memory and gives NaN outputs for that token (callers validate
 * positions first; without positions table_rows < S is an error).
 * backward != 0 rotates by -theta.  Any q/k/out strides; in place
 * (q_out == q, k_out == k) is allowed.
 * Replaces `_forge_rope_v3_kernel` + `_launch_kernel`
 * (kernels/rope/forge_rope_v3.py:32-132). */
int forge_rope(int dtype,
               const void* q, int64_t q_sb, int64_t q_sh, int64_t q_ss,
               const void* k, int64_t k_sb, int64_t k_sh, int64_t k_ss,
               void* q_out, int64_t qo_sb, int64_t qo_sh, int64_t qo_ss,
               void* k_out, int64_t ko_sb, int64_t ko_sh, int64_t ko_ss,
               const void* cos, int64_t cos_sb, int64_t cos_ss,
               const void* sin, int64_t sin_sb, int64_t sin_ss,
               int table_dtype, int64_t table_rows,
               const int64_t* positions,
               int64_t batch, int64_t n_q, int64_t n_kv, int64_t seq_len,
               int64_t head_dim, int backward, void* stream);

/* ------------------------------------------------------------------------
 * Cross-entropy (online softmax, dlogits written in place)
 * ------------------------------------------------------------------------ */

enum {
  FORGE_CE_HAS_GRADIENTS = 1,
  FORGE_CE_HAS_WEIGHT = 2,
  FORGE_CE_HAS_SOFTCAP = 4,
  FORGE_CE_RETURN_Z_LOSS = 8,
  FORGE_CE_RETURN_ACCURACY = 16,
  FORGE_CE_RETURN_PREDICTED = 32,
  FORGE_CE_REDUCTION_MEAN = 64,
};

/* Per row of logits [n_rows, n_cols] (row stride ld): loss (fp32, [n_rows]),
 * optional z_loss (fp32), token accuracy (fp32), predicted token (int64),
 * and — with FORGE_CE_HAS_GRADIENTS — dloss/dlogits written over the logits
 * (ignored rows are zero-filled).  weight (fp32 [n_cols]) is read only with
 * FORGE_CE_HAS_WEIGHT.  Scalars follow the reference kernel's arguments.
 * stats (optional, device int64[4] from forge_ce_target_stats on the same
 * stream): when given, n_non_ignore (and sum_non_ignore_weight without
 * weights) are taken from stats[0] on the device, and nothing is written if
 * stats[3] == 0 (targets out of range).  A row whose target is neither
 * ignore_index nor in [0, n_cols) is always left untouched.
 * Replaces `forge_cross_entropy_kernel`
 * (kernels/cross_entropy/experiments/v2/cross_entropy_kernel_v2.py:65-338)
 * launched by `cross_entropy_forward` (same file :346-458). */
int forge_ce_fwd(int dtype, void* logits, int64_t ld, int64_t n_rows, int64_t n_cols,
                 const int64_t* target, int64_t target_stride,
                 const float* weight,
                 float* loss, float* z_loss, float* token_accuracy,
                 int64_t* predicted_tokens,
                 int64_t ignore_index, float n_non_ignore, float sum_non_ignore_weight,
                 float weight_sum, float lse_square_scale, float label_smoothing,
                 float softcap, int flags, const int64_t* stats, void* stream);

/* stats[0] = number of targets != ignore_index; stats[1], stats[2] = min and
 * max of target * (target != ignore_index); stats[3] = 1 if that range lies in
 * [0, n_cols), else 0.  Device int64[4], written on `stream`.  Replaces the
 * host-side `.item()` reads and bounds asserts of `cross_entropy_forward`
 * (kernels/cross_entropy/experiments/v2/cross_entropy_kernel_v2.py:374-387),
 * whose values the host still reads (for the same AssertionError) after the
 * main kernel is queued. */
int forge_ce_target_stats(const int64_t* target, int64_t target_stride, int64_t n_rows,
                          int64_t ignore_index, int64_t n_cols, int64_t* stats, void* stream);

/* forge_ce_fwd in one launch with the target statistics and the loss
 * reduction inside it (no class weights: FORGE_CE_HAS_WEIGHT is rejected).
 * The launch computes the statistics of forge_ce_target_stats itself (n_valid
 * for the mean; when the targets are out of range it writes no per-row output
 * and no gradient, and the sums, if requested, as 0) and copies them to
 * pinned host memory, tagged with the call's
 * *ticket; forge_ce_stats_wait(ticket) returns them on the host (for the
 * reference's bounds asserts) as soon as the launch has computed them,
 * without waiting for the rest of it.  loss (and z_loss) [n_rows] receive the
 * per-row values.  With loss_sum non-NULL the launch also stores their fp32
 * sum there (and z_loss's in z_sum), summed in a fixed order (deterministic),
 * and, when loss_cast / z_cast are given, the sums rounded to cast_dtype.
 * The library keeps 64 call slots per device (allocated on the first call):
 * call t uses slot t % 64, so at most 64 calls per device may be in flight
 * at once (launched and not yet finished on the device; calls on one stream
 * never overlap), and forge_ce_stats_wait must be called before 64 later
 * calls on the device have been made.
 * Replaces `forge_cross_entropy_kernel` with the `.item()` reads and bounds
 * asserts before it and the `torch.sum` after it
 * (kernels/cross_entropy/experiments/v2/cross_entropy_kernel_v2.py:374-387,
 * 414-441, 451). */
int forge_ce_fwd_reduce(int dtype, void* logits, int64_t ld, int64_t n_rows, int64_t n_cols,
                        const int64_t* target, int64_t target_stride,
                        float* loss, float* z_loss, float* token_accuracy, int64_t* predicted_tokens,
                        int64_t ignore_index, float lse_square_scale, float label_smoothing, float softcap,
                        int flags, float* loss_sum, float* z_sum, void* loss_cast, void* z_cast, int cast_dtype,
                        uint64_t* ticket, void* stream);

/* Host: waits until the launch of `ticket` (forge_ce_fwd_reduce on a stream of
 * the same device as `stream`) has computed its target statistics, then
 * stores them in stats[4] (host memory), laid out as forge_ce_target_stats'.
 * Returns an error if the stream finishes without them. */
int forge_ce_stats_wait(uint64_t ticket, int64_t* stats, void* stream);

/* x[r, :] *= *grad_output (device scalar of grad_dtype: fp32, bf16 or fp16),
 * in place; a no-op when *grad_output == 1 (the reference's torch.equal
 * skip, :465-467, decided on the device so the host does not wait).
 * Replaces `_element_mul_kernel`
 * (kernels/cross_entropy/experiments/v2/cross_entropy_kernel_v2.py:49-62). */
int forge_ce_scale(int dtype, void* x, int64_t ld, int64_t n_rows, int64_t n_cols,
                   const void* grad_output, int grad_dtype, void* stream);

/* Sum of an fp32 vector into out[0] (fp32), deterministic two-level tree;
 * when out_cast is given the sum is also stored there rounded to cast_dtype
 * (fp32, bf16 or fp16: the loss in the logits' dtype).  Used for the loss
 * reduction in place of `torch.sum(loss_1d)` and the cast that follows
 * (kernels/cross_entropy/experiments/v2/cross_entropy_kernel_v2.py:451). */
int forge_sum_f32(const float* x, int64_t n, float* out, void* out_cast, int cast_dtype, void* stream);

/* Token scaling of the fused linear + cross-entropy path: prob[r] = the
 * softmax probability of row r's target class after the optional softcap
 * (softcap <= 0: none), rounded to the logits dtype; 0 for ignored rows.
 * Replaces the `use_token_scaling` block of `fused_linear_cross_entropy_forward`
 * (kernels/cross_entropy/experiments/v2/fused_linear_cross_entropy.py:148-160). */
int forge_ce_target_prob(int dtype, const void* logits, int64_t ld, int64_t n_rows, int64_t n_cols,
                         const int64_t* target, int64_t target_stride, int64_t ignore_index, float softcap,
                         float* prob, void* stream);

/* x[r, :n_cols] *= scale[r] (fp32 scales), in place, rounded to x's dtype
 * (fp32, bf16 or fp16).  Replaces the loss and dlogits multiplications by the
 * token scaling factors (fused_linear_cross_entropy.py:196-205). */
int forge_row_scale(int dtype, void* x, int64_t ld, int64_t n_rows, int64_t n_cols, const float* scale,
                    void* stream);

/* ------------------------------------------------------------------------
 * RMSNorm (forward + backward, deterministic weight gradient)
 * ------------------------------------------------------------------------ */

enum { FORGE_RMS_LLAMA = 0, FORGE_RMS_GEMMA = 1, FORGE_RMS_NONE = 2 };

/* y[r, :] = RMSNorm(x[r, :]) * (w + offset) with rstd[r] = rsqrt(mean(x^2) + eps)
 * written to rstd (fp32; fp64 for fp64 x).  casting_mode FORGE_RMS_LLAMA /
 * GEMMA / NONE selects where products are rounded to the storage dtype (see
 * forge_rmsnorm_v4.py:73-128).  Dtypes: x, w, y all equal (fp32, fp64, bf16,
 * fp16), or a 16-bit x with an fp32 weight and y of x's dtype or fp32.
 * Replaces `_rmsnorm_v4_forward_kernel` (kernels/rmsnorm/forge_rmsnorm_v4.py:
 * 73-128, launched by rmsnorm_v4_forward :242-270; the v2/v3 kernels are the
 * same) and `_rmsnorm_v1_forward_kernel` (forge_rmsnorm_v1.py:32-58, llama
 * mode with offset 0 and y of the promoted dtype). */
int forge_rmsnorm_fwd(int dtype, int w_dtype, int y_dtype, const void* x, int64_t ldx, const void* w,
                      void* y, int64_t ldy, void* rstd, int64_t rows, int64_t cols, double eps,
                      double offset, int casting_mode, void* stream);

/* dx = rstd (s - x rstd^2 sum(s x) / H) with s = dy (w + offset), written
 * to dx (may alias dy: the in-place backward); when dw is given, dw =
 * sum over rows of dy x rstd in w's dtype, through per-workgroup partial
 * sums in `work` (forge_rmsnorm_bwd_workspace bytes, caller-allocated) added
 * in a fixed order.  variant 1 = v1's roundings (s and the dw terms rounded
 * to x's dtype).  Replaces `_rmsnorm_v4_backward_kernel`
 * (forge_rmsnorm_v4.py:131-184) with the host reduction of its partials
 * (:273-336), and `_rmsnorm_v1_backward_kernel` (forge_rmsnorm_v1.py:61-106). */
int forge_rmsnorm_bwd(int dtype, int w_dtype, const void* dy, int64_t lddy, const void* x, int64_t ldx,
                      const void* w, const void* rstd, void* dx, int64_t lddx, void* dw, void* work,
                      int64_t rows, int64_t cols, double offset, int variant, void* stream);

/* Bytes of the dw partial-sum workspace forge_rmsnorm_bwd needs. */
int64_t forge_rmsnorm_bwd_workspace(int dtype, int64_t rows, int64_t cols);

/* ------------------------------------------------------------------------
 * Generic GEMM (any strides, fp32 / fp16 / bf16 operands, fp32 accumulation)
 * ------------------------------------------------------------------------ */

/* C[m, n] = act(alpha * sum_k A[m*a_sm + k*a_sk] * B[k*b_sk + n*b_sn]
 *               + beta * C[m, n] + bias[n])   (bias of the operand dtype,
 * optional; act = FORGE_GEMM_ACT_NONE, _SILU, _RELU or _GELU, the tanh form)
 * with one fp32 fmaf per k in increasing k order (deterministic).  Operands
 * of `dtype` (fp32, fp16 or bf16); C of c_dtype = fp32 or dtype, row stride
 * ldc.  Any shape and stride: the path for fp32 / fp16 models and for K or
 * pitches that are not multiples of 8, which the bf16 MFMA core does not take.
 * Replaces the cuBLAS products of the fused linear + cross-entropy path
 * (kernels/cross_entropy/experiments/v2/fused_linear_cross_entropy.py:142-144,
 * 207-219: logits = X W^T + b, dX = dlogits W, dW += dlogits^T X,
 * db += colsum(dlogits)). */
int forge_gemm_generic(int64_t M, int64_t N, int64_t K, int dtype,
                       const void* a, int64_t a_sm, int64_t a_sk,
                       const void* b, int64_t b_sk, int64_t b_sn,
                       void* c, int64_t ldc, int c_dtype, float alpha, float beta,
                       const void* bias, int act, void* stream);

/* ------------------------------------------------------------------------
 * bf16 MFMA GEMM core (fp32 accumulation) with fused LoRA epilogues
 * ------------------------------------------------------------------------ */

/* Operand layouts. For A (M x K): ROW = [M][K] row-major (K contiguous),
 * COL = [K][M] (M contiguous).  For B (K x N): COL = [N][K] (K contiguous,
 * i.e. an nn.Linear weight used as W^T), ROW = [K][N] (N contiguous). */
enum { FORGE_LAYOUT_ROW = 0, FORGE_LAYOUT_COL = 1 };

/* One K-segment of a multi-segment product C = sum_s A_s @ B_s.  With
 * n_lo < n_hi the segment applies only to output columns [n_lo, n_hi) and B's
 * first column (row, for B as [N][K]) is output column n_lo; n_lo = n_hi = 0
 * means every column.  Segments with disjoint column ranges make several
 * independent products one launch (e.g. [dQ B_q | dK B_k | dV B_v]). */
typedef struct forge_gemm_segment {
  const void* a;  /* bf16 */
  int64_t lda;    /* multiple of 8, at most 4,194,303 (256 rows < 2^31 bytes) */
  const void* b;  /* bf16 */
  int64_t ldb;    /* as lda */
  int64_t k;      /* extent of this segment along K (multiple of 8) */
  int64_t n_lo, n_hi;
} forge_gemm_segment;

enum {
  FORGE_EPI_STORE = 0,          /* C = alpha*acc + beta*C (C dtype = c_dtype) */
  FORGE_EPI_ATOMIC_F32 = 1,     /* C(fp32) += alpha*acc  (split-K partials) */
  FORGE_EPI_SILU = 2,           /* C = silu(alpha*acc + beta*C)  (split_k 1) */
  FORGE_EPI_RELU = 3,           /* C = relu(alpha*acc + beta*C)  (split_k 1) */
  FORGE_EPI_GELU = 4,           /* C = gelu_tanh(alpha*acc + beta*C)  (split_k 1) */
};

/* Activation of forge_gemm_generic's result. */
enum {
  FORGE_GEMM_ACT_NONE = 0,
  FORGE_GEMM_ACT_SILU = 1,
  FORGE_GEMM_ACT_RELU = 2,
  FORGE_GEMM_ACT_GELU = 3,
};

/* C[M, N] = alpha * sum_s A_s @ B_s + beta * C.  A and B layouts are shared by
 * all segments.  c_dtype is FORGE_DTYPE_BF16 or FORGE_DTYPE_F32.  The SILU /
 * RELU / GELU epilogues store the activation of that value (the SiLU one
 * replaces the cuBLASLt SWISH-epilogue GEMM of the LoRA-MLP inference path,
 * kernels/lora_mlp/experiments/v4/cublaslt_silu.cu:9-92, with the tanh GELU
 * and ReLU of the same wrapper's epilogue map).  split_k > 1
 * partitions the K range across workgroups: with FORGE_EPI_ATOMIC_F32 they
 * accumulate into C; with FORGE_EPI_STORE and an fp32 C (beta = 0) split z
 * writes its partial sums to C + z*M*ldc (C holds split_k slices of [M, ldc]),
 * to be summed by forge_splitk_reduce (deterministic order).
 * Replaces the cuBLAS calls (`torch.matmul` / `addmm_`) of the LoRA paths:
 * kernels/lora_mlp/experiments/v6/lora_mlp_kernel_v6.py:373-443, 623-653;
 * kernels/lora_qkv/experiments/v4/lora_qkv_kernel_v4.py:248-287. */
int forge_gemm(int64_t M, int64_t N, const forge_gemm_segment* segs, int n_segs,
               int a_layout, int b_layout,
               void* c, int64_t ldc, int c_dtype, float alpha, float beta,
               int epilogue, int split_k, void* stream);

/* ------------------------------------------------------------------------
 * Fused LoRA entry points (bf16 storage, fp32 accumulation)
 * ------------------------------------------------------------------------ */

/* Gated activation of the fused LoRA-MLP entry points. */
enum {
  FORGE_ACT_SILU = 0,       /* SwiGLU: h = silu(e) g */
  FORGE_ACT_GELU_TANH = 1,  /* GeGLU, tanh-approximate GELU */
  FORGE_ACT_GELU_ERF = 2,   /* GeGLU, exact (erf) GELU */
};

/* LoRA-MLP forward, gate and up projections with the gated-activation epilogue:
 *   e = X Wg^T + xa[:, :r] Bg^T,  g = X Wu^T + xa[:, r:2r] Bu^T,
 *   h = silu(e) g                        (FORGE_ACT_SILU, on the fp32 e, g)
 *   h = round(gelu(round(e))) round(g)   (FORGE_ACT_GELU_*: forge_geglu_fwd on
 *                                         the stored bf16 e, g)
 * X [M, H] (row pitch ldx), Wg/Wu [I, H] (pitch ldw), xa [M, 2r] holding
 * (sg X Ag^T | su X Au^T) (pitch ld_xa; NULL or r = 0 disables LoRA),
 * Bg/Bu [I, r] (pitch ldb).  Writes e, g, h [M, I] (pitch ld_out); with
 * e = g = NULL only h is written (the merged-weight inference path: h =
 * silu(X Wg_eff^T) (X Wu_eff^T) in one GEMM, in place of the SWISH-epilogue
 * GEMM, plain GEMM and product of lora_mlp_kernel_v5.py:425-460).
 * SiLU replaces phases 1-3 of `_v6_forward_impl`
 * (kernels/lora_mlp/experiments/v6/lora_mlp_kernel_v6.py:373-415: two cuBLAS
 * GEMMs + `_fused_lora_swiglu_kernel`, experiments/v3/lora_mlp_kernel_v3.py:45-138);
 * GELU replaces the Gemma path's gate_proj(x), up_proj(x) and geglu(gate, up)
 * (forge/forge/patching/kernels/lora.py:184-188 with
 * kernels/geglu/geglu.py:126-148). */
int forge_lora_mlp_gate_up(int64_t M, int64_t H, int64_t I, int64_t r,
                           const void* x, int64_t ldx,
                           const void* w_gate, const void* w_up, int64_t ldw,
                           const void* xa, int64_t ld_xa,
                           const void* b_gate, const void* b_up, int64_t ldb,
                           void* e, void* g, void* h, int64_t ld_out, int activation, void* stream);

/* forge_lora_mlp_gate_up that also forms the forward's down-projection
 * LoRA-A product h A_down^T while its epilogue holds h:
 *   v_part[t][m][j] = sum over the h columns i of column tile t (128 wide)
 *                     of h[m, i] A_down[j, i]          (j < rd)
 * with a_down = A_down [rd][I] (pitch ld_ad).  v_part is fp32
 * [ceil(I / 128)][M][rd]; forge_splitk_reduce over its ceil(I / 128) slices
 * (fixed order) gives s_down h A_down^T, scaled and rounded once.  e and g
 * must be given (training); rd: 8..64, a multiple of 8; I a multiple of 8;
 * every buffer 16-byte aligned and ld_out a multiple of 8 (else an error, no
 * launch).  Replaces the LoRA-A product of the down projection that re-reads
 * h (kernels/lora_mlp/experiments/v6/lora_mlp_kernel_v6.py:423-442). */
int forge_lora_mlp_gate_up_v(int64_t M, int64_t H, int64_t I, int64_t r,
                             const void* x, int64_t ldx,
                             const void* w_gate, const void* w_up, int64_t ldw,
                             const void* xa, int64_t ld_xa,
                             const void* b_gate, const void* b_up, int64_t ldb,
                             void* e, void* g, void* h, int64_t ld_out, int activation,
                             const void* a_down, int64_t ld_ad, int64_t rd, float* v_part, void* stream);

/* LoRA-MLP backward through the down projection and the gated activation:
 *   DW = dY Wd + t Ad   (dY [M, H], Wd [H, I], t = sd dY Bd [M, r], Ad [r, I])
 *   then in place, with D = round(DW):
 *   FORGE_ACT_SILU:   f = round(silu(e)), h_out = f g, e <- D f,
 *                     g <- round(D g) sig(e) (1 + e (1 - sig(e)))
 *   FORGE_ACT_GELU_*: a = round(gelu(e)), h_out = a g, e <- D a (d up),
 *                     g <- D g gelu'(e) (d gate): forge_geglu_bwd with dout = D
 * w_layout FORGE_LAYOUT_ROW: w_down = Wd [H, I], a_down = Ad [r, I];
 * FORGE_LAYOUT_COL: w_down = Wd^T [I, H], a_down = Ad^T [I, r] (K-contiguous,
 * the faster engine; callers with frozen weights keep the transpose).
 * SiLU replaces `matmul_lora(dY, W_down^T, ...)` + `_DWf_DW_dfg_kernel`
 * (kernels/lora_mlp/experiments/v6/lora_mlp_kernel_v6.py:632-634;
 * kernels/lora_mlp/reference/unsloth_baseline.py:34-55, 118-168); GELU
 * replaces the backward of down_proj and geglu on the Gemma path
 * (forge/forge/patching/kernels/lora.py:186-188, kernels/geglu/geglu.py:151-182). */
int forge_lora_mlp_down_bwd(int64_t M, int64_t H, int64_t I, int64_t r,
                            const void* dy, int64_t lddy,
                            const void* w_down, int64_t ldwd,
                            const void* t_d, int64_t ld_t,
                            const void* a_down, int64_t ld_ad, int w_layout,
                            void* h_out, void* e_df, void* g_de, int64_t ld, int activation, void* stream);

/* forge_lora_mlp_down_bwd (W_down given as W^T [I][H], A_down as A^T [I][r])
 * that also forms the up / gate rank-rv products of the LoRA backward from
 * df and de while its epilogue holds them:
 *   v_part[t][m][j]      = sum over the columns i of column tile t (256 wide)
 *                          of df[m, i] B_u[i, j]          (j < rv)
 *   v_part[t][m][rv + j] = the same of de[m, i] B_g[i, j]
 * with b_up_t = B_u^T, b_gate_t = B_g^T ([rv][I], pitch ld_bt).  v_part is
 * fp32 [ceil(I / 256)][M][2 rv]; forge_splitk_reduce over its ceil(I / 256)
 * slices (fixed order) gives [df B_u | de B_g], scaled and rounded once.
 * With w_part (may be NULL) it also forms the LoRA B gradients' token
 * reductions:
 *   w_part[t][0][i][j] = sum over the rows m of row tile t (256 tall)
 *                        of df[m, i] xa_up[m, j]        (j < rv)
 *   w_part[t][1][i][j] = the same of de[m, i] xa_gate[m, j]
 * with xa_t_up = xa_up^T, xa_t_gate = xa_gate^T ([rv][M], pitch ld_xat >= M,
 * a multiple of 8).  w_part is fp32 [ceil(M / 256)][2][I][rv];
 * forge_splitk_reduce over its ceil(M / 256) slices (stride 2 I rv) from
 * block 0 or 1 gives df^T xa_up = dB_up or de^T xa_gate = dB_gate when xa
 * holds the scaled products s X A^T.
 * rv: 8..64, a multiple of 8; I a multiple of 8; every buffer 16-byte aligned
 * and ld a multiple of 8 (else an error, no launch).
 * Replaces the rank-r products of the LoRA up / gate backward that re-read df
 * and de (kernels/lora_mlp/experiments/v6/lora_mlp_kernel_v6.py:643-653), and
 * with w_part their B-gradient products (:646, :648). */
int forge_lora_mlp_down_bwd_v(int64_t M, int64_t H, int64_t I, int64_t r,
                              const void* dy, int64_t lddy,
                              const void* w_down_t, int64_t ldwd,
                              const void* t_d, int64_t ld_t,
                              const void* a_down_t, int64_t ld_ad,
                              void* h_out, void* e_df, void* g_de, int64_t ld, int activation,
                              const void* b_up_t, const void* b_gate_t, int64_t ld_bt, int64_t rv,
                              float* v_part, const void* xa_t_up, const void* xa_t_gate,
                              int64_t ld_xat, float* w_part, void* stream);

/* The gated-activation backward of forge_lora_mlp_down_bwd on its own:
 * (D, e, g) -> h [M, I] (pitch ld_h), df over e and de over g (pitch ld_eg)
 * for a bf16 D = dY Wd + t Ad [M, I] (pitch ld_d) that the caller computed,
 * with that entry point's per-element formulas.  I and the pitches multiples
 * of 8, pointers 16-byte aligned (else FORGE_ERR_UNSUPPORTED).  With
 * FORGE_ACT_SILU it replaces Unsloth's in-place `_DWf_DW_dfg_kernel`
 * (`swiglu_DWf_DW_dfg_kernel`, kernels/lora_mlp/reference/unsloth_baseline.py
 * :118-168, called by experiments/v6/lora_mlp_kernel_v6.py:632-640); the
 * GELU activations give the GeGLU backward (kernels/geglu/geglu.py:151-182). */
int forge_lora_mlp_glu_bwd(int64_t M, int64_t I, const void* d, int64_t ld_d, void* e_df, void* g_de,
                           int64_t ld_eg, void* h, int64_t ld_h, int activation, void* stream);

/* LoRA-QKV forward with GQA-asymmetric widths and optional fused RoPE:
 *   out[:, 0:hq]          = X Wq^T + xa[:, 0:r]   Bq^T   (rotated if apply_rope)
 *   out[:, hq:hq+hkv]     = X Wk^T + xa[:, r:2r]  Bk^T   (rotated if apply_rope)
 *   out[:, hq+hkv:hq+2hkv]= X Wv^T + xa[:, 2r:3r] Bv^T
 * xa holds (sq X Aq^T | sk X Ak^T | sv X Av^T).  RoPE (head_dim 64 or 128)
 * uses bf16 cos/sin tables [cs_rows, head_dim] with row pitch cs_ld and row
 * positions[m] for token m (NULL: m, then cs_rows >= M is required); a
 * position outside [0, cs_rows) reads no table memory and gives NaN in that
 * token's Q/K (callers validate positions first).  Q/K are rounded to bf16
 * before the rotation, as in the unfused path.
 * Replaces `lora_qkv_v2_3` (kernels/lora_qkv/experiments/v2/lora_qkv_kernel_v2_3.py
 * :177-267: one cuBLAS GEMM + `_fused_qkv_epilogue_packed_kernel`) followed by
 * the caller's RoPE (forge/forge/patching/kernels/lora.py:250-264). */
int forge_lora_qkv_rope(int64_t M, int64_t K, int64_t hq, int64_t hkv, int64_t r,
                        const void* x, int64_t ldx,
                        const void* w_q, const void* w_k, const void* w_v, int64_t ldw,
                        const void* xa, int64_t ld_xa,
                        const void* b_q, const void* b_k, const void* b_v, int64_t ldb,
                        void* out, int64_t ld_out,
                        const void* cos, const void* sin, int64_t cs_ld, int64_t cs_rows,
                        const int64_t* positions, int64_t head_dim, int apply_rope,
                        void* stream);

/* LoRA-QKV backward through RoPE with the LoRA-B products of its outputs, in
 * one pass over the gradients (head_dim 128, an even number of Q and of KV
 * heads; 32/8, 32/32, 64/8, 16/8, 8/2 and 4/2 Q/KV heads are built):
 *   dq_out = rotate(dq, -theta), dk_out = rotate(dk, -theta)   (forge_rope's
 *            backward: the same formula and rounding, bitwise equal)
 *   t[m]   = alpha [dq_out[m] B_q | dk_out[m] B_k | dv[m] B_v]   (bf16 [M, 3r],
 *            fp32 sums rounded once)
 * dq [M, hq], dk / dv [M, hkv] (row pitches ld_*); cos / sin bf16 [cs_rows,
 * >= 64] with row pitch cs_ld, read at the token's position (positions
 * int64 [M], or the row index when NULL); b*_t = B^T [r][width] (pitch ld_b*).
 * r: 16, 32, 48 or 64.  Every buffer 16-byte aligned, pitches multiples of 8
 * (ld_t of 4), else an error and no launch.  Replaces the RoPE backward
 * (kernels/rope/forge_rope_v3.py:32-132) and the three LoRA-B products of the
 * QKV backward (kernels/lora_qkv/experiments/v4/lora_qkv_kernel_v4.py:264-266),
 * which read the gradients a second time. */
int forge_lora_qkv_rope_bwd(int64_t M, int64_t hq, int64_t hkv, int64_t r, int64_t head_dim,
                            const void* dq, int64_t ld_dq, const void* dk, int64_t ld_dk,
                            const void* dv, int64_t ld_dv,
                            const void* cos, const void* sin, int64_t cs_ld, int64_t cs_rows,
                            const int64_t* positions,
                            void* dq_out, int64_t ld_qo, void* dk_out, int64_t ld_ko,
                            const void* bq_t, const void* bk_t, const void* bv_t,
                            int64_t ld_bq, int64_t ld_bk, int64_t ld_bv,
                            void* t, int64_t ld_t, float alpha, void* stream);

/* Rank-r LoRA-A projections of one input, one GEMM:
 *   out[:, p*r:(p+1)*r] = scales[p] * X @ A_p^T     for p < n_proj (<= 4)
 * X [M, K] (row pitch ldx), A_p [r, K] (pitch lda), out [M, n_proj*r] bf16.
 * scales is a host array.  split_k > 1 spreads K over split_k workgroups
 * per output tile, each writing fp32 partial sums to its slice of `work`
 * (fp32 [split_k][M][n_proj*r], caller-owned, no initialisation needed),
 * summed in a fixed order and rounded to bf16.  Replaces the LoRA-A GEMMs X @ A^T of the
 * reference (the stacked [W; A_g; A_u] cuBLAS call,
 * kernels/lora_mlp/experiments/v6/lora_mlp_kernel_v6.py:373-381, and
 * `XA_all = X @ A_packed^T`, kernels/lora_qkv/experiments/v4/lora_qkv_kernel_v4.py:260). */
int forge_lora_a(int64_t M, int64_t K, int64_t r, int n_proj, const void* x, int64_t ldx,
                 const void* const* a_mats, int64_t lda, const float* scales, void* out,
                 int64_t ld_out, float* work, int split_k, void* stream);

/* Bytes of the per-GPU scratch array behind forge_lora_a_noalloc. */
#define FORGE_LORA_A_SCRATCH_BYTES (16LL * 1024 * 1024)

/* forge_lora_a with no workspace argument and no allocation: the split-K
 * partials live in a file-scope device array of FORGE_LORA_A_SCRATCH_BYTES
 * per GPU (held until the process ends), so split_k * M * n_proj * r fp32
 * values must fit in it (larger calls return FORGE_ERR_INVALID).  Calls no
 * hipMalloc / hipFree.  Calls that overlap on one GPU (different streams)
 * share the array and race; serialise them.  Same results as forge_lora_a,
 * bit for bit.  No counterpart in the reference: it is for callers that
 * cannot allocate (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). */
int forge_lora_a_noalloc(int64_t M, int64_t K, int64_t r, int n_proj, const void* x, int64_t ldx,
                         const void* const* a_mats, int64_t lda, const float* scales, void* out,
                         int64_t ld_out, int split_k, void* stream);

/* Utilities for split-K reductions (no counterpart in the reference, which
 * delegates these to cuBLAS): zero an fp32 workspace with a fill kernel, and
 * cast a reduced fp32 [rows, cols] block to bf16. */
int forge_zero(void* ptr, int64_t bytes, void* stream);

/* Copies `bytes` bytes from src to dst (both 16-byte aligned, not
 * overlapping) with 16-byte nontemporal loads and stores.  No counterpart in
 * the reference: a plain device copy with the access pattern of this
 * library's streaming kernels, the ceiling that the HBM-bound kernels' rates
 * are read against. */
int forge_copy(void* dst, const void* src, int64_t bytes, void* stream);

/* out[m, n] = alpha * sum_{z < n_split} parts[z*split_stride + m*ld_parts + n],
 * summed in z order (deterministic), rounded once to out_dtype (fp32, bf16 or
 * fp16).  The reduction of forge_gemm / forge_lora_a split-K partials; no
 * reference counterpart (the reference's cuBLAS GEMMs do not split K). */
int forge_splitk_reduce(const float* parts, int64_t split_stride, int n_split, int64_t rows, int64_t cols,
                        int64_t ld_parts, void* out, int64_t ld_out, int out_dtype, float alpha, void* stream);
int forge_cast_f32_bf16(const float* src, int64_t ld_src, void* dst, int64_t ld_dst, int64_t rows,
                        int64_t cols, void* stream);

/* dst[c, r] = src[r, c] for 2-byte elements (bf16 / fp16), src [rows, cols]
 * with row pitch ld_src, dst [cols, rows] with row pitch ld_dst.  Makes the
 * token-reduction weight gradient of the fused linear + cross-entropy path
 * (dW = dlogits^T X, fused_linear_cross_entropy.py:211-212) a K-contiguous
 * product for the LDS-DMA GEMM; no reference counterpart (cuBLAS reads the
 * transposed operands directly). */
int forge_transpose_2b(const void* src, int64_t ld_src, int64_t rows, int64_t cols, void* dst, int64_t ld_dst,
                       void* stream);

/* Up to FORGE_TRANSPOSE_BATCH_MAX of the above in one launch: matrix i is
 * src[i] [rows[i], cols[i]] (pitch ld_src[i]) -> dst[i] [cols[i], rows[i]]
 * (pitch ld_dst[i]).  The transposed rank-r LoRA matrices that the backward
 * passes read K-contiguous (B^T for dY B, A^T for the dX LoRA segments), in
 * one launch per backward instead of one each; no reference counterpart. */
#define FORGE_TRANSPOSE_BATCH_MAX 8
int forge_transpose_2b_batch(int n, const void* const* src, const int64_t* ld_src, const int64_t* rows,
                             const int64_t* cols, void* const* dst, const int64_t* ld_dst, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FORGE_HIP_H */
