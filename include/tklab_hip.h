/*
 * tklab_hip.h — C ABI of libtklab_hip.so, the gfx950 (MI355X) kernels behind
 * the tklab Python entry points.
 *
 * Each entry point replaces one `kernel[grid](...)` launch of the reference's
 * Python launchers (v1olegrace/triton-kernel-lab, src/tklab/kernels/<kernel>.py); the
 * replaced launch is cited above every declaration. Validation, allocation and
 * autograd stay in Python exactly as in the reference; these functions only
 * check what the kernels themselves assume and then enqueue work.
 *
 * Conventions
 *   - Pointers are device pointers; `const` marks inputs. Nothing here
 *     allocates or frees device memory: every output and workspace is passed in.
 *   - Sizes and strides are in ELEMENTS, as int64_t. Every feature dimension is
 *     unit-stride; the strides given are the remaining (row/batch/head) ones.
 *     Strides are >= 0 (0 repeats one row, e.g. a broadcast table); a negative
 *     stride, a size <= 0 or sizes whose product leaves the kernels' index range
 *     are rejected before anything is enqueued.
 *   - `dtype` is one of TK_DTYPE_*; all tensors of one call share it unless a
 *     parameter says otherwise (statistics and workspaces are float32).
 *   - `stream` is a hipStream_t (0 = the null stream). Work is enqueued
 *     asynchronously; no function synchronizes the device.
 *   - Return value: 0 on success; non-zero when the arguments break a kernel
 *     assumption or the launch failed. tk_last_error() then returns a message
 *     (thread-local, valid until the next failing call on the same thread).
 */
#ifndef TKLAB_HIP_H
#define TKLAB_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TK_ABI_VERSION 1

enum tk_dtype { TK_DTYPE_F32 = 0, TK_DTYPE_F16 = 1, TK_DTYPE_BF16 = 2 };

/* ABI version of the loaded library (TK_ABI_VERSION at build time). */
int tk_abi_version(void);

/* Message of the last failing call on this thread ("" if none). */
const char* tk_last_error(void);

/* Row-wise softmax y = exp(x - max) / sum, float32 math, stored in `dtype`.
 * Replaces `_softmax_kernel[(rows,)](...)`, src/tklab/kernels/fused_softmax.py:116-124.
 * cols <= 65536. */
int tk_softmax_fwd(int dtype, const void* x, void* y, int64_t rows, int64_t cols,
                   int64_t x_row_stride, int64_t y_row_stride, void* stream);

/* Online softmax for rows of any width: the same y = exp(x - max) / sum per row,
 * for the rows the single-pass kernel rejects (more than 65536 columns). No
 * reference kernel exists; the reference's validator points callers there
 * (src/tklab/kernels/fused_softmax.py:75-79, "use an online softmax").
 * Each row is split into chunks of 16384 columns whose (max, sum of exp) partials
 * are folded in a fixed order; deterministic, cols <= 2^31 - 1.
 * `partials` is the workspace, float32[2 * rows * ceil(cols / 16384)], 8-byte aligned; the
 * call overwrites it (no clearing needed). Rows of at most 64 chunks (1 048 576 columns)
 * take one launch that reads x once (one read and one write per element; the workgroups
 * of a row exchange their partials through the workspace, after a small kernel clears
 * it); wider rows take two launches (partials, then fold and write: two reads, one
 * write). */
int tk_softmax_online_fwd(int dtype, const void* x, void* y, float* partials, int64_t rows,
                          int64_t cols, int64_t x_row_stride, int64_t y_row_stride,
                          void* stream);

/* RMSNorm forward with an optional fused residual add.
 *   s = residual ? round_dtype(x + residual) : x
 *   rstd = 1 / sqrt(mean(s^2) + eps);  y = s * rstd * weight
 * `residual`, `residual_sum` (written when non-null) and `rstd` (float32[rows],
 * written when non-null) may be NULL. `y` may be NULL when `rstd` is not
 * (statistics mode: only s and rstd are written and `weight` is not read; the
 * statistics pass of tk_gemm_rowscale's normalized GEMM).
 * Replaces `_rms_norm_forward_kernel[(rows,)]`, src/tklab/kernels/rms_norm.py:248-260,
 * and `_residual_rms_norm_forward_kernel[(rows,)]`,
 * src/tklab/kernels/residual_rms_norm.py:149-167. cols * sizeof(dtype) <= 65536. */
int tk_rmsnorm_fwd(int dtype, const void* x, const void* residual, const void* weight,
                   void* residual_sum, void* y, float* rstd, int64_t rows, int64_t cols,
                   int64_t x_row_stride, int64_t residual_row_stride,
                   int64_t residual_sum_row_stride, int64_t y_row_stride, float eps,
                   void* stream);

/* RMSNorm backward, stage 1: per-row dx (plus `incoming_dx` when non-null) and
 * one float32 dweight partial row per group, partial_dw[group_count][cols].
 * Group g (g < group_count = min(group_size, rows)) owns the contiguous rows
 * [g*q, min((g+1)*q, rows)) with q = ceil(rows / group_count) and writes
 * partial_dw[g] with a plain store, in a fixed summation order (deterministic,
 * no atomics); a group past the last row writes a zero partial row. `locks` is int32[2*group_size]:
 * the first half is left untouched (zero), the second half gets 1 in every
 * slot g < group_count, marking partial row g as written.
 * Replaces `_rms_norm_backward_stage1_kernel[(rows,)]`, src/tklab/kernels/rms_norm.py:309-327. */
int tk_rmsnorm_bwd_stage1(int dtype, void* dx, const void* dy, const void* incoming_dx,
                          float* partial_dw, const void* x, const void* weight,
                          const float* rstd, int32_t* locks, int64_t rows, int64_t cols,
                          int64_t x_row_stride, int64_t dy_row_stride,
                          int64_t incoming_dx_row_stride, int64_t dx_row_stride,
                          int64_t group_size, void* stream);

/* RMSNorm backward, stage 2: dw[c] = sum_{g < group_count} partial_dw[g][c], summed
 * in increasing g, stored in `dtype`.
 * Replaces `_rms_norm_backward_stage2_kernel[...]`, src/tklab/kernels/rms_norm.py:335-343. */
int tk_rmsnorm_bwd_stage2(int dtype, const float* partial_dw, void* dw, int64_t group_count,
                          int64_t cols, void* stream);

/* Size of the device array that holds tk_rmsnorm_bwd_noalloc's partial rows (16 MiB per GPU). */
#define TK_RMSNORM_NOALLOC_SCRATCH_BYTES (16LL << 20)

/* RMSNorm backward, both stages, allocating nothing: the same kernels and results as
 * tk_rmsnorm_bwd_stage1 (no `locks` counts) followed by tk_rmsnorm_bwd_stage2 with the same
 * group_size, so dx and dw are bitwise those of the two-call path. The float32 partial rows
 * (group_count = min(group_size, rows) rows of `cols`) live in a library-owned device array of
 * TK_RMSNORM_NOALLOC_SCRATCH_BYTES on each GPU, kept until the process ends; a problem needing
 * more (group_count * cols * 4 bytes) is rejected with an error, before any launch. The call
 * makes no hipMalloc/hipFree and no memset: every partial row read is written first.
 * All calls on one GPU share that array, so calls that overlap on one GPU (different streams or
 * threads) race; serialize them. The stream must belong to the current device.
 * No counterpart in the reference: for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid allocation). */
int tk_rmsnorm_bwd_noalloc(int dtype, void* dx, void* dw, const void* dy, const void* incoming_dx,
                           const void* x, const void* weight, const float* rstd, int64_t rows,
                           int64_t cols, int64_t x_row_stride, int64_t dy_row_stride,
                           int64_t incoming_dx_row_stride, int64_t dx_row_stride,
                           int64_t group_size, void* stream);

/* SwiGLU forward y = value * gate * sigmoid(gate).
 * Replaces `_swiglu_forward_kernel[...]`, src/tklab/kernels/swiglu.py:157-167. */
int tk_swiglu_fwd(int dtype, const void* value, const void* gate, void* y, int64_t rows,
                  int64_t cols, int64_t value_row_stride, int64_t gate_row_stride,
                  int64_t y_row_stride, void* stream);

/* SwiGLU backward: dvalue = dy * silu(gate), dgate = dy * value * silu'(gate).
 * Replaces `_swiglu_backward_kernel[...]`, src/tklab/kernels/swiglu.py:185-199. */
int tk_swiglu_bwd(int dtype, const void* dy, const void* value, const void* gate,
                  void* dvalue, void* dgate, int64_t rows, int64_t cols,
                  int64_t dy_row_stride, int64_t value_row_stride, int64_t gate_row_stride,
                  int64_t dvalue_row_stride, int64_t dgate_row_stride, void* stream);

/* Rotate-half RoPE forward on x[rows][2*half_dim] with cos/sin[rows][half_dim]:
 *   y1 = x1*cos - x2*sin,  y2 = x2*cos + x1*sin.
 * Replaces `_rope_forward_kernel[...]`, src/tklab/kernels/rope.py:213-225. */
int tk_rope_fwd(int dtype, const void* x, const void* cos, const void* sin, void* y,
                int64_t rows, int64_t half_dim, int64_t x_row_stride, int64_t cos_row_stride,
                int64_t sin_row_stride, int64_t y_row_stride, void* stream);

/* RoPE backward: dx = RoPE(dy, cos, -sin); when non-null,
 * dcos = dy1*x1 + dy2*x2 and dsin = -dy1*x2 + dy2*x1 (x is read only then).
 * Replaces `_rope_backward_kernel[...]`, src/tklab/kernels/rope.py:251-271. */
int tk_rope_bwd(int dtype, const void* dy, const void* x, const void* cos, const void* sin,
                void* dx, void* dcos, void* dsin, int64_t rows, int64_t half_dim,
                int64_t dy_row_stride, int64_t x_row_stride, int64_t cos_row_stride,
                int64_t sin_row_stride, int64_t dx_row_stride, int64_t dcos_row_stride,
                int64_t dsin_row_stride, void* stream);

/* Rotate-half RoPE over `rows` rows of [batch, heads, seq, D] (uniform row strides)
 * with position-indexed tables cos/sin [>= seq][D/2] (row stride table_row_stride):
 * row r uses table row r mod seq. inverse == 0: tk_rope_fwd's arithmetic; inverse != 0:
 * the input gradient, tk_rope_bwd's dx (RoPE with -sin). No reference counterpart:
 * the reference's tables are per row (src/tklab/kernels/rope.py:213-225); this is the
 * position-indexed form the attention prologue uses (see tk_attn_fwd_rope). */
int tk_rope_positions(int dtype, const void* x, const void* cos, const void* sin, void* y,
                      int64_t rows, int64_t seq, int64_t half_dim, int64_t x_row_stride,
                      int64_t table_row_stride, int64_t y_row_stride, int inverse,
                      void* stream);

/* GEMM C[M][N] = A[M][K] * B[K][N] on MFMA, float32 accumulation, C stored in
 * `dtype` (TK_DTYPE_F16 or TK_DTYPE_BF16). All strides are element strides
 * and must be positive. `acc_fp16` != 0 requests the reference's FP16
 * accumulation mode; gfx950 MFMA accumulates f16/bf16 products in float32
 * only, so the flag is accepted and the result is the FP32-accumulated one.
 * Replaces `_matmul_kernel[grid](...)`, src/tklab/kernels/matmul.py:217-232. */
int tk_gemm(int dtype, const void* a, const void* b, void* c, int64_t m, int64_t n,
            int64_t k, int64_t stride_am, int64_t stride_ak, int64_t stride_bk,
            int64_t stride_bn, int64_t stride_cm, int64_t stride_cn, int acc_fp16,
            void* stream);

/* GEMM with the SwiGLU nonlinearity fused into its epilogue:
 *   y = value * gate * sigmoid(gate), gate = a * b_gate, value = a * b_up,
 * with a [m, k] and both weights [k, n]; gate and value are rounded to `dtype`
 * before the nonlinearity, exactly as when two tk_gemm calls store them and
 * tk_swiglu_fwd reads them back, so the result is bitwise that composition's while
 * the two m x n intermediates never reach HBM. No reference kernel exists: the
 * reference lists this fusion among its next steps around
 * src/tklab/kernels/swiglu.py:28-59 and matmul.py:72-164. Needs unit inner
 * strides, 16-byte aligned rows, k % 32 == 0, n % 8 == 0 and operand extents
 * below 2 GiB (otherwise non-zero status: compose tk_gemm and tk_swiglu_fwd).
 * dtype TK_DTYPE_F16 or TK_DTYPE_BF16. */
int tk_gemm_swiglu(int dtype, const void* a, const void* b_gate, const void* b_up, void* y,
                   int64_t m, int64_t n, int64_t k, int64_t stride_am, int64_t stride_ak,
                   int64_t stride_gk, int64_t stride_gn, int64_t stride_uk, int64_t stride_un,
                   int64_t stride_ym, int64_t stride_yn, void* stream);

/* GEMM with a per-row float32 scale in its epilogue:
 *   c[i, :] = round_dtype(row_scale[i] * (a * b)[i, :])   (float32 accumulation)
 * The normalized GEMM rms_norm(s; w) * W = diag(rstd) * s * (diag(w) * W): with
 * row_scale = rstd from tk_rmsnorm_fwd's statistics mode and b = tk_scale_rows(W, w)
 * (the norm weight folded into the projection once per weight version), the
 * normalized activations are never written. No reference kernel exists: the
 * reference lists the residual-RMSNorm -> projection fusion among its next steps
 * around src/tklab/kernels/residual_rms_norm.py:28-82 and matmul.py:72-164.
 * Operand requirements are tk_gemm_swiglu's (otherwise non-zero status: compose
 * tk_rmsnorm_fwd and tk_gemm). dtype TK_DTYPE_F16 or TK_DTYPE_BF16. */
int tk_gemm_rowscale(int dtype, const void* a, const void* b, const float* row_scale, void* c,
                     int64_t m, int64_t n, int64_t k, int64_t stride_am, int64_t stride_ak,
                     int64_t stride_bk, int64_t stride_bn, int64_t stride_cm, int64_t stride_cn,
                     void* stream);

/* Row scaling y[r, c] = round_dtype(x[r, c] * scale[r]) for x, y [rows, cols]
 * (unit column stride) and scale[rows] in the same dtype: folds a normalization
 * weight into the projection that follows it (see tk_gemm_rowscale). Helper of
 * that fusion; no reference counterpart. */
int tk_scale_rows(int dtype, const void* x, const void* scale, void* y, int64_t rows,
                  int64_t cols, int64_t x_row_stride, int64_t y_row_stride, void* stream);

/* Flash attention forward over q/k/v/o[batch][heads][seq][head_dim]
 * (head_dim unit-stride; strides given for batch, head and seq), head_dim in
 * {64, 128}, dtype TK_DTYPE_F16 or TK_DTYPE_BF16. Online softmax in base 2
 * with scale*log2(e); O = acc / l. When `lse` (float32[batch][heads][seq],
 * contiguous) is non-null it receives m + log2(l), the base-2 log-sum-exp of
 * the scaled scores.
 * Replaces `_flash_attention_forward_kernel[grid](...)`,
 * src/tklab/kernels/flash_attention.py:331-347. */
int tk_attn_fwd(int dtype, const void* q, const void* k, const void* v, void* o, float* lse,
                int64_t batch, int64_t heads, int64_t seq, int64_t head_dim,
                const int64_t* q_strides, const int64_t* k_strides, const int64_t* v_strides,
                const int64_t* o_strides, float sm_scale, int causal, void* stream);

/* Attention backward preprocess: delta[b][h][i] = sum_d o[i][d] * do[i][d] (float32).
 * o and do share `strides` (batch, head, seq).
 * Replaces `_attn_bwd_preprocess_kernel[...]`, src/tklab/kernels/flash_attention.py:560-569. */
int tk_attn_bwd_preprocess(int dtype, const void* o, const void* dout, float* delta,
                           int64_t batch, int64_t heads, int64_t seq, int64_t head_dim,
                           const int64_t* strides, void* stream);

/* Attention backward, dK and dV for every key block (single writer per block):
 *   P = exp2(S*scale*log2e - lse) (masked), dV = P^T dO, dS = P (dO V^T - delta),
 *   dK = scale * dS^T Q.  All of q/k/v/dout/dk/dv share `strides`.
 * Replaces `_attn_bwd_dkdv_kernel[...]`, src/tklab/kernels/flash_attention.py:570-587. */
int tk_attn_bwd_dkdv(int dtype, const void* q, const void* k, const void* v, const void* dout,
                     void* dk, void* dv, const float* lse, const float* delta, int64_t batch,
                     int64_t heads, int64_t seq, int64_t head_dim, const int64_t* strides,
                     float sm_scale, int causal, void* stream);

/* Attention backward, dQ = scale * dS K for every query block (single writer).
 * Replaces `_attn_bwd_dq_kernel[...]`, src/tklab/kernels/flash_attention.py:588-605. */
int tk_attn_bwd_dq(int dtype, const void* q, const void* k, const void* v, const void* dout,
                   void* dq, const float* lse, const float* delta, int64_t batch,
                   int64_t heads, int64_t seq, int64_t head_dim, const int64_t* strides,
                   float sm_scale, int causal, void* stream);

/* Grouped-query attention (prefill / training): q, o, dO, dQ have `heads` heads, k, v,
 * dK, dV have `kv_heads` (heads % kv_heads == 0) and query head h uses K/V head
 * h / (heads / kv_heads). Same arithmetic as tk_attn_fwd / tk_attn_bwd_dkdv /
 * tk_attn_bwd_dq (which are the kv_heads == heads case); delta comes from
 * tk_attn_bwd_preprocess with the query-side strides. dK and dV sum a KV head's query
 * heads in a fixed order (deterministic). Strides: q_strides {batch, head, seq} of the
 * query side, kv_strides of the KV side. Needs each head's rows below 2 GiB.
 * No reference kernel exists: the reference lists grouped-query attention among its
 * next steps (README.md:509-514; docs/research/gqa_decode_model.md fixes the head
 * mapping). */
int tk_attn_fwd_gqa(int dtype, const void* q, const void* k, const void* v, void* o, float* lse,
                    int64_t batch, int64_t heads, int64_t kv_heads, int64_t seq,
                    int64_t head_dim, const int64_t* q_strides, const int64_t* k_strides,
                    const int64_t* v_strides, const int64_t* o_strides, float sm_scale,
                    int causal, void* stream);
/* Grouped-query attention forward with rotate-half RoPE applied to Q and K first,
 * from position-indexed tables cos/sin [table_rows >= seq][head_dim / 2]: query and
 * key i use row i. Q is rotated in the kernel's prologue as it is loaded (the rotate-half
 * pairs sit in one lane's MFMA fragments); K is rotated once by tk_rope_positions into
 * the workspace `k_rot` (contiguous [batch][kv_heads][seq][head_dim]), since every
 * query block re-reads each K block. Bitwise the composition tk_rope_fwd(q), tk_rope_fwd(k),
 * tk_attn_fwd_gqa; k_rot holds the rotated K afterwards (the backward needs it). K must be
 * [batch][kv_heads][seq] rows of one row stride. No reference kernel exists: the
 * reference lists RoPE in the attention prologue among its next steps around
 * src/tklab/kernels/rope.py:26-73 and flash_attention.py:120-264. */
int tk_attn_fwd_rope(int dtype, const void* q, const void* k, const void* v, void* o, float* lse,
                     const void* rope_cos, const void* rope_sin, int64_t table_rows,
                     int64_t table_row_stride, void* k_rot, int64_t batch, int64_t heads,
                     int64_t kv_heads, int64_t seq, int64_t head_dim, const int64_t* q_strides,
                     const int64_t* k_strides, const int64_t* v_strides,
                     const int64_t* o_strides, float sm_scale, int causal, void* stream);
int tk_attn_bwd_dkdv_gqa(int dtype, const void* q, const void* k, const void* v,
                         const void* dout, void* dk, void* dv, const float* lse,
                         const float* delta, int64_t batch, int64_t heads, int64_t kv_heads,
                         int64_t seq, int64_t head_dim, const int64_t* q_strides,
                         const int64_t* kv_strides, float sm_scale, int causal, void* stream);
int tk_attn_bwd_dq_gqa(int dtype, const void* q, const void* k, const void* v,
                       const void* dout, void* dq, const float* lse, const float* delta,
                       int64_t batch, int64_t heads, int64_t kv_heads, int64_t seq,
                       int64_t head_dim, const int64_t* q_strides, const int64_t* kv_strides,
                       float sm_scale, int causal, void* stream);

/* Variable-length attention: packed q, o, dO, dQ [total][heads][head_dim] and k, v,
 * dK, dV [total][kv_heads][head_dim] (strides {token, head}; head_dim unit-stride),
 * int32 cu_seqlens[batch + 1]: sequence b is rows cu_seqlens[b] .. cu_seqlens[b+1]
 * (max_seqlen the longest). Same arithmetic as tk_attn_fwd_gqa / _bwd_*_gqa per
 * sequence; LSE and delta are float32 [heads][total] (delta from tk_attn_bwd_preprocess
 * with batch 1, seq total, strides {total * token, head, token}). Lengths are clamped
 * into [0, total] and to max_seqlen inside the kernels. No reference kernel exists: the
 * reference lists variable-length batches among its next steps (README.md:509-514). */
int tk_attn_fwd_varlen(int dtype, const void* q, const void* k, const void* v, void* o,
                       float* lse, const int32_t* cu_seqlens, int64_t batch, int64_t heads,
                       int64_t kv_heads, int64_t max_seqlen, int64_t total, int64_t head_dim,
                       const int64_t* q_strides, const int64_t* kv_strides,
                       const int64_t* o_strides, float sm_scale, int causal, void* stream);
int tk_attn_bwd_dkdv_varlen(int dtype, const void* q, const void* k, const void* v,
                            const void* dout, void* dk, void* dv, const float* lse,
                            const float* delta, const int32_t* cu_seqlens, int64_t batch,
                            int64_t heads, int64_t kv_heads, int64_t max_seqlen, int64_t total,
                            int64_t head_dim, const int64_t* q_strides,
                            const int64_t* kv_strides, float sm_scale, int causal, void* stream);
int tk_attn_bwd_dq_varlen(int dtype, const void* q, const void* k, const void* v,
                          const void* dout, void* dq, const float* lse, const float* delta,
                          const int32_t* cu_seqlens, int64_t batch, int64_t heads,
                          int64_t kv_heads, int64_t max_seqlen, int64_t total, int64_t head_dim,
                          const int64_t* q_strides, const int64_t* kv_strides, float sm_scale,
                          int causal, void* stream);

/* ---- Registry kernels outside the transformer hot path ---------------- */

/* out[i*out_stride] = x[i*x_stride] + y[i*y_stride], i < n (strides may be 0).
 * Replaces `_vector_add_kernel[grid](...)`, src/tklab/kernels/vector_add.py:98-107. */
int tk_vector_add(int dtype, const void* x, const void* y, void* out, int64_t n,
                  int64_t x_stride, int64_t y_stride, int64_t out_stride, void* stream);

/* Pointwise activation forward, kind 0 = ReLU, 1 = exact (erf) GELU,
 * 2 = SiLU, 3 = tanh (as 2*sigmoid(2x) - 1).
 * Replaces `_activation_forward_kernel[...]`, src/tklab/kernels/activations.py:173-182. */
int tk_activation_fwd(int dtype, int kind, const void* x, void* y, int64_t rows, int64_t cols,
                      int64_t x_row_stride, int64_t y_row_stride, void* stream);

/* dx = dy * activation'(x).
 * Replaces `_activation_backward_kernel[...]`, src/tklab/kernels/activations.py:195-206. */
int tk_activation_bwd(int dtype, int kind, const void* dy, const void* x, void* dx, int64_t rows,
                      int64_t cols, int64_t dy_row_stride, int64_t x_row_stride,
                      int64_t dx_row_stride, void* stream);

/* LayerNorm forward y = (x - mean) * rstd * w + b; mean/rstd (float32[rows])
 * written when non-null.
 * Replaces `_layer_norm_forward_kernel[(rows,)]`, src/tklab/kernels/layer_norm.py:254-267. */
int tk_layernorm_fwd(int dtype, const void* x, const void* weight, const void* bias, void* y,
                     float* mean, float* rstd, int64_t rows, int64_t cols, int64_t x_row_stride,
                     int64_t y_row_stride, float eps, void* stream);

/* LayerNorm backward stage 1: dx per row and float32 dweight/dbias partial rows
 * per group, with the same count and determinism contract as
 * tk_rmsnorm_bwd_stage1; group g owns the rows r with r % group_size == g.
 * Replaces `_layer_norm_backward_stage1_kernel[(rows,)]`, src/tklab/kernels/layer_norm.py:316-333. */
int tk_layernorm_bwd_stage1(int dtype, void* dx, const void* dy, float* partial_dw,
                            float* partial_db, const void* x, const void* weight,
                            const float* mean, const float* rstd, int32_t* locks, int64_t rows,
                            int64_t cols, int64_t x_row_stride, int64_t dy_row_stride,
                            int64_t dx_row_stride, int64_t group_size, void* stream);

/* LayerNorm backward stage 2: fixed-order column sums of both partial buffers.
 * Replaces `_layer_norm_backward_stage2_kernel[...]`, src/tklab/kernels/layer_norm.py:341-350. */
int tk_layernorm_bwd_stage2(int dtype, const float* partial_dw, const float* partial_db, void* dw,
                            void* db, int64_t group_count, int64_t cols, void* stream);

/* Grouped-query attention decode: for each (batch b, query head h) one query row
 * q[b][h] attends to the first clamp(seqlens[b], 0, max_len) keys of KV head
 * h / (q_heads / kv_heads) (all max_len when `seqlens` is NULL); o[b][h] in the
 * storage dtype, `lse` (nullable) float32 [batch][q_heads], base 2.
 * No reference kernel exists: the workload and head mapping are the reference's
 * decode model (docs/research/gqa_decode_model.md, "Canonical decode workload",
 * "Semantic GQA mapping"); the arithmetic is its attention forward for one query
 * row (src/tklab/kernels/flash_attention.py:90-117, 248-264).
 * Strides in elements: q_strides/o_strides {batch, head}, k/v_strides {batch,
 * head, position}; the head dimension is unit-stride; bases 16-byte aligned and
 * strides multiples of 8. dtype F16 or BF16; head_dim 64 or 128; q_heads /
 * kv_heads in {1, 2, 4, 8}. `partials` is float32 workspace of
 * batch * q_heads * ceil(max_len / split_len) * (head_dim + 4) elements;
 * split_len (keys per split-kernel wave) is a positive multiple of 64. */
int tk_gqa_decode(int dtype, const void* q, const void* k, const void* v, void* o, float* lse,
                  float* partials, const int32_t* seqlens, int64_t batch, int64_t q_heads,
                  int64_t kv_heads, int64_t max_len, int64_t head_dim, int64_t split_len,
                  const int64_t* q_strides, const int64_t* k_strides, const int64_t* v_strides,
                  const int64_t* o_strides, float scale, void* stream);

/* ---- Calibration kernels (no counterpart in the reference). They measure the
 * roofs this GPU sustains, so that the kernels above can be priced against
 * measured ceilings beside the published peaks. */

/* Copy `bytes` (a multiple of 16; 16-byte aligned pointers) from src to dst with
 * 16-byte non-temporal accesses, four loads in flight per thread: the streaming roof. */
int tk_roof_copy(const void* src, void* dst, int64_t bytes, void* stream);

/* `reads` source arrays and `writes` destination arrays of `bytes` each (src holds
 * reads * bytes, dst writes * bytes, at least `bytes` when writes is 0), cut into tiles of
 * `tile_kib` (8 or 16) KiB per array: one workgroup per tile (max_workgroups 0) or at most
 * max_workgroups workgroups walking the tiles grid-stride. 16-byte non-temporal loads,
 * stores non-temporal (store_policy 0) or sc1 (1); each written 16-byte chunk i is
 * {i, 0, 0, 0} xor the chunks read at its position. Mixes (reads:writes) 1:0, 0:1, 1:1, 2:1,
 * 3:1, 2:2 and 3:2. HBM traffic: (reads + writes) * bytes. */
int tk_roof_stream(const void* src, void* dst, int64_t bytes, int reads, int writes,
                   int store_policy, int tile_kib, int64_t max_workgroups, void* stream);

/* Dense MFMA issue with no memory traffic: `waves` waves (a multiple of 4) each
 * run `iters` (a multiple of 8) iterations of 16 independent v_mfma_f32_16x16x32
 * (dtype TK_DTYPE_F16 or TK_DTYPE_BF16) on random operand bits held in
 * registers, and write one float to out[wave]. Work: waves * iters * 8 * 32768 FLOP. */
int tk_roof_mfma(int dtype, float* out, int64_t waves, int64_t iters, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TKLAB_HIP_H */
