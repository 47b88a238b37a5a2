/*
 * ksdraft_amd.h — C ABI of libksdraft_amd.so, the MI355X (gfx950) kernels behind
 * KSDraft's INT8 tier (the reference's ksdraft/kernels package).
 *
 * Conventions shared by every entry point:
 *   - All pointers are device pointers (HBM) unless stated otherwise. The library
 *     allocates nothing: callers own inputs and outputs.
 *   - `stream` is a hipStream_t passed as void*; work is enqueued on it and the call
 *     returns without synchronising.
 *   - Tensors are dense row-major. int8 codes, fp16 scales (passed as uint16_t bit
 *     patterns), fp32 accumulators.
 *   - Return value: KSD_OK (0) or an error class. The message of the last error on the
 *     calling thread is copied out by ksd_last_error(). Calls keep no global mutable
 *     state besides that thread-local message, so they are reentrant.
 *   - "group" is the quantisation group size along the quantised axis; 32, 64 and
 *     128 are supported (128 is the KSDraft default, GROUP_SIZE in
 *     reference ksdraft/kernels/quant.py:20).
 */
#ifndef KSDRAFT_AMD_H
#define KSDRAFT_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* status codes (mapped to Python exception classes by the host wrapper) */
#define KSD_OK 0
#define KSD_EINVAL 1   /* ValueError: shape / group / argument mismatch */
#define KSD_ETYPE 2    /* TypeError: unsupported dtype                  */
#define KSD_EHIP 3     /* RuntimeError: HIP launch / runtime failure     */

/* element types for typed float buffers */
#define KSD_F32 0
#define KSD_BF16 1
#define KSD_F16 2
#define KSD_F16_SAT 3  /* output only: fp16 rounded then clamped to +-65504 */

/* ABI version, bumped on any signature change. */
int ksd_abi_version(void);

/* Copies the calling thread's last error message (NUL-terminated) into buf. */
int ksd_last_error(char *buf, size_t len);

/*
 * Q1 / Q3 — quantize along the last dim.
 * Replaces quantize_last_dim (reference ksdraft/kernels/quant.py:30-52) and, with
 * noise != NULL, quantize_last_dim_dithered (reference ksdraft/train/stages.py:27-50).
 *   x       (rows, K) of type x_dtype, row stride x_stride elements
 *   codes   (rows, K) int8, dense
 *   scales  (rows, ceil(K/group)) fp16
 *   noise   NULL, or (rows, ceil(K/group)*group) fp32 uniform [0,1) draws (torch.rand of
 *           the padded grouped shape); code_value += (noise - 0.5) * dither2 before rounding,
 *           dither2 = fp32(2 * dither).
 */
int ksd_quantize_lastdim(const void *x, int x_dtype, int64_t rows, int64_t K,
                         int64_t x_stride, int group, int8_t *codes, uint16_t *scales,
                         const float *noise, float dither2, void *stream);

/*
 * Q2 — dequantize along the last dim: out = float(code) * float(scale) per group.
 * Replaces dequantize_last_dim (reference ksdraft/kernels/quant.py:55-67).
 *   codes (rows, K) int8; scales (rows, n_scales) fp16; out (rows, K) fp32.
 *   group is already resolved by the caller (the reference's group=None inference).
 */
int ksd_dequantize_lastdim(const int8_t *codes, const uint16_t *scales, int64_t rows,
                           int64_t K, int64_t n_scales, int group, float *out,
                           void *stream);

/*
 * Transposed quantization: quantize_last_dim(x.t().contiguous(), group) without the
 * transpose copy. Used for the dW operands (reference ksdraft/kernels/ks3_int8.py:418,422).
 *   x       (R, C) of type x_dtype, dense
 *   codes   (C, R) int8; scales (C, ceil(R/group)) fp16
 */
int ksd_quantize_transpose(const void *x, int x_dtype, int64_t R, int64_t C, int group,
                           int8_t *codes, uint16_t *scales, void *stream);

/*
 * Requant-transpose: quantize_last_dim(dequantize_last_dim(codes, scales).t(), group).
 * Replaces the dequantize -> transpose -> requantize operand builds of
 * reference ksdraft/kernels/ks3_int8.py:349-351, 407-408, 417-419, 423.
 *   codes (R, C) int8 with scales (R, ceil(C/group_in)) fp16
 *   out_codes (C, R) int8; out_scales (C, ceil(R/group)) fp16
 */
int ksd_requant_transpose(const int8_t *codes, const uint16_t *scales, int64_t R,
                          int64_t C, int group_in, int group, int8_t *out_codes,
                          uint16_t *out_scales, void *stream);

/*
 * ksd_requant_transpose (group 128 in and out) of many tensors in one launch: the weight
 * transposes W^T = quant(dequant(W)^T) that a training step's dX GEMMs use (reference
 * ksdraft/kernels/ks3_int8.py:349-351, 403-424), built for every registered master right
 * after the optimizer step instead of once per layer inside the backward. Results equal n
 * ksd_requant_transpose calls; the list is read during the call only. No reference
 * counterpart as one call.
 */
typedef struct KsdRequantT {
  const int8_t *codes;    /* (R, C) int8 */
  const uint16_t *scales; /* (R, ceil(C/128)) fp16 */
  int64_t R, C;
  int8_t *codes_t;        /* (C, R) int8 */
  uint16_t *scales_t;     /* (C, ceil(R/128)) fp16 */
} KsdRequantT;
int ksd_requant_transpose_multi(const KsdRequantT *list, int n, int group, void *stream);

/*
 * Both layouts of one tensor in one pass: the row codes quantize_last_dim(x, group) and
 * the column codes quantize_last_dim(x.t(), group) (t_from_codes = 0: the dY and dY^T
 * operands of the linear backward, reference ksdraft/kernels/ks3_int8.py:410, 418), or
 * the column codes of the row-quantized values, quantize_last_dim(dequantize_last_dim(
 * codes, scales).t(), group) (t_from_codes = 1: the X and X^T operands, :417-420), or both
 * layouts of x rounded to fp16 first (t_from_codes = 2: the KS3 cell's g16 = grad.to(
 * float16) operands, :345-348, :421-422; needs group 128, C % 8 == 0, 16-byte rows).
 * No reference counterpart as one call; the results equal those of ksd_quantize_lastdim
 * followed by ksd_quantize_transpose or ksd_requant_transpose (of x.to(float16) for mode 2).
 *   x       (R, C) of type x_dtype (KSD_F32, KSD_BF16, KSD_F16), dense
 *   codes   (R, C) int8;  scales   (R, ceil(C/group)) fp16
 *   codes_t (C, R) int8;  scales_t (C, ceil(R/group)) fp16
 */
int ksd_quantize_dual(const void *x, int x_dtype, int64_t R, int64_t C, int group,
                      int t_from_codes, int8_t *codes, uint16_t *scales, int8_t *codes_t,
                      uint16_t *scales_t, void *stream);
/*
 * ksd_quantize_dual with t_from_codes = 1 (the X-operand recipe) of two tensors of one dtype
 * in one launch: a linear layer's fp32 weight and its input when both are quantized for a
 * training forward (reference ksdraft/kernels/linear.py:46-56 and :69 with the X^T recipe of
 * ks3_int8.py:417-420). The outputs are those of two ksd_quantize_dual calls; shapes the
 * fused kernel does not take (C % 8 != 0, unaligned rows) run as two calls. Group 128.
 */
int ksd_quantize_dual2(const void *x0, int64_t R0, int64_t C0, int8_t *codes0, uint16_t *scales0,
                       int8_t *codes_t0, uint16_t *scales_t0, const void *x1, int64_t R1,
                       int64_t C1, int8_t *codes1, uint16_t *scales1, int8_t *codes_t1,
                       uint16_t *scales_t1, int x_dtype, int group, void *stream);
/*
 * ksd_quantize_dual (t_from_codes = 0, group 128) of an upstream gradient dY, plus its column
 * sums: the bias gradient db = dY.float().sum(0) of an Int8Linear's backward (reference
 * ksdraft/kernels/linear.py:75-97 through autograd's bias grad), from the same read of dY.
 * Each 128-row tile sums its column in four 32-row parts ((p0 + p1) + (p2 + p3)); the tiles'
 * sums are added in tile order (an fp32 sum in another order than torch's: TOL).
 *   colsum     (C,) fp32
 *   workspace  fp32 scratch of ceil(R/128) * C * 4 bytes; R > 0, C % 8 == 0, aligned rows
 */
int ksd_quantize_dual_colsum(const void *x, int x_dtype, int64_t R, int64_t C, int group,
                             int8_t *codes, uint16_t *scales, int8_t *codes_t, uint16_t *scales_t,
                             float *colsum, float *workspace, int64_t workspace_bytes, void *stream);

/*
 * Cross entropy over the rows of fp32 logits (R, C) with class targets, the
 * F.cross_entropy(logits, tgt) of reference ksdraft/train/__init__.py:77 (mean reduction,
 * torch's default ignore_index semantics). Row statistics, one read of the logits:
 *   row_max[r]     = max_c y[r, c]
 *   row_inv_sum[r] = 1 / sum_c exp(y[r, c] - row_max[r])
 *   row_loss[r]    = row_max[r] + log(1 / row_inv_sum[r]) - y[r, t_r], or 0 when t_r is
 *                    ignore_index or outside [0, C) (the caller validates targets)
 * The mean loss is sum(row_loss) / (number of counted rows), as torch computes it.
 */
int ksd_ce_row_stats(const float *logits, int64_t R, int64_t C, const int64_t *targets,
                     int64_t ignore_index, float *row_max, float *row_inv_sum, float *row_loss,
                     void *stream);

/*
 * The backward of that cross entropy, quantized straight into both int8 operand layouts of
 * the LM head's int8 backward (dY for dX = dY.W, dY^T for dW = dY^T.X; the recipe of
 * reference ksdraft/kernels/ks3_int8.py:403-424), without writing dY:
 *   dY[r, c] = (exp(y[r, c] - row_max[r]) * row_inv_sum[r] - [c == t_r]) * grad_scale[0]
 * for counted rows and 0 for ignored ones; grad_scale is a device fp32 scalar (d loss /
 * d mean-CE divided by the counted-row count). codes/scales and codes_t/scales_t are
 * exactly ksd_quantize_dual(dY, t_from_codes = 0) of these dY values. No reference
 * counterpart as one call (the reference's autograd materialises dY in fp32).
 *   group 128; dy_out (R, C) fp32 optional: when given, dY is also written there. Shapes
 *   with C % 8 != 0 (or unaligned buffers) require dy_out, which then serves as the
 *   staging buffer of the two-pass path.
 */
int ksd_ce_backward_quant_dual(const float *logits, int64_t R, int64_t C, const float *row_max,
                               const float *row_inv_sum, const int64_t *targets,
                               int64_t ignore_index, const float *grad_scale, int group,
                               int8_t *codes, uint16_t *scales, int8_t *codes_t,
                               uint16_t *scales_t, float *dy_out, void *stream);

/*
 * One torch.optim.AdamW step on fp32 masters with the int8 repack of the updated masters:
 * the optimizer step of reference ksdraft/train/__init__.py:114-116, 166 (AdamW with
 * decoupled weight decay after clip_grad_norm_) fused with the per-call weight quantization
 * of ksdraft/kernels/linear.py:46-56 (and the master repack of ks3_int8.py:262-277).
 * Elementwise, in the order of torch's single-tensor AdamW, each op one fp32 rounding:
 *   g  = grad * clip_coef[0]          (when clip_coef is non-null: clip_grad_norm_'s mul_)
 *   p  = param * decay                (decay = 1 - lr * weight_decay)
 *   m  = m + one_minus_beta1 * (g - m)
 *   v  = v * beta2 + (one_minus_beta2 * g) * g
 *   p  = p + (-step_size) * (m / (sqrt(v) / bias_correction2_sqrt + eps))
 * param, exp_avg, exp_avg_sq are updated in place; grad is read only. The scalars are
 * torch's python-double values rounded to fp32: step_size = lr / (1 - beta1^step),
 * bias_correction2_sqrt = (1 - beta2^step)^0.5. When codes/scales are non-null they
 * receive quantize_last_dim(p) (rows, K) int8 / (rows, ceil(K/128)) fp16. group 128.
 * No reference counterpart as one call.
 */
int ksd_adamw_requant(float *param, const float *grad, float *exp_avg, float *exp_avg_sq,
                      int64_t rows, int64_t K, const float *clip_coef, float decay,
                      float one_minus_beta1, float beta2, float one_minus_beta2, float eps,
                      float step_size, float bias_correction2_sqrt, int group, int8_t *codes,
                      uint16_t *scales, void *stream);

/*
 * ksd_adamw_requant over many masters in a few launches (the optimizer step of a whole
 * model: torch's foreach AdamW over a parameter group, reference ksdraft/train/__init__.py:
 * 114-116, 166). Each entry is one master with its own step scalars; the shared scalars
 * and clip_coef are those of ksd_adamw_requant. Results equal n ksd_adamw_requant calls.
 * The list is read during the call only. No reference counterpart as one call.
 */
typedef struct KsdAdamTensor {
  float *param;
  const float *grad;
  float *exp_avg;
  float *exp_avg_sq;
  int8_t *codes;    /* (rows, K) int8, or NULL (no repack; scales NULL too) */
  uint16_t *scales; /* (rows, ceil(K/128)) fp16 */
  int64_t rows, K;
  float step_size, bias_correction2_sqrt;
} KsdAdamTensor;
int ksd_adamw_requant_multi(const KsdAdamTensor *tensors, int n, const float *clip_coef, float decay,
                            float one_minus_beta1, float beta2, float one_minus_beta2, float eps,
                            int group, void *stream);

/*
 * LayerNorm forward fused with the GS128 quantization of its output: the pre-norm of
 * every block (reference ksdraft/model/block.py:27-41, nn.LayerNorm ln_attn / ln_ffn)
 * followed by the Int8Linear A-operand quantization (ksdraft/kernels/linear.py:69,
 * quantize_last_dim). No reference counterpart as one call.
 *   x       (rows, d) of type x_dtype, row stride x_stride elements; 1 <= d <= 4096
 *   weight, bias  (d,) fp32 or NULL (weight 1, bias 0: elementwise_affine=False)
 *   y = (x - mean) * rstd * weight + bias, rstd = 1 / sqrt(biased var + eps), computed in
 *           fp32 and rounded to x_dtype; codes/scales = quantize_last_dim(y, 128):
 *   codes   (rows, d) int8; scales (rows, ceil(d/128)) fp16; group must be 128
 *   y_out   NULL or (rows, d) of x_dtype; mean_out, rstd_out NULL or (rows,) fp32
 */
int ksd_layernorm_quant(const void *x, int x_dtype, int64_t rows, int64_t d, int64_t x_stride,
                        const float *weight, const float *bias, float eps, int group,
                        int8_t *codes, uint16_t *scales, void *y_out, float *mean_out,
                        float *rstd_out, void *stream);

/*
 * §8(f) rank 4 — int8 embedding gather: rows of a per-row GS-quantized embedding table
 * (the tied table of reference ksdraft/model/draft.py:34, 51; quantized as the head's
 * weight, kernels/quant.py:30-52), dequantized by token id (nn.Embedding's lookup,
 * draft.py:68): out[i, :] = codes[ids[i], :] * scales[ids[i], :/group], exact in fp32.
 *   codes (V, d) int8, scales (V, ceil(d/group)) fp16, ids (n,) int64
 *   out (n, d) of out_dtype (KSD_F32, KSD_BF16, KSD_F16); an id outside [0, V) gives zeros
 */
int ksd_embedding_gather_int8(const int8_t *codes, const uint16_t *scales, const int64_t *ids,
                              int64_t n, int64_t V, int64_t d, int group, void *out,
                              int out_dtype, void *stream);

/*
 * G1 / G2 — W8A8 GEMM, "NT" layout: Y = dequant(A) . dequant(W)^T with the ordered
 * per-group contract
 *     acc = 0;  for g in 0..K/group-1:  acc = fmaf(float(P_g), sa[m,g]*sw[n,g], acc)
 * where P_g = sum_{k in g} A[m,k]*W[n,k] is exact int32 and sa*sw is exact in fp32.
 * Replaces _w8a8_gemm_kernel / w8a8_gemm (reference ksdraft/kernels/gemm.py:18-50, 53-90).
 *   a (M, K) int8, a_scales (M, K/group) fp16; w (N, K) int8, w_scales (N, K/group)
 *   K must be a multiple of 128 (the host wrapper zero-pads like gemm.py:71-73).
 *   bias    NULL or (N,) fp32, added in fp32 after the group sum (linear.py:71-72)
 *   y       (M, N) of type y_dtype (KSD_F32, KSD_BF16, KSD_F16, KSD_F16_SAT)
 */
int ksd_w8a8_gemm_nt(const int8_t *a, const uint16_t *a_scales, const int8_t *w,
                     const uint16_t *w_scales, int64_t M, int64_t N, int64_t K, int group,
                     const float *bias, void *y, int y_dtype, void *stream);

/*
 * G1 / G2 with split K — the same GEMM for launches with few output tiles (the dW of a
 * narrow layer: N x K output, K = tokens). For group 128, a shape with fewer than 192
 * tiles of 128 x 128 is split into S = ksd_w8a8_gemm_splits(M, N, K) contiguous K parts
 * (S = min(256 / tiles, K/128 / 8, 8), at least 1; a function of the shape only). Part p
 * covers the groups [floor(p*G/S), floor((p+1)*G/S)), G = K/128, each summed in the ordered
 * contract above from zero; the parts are then added in ascending order in fp32, then the
 * bias: y = ((part_0 + part_1) + ...) + bias. With S = 1 this is ksd_w8a8_gemm_nt exactly.
 * Replaces _w8a8_gemm_kernel / w8a8_gemm (reference ksdraft/kernels/gemm.py:18-50, 53-90).
 *   workspace  16-byte aligned fp32 scratch of at least S*M*N*4 bytes (unused when S = 1)
 */
int ksd_w8a8_gemm_splits(int64_t M, int64_t N, int64_t K, int group, int *splits);
/*
 * The general entry: split K as above, plus an optional residual operand added in the
 * store (the residual adds of reference ksdraft/model/block.py:39-41, h = x + linear(...)):
 *   residual  NULL or (M, N) of type y_dtype (KSD_F32, KSD_BF16 or KSD_F16; group 128):
 *             y = out(out(gemm + bias) + residual), one rounding to the output type per
 *             op as the torch add on tensors of that dtype; may alias y
 */
int ksd_w8a8_gemm_nt_ex(const int8_t *a, const uint16_t *a_scales, const int8_t *w,
                        const uint16_t *w_scales, int64_t M, int64_t N, int64_t K, int group,
                        const float *bias, const void *residual, void *y, int y_dtype,
                        float *workspace, int64_t workspace_bytes, void *stream);
int ksd_w8a8_gemm_nt_ws(const int8_t *a, const uint16_t *a_scales, const int8_t *w,
                        const uint16_t *w_scales, int64_t M, int64_t N, int64_t K, int group,
                        const float *bias, void *y, int y_dtype, float *workspace,
                        int64_t workspace_bytes, void *stream);

/*
 * Two independent group-128 GEMMs in one persistent launch: the dX = dY . W and
 * dW = dY^T . X pair of a linear layer's backward (reference ksdraft/kernels/ks3_int8.py:
 * 403-424, two w8a8_gemm calls of gemm.py:53-90), or any two GEMMs with no data dependence.
 * Problem i: y_i (M_i, N_i) = a_i (M_i, K_i) . w_i (N_i, K_i)^T in output type y_i_dtype
 * (KSD_F32, KSD_BF16 or KSD_F16), no bias, no residual, each with exactly the numeric
 * contract of ksd_w8a8_gemm_nt_ex on its own (including its K split). The workgroups take
 * balanced runs of both problems' tiles, so a problem with few long tiles (dW) shares the
 * device with one of many short tiles (dX) instead of leaving CUs idle.
 *   workspace  16-byte aligned fp32 scratch: the sum over split problems of S*M*N*4 bytes
 *              (NULL when neither problem splits)
 */
int ksd_w8a8_gemm_pair(const int8_t *a0, const uint16_t *a0_scales, const int8_t *w0,
                       const uint16_t *w0_scales, int64_t M0, int64_t N0, int64_t K0, void *y0,
                       int y0_dtype, const int8_t *a1, const uint16_t *a1_scales, const int8_t *w1,
                       const uint16_t *w1_scales, int64_t M1, int64_t N1, int64_t K1, void *y1,
                       int y1_dtype, float *workspace, int64_t workspace_bytes, void *stream);

/*
 * Test-only export of the exact int32 group partials P_g of the GEMM above
 * (the tl.dot result of reference ksdraft/kernels/gemm.py:42).
 *   partials (K/group, M, N) int32
 */
int ksd_w8a8_group_partials(const int8_t *a, const int8_t *w, int64_t M, int64_t N,
                            int64_t K, int group, int32_t *partials, void *stream);

/*
 * K6 (+ the requantization that follows it) — KS3 int8-mode spine features, rank 1, of
 * the composed contract: _spine_features 'int8' (reference ksdraft/kernels/ks3_int8.py:205-234)
 * on the coordinates of _project (:241-242), then quantize_last_dim(h, group) (:309, :330).
 *   coords            (M, F) fp16: fp16(GEMM(x, down)) clamped to +-65504 (ksd_w8a8_gemm_nt
 *                     with KSD_F16_SAT writes exactly this)
 *   spine_codes       (F, 6) int8, spine_scale (F,) fp16            (pack_spine, :87-92)
 *   warp_scale, warp_shift (F,) fp16: _warp_scalars(FP16), i.e. fp16(dequantize) of the
 *                     one-element warp groups                       (:158-165)
 *   tanh_lut          (256,) int8, 4-byte aligned                   (make_tanh_lut, :50-54)
 *   h                 NULL or (M, F) fp32: the features (_spine_features' return value)
 *   h_codes, h_scales NULL, or (M, F) int8 and (M, ceil(F/group)) fp16: quantize_last_dim(h)
 *   table             workspace, (F, 256) fp16, 16-byte aligned, overwritten: the per-chart
 *                     spine increment for each of the 256 LUT indices (it depends on the
 *                     chart's spine and warp parameters only)
 */
int ksd_ks3_spine_fwd(const uint16_t *coords, int64_t M, int64_t F, const int8_t *spine_codes,
                      const uint16_t *spine_scale, const uint16_t *warp_scale,
                      const uint16_t *warp_shift, const int8_t *tanh_lut, int group, float *h,
                      int8_t *h_codes, uint16_t *h_scales, uint16_t *table, void *stream);

/*
 * ksd_ks3_spine_fwd without the table workspace, for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). It has no counterpart in the reference. The per-chart table lives in a
 * library-owned device array of 8192 charts x 256 fp16 (4 MiB per GPU, held until the
 * process ends); F > 8192 returns KSD_EINVAL. The call allocates nothing. The stream must
 * belong to the current device. Calls that overlap on one GPU share the array and race.
 * Arguments and outputs otherwise as ksd_ks3_spine_fwd.
 */
int ksd_ks3_spine_fwd_noalloc(const uint16_t *coords, int64_t M, int64_t F,
                              const int8_t *spine_codes, const uint16_t *spine_scale,
                              const uint16_t *warp_scale, const uint16_t *warp_shift,
                              const int8_t *tanh_lut, int group, float *h, int8_t *h_codes,
                              uint16_t *h_scales, void *stream);

/*
 * K8 — the spine + requantization stage of project_fused / _fused_gemm_spine, 'int8' mode
 * (reference ksdraft/kernels/ks3_triton.py:47-75, 137-156 and 159-195), applied to the
 * fp32 down-projection accumulator. This is the reference's GPU-eval contract, which
 * differs from the composed one (fp32 coordinates, fp32 LUT index, no truncation, pre-ReLU
 * group pre-scale, exact squares, a second per-group requantization).
 *   acc        (M, F) fp32: w8a8_gemm(xq, xs, down_codes, down_scales)
 *   spine/warp buffers and tanh_lut as for ksd_ks3_spine_fwd
 *   h_codes (M, F) int8, h_scales (M, ceil(F/group)) fp16
 *   table      workspace, (F, 256) fp32, 16-byte aligned, overwritten (per-chart increments)
 */
int ksd_ks3_spine_fused(const float *acc, int64_t M, int64_t F, const int8_t *spine_codes,
                        const uint16_t *spine_scale, const uint16_t *warp_scale,
                        const uint16_t *warp_shift, const int8_t *tanh_lut, int group,
                        int8_t *h_codes, uint16_t *h_scales, float *table, void *stream);

/*
 * K8 — project_fused / _fused_gemm_spine, 'int8' mode, group 128, as one GEMM launch
 * (reference ksdraft/kernels/ks3_triton.py:100-156 and 159-195): the input-projection
 * GEMM xq . down_codes^T whose epilogue applies the spine, ReLU^2 and the per-group
 * requantization of ksd_ks3_spine_fused to each finished fp32 accumulator tile, so the
 * (M, F) accumulator never reaches memory. The accumulator is the ordered sum over all K
 * groups (K is never split). A small kernel fills the table workspace first.
 *   a, a_scales     (M, K) int8 codes, 16-byte aligned; (M, K/128) fp16 scales
 *   w, w_scales     (F, K) int8 down-projection codes, 16-byte aligned; (F, K/128) fp16
 *   K               a multiple of 128, > 0
 *   spine/warp buffers and tanh_lut as for ksd_ks3_spine_fwd
 *   group           128 (groups 32 and 64: ksd_w8a8_gemm_nt, then ksd_ks3_spine_fused)
 *   h_codes (M, F) int8, h_scales (M, ceil(F/128)) fp16
 *   table           workspace, (F, 256) fp32, 16-byte aligned, overwritten
 */
int ksd_ks3_project_fused(const int8_t *a, const uint16_t *a_scales, const int8_t *w,
                          const uint16_t *w_scales, int64_t M, int64_t F, int64_t K,
                          const int8_t *spine_codes, const uint16_t *spine_scale,
                          const uint16_t *warp_scale, const uint16_t *warp_shift,
                          const int8_t *tanh_lut, int group, int8_t *h_codes, uint16_t *h_scales,
                          float *table, void *stream);

/*
 * K6/K8, the 'fp32' and 'fp16' nonlinear modes — _spine_features (reference
 * ksdraft/kernels/ks3_int8.py:172-203, rank 1) followed by quantize_last_dim(h), or the
 * same stage of project_fused for NL = 0 / 1 (ksdraft/kernels/ks3_triton.py:76-98, 137-156).
 *   x          (M, F): KSD_F16 coordinates (composed path) or the KSD_F32 down-projection
 *              accumulator (project_fused contract; clamped to +-65504)
 *   spine_codes (F, 6) int8, spine_scale (F,) fp16: pack_spine's buffers
 *   warp_scale, warp_shift (F,) fp32: the dequantized warp scalars in the path's
 *              arithmetic (composed 'fp32': fp32; composed 'fp16' and both fused modes: fp16
 *              values), softplus/tanh already applied (KS3Int8Cell._warp_scalars)
 *   mode       0 = 'fp32', 1 = 'fp16'
 *   h          optional (M, F) fp32 features; h_codes (M, F) int8 + h_scales
 *              (M, ceil(F/group)) fp16 optional, together
 */
int ksd_ks3_spine_float(const void *x, int x_dtype, int64_t M, int64_t F,
                        const int8_t *spine_codes, const uint16_t *spine_scale,
                        const float *warp_scale, const float *warp_shift, int mode, int group,
                        float *h, int8_t *h_codes, uint16_t *h_scales, void *stream);

/*
 * Number of row blocks (the first dim of the partials workspace) ksd_ks3_vjp uses for M
 * rows: ceil(M / 512). Fixes the order of the column reductions.
 */
int ksd_ks3_vjp_row_blocks(int64_t M, int64_t *n_row_blocks);

/*
 * K10 steps 2-4 — the fp16 geometry VJP of _KS3Int8Train.backward, rank 1
 * (reference ksdraft/kernels/ks3_int8.py:354-401), with dc emitted directly as the two
 * int8 operands of the backward GEMMs.
 *   value      (M, F) fp16: fp16(GEMM(quant(g), quant(dequant(up)^T)))  (:345-352)
 *   coords     (M, F) fp16, as saved by the forward
 *   spine_codes, spine_scale, warp_scale, warp_shift as for ksd_ks3_spine_fwd;
 *              c_k = fp16(code_k * spine_scale)                           (:355-362)
 *   dc         NULL or (M, F) fp16: value + dmean                        (:398-401)
 *   dc_codes, dc_scales    NULL or (M, F) int8, (M, ceil(F/group)) fp16:
 *                          quantize_last_dim(dc, group)                   (:410)
 *   dct_codes, dct_scales  NULL or (F, M) int8, (F, ceil(M/group)) fp16:
 *                          quantize_last_dim(dc.t(), group)               (:417)
 *   partials   (n_row_blocks, 8, F) fp32 workspace: per-block column sums of the eight
 *              reduction terms d0..d5, dscale_t, 2*dshift_t (:379-388)
 */
int ksd_ks3_vjp(const uint16_t *value, const uint16_t *coords, int64_t M, int64_t F,
                const int8_t *spine_codes, const uint16_t *spine_scale, const uint16_t *warp_scale,
                const uint16_t *warp_shift, int group,
                uint16_t *dc, int8_t *dc_codes, uint16_t *dc_scales, int8_t *dct_codes,
                uint16_t *dct_scales, float *partials, int64_t n_row_blocks, void *stream);

/*
 * K10 step 3 — reduce the partials of ksd_ks3_vjp in fixed block order and apply the
 * reference's fp16 roundings and STE chain (reference ksdraft/kernels/ks3_int8.py:379-395).
 *   warp_scale_raw, warp_shift_raw (F,) fp32 master parameters
 *   sums    NULL or (8, F) fp32: the column sums before fp16 rounding
 *   dcoeff  (F, 6) fp16; dscale, dshift (F,) fp16
 */
int ksd_ks3_vjp_finalize(const float *partials, int64_t n_row_blocks, int64_t F,
                         const float *warp_scale_raw, const float *warp_shift_raw, float *sums,
                         uint16_t *dcoeff, uint16_t *dscale, uint16_t *dshift, void *stream);

/*
 * Test-only export: fp16 tanh of n fp16 values through the table the VJP reads,
 * i.e. torch.tanh on an fp16 tensor (reference ksdraft/kernels/ks3_int8.py:365-366).
 */
/*
 * K11 — _grad_handoff (reference ksdraft/kernels/ks3_int8.py:75-84) on the device: out =
 * fp32(fp16(t)) when every fp16(t[i]) is finite, else t, decided by *flag (int32, zeroed by
 * the caller; set to 1 here when an element overflows fp16 or is NaN). t, out (n,) fp32;
 * out may alias t.
 */
int ksd_grad_handoff(const float *t, int64_t n, int *flag, float *out, void *stream);

int ksd_ks3_tanh16(const uint16_t *x, int64_t n, uint16_t *y, void *stream);

/*
 * R1 — RosaMixer._shifted fused with the quantization of each projection input
 * (reference ksdraft/model/rosa.py:128-133, then Int8Linear's quantize_last_dim,
 * ksdraft/kernels/linear.py:69): for every token row r = (b, t) and feature i,
 *     m_in = prev + (x - prev) * sig_m,  prev = x[b, t-1] (0 at t = 0),
 * with x - prev rounded to x's dtype and the rest in fp32, then quantized per group.
 *   x        (B, T, d) of type x_dtype (KSD_F32, KSD_BF16, KSD_F16), dense
 *   sig_q/k/v (d,) fp32: torch.sigmoid(time_mix_q/k/v)
 *   *_codes  (B*T, d) int8; *_scales (B*T, ceil(d/group)) fp16
 */
int ksd_rosa_shift_quant(const void *x, int x_dtype, int64_t B, int64_t T, int64_t d,
                         const float *sig_q, const float *sig_k, const float *sig_v, int group,
                         int8_t *q_codes, uint16_t *q_scales, int8_t *k_codes, uint16_t *k_scales,
                         int8_t *v_codes, uint16_t *v_scales, void *stream);

/*
 * R1, training form — RosaMixer._shifted (reference ksdraft/model/rosa.py:128-133) fused
 * with the training quantization of each projection input: the row codes of the forward
 * GEMM (Int8Linear, ksdraft/kernels/linear.py:69) and dW's operand, the input transposed and
 * requantized along the tokens from those row codes (the recipe of
 * ksdraft/kernels/ks3_int8.py:417-420). Group 128. m = 0, 1, 2 is q, k, v:
 *   x            (B, T, d) of type x_dtype, dense, d % 8 == 0, 16-byte aligned
 *   sig_q/k/v    (d,) fp32: torch.sigmoid(time_mix_q/k/v), 16-byte aligned
 *   codes[m]     (B*T, d) int8;   scales[m]   (B*T, ceil(d/128)) fp16
 *   codes_t[m]   (d, B*T) int8;   scales_t[m] (d, ceil(B*T/128)) fp16
 */
int ksd_rosa_shift_quant_dual(const void *x, int x_dtype, int64_t B, int64_t T, int64_t d,
                              const float *sig_q, const float *sig_k, const float *sig_v,
                              int8_t *const *codes, uint16_t *const *scales,
                              int8_t *const *codes_t, uint16_t *const *scales_t, void *stream);

/*
 * Backward of the time shift of RosaMixer._shifted (reference ksdraft/model/rosa.py:128-133,
 * the autograd of its three lerps): given g_m = dL/dm_in (fp32, (B, T, d)),
 *   dx[r]     = sum_m g_m[r] sig_m + [t(r) + 1 < T] (g_m[r+1] - g_m[r+1] sig_m)   (x's dtype)
 *   dsig_m[i] = sum_r g_m[r, i] (x[r, i] - prev[r, i])
 * dsig comes as per-row-block partials (n_blocks, 3, d) fp32, n_blocks from
 * ksd_rosa_shift_backward_blocks; their sum over the first axis is dL/dsig_m.
 */
int ksd_rosa_shift_backward_blocks(int64_t B, int64_t T, int64_t *n_blocks);
int ksd_rosa_shift_backward(const void *x, int x_dtype, int64_t B, int64_t T, int64_t d,
                            const float *g_q, const float *g_k, const float *g_v,
                            const float *sig_q, const float *sig_k, const float *sig_v,
                            void *dx, float *dsig_partials, void *stream);

/*
 * The (x > 0) symbol bits of Rosa projections (reference ksdraft/model/rosa.py:156-158,
 * ksdraft/kernels/rosa_credit_gpu.py:68-70), packed per stream along T.
 *   x     (B, T, S) of type x_dtype, dense
 *   bits  (B, S, ceil(T/32)) uint32: bit b of word w is position 32w + b
 */
int ksd_rosa_pack_bits(const void *x, int x_dtype, int64_t B, int64_t T, int64_t S,
                       uint32_t *bits, void *stream);
/* The same for q, k and v of one shape in one launch (the three pack_bits of
 * rosa_credit_gpu.py:68-70). */
int ksd_rosa_pack_bits3(const void *q, const void *k, const void *v, int x_dtype, int64_t B,
                        int64_t T, int64_t S, uint32_t *q_bits, uint32_t *k_bits, uint32_t *v_bits,
                        void *stream);

/*
 * R2 — _match_payload_sign (reference ksdraft/model/rosa.py:40-98) on packed bits: for
 * each stream and position t the latest endpoint j < t of the longest common suffix of
 * q[..t] and k[..j], lengths capped at min(j + 1, lmax); sign = v[j + 1] ? +1 : -1, or -1
 * when nothing matches.
 *   q/k/v_bits  (n_streams, ceil(T/32)) uint32 as from ksd_rosa_pack_bits
 *   lmax        the reference's max_match_len rule, resolved by the caller (<= 63)
 *   sign        (n_streams, T) int8 in {-1, +1}
 *   match_j     NULL or (n_streams, T) int32 endpoint (-1 when nothing matches)
 *   T <= 65536.
 */
int ksd_rosa_match(const uint32_t *q_bits, const uint32_t *k_bits, const uint32_t *v_bits,
                   int64_t n_streams, int64_t T, int lmax, int8_t *sign, int32_t *match_j,
                   void *stream);

/*
 * R4 forward output — payload[s] * sign, transposed from (B, S, T) to (B, T, S)
 * (reference ksdraft/kernels/rosa_credit_gpu.py:75).
 *   out (B, T, S) of type out_dtype (KSD_F32, KSD_BF16, KSD_F16)
 */
int ksd_rosa_hard(const int8_t *sign, const float *payload, int64_t B, int64_t T, int64_t S,
                  void *out, int out_dtype, void *stream);

/*
 * R5 — exact first-order single-bit counterfactual credits of HardRosaGPU.backward
 * (reference ksdraft/kernels/rosa_credit_gpu.py:28-51, 78-104): for every q, k and v bit
 * of every stream, sum over positions t of (sign after flipping that bit - sign) * g(t),
 * g = grad[b, t, s] * payload[s]. No length guard: any T up to 65535.
 *   q/k/v_bits  (B*S, ceil(T/32)) uint32 from ksd_rosa_pack_bits
 *   match_j     (B*S, T) int32 endpoints from ksd_rosa_match
 *   grad        (B, T, S) fp32 upstream gradient of the hard output
 *   credits     (B*S, 3, T) fp32, written by the call (rows q, k, v)
 *   payload_partial (B*S,) fp32: sum over t of grad * sign per stream (fixed order)
 *   credit_sums (B*S, 3, T) int64 workspace (required). Every credit is an exact
 *               fixed-point sum of +-2 g(t) (g rounded once, at 2^-48 of the stream's
 *               largest |grad * payload|), so the credits are identical on every run. A
 *               stream whose g holds inf or NaN gets what the reference's dense sum over t
 *               of delta * g gives (rosa_credit_gpu.py:48): NaN where any g(t) is NaN or
 *               some infinite g(t) leaves the entry's sign unchanged (0 * inf), else +-inf
 *               (NaN if its infinite terms have both signs)
 * The credits buffer is the call's scratch until it returns (three launches on the stream:
 * per-stream set-up, the contributions, the conversion to fp32). For T <= 2048 the
 * contributions are formed by waves that take (stream, 64-position chunk) items from a
 * counter, so the cost of streams with long matches spreads over the whole device.
 */
int ksd_rosa_credits(const uint32_t *q_bits, const uint32_t *k_bits, const uint32_t *v_bits,
                     const int32_t *match_j, const float *grad, const float *payload, int64_t B,
                     int64_t T, int64_t S, int lmax, float *credits, float *payload_partial,
                     int64_t *credit_sums, void *stream);

/*
 * R5 projection-space gradients (reference ksdraft/kernels/rosa_credit_gpu.py:99-111):
 * g_x = credit * (1 - 2 * bit) * sigmoid(x) * (1 - sigmoid(x)) in x's dtype, and
 * d payload[s] = sum over b of payload_partial[b, s] (fixed order).
 *   q/k/v   (B, T, S) pre-bit projections of type dtype
 *   payload_partial (B*S,) fp32 from ksd_rosa_credits
 *   gq/gk/gv (B, T, S) of type dtype; gpayload (S,) fp32
 */
int ksd_rosa_credit_grads(const float *credits, const void *q, const void *k, const void *v,
                          int dtype, const float *payload_partial, int64_t B, int64_t T, int64_t S,
                          void *gq, void *gk, void *gv, float *gpayload, void *stream);

/*
 * The transfer-space term of distillation_losses (reference ksdraft/train/__init__.py:79-85),
 * per layer feature f (M, d) fp32 against e_hat = normalize(embedding[targets]) (M, d) fp32:
 *   ksd_transfer_cos   cos[r] = <f_r, e_r> / max(|f_r|, 1e-12), norm[r] = |f_r|
 *   ksd_transfer_grad  df = d/df of coef * (1 - cos) (F.normalize's gradient), and
 *                      grad_e (+)= -coef * f_r / max(|f_r|, 1e-12) (written when first != 0);
 *                      coef a device fp32 scalar (upstream gradient x weight / M)
 */
int ksd_transfer_cos(const float *f, const float *e_hat, int64_t M, int64_t d, float *cos_out,
                     float *norm_out, void *stream);
int ksd_transfer_grad(const float *f, const float *e_hat, const float *cos_in,
                      const float *norm_in, const float *coef, int64_t M, int64_t d, float *df,
                      float *grad_e, int first, void *stream);

/*
 * The gated update of the DSpine adjacent injection (reference ksdraft/model/spine.py:62-68):
 *   out = z + sigmoid(pre) * u,  pre = bias + zs[:, 0:64] . wc^T,  u = zs[:, 64:96] . wiu^T
 * zs (M, 96) fp32 = [gate_q.down(z) | gate_p.down(p_prev) | inject.down(p_prev)], wc (d, 64)
 * = [gate_q.up.weight | gate_p.up.weight], wiu (d, 32) = inject.up.weight, bias (d,) or NULL;
 * z, out (M, d) fp32. The backward writes dpre = g u s (1 - s) and du = g s (s = sigmoid(pre))
 * for the upstream gradient g, recomputing pre and u.
 */
int ksd_injection_update(const float *zs, const float *wc, const float *wiu, const float *bias,
                         const float *z, int64_t M, int64_t d, float *out, void *stream);
int ksd_injection_update_backward(const float *zs, const float *wc, const float *wiu,
                                  const float *bias, const float *grad_out, int64_t M, int64_t d,
                                  float *dpre, float *du, void *stream);

/*
 * nn.LayerNorm's backward (reference ksdraft/model/block.py:27-41) fused with the gradient
 * of the residual branch that reads the same input (the block's x + mixer(ln(x)),
 * block.py:39-41): dx = LN_backward(dy) + dres (dres may be NULL), and per-block partial
 * sums of dweight = sum dy xhat and dbias = sum dy, partials (n_blocks, 2, d) fp32 with
 * n_blocks from ksd_layernorm_backward_blocks; their sum over the first axis is (dw, db).
 * x, dy, dres, dx (M, d) fp32 with d a multiple of 256 (<= 2048), 16-byte aligned rows;
 * mean, rstd (M,) fp32 from the forward; weight (d,) fp32.
 */
int ksd_layernorm_backward_blocks(int64_t M, int64_t *n_blocks);
int ksd_layernorm_backward(const float *x, const float *dy, const float *dres, const float *mean,
                           const float *rstd, const float *weight, int64_t M, int64_t d,
                           float *dx, float *partials, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* KSDRAFT_AMD_H */
