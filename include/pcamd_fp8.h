/*
 * pcamd_fp8.h - C ABI of the MI355X (gfx950) FP8 hot path.
 *
 * One shared library, libpcamd_fp8.so, exports these functions. They take raw
 * device pointers, element strides (in elements, not bytes) and sizes, launch
 * asynchronously on the given hipStream_t (passed as void*), never allocate
 * device memory, keep no mutable global state and are reentrant. Every
 * function returns PCAMD_OK (0) or a negative status; pcamd_last_error()
 * returns a thread-local description of the most recent failure.
 *
 * Reference interfaces replaced (paths relative to xuOAO/practice_cuda):
 *   pcamd_quant_block   <- fp8_training/fp8_bench/impls/triton_per_block.py:60-150
 *                          (launches kernels/quant/per_block.py:6-48)
 *   pcamd_quant_block_dual <- no single counterpart: the block_m = 1 and
 *                          block_n = 1 calls of pcamd_quant_block on one tensor
 *   pcamd_quant_block_ex, pcamd_quant_block_dual_ex <- the two above with an
 *                          output store policy (flags)
 *   pcamd_quant_channel <- fp8_training/fp8_bench/impls/triton_per_channel.py:90-219
 *                          (launches kernels/quant/per_channel.py:35-102, :105-267)
 *   pcamd_quant_tensor  <- fp8_training/fp8_bench/impls/triton_per_tensor.py:28-95
 *                          and kernels/fp8_bmm/fp8_warper.py:9-77
 *   pcamd_bmm_quant_a   <- kernels/fp8_bmm/kernel/fp8_quant_bmm_fused_kernel.py:30-146
 *                          (its intent: the activation quantized inside the GEMM)
 *   pcamd_repack_fp8    <- the `.contiguous()` copies of the do_transpose_a /
 *                          do_transpose_b BMM variants
 *                          (impls/triton_per_block.py:254-272)
 *   pcamd_bmm_scaled    <- impls/triton_per_block.py:232-420 (block scales),
 *                          impls/triton_per_channel.py:271-427 (channel scales),
 *                          impls/triton_per_tensor.py:140-306 and
 *                          kernels/fp8_bmm/fp8_warper.py:79-129 (tensor scale)
 *   pcamd_bmm_scaled_mixed <- the same GEMM with an e5m2 and an e4m3fn operand:
 *                          fp8_training/fp8_bench/modules/bmm_linear.py:121-227
 *                          (custom op fp8_bench::bmm_linear_tma, called for
 *                          dgrad / wgrad at :402-410, :441-446 with torchao's
 *                          e5m2 grad_output and e4m3fn input / weight, :43-46)
 */
#ifndef PCAMD_FP8_H
#define PCAMD_FP8_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PCAMD_ABI_VERSION 4 /* 2: pcamd_bmm_scaled_mixed; 3: pcamd_quant_block_ex, pcamd_quant_block_dual_ex;
                              4: PCAMD_F64 scale arithmetic of pcamd_quant_tensor */

/* status codes */
#define PCAMD_OK 0
#define PCAMD_ERR_INVALID (-1)     /* bad argument (shape, stride, pointer, code) */
#define PCAMD_ERR_UNSUPPORTED (-2) /* valid but not implemented combination */
#define PCAMD_ERR_LAUNCH (-3)      /* hipGetLastError() after launch */

/* element type codes */
#define PCAMD_F32 0
#define PCAMD_BF16 1
#define PCAMD_F16 2
#define PCAMD_E4M3FN 3 /* OCP fp8 e4m3fn: max 448, no inf, NaN = 0x7f/0xff */
#define PCAMD_E5M2 4   /* OCP fp8 e5m2: max 57344, inf = 0x7c */
#define PCAMD_F64 5    /* scale arithmetic only (pcamd_quant_tensor) */

/* BMM scale modes */
#define PCAMD_SCALE_BLOCK 0   /* sa[b, m/qbm, k/qbk], sb[b, k/qbk, n/qbn] */
#define PCAMD_SCALE_CHANNEL 1 /* sa[b, m], sb[b, n] */
#define PCAMD_SCALE_TENSOR 2  /* sa[0] (and sb[0] when scales_are_quant) */

/* quantizer flags (the _ex entry points) */
#define PCAMD_QUANT_CACHED_OUTPUT 1 /* write y and the scales with ordinary, cache-allocating stores */

/* BMM epilogue activations */
#define PCAMD_ACT_NONE 0
#define PCAMD_ACT_GELU 1 /* exact: 0.5 x (1 + erf(x / sqrt 2)) */

int pcamd_abi_version(void);
const char *pcamd_last_error(void);

/*
 * Per-block quantization of x[batch, m, n] into fp8 y with one fp32 dequant
 * scale per block_m x block_n tile (block sizes are powers of two).
 * Per block: amax = max|x|; s = max(amax, eps); qs = fp8_max / s;
 * scale[b, i, j] = 1 / qs; y = fp8_rne(clamp(x * qs, -fp8_max, fp8_max)).
 * Replaces fp8_training/fp8_bench/impls/triton_per_block.py:60-150.
 */
int pcamd_quant_block(const void *x, int x_dtype, int64_t batch, int64_t m,
                      int64_t n, int64_t sxb, int64_t sxm, int64_t sxn,
                      void *y, int y_dtype, int64_t syb, int64_t sym,
                      int64_t syn, float *scale, int64_t ssb, int64_t ssm,
                      int64_t ssn, int64_t block_m, int64_t block_n,
                      float fp8_max, float eps, void *stream);

/*
 * Both block quantizations the block-scaled training recipe applies to one
 * tensor, from a single read of x: y_row / scale_row are exactly
 * pcamd_quant_block(block_m = 1, block_n = block) and y_col / scale_col
 * exactly pcamd_quant_block(block_m = block, block_n = 1). y_row has strides
 * syb, sym, syn and y_col its own ycb, ycm, ycn: the same layout, or stored
 * transposed (ycm = 1, element (r, c) at c * ycn + r), which makes it the
 * K-major operand of a GEMM reducing over m. scale_row is
 * [batch, m, ceil(n / block)] and scale_col [batch, ceil(m / block), n]
 * (strides in elements). One kernel serves row-contiguous x with block = 128
 * (transposed y_col: m and n multiples of 128, 16-byte aligned rows); other
 * layouts and block sizes run the two quantizers in turn. The reference has no
 * single counterpart: its per-block training module is unfinished
 * (fp8_training/fp8_bench/modules/per_block.py:13-67), and this pairs the
 * act/grad 1x128 quantization (impls/triton_per_block.py:60-150, block_m = 1)
 * with the wgrad re-quantization along the reduction dimension.
 */
int pcamd_quant_block_dual(const void *x, int x_dtype, int64_t batch,
                           int64_t m, int64_t n, int64_t sxb, int64_t sxm,
                           int64_t sxn, void *y_row, int64_t syb, int64_t sym,
                           int64_t syn, void *y_col, int64_t ycb, int64_t ycm,
                           int64_t ycn, int y_dtype, float *scale_row,
                           int64_t srb, int64_t srm, int64_t srn,
                           float *scale_col, int64_t scb, int64_t scm,
                           int64_t scn, int64_t block, float fp8_max, float eps,
                           void *stream);

/*
 * pcamd_quant_block and pcamd_quant_block_dual with flags. By default the
 * quantizers write their fp8 outputs and scales with non-temporal stores
 * (the fastest for a quantization on its own); PCAMD_QUANT_CACHED_OUTPUT
 * writes them with ordinary stores, which leave them in the GPU's caches
 * (the 256 MB memory-side cache included) for a kernel that reads them next,
 * e.g. the GEMM after the training layer's quantization. Bytes and scales
 * are the same either way; flags = 0 is exactly the call without _ex; other
 * bits return PCAMD_ERR_INVALID. The reference interfaces are those of
 * pcamd_quant_block / pcamd_quant_block_dual (the Triton kernels there pick
 * their own cache policy). Available from PCAMD_ABI_VERSION 3.
 */
int pcamd_quant_block_ex(const void *x, int x_dtype, int64_t batch, int64_t m,
                         int64_t n, int64_t sxb, int64_t sxm, int64_t sxn,
                         void *y, int y_dtype, int64_t syb, int64_t sym,
                         int64_t syn, float *scale, int64_t ssb, int64_t ssm,
                         int64_t ssn, int64_t block_m, int64_t block_n,
                         float fp8_max, float eps, int flags, void *stream);
int pcamd_quant_block_dual_ex(const void *x, int x_dtype, int64_t batch,
                              int64_t m, int64_t n, int64_t sxb, int64_t sxm,
                              int64_t sxn, void *y_row, int64_t syb,
                              int64_t sym, int64_t syn, void *y_col,
                              int64_t ycb, int64_t ycm, int64_t ycn,
                              int y_dtype, float *scale_row, int64_t srb,
                              int64_t srm, int64_t srn, float *scale_col,
                              int64_t scb, int64_t scm, int64_t scn,
                              int64_t block, float fp8_max, float eps,
                              int flags, void *stream);

/*
 * Per-channel quantization. channel_axis = -2: one scale per row (reduce over
 * n); channel_axis = -1: one scale per column (reduce over m).
 * s = max(amax, eps); qs = fp8_max / s; scale[b, c] = s / fp8_max;
 * y = fp8_rne(clamp(x * qs, -fp8_max, fp8_max)).
 * Replaces fp8_training/fp8_bench/impls/triton_per_channel.py:90-219.
 */
int pcamd_quant_channel(const void *x, int x_dtype, int64_t batch, int64_t m,
                        int64_t n, int64_t sxb, int64_t sxm, int64_t sxn,
                        void *y, int y_dtype, int64_t syb, int64_t sym,
                        int64_t syn, float *scale, int64_t ssb, int64_t ssc,
                        int channel_axis, float fp8_max, float eps,
                        void *stream);

/*
 * Per-tensor quantization: amax over the whole tensor, s = max(amax, eps),
 * qs = reciprocal(s) * fp8_max, scale[0] = reciprocal(qs),
 * y = fp8_rne(clamp(x * qs)). quant_scale_out (may be NULL) receives qs. Both
 * scalars are device fp32. scale_dtype (PCAMD_F32 / PCAMD_BF16 / PCAMD_F16) is
 * the dtype the scalar steps are rounded to: PCAMD_F32 for
 * fp8_training/fp8_bench/impls/triton_per_tensor.py:28-95; the input's dtype
 * for the legacy kernels/fp8_bmm/fp8_warper.py:9-77, whose torch ops on 0-d
 * tensors of the input's dtype round every step (the results are then
 * exactly representable in that dtype). PCAMD_F64 (from PCAMD_ABI_VERSION 4)
 * is torchao's tensorwise scale, which the reference's Float8BMMLinear
 * quantizes with (fp8_training/fp8_bench/modules/float8/float8_utils.py:
 * 45-48, used through float8_scaling_utils.py): qs = fp32(fp8_max /
 * max(fp64(amax), eps)) with the division in fp64, scale[0] = reciprocal(qs)
 * in fp32 (the reciprocal its scaled GEMMs take), then the same
 * fp8_rne(clamp(x * qs)) (float8_training_tensor.py:153-154).
 */
int pcamd_quant_tensor(const void *x, int x_dtype, int64_t batch, int64_t m,
                       int64_t n, int64_t sxb, int64_t sxm, int64_t sxn,
                       void *y, int y_dtype, int64_t syb, int64_t sym,
                       int64_t syn, float *scale, float *quant_scale_out,
                       float fp8_max, float eps, int scale_dtype,
                       void *stream);

/*
 * Scaled FP8 batched GEMM: c[b, m, n] = act(sum_k a[b, m, k] b[b, k, n] *
 * scale + bias[b, m, n]) with fp32 accumulation, a/b fp8 of the same code.
 * Block mode applies sa[b, m/qbm, kq] * sb[b, kq, n/qbn] to each qbk-wide
 * partial sum (qbk a multiple of 128); channel mode multiplies the full sum by
 * sa[b, m] * sb[b, n]; tensor mode by sa[0]. scales_are_quant = 1 means the
 * scales are quant scales and the product is inverted (1 / (sa * sb)).
 * bias may be NULL. Strides are in elements; a must be contiguous along k or
 * m, b along n or k, c and bias along n.
 */
int pcamd_bmm_scaled(const void *a, const void *b, int ab_dtype,
                     int64_t batch, int64_t m, int64_t n, int64_t k,
                     int64_t sab, int64_t sam, int64_t sak, int64_t sbb,
                     int64_t sbk, int64_t sbn, void *c, int c_dtype,
                     int64_t scb, int64_t scm, int64_t scn, const void *bias,
                     int bias_dtype, int64_t sbiasb, int64_t sbiasm,
                     int64_t sbiasn, const float *sa, int64_t ssab,
                     int64_t ssa1, int64_t ssa2, const float *sb,
                     int64_t ssbb, int64_t ssb1, int64_t ssb2, int scale_mode,
                     int scales_are_quant, int64_t qbm, int64_t qbk,
                     int64_t qbn, int activation, void *stream);

/*
 * pcamd_bmm_scaled with a format code per operand (a_dtype, b_dtype:
 * PCAMD_E4M3FN or PCAMD_E5M2, equal or not): the training recipe's e5m2
 * gradient times an e4m3fn weight or activation. Every other argument and
 * the math are those of pcamd_bmm_scaled, which is this call with a_dtype ==
 * b_dtype. Available from PCAMD_ABI_VERSION 2.
 */
int pcamd_bmm_scaled_mixed(const void *a, int a_dtype, const void *b,
                           int b_dtype, int64_t batch, int64_t m, int64_t n,
                           int64_t k, int64_t sab, int64_t sam, int64_t sak,
                           int64_t sbb, int64_t sbk, int64_t sbn, void *c,
                           int c_dtype, int64_t scb, int64_t scm, int64_t scn,
                           const void *bias, int bias_dtype, int64_t sbiasb,
                           int64_t sbiasm, int64_t sbiasn, const float *sa,
                           int64_t ssab, int64_t ssa1, int64_t ssa2,
                           const float *sb, int64_t ssbb, int64_t ssb1,
                           int64_t ssb2, int scale_mode, int scales_are_quant,
                           int64_t qbm, int64_t qbk, int64_t qbn,
                           int activation, void *stream);

/*
 * Block-scaled FP8 GEMM with the activation quantization fused into the K
 * loop: a (bf16 or fp16, [batch, m, k], contiguous along k with 16-byte
 * aligned rows) is quantized in 1 x 128 groups along k inside the kernel -
 * bytes and dequant scales exactly those of pcamd_quant_block(block_m = 1,
 * block_n = 128, fp8_max, eps) into ab_dtype - and multiplied by the fp8 b
 * (block scales sb[b, k/128, n/qbn], quant-K block 128) as pcamd_bmm_scaled
 * would with those A scales. qa_out / sa_out (both or neither; qa_out
 * contiguous along k, 8-byte aligned rows) receive the quantized A and its
 * scales [batch, m, k/128]. k must be a positive multiple of 128; other
 * layouts return PCAMD_ERR_UNSUPPORTED (quantize, then pcamd_bmm_scaled).
 * The call pays off for n <= 256 (with n a multiple of 16, k a multiple of
 * 256 and quant-N blocks of at least 128, one workgroup holds every column
 * and reads a once; any bias, activation and output type); wider products quantize each 128-row block of a once per
 * 256-column tile of c, where quantizing first and then multiplying is
 * faster. Replaces the intent of the reference's fused quant + BMM kernel
 * (kernels/fp8_bmm/kernel/fp8_quant_bmm_fused_kernel.py:30-146), whose
 * per-tile scale helper is unfinished there, with the per-block recipe of
 * fp8_training/fp8_bench/impls/triton_per_block.py:60-150 (A) and :232-420
 * (GEMM).
 */
int pcamd_bmm_quant_a(const void *a, int a_dtype, const void *b, int ab_dtype,
                      int64_t batch, int64_t m, int64_t n, int64_t k,
                      int64_t sab, int64_t sam, int64_t sak, int64_t sbb,
                      int64_t sbk, int64_t sbn, void *c, int c_dtype,
                      int64_t scb, int64_t scm, int64_t scn, const void *bias,
                      int bias_dtype, int64_t sbiasb, int64_t sbiasm,
                      int64_t sbiasn, const float *sb, int64_t ssbb,
                      int64_t ssb1, int64_t ssb2, int64_t qbn, void *qa_out,
                      int64_t sqab, int64_t sqam, int64_t sqak, float *sa_out,
                      int64_t soab, int64_t soam, int64_t soak, float fp8_max,
                      float eps, int activation, void *stream);

/*
 * Transposing byte copy of an fp8 tensor: y[b, r, c] = x[b, r, c] for a
 * view x contiguous along rows (sxr == 1) into a view y contiguous along
 * columns (syc == 1); strides in elements (= bytes). This is the copy of the
 * BMM wrappers' transpose variants - an M-major A made K-major, or an
 * N-major B made K-major - that the reference makes with `.contiguous()`
 * on the strided view (fp8_training/fp8_bench/impls/triton_per_block.py:
 * 254-272). Other stride patterns return PCAMD_ERR_UNSUPPORTED.
 */
int pcamd_repack_fp8(const void *x, int64_t batch, int64_t rows,
                     int64_t cols, int64_t sxb, int64_t sxr, int64_t sxc,
                     void *y, int64_t syb, int64_t syr, int64_t syc,
                     void *stream);

#ifdef __cplusplus
}
#endif

#endif /* PCAMD_FP8_H */
