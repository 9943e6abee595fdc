/* tcfp_hip.h -- C ABI of the MI355X-native TCFP-12 kernel library
 * (libtcfp_hip.so, hand-written HIP for gfx950).
 *
 * Every entry point takes raw device pointers, int64 sizes/leading
 * dimensions and a hipStream_t (passed as void*), enqueues its kernels on
 * that stream and returns a status code.  No torch types cross this
 * boundary; the library does not allocate device memory.  Scalars that the
 * reference keeps as (1,) fp32 device tensors (per-tensor inverse scales)
 * are device pointers here too, so no call synchronises with the host.
 *
 * Layout conventions (all row-major, innermost index contiguous):
 *   activations  [M, K]        (K = in_features)
 *   weights      [N, K]        (nn.Linear layout, N = out_features)
 *   block exps   [K/bs, rows]  int8, scale = 2^e (reference layout,
 *                              tcfp/kernels.py:1700)
 *
 * Each declaration cites the reference interface (path:line under the
 * reference tree) whose behaviour it replaces.
 */
#ifndef TCFP_HIP_H_
#define TCFP_HIP_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- enums ------------------------------------------------------------- */
#define TCFP_FP8_E4M3 0 /* OCP float8_e4m3fn */
#define TCFP_FP8_E5M2 1 /* OCP float8_e5m2   */

#define TCFP_DTYPE_F32 0
#define TCFP_DTYPE_BF16 1

/* ---- status codes ------------------------------------------------------ */
#define TCFP_OK 0
#define TCFP_ERR_SHAPE 1     /* bad size / leading dimension / divisibility */
#define TCFP_ERR_DTYPE 2     /* unsupported dtype / format code            */
#define TCFP_ERR_ALIGN 3     /* pointer or leading dimension misaligned    */
#define TCFP_ERR_HIP 4       /* a HIP runtime call failed                  */
#define TCFP_ERR_WORKSPACE 5 /* workspace missing or too small             */
#define TCFP_ERR_EXCLUSIVE 6 /* mutually exclusive options requested       */
#define TCFP_ERR_DEVICE 7    /* stream not on the current device           */

/* Human-readable text for a status code (static storage). */
const char* tcfp_status_string(int status);

/* Bytes of device workspace the per-tensor reductions need.  Reducing
 * kernels store one partial maximum per workgroup there and the kernel that
 * consumes the scale reduces them again.  Its contents need no
 * initialisation.  Calls that may run concurrently (different streams) need different
 * workspaces; calls ordered on one stream can share one. */
size_t tcfp_workspace_bytes(void);

/* ---- per-tensor quantisation ------------------------------------------- */

/* Per-tensor FP8 quantisation of x [rows, cols] (f32 or bf16).
 * Replaces tcfp.core.to_fp8_e4m3 (tcfp/core.py:85-106) and to_fp8_e5m2
 * (tcfp/core.py:137-158), used for activations at tcfp/nn/__init__.py:390
 * and gradients at :494.
 *   scale_in  optional device fp32 scalar: use it instead of the amax rule.
 *   q         [rows, cols] fp8 codes; may be NULL when q_t is given and
 *             cols % 8 == 0 (only the transposed copy is written).
 *   q_t       optional [cols, rows] transposed codes (wgrad operand).
 *   scale_out optional device fp32 scalar receiving the scale used.
 *   inv_out   device fp32 scalar receiving 1/scale.
 * Without scale_in: amax = max|x| (NaN-propagating), clamped at 1e-12,
 * scale = reciprocal(amax) * FP8_MAX with both ops rounded to x's dtype,
 * q = RNE(clamp(x * scale, +-FP8_MAX)), inv = 1/scale (IEEE fp32). */
int tcfp_quantize_per_tensor(const void* x, int x_dtype, int64_t rows, int64_t cols,
                             int fp8_fmt, const float* scale_in, uint8_t* q, uint8_t* q_t,
                             float* scale_out, float* inv_out, void* workspace,
                             void* stream);

/* Per-tensor FP8 E4M3 quantisation with stochastic rounding.  Replaces
 * tcfp.core.to_fp8_e4m3_sr (tcfp/core.py:109-134), which applies
 * stochastic_round_to_fp8_e4m3 (tcfp/core.py:418-464) to the scaled values;
 * with *scale_in == 1 it is that function on already clamped values.
 *   scale as tcfp_quantize_per_tensor (amax rule, or scale_in);
 *   c = clamp(x * scale, +-448); code = RNE(c) or its neighbour toward c,
 *   the neighbour with probability |c - RNE(c)| / gap (the reference's
 *   candidate rule: nudge 2^-7, retry 0.25 * max(|lo|, 2^-6)); exact values
 *   keep their code.  Uniforms from Philox4x32-10 keyed by (seed, offset).
 *   q [rows, cols] (8-byte aligned when >= 8 elements), inv_out (and the
 *   optional scale_out) device fp32 scalars. */
int tcfp_quantize_per_tensor_sr(const void* x, int x_dtype, int64_t rows, int64_t cols,
                                const float* scale_in, uint64_t seed, uint64_t offset,
                                uint8_t* q, float* scale_out, float* inv_out, void* workspace,
                                void* stream);

/* Power-of-two block scales.  Replaces tcfp.core.compute_block_scales
 * (tcfp/core.py:221-252): for each run of `block` elements of the rows of
 * x [rows, cols] (f32 or bf16), scale = 2^ceil(log2(max(amax, 1e-12) /
 * fp8_max)) with every step rounded to x's dtype as torch rounds it (bf16:
 * the quotient and its log2 are rounded to bf16 before the ceil), written
 * in x's dtype to scales [rows, cols / block] (row-major: the reference's
 * (..., D // block) layout, not the kernels' [K / block, rows]).  NaN
 * propagates.  cols % block == 0, fp8_max > 0. */
int tcfp_block_scales(const void* x, int x_dtype, int64_t rows, int64_t cols, int block,
                      float fp8_max, void* scales, void* stream);

/* Per-tensor quantisation that also returns the column sums of x
 * (col_sum [cols] fp32 = sum over rows), read in the same pass as the
 * amax.  For the gradient this is the bias gradient the reference computes
 * separately as grad_2d.sum(0) (tcfp/nn/__init__.py:558) next to the E5M2
 * quantisation at :494.  Scale rule as tcfp_quantize_per_tensor (no
 * explicit scale).  cols % 8 == 0; colsum_ws holds
 * tcfp_colsum_workspace_bytes(rows, cols) bytes of scratch (16-byte
 * aligned).  The sums are fp32 in one fixed order, shared by every entry
 * point that returns column sums: per 64-row group q and column c,
 * y[l] = x[64q + l][c] + x[64q + 32 + l][c] (l < 32; missing rows +0), then
 * the halving folds y[l] += y[l + d] for l < d, d = 16, 8, 4, 2, 1, give the
 * group sum y[0]; a finalising pass adds the group sums (its own fixed
 * order: eight interleaved lanes of four accumulators each, then the lanes
 * in turn). */
size_t tcfp_colsum_workspace_bytes(int64_t rows, int64_t cols);
int tcfp_quantize_per_tensor_colsum(const void* x, int x_dtype, int64_t rows, int64_t cols,
                                    int fp8_fmt, uint8_t* q, uint8_t* q_t, float* inv_out,
                                    float* col_sum, void* workspace, void* colsum_ws,
                                    size_t colsum_ws_bytes, void* stream);

/* Producer-fused per-tensor quantisation across a GELU (erf form) between
 * two TCFP-12 layers.  No single reference function: it replaces the
 * model's torch GELU followed by the next layer's to_fp8_e4m3 of its input
 * (tcfp/nn/__init__.py:390 on the GELU output).  h [rows, cols] fp32 is the
 * first layer's output; gelu(h) (as torch's GELU computes it, bit for bit)
 * is quantised by the tcfp_quantize_per_tensor rule (q, optional transposed
 * q_t, inv_out).  Written when not NULL: act = gelu(h) and dgelu = the
 * derivative factor of torch's GELU backward (cdf(h) + h * pdf(h), so that
 * dy * dgelu is the backward bit for bit), both [rows, cols] fp32.  One
 * amax pass, then a quantising pass that recomputes gelu(h) from h.
 * h, act, dgelu 16-byte aligned.  cols % 8 != 0 takes a flat path that
 * needs act (written by the amax pass) and no dgelu. */
int tcfp_gelu_quantize_per_tensor(const float* h, int64_t rows, int64_t cols, int fp8_fmt,
                                  float* act, float* dgelu, uint8_t* q, uint8_t* q_t,
                                  float* inv_out, void* workspace, void* stream);

/* The backward counterpart: grad = dGELU/dh * dy (fp32, bit for bit as
 * torch's GELU backward) is written in the same pass that takes its amax and
 * its column sums, then quantised as tcfp_quantize_per_tensor_colsum does
 * (tcfp/nn/__init__.py:494 and :558 applied to the GELU's input gradient,
 * which the reference gets from torch's GELU backward).  dy, h, grad
 * [rows, cols] fp32, cols % 8 == 0; colsum_ws as for
 * tcfp_quantize_per_tensor_colsum.  dy and grad may be the same buffer.
 * col_sum may be NULL (no sums; colsum_ws unused). */
int tcfp_gelu_backward_quantize_per_tensor_colsum(const float* dy, const float* h, int64_t rows,
                                                  int64_t cols, int fp8_fmt, float* grad,
                                                  uint8_t* q, uint8_t* q_t, float* inv_out,
                                                  float* col_sum, void* workspace,
                                                  void* colsum_ws, size_t colsum_ws_bytes,
                                                  void* stream);

/* The first layer of a TCFP-12 -> GELU -> TCFP-12 pair with the GELU's
 * amax taken from the GEMM's epilogue.  No single reference function: it
 * replaces fused_dual_gemm_forward (tcfp/kernels.py:1545-1601) of the first
 * layer, the model's torch GELU and the second layer's to_fp8 of its input
 * (tcfp/nn/__init__.py:390 on the GELU output).
 *   h = s_a*s_hi * A B_hi^T + s_a*s_lo * A B_lo^T (+ bias), [m, n] fp32
 *   contiguous, written exactly as tcfp_dual_gemm writes it;
 *   q (+ q_t) / inv_out / act / dgelu: as tcfp_gelu_quantize_per_tensor
 *   gives them from h (act and dgelu optional).
 * Operands and scales as tcfp_dual_gemm (b_lo may be NULL).  On the
 * persistent launch's shapes (m % 256 == 0, n % 128 == 0, k % 128 == 0,
 * k > 128, more 256 x 128 tiles than CUs, fp8 operands, b_lo given) the
 * epilogue records the max of h, and max |gelu(h)| is gelu(max h) whenever
 * the premises of that rule hold: gelu non-decreasing on [+0, +inf] and
 * |gelu| below a bound T on the negative numbers, both checked over every
 * fp32 input once per device (the first call launches the check on its
 * stream, unless the stream is being captured), and gelu(max h) >= T with
 * no NaN or -inf in h.  Otherwise a full GELU amax pass runs on the device
 * in its place.  On any other shape this is tcfp_dual_gemm followed by
 * tcfp_gelu_quantize_per_tensor.  Same bits in every case. */
int tcfp_dual_gemm_gelu_quantize(const uint8_t* a, int a_fmt, int64_t lda, const uint8_t* b_hi,
                                 const uint8_t* b_lo, int b_fmt, int64_t ldb, int64_t m,
                                 int64_t n, int64_t k, const float* s_a, const float* s_hi,
                                 const float* s_lo, const float* bias, float* h, float* act,
                                 float* dgelu, int fp8_fmt, uint8_t* q, uint8_t* q_t,
                                 float* inv_out, void* workspace, void* stream);

/* State of the premise check of tcfp_dual_gemm_gelu_quantize's amax rule on
 * the current device: checked (the check has completed), holds (gelu is
 * non-decreasing on [+0, +inf] for this build), bound (T, the largest
 * |gelu| over the negative numbers).  Synchronous (a copy from the device).
 * No reference counterpart. */
int tcfp_gelu_amax_rule_status(int* checked, int* holds, float* bound);

/* The backward counterpart, with the GELU backward in the dgrad GEMM's
 * epilogue: replaces fused_dual_gemm_backward_dx (tcfp/kernels.py:1604-1666)
 * of the second layer, torch's GELU backward, and the first layer's E5M2
 * gradient quantisation and bias gradient (tcfp/nn/__init__.py:494, :558).
 *   grad = (s_a*s_hi * A B_hi^T + s_a*s_lo * A B_lo^T) * dgelu, [m, n] fp32
 *   contiguous (A the quantised output gradient, B the transposed weight
 *   codes, dgelu the derivative factors tcfp_dual_gemm_gelu_quantize wrote):
 *   torch's GELU backward of tcfp_dual_gemm's output, bit for bit;
 *   q (+ q_t) / inv_out / col_sum: grad quantised as
 *   tcfp_quantize_per_tensor_colsum quantises it.
 * n % 8 == 0; col_sum may be NULL; q may be NULL when q_t is given;
 * colsum_ws as for tcfp_quantize_per_tensor_colsum.  On the persistent
 * launch's shapes (the 256 x 64 tile with the factors staged in LDS for
 * k <= 2048, else the 256 x 128 tile) the
 * epilogue writes grad with its per-workgroup maxima and 64-row column
 * partials; otherwise the GEMM, a multiply-and-amax pass and the
 * quantising pass run in turn.  Same bits either way. */
int tcfp_dual_gemm_dgelu_quantize_colsum(const uint8_t* a, int a_fmt, int64_t lda,
                                         const uint8_t* b_hi, const uint8_t* b_lo, int b_fmt,
                                         int64_t ldb, int64_t m, int64_t n, int64_t k,
                                         const float* s_a, const float* s_hi, const float* s_lo,
                                         const float* dgelu, float* grad, int fp8_fmt,
                                         uint8_t* q, uint8_t* q_t, float* inv_out,
                                         float* col_sum, void* workspace, void* colsum_ws,
                                         size_t colsum_ws_bytes, void* stream);

/* ---- batched per-tensor quantisation ------------------------------------ */

#define TCFP_JOB_DUAL 0 /* dual quantisation of a weight (W + EF -> W_hi, W_lo)  */
#define TCFP_JOB_ACT 1  /* per-tensor quantisation of an activation / gradient */

/* One tensor of tcfp_quantize_batch.  x [rows, cols] (f32 or bf16),
 * cols % 8 == 0, rows, cols > 0.
 *   TCFP_JOB_DUAL: as tcfp_dual_quantize_per_tensor without stochastic
 *     rounding: ef optional (updated in place when update_ef), q / q_lo the
 *     W_hi / W_lo codes, inv / inv_lo their inverse scales, q_t / q_lo_t
 *     optional transposed copies.
 *   TCFP_JOB_ACT: as tcfp_quantize_per_tensor without an explicit scale:
 *     fp8_fmt, q (may be NULL when q_t is given), q_t optional, inv. */
typedef struct tcfp_quant_job {
  int kind;
  const void* x;
  int x_dtype;
  int64_t rows;
  int64_t cols;
  float* ef;
  int update_ef;
  int fp8_fmt;
  uint8_t* q;
  uint8_t* q_t;
  float* inv;
  uint8_t* q_lo;
  uint8_t* q_lo_t;
  float* inv_lo;
} tcfp_quant_job;

/* Workspace bytes tcfp_quantize_batch needs for `count` jobs. */
size_t tcfp_quantize_batch_workspace_bytes(int count);

/* Up to 4 independent per-tensor quantisations in three launches in all,
 * instead of two (activation) or three (weight) each: the amax passes of
 * every job share one launch, the W_hi passes of the weights a second, and
 * the final passes (W_lo + EF + transposed codes; activation codes) a third.
 * Results are those of the single-tensor entry points, bit for bit.  No
 * reference counterpart: it serves TCFPMLP's forward, whose two weights and
 * input the reference quantises one call at a time (tcfp/nn/__init__.py:
 * 343-390, once per layer).  workspace: tcfp_quantize_batch_workspace_bytes
 * (count) bytes, any contents; jobs must not alias each other's outputs. */
int tcfp_quantize_batch(int count, const tcfp_quant_job* jobs, void* workspace,
                        size_t workspace_bytes, void* stream);

/* Tuning switch of tcfp_dual_quantize_per_tensor (and its workspace-free
 * variant) without delayed or NF-aware scaling, on tensors of 2^23 elements
 * or more (no counterpart in the reference): on = 1 (default) keeps the
 * candidates for the residual amax during the amax pass and skips the full
 * residual pass whenever they decide it; on = 0 always runs the full pass.
 * Results do not depend on it.  While the candidates are kept, the
 * caller's w_lo buffer (all n * k bytes of it, as up to n * k / 4 fp32
 * values) holds them between the amax pass and the W_lo pass (see the w_lo
 * note of tcfp_dual_quantize_per_tensor). */
int tcfp_dual_quantize_set_candidates(int on);

/* Per-tensor dual quantisation with optional error feedback.
 * Three launches (amax; W_hi + residual amax; W_lo + EF + transposed
 * codes), each re-reading W and EF.
 * Replaces the body of _TCFP12TensorCoreFunction.forward that builds
 * W_hi/W_lo (tcfp/nn/__init__.py:343-383, with ErrorFeedbackState
 * get_error/update_error, tcfp/core.py:320-326).
 *   w       [n, k] f32 or bf16 master weight.
 *   ef      optional [n, k] fp32 error buffer; read as e_prev, and if
 *           update_ef != 0 overwritten in place with
 *           e_new = W - (hi*inv_hi + lo*inv_lo).
 *   stochastic_lo  round W_lo stochastically (SRR, tcfp/core.py:109-134,
 *           418-464) with Philox4x32-10 keyed by (seed, offset).
 *   w_hi_t, w_lo_t optional [k, n] transposed codes (dgrad operands).
 *   w_lo    is also scratch during the call: on tensors of 2^23 elements or
 *           more (candidate pass on, the default; no delayed or NF-aware
 *           scaling) the amax pass stores fp32 candidate values in it, which
 *           the final pass overwrites with the W_lo codes.  So w_lo must not
 *           alias any input (w, ef) and must not be read, on any stream,
 *           before the call's work on `stream` has completed; a persistent
 *           w_lo buffer shared with concurrent readers needs
 *           tcfp_dual_quantize_set_candidates(0). */
int tcfp_dual_quantize_per_tensor(const void* w, int w_dtype, int64_t n, int64_t k,
                                  float* ef, int update_ef, int stochastic_lo,
                                  uint64_t seed, uint64_t offset, uint8_t* w_hi,
                                  uint8_t* w_lo, float* inv_hi, float* inv_lo,
                                  uint8_t* w_hi_t, uint8_t* w_lo_t, void* workspace,
                                  void* stream);

/* tcfp_dual_quantize_per_tensor without the workspace argument, for callers
 * that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc).  No counterpart in the
 * reference.  Same arguments, kernels and results (bit for bit) as
 * tcfp_dual_quantize_per_tensor; the reduction partials live in a
 * library-owned static device array of 49408 bytes per GPU (held until the
 * process ends; the per-tensor reductions need at most that for any weight
 * size, so no size is rejected for scratch).  The call allocates nothing:
 * no hipMalloc/hipFree, no allocating library routine; its first call on a
 * device looks up the array's device address once.  The stream must belong
 * to the current device (TCFP_ERR_DEVICE otherwise).  Every call on one GPU
 * shares that array: calls that overlap on one GPU (e.g. on two streams
 * without ordering between them) race and give wrong scales; calls ordered
 * on one stream are safe.  w_lo is scratch during the call as in
 * tcfp_dual_quantize_per_tensor (same aliasing rule). */
int tcfp_dual_quantize_per_tensor_noalloc(const void* w, int w_dtype, int64_t n, int64_t k,
                                          float* ef, int update_ef, int stochastic_lo,
                                          uint64_t seed, uint64_t offset, uint8_t* w_hi,
                                          uint8_t* w_lo, float* inv_hi, float* inv_lo,
                                          uint8_t* w_hi_t, uint8_t* w_lo_t, void* stream);

/* Per-tensor dual quantisation with delayed ("predictive dual-track")
 * scaling: _TCFP12TensorCoreFunction.forward with delayed_scaling=True
 * (tcfp/nn/__init__.py:250-309, 343-383; ErrorFeedbackState tcfp/core.py:
 * 341-403).
 *   W_hi scale = 448 / D with D = a*amax_prev + b*amax (EMA, three rounded
 *   fp32 ops; D = amax on the first call, amax_prev == NULL), amax =
 *   max|W + ef| clamped to 1e-12.
 *   validate != 0: W_lo scale from the measured residual amax A, and the
 *   ratio EMA r' = a*ratio_prev + b*(A / D) (r' = A / D when ratio_prev ==
 *   NULL) is written to *ratio_out.
 *   validate == 0: W_lo scale = 448 / max(D * ratio_prev, 1e-12) (D / 8
 *   when ratio_prev == NULL); no residual reduction, so the weight is read
 *   twice instead of three times.
 *   a = fp32(ema_decay), b = fp32(1 - ema_decay) as the caller's Python
 *   float arithmetic rounds them.  *amax_out receives D.  The previous
 *   state and the outputs must not alias.  Otherwise as
 *   tcfp_dual_quantize_per_tensor (no stochastic rounding: the reference
 *   disables delayed scaling under SRR). */
int tcfp_dual_quantize_per_tensor_delayed(const void* w, int w_dtype, int64_t n, int64_t k,
                                          float* ef, int update_ef, const float* amax_prev,
                                          const float* ratio_prev, float ema_decay,
                                          float one_minus_decay, int validate, float* amax_out,
                                          float* ratio_out, uint8_t* w_hi, uint8_t* w_lo,
                                          float* inv_hi, float* inv_lo, uint8_t* w_hi_t,
                                          uint8_t* w_lo_t, void* workspace, void* stream);

/* Per-tensor dual quantisation with NF-aware (sigma-based) W_hi scaling:
 * _TCFP12TensorCoreFunction.forward with nf_aware_scaling=True
 * (tcfp/nn/__init__.py:350-360 -> to_fp8_e4m3_nf_aware, tcfp/core.py:
 * 161-193; with delayed scaling, _delayed_quantise_w_hi's NF branch,
 * :263-275).
 *   W_hi target T = fp32(sigma_factor) * S, S = std(W + ef) (unbiased,
 *   computed in fp64 and rounded once to fp32, clamped to 1e-12); T = the
 *   clamped amax when S < 1e-6.  Fewer than two elements give S = NaN, as
 *   torch.std does.  W_hi scale = 448 / T (values beyond +-448 saturate).
 *   stochastic_hi != 0 rounds the W_hi codes stochastically (Philox4x32-10
 *   keyed by seed / offset, counters apart from W_lo's); stochastic_lo as in
 *   tcfp_dual_quantize_per_tensor.
 *   amax_out != NULL selects delayed scaling with the arguments of
 *   tcfp_dual_quantize_per_tensor_delayed: T replaces the amax in the EMA
 *   and the residual prediction uses the delayed T.
 *   Empty weights return TCFP_ERR_SHAPE (the reference's residual amax of
 *   an empty tensor raises). */
int tcfp_dual_quantize_per_tensor_nf(const void* w, int w_dtype, int64_t n, int64_t k, float* ef,
                                     int update_ef, float sigma_factor, int stochastic_hi,
                                     int stochastic_lo, uint64_t seed, uint64_t offset,
                                     const float* amax_prev, const float* ratio_prev,
                                     float ema_decay, float one_minus_decay, int validate,
                                     float* amax_out, float* ratio_out, uint8_t* w_hi,
                                     uint8_t* w_lo, float* inv_hi, float* inv_lo,
                                     uint8_t* w_hi_t, uint8_t* w_lo_t, void* workspace,
                                     void* stream);

/* ---- per-block quantisation -------------------------------------------- */

/* Per-(row, K-block) FP8 quantisation.  Replaces block_quantize_fp8
 * (tcfp/kernels.py:1675-1722, kernel :205-275).
 *   x [m, k] f32/bf16; block in {32, 64, 128}; k % block == 0.
 *   q [m, k] codes; exps [k/block, m] int8 with
 *   e = max(ceil(log2(max(amax,1e-12)/FP8_MAX)), -126), q = RNE(clamp(x/2^e)). */
int tcfp_block_quantize(const void* x, int x_dtype, int64_t m, int64_t k, int block,
                        int fp8_fmt, uint8_t* q, int8_t* exps, void* stream);

/* Fused block dual quantisation.  Replaces fused_dual_quantize_fp8
 * (tcfp/kernels.py:1749-1875, kernel :288-459) including the error update
 * the reference performs afterwards (:1867-1873), in one pass.
 *   ef      optional [n, k] fp32 buffer, read then overwritten in place
 *           with W - deq(hi) - deq(lo) unless update_ef == 0.
 *   e_lo    holds -128 for blocks whose residual amax < 1e-12.
 *   stochastic_lo and ef are mutually exclusive (TCFP_ERR_EXCLUSIVE). */
int tcfp_block_dual_quantize(const void* w, int w_dtype, int64_t n, int64_t k, int block,
                             float* ef, int update_ef, int stochastic_lo, uint64_t seed,
                             uint64_t offset, uint8_t* w_hi, uint8_t* w_lo, int8_t* e_hi,
                             int8_t* e_lo, void* stream);

/* Re-blocking of a block dual-quantised weight along its other axis, for an
 * FP8 block dgrad.  No single reference function: it is the operand step of
 * the "FP8 block dgrad via a D_out-major re-quantised W^T" that would
 * replace the reference's fp32 dequantise-then-dot dgrad
 * (fused_block_scaled_dual_gemm_backward_dx, tcfp/kernels.py:2428-2469,
 * kernel :2326-2425) when a caller opts in.  W_hi / W_lo [d_out, d_in] with
 * exponents e_hi / e_lo [d_in/block, d_out] (tcfp_block_dual_quantize's
 * output) are summed in fp32, v = 2^e_hi W_hi + 2^e_lo W_lo (e_lo = -128:
 * no lo term), transposed to [d_in, d_out], and dual-quantised again by
 * the tcfp_block_dual_quantize rule (RNE, no error buffer) along d_out:
 * wt_hi / wt_lo [d_in, d_out], et_hi / et_lo [d_out/block, d_in], i.e. the
 * B operands of tcfp_block_dual_gemm for dX = G W with G block-quantised
 * along d_out.  The re-quantised product differs from the exact one by the
 * dual-FP8 rounding of v (relative ~2^-9 of each block's maximum).  One pass: v never leaves
 * the chip.
 *   w_lo / e_lo may both be NULL (W_hi alone); d_out % block == 0,
 *   d_in % block == 0; code pointers 16-byte aligned. */
int tcfp_block_requant_t(const uint8_t* w_hi, const uint8_t* w_lo, const int8_t* e_hi,
                         const int8_t* e_lo, int64_t d_out, int64_t d_in, int block,
                         uint8_t* wt_hi, uint8_t* wt_lo, int8_t* et_hi, int8_t* et_lo,
                         void* stream);

/* Block dequantisation fp8 * 2^e -> fp32 (tcfp/kernels.py:1725-1746).
 * A -128 exponent is decoded as 2^-128 like the reference's exp2. */
int tcfp_block_dequantize(const uint8_t* q, int fp8_fmt, const int8_t* exps, int64_t m,
                          int64_t k, int block, float* out, void* stream);

/* fp32 block scales (non-power-of-two).  The reference quantises blocks
 * only with power-of-two exponents; these variants apply its per-tensor
 * rule to_fp8_e4m3 / to_fp8_e5m2 (tcfp/core.py:85-106, 137-158) to each
 * (row, K-block): scale = FP8_MAX / max(amax, 1e-12) with the reciprocal and
 * the product rounded to the input dtype, q = RNE(clamp(x * scale)), and
 * store the fp32 dequantisation multiplier 1 / scale in inv_scales
 * [k/block, m].  Layout, block sizes and constraints as above. */
int tcfp_block_quantize_f32s(const void* x, int x_dtype, int64_t m, int64_t k, int block,
                             int fp8_fmt, uint8_t* q, float* inv_scales, void* stream);

/* Fused block dual quantisation with fp32 block scales: W' = W (+ ef),
 * hi by the fp32 block rule on W', r = W' - hi * inv_hi, lo by the same rule
 * on r (RNE, or stochastic as tcfp_block_dual_quantize), and the error
 * update ef = (W - hi * inv_hi) - lo * inv_lo in place (the reference's
 * block error update order, tcfp/kernels.py:1867-1873).  A zero residual
 * block gets zero codes and the 1e-12-clamped multiplier (no sentinel). */
int tcfp_block_dual_quantize_f32s(const void* w, int w_dtype, int64_t n, int64_t k, int block,
                                  float* ef, int update_ef, int stochastic_lo, uint64_t seed,
                                  uint64_t offset, uint8_t* w_hi, uint8_t* w_lo, float* inv_hi,
                                  float* inv_lo, void* stream);

/* fp8 * inv_scales[c / block, r] -> fp32. */
int tcfp_block_dequantize_f32s(const uint8_t* q, int fp8_fmt, const float* inv_scales,
                               int64_t m, int64_t k, int block, float* out, void* stream);

/* ---- GEMMs ------------------------------------------------------------- */

/* Fused dual FP8 GEMM, both operands K-contiguous ("NT"):
 *   out[i,j] = s_a*s_hi * sum_k A[i,k] B_hi[j,k] + s_a*s_lo * sum_k A[i,k] B_lo[j,k]
 *              (+ bias[j]).
 * Replaces fused_dual_gemm_forward (tcfp/kernels.py:1545-1601),
 * cuda_ext_dual_gemm_forward (tcfp/cuda_ext.py:241-259, C++
 * tcfp/csrc/fused_dual_gemm.cu:119-274) and, with B = W^T, the dgrad
 * fused_dual_gemm_backward_dx (tcfp/kernels.py:1604-1666).
 * With b_lo == NULL it is the single scaled GEMM s_a*s_hi*(A B_hi^T): the
 * FP8 wgrad of tcfp/nn/__init__.py:546-555 (A = G^T, B = X^T).
 *   a [m, k] (lda), b_hi/b_lo [n, k] (ldb); k % 16 == 0; lda, ldb % 16 == 0;
 *   pointers (bias included) 16-byte aligned.  s_* are device fp32 scalars
 *   (inverse scales).  out [m, n] (ldo) fp32 or bf16; accumulation is fp32.
 *   An operand panel of 256 rows must span less than 2 GiB
 *   (256 * ld + k < 2^31 - 2^20), else TCFP_ERR_SHAPE; the block GEMMs below
 *   share these constraints. */
int tcfp_dual_gemm(const uint8_t* a, int a_fmt, int64_t lda, const uint8_t* b_hi,
                   const uint8_t* b_lo, int b_fmt, int64_t ldb, int64_t m, int64_t n,
                   int64_t k, const float* s_a, const float* s_hi, const float* s_lo,
                   const float* bias, void* out, int out_dtype, int64_t ldo, void* stream);

/* Block-scaled dual FP8 GEMM, both operands K-contiguous ("NT"):
 *   out[i,j] = sum_kb 2^ea[kb,i] * ( 2^ehi[kb,j] * sum_{k in kb} A[i,k] B_hi[j,k]
 *                                  + 2^elo[kb,j] * sum_{k in kb} A[i,k] B_lo[j,k] ) (+ bias[j])
 * with int8 exponent arrays e_a [k/block, m], e_hi / e_lo [k/block, n]
 * (the layout block_quantize / block_dual_quantize produce).  An exponent
 * of -128 in e_lo (a zero-residual block) contributes nothing.
 * Replaces fused_block_scaled_dual_gemm_forward (tcfp/kernels.py:1939-2028,
 * kernel :628-796); with b_lo == NULL it is the single block-scaled GEMM
 * block_scaled_gemm (tcfp/kernels.py:1878-1936, kernel :491-600).
 *   block in {32, 64, 128}; k % block == 0; other constraints as
 *   tcfp_dual_gemm.  The exponents are applied by the MFMA's E8M0 scale
 *   operands (exact powers of two); accumulation is fp32. */
int tcfp_block_dual_gemm(const uint8_t* a, int a_fmt, int64_t lda, const int8_t* e_a,
                         const uint8_t* b_hi, const uint8_t* b_lo, int b_fmt, int64_t ldb,
                         const int8_t* e_hi, const int8_t* e_lo, int64_t m, int64_t n,
                         int64_t k, int block, const float* bias, void* out, int out_dtype,
                         int64_t ldo, void* stream);

/* Activation block quantisation + block dual FP8 GEMM in one launch.
 * Replaces fused_act_quant_dual_gemm_forward (tcfp/kernels.py:2031-2149,
 * kernel :826-1041): act [m, k] (f32 or bf16, row stride lda elements) is
 * block-quantised to E4M3 along k by tcfp_block_quantize's rule inside the
 * GEMM, and out [m, n] (fp32, row stride ldo) = the block dual GEMM of those
 * codes with w_hi / w_lo [n, k] E4M3 and e_hi / e_lo [k/block, n]
 * (+ bias[j]).  act_fp8 [m, k] (row stride k) and act_scales [k/block, m]
 * receive the codes and exponents (bitwise tcfp_block_quantize's), or are
 * both NULL (the reference's save_side_outputs=False).
 *   block in {32, 64, 128}; k % block == 0; act, w_hi, w_lo, act_fp8 and
 *   bias 16-byte aligned; lda * element bytes and ldb multiples of 16. */
int tcfp_act_quant_block_dual_gemm(const void* act, int act_dtype, int64_t lda,
                                   const uint8_t* w_hi, const uint8_t* w_lo, int64_t ldb,
                                   const int8_t* e_hi, const int8_t* e_lo, int64_t m, int64_t n,
                                   int64_t k, int block, const float* bias, float* out,
                                   int64_t ldo, uint8_t* act_fp8, int8_t* act_scales,
                                   void* stream);

/* Block-scaled dual FP8 GEMM with fp32 block multipliers (non-power-of-two
 * block scales, e.g. the 448 / amax rule of tcfp_block_quantize_f32s):
 *   out[i,j] = sum_kb s_a[kb,i] * ( s_hi[kb,j] * sum_{k in kb} A[i,k] B_hi[j,k]
 *                                 + s_lo[kb,j] * sum_{k in kb} A[i,k] B_lo[j,k] ) (+ bias[j])
 * with fp32 dequantisation multipliers s_a [k/block, m], s_hi / s_lo
 * [k/block, n].  Same operation as tcfp_block_dual_gemm with the reference's
 * int8 exponents replaced by arbitrary fp32 scales (the reference kernel
 * multiplies by exp2 of its exponents in-loop, tcfp/kernels.py:577-585,
 * :757-776); b_lo == NULL gives the single GEMM.  The per-block products
 * are accumulated on the MFMA and folded into the output with the fp32
 * multipliers on the VALU.
 *   block in {32, 64, 128}; k % block == 0; m % 4 == 0; n % 4 == 0;
 *   s_* 16-byte aligned; other constraints as tcfp_dual_gemm. */
int tcfp_block_dual_gemm_f32s(const uint8_t* a, int a_fmt, int64_t lda, const float* s_a,
                              const uint8_t* b_hi, const uint8_t* b_lo, int b_fmt, int64_t ldb,
                              const float* s_hi, const float* s_lo, int64_t m, int64_t n,
                              int64_t k, int block, const float* bias, void* out,
                              int out_dtype, int64_t ldo, void* stream);

/* Weight quantisation + block dual GEMM in one call.  Replaces
 * fused_wtquant_block_scaled_dual_gemm_forward (tcfp/kernels.py:2152-2323,
 * kernel :1233-1531): W [n, k] f32/bf16 (+ ef) is dual-quantised as
 * tcfp_block_dual_quantize (error buffer updated in place, or W_lo
 * stochastically rounded) into the caller's w_hi / w_lo [n, k] and
 * e_hi / e_lo [k/block, n], then out = tcfp_block_dual_gemm(a, ...).
 * Runs as two launches on `stream`: one streaming pass over W and the
 * GEMM.  w_hi/w_lo are always written (the GEMM reads them).
 *   constraints as tcfp_block_dual_quantize and tcfp_block_dual_gemm. */
int tcfp_wtquant_block_dual_gemm(const uint8_t* a, int a_fmt, int64_t lda, const int8_t* e_a,
                                 const void* w, int w_dtype, int64_t m, int64_t n, int64_t k,
                                 int block, float* ef, int stochastic_lo, uint64_t seed,
                                 uint64_t offset, uint8_t* w_hi, uint8_t* w_lo, int8_t* e_hi,
                                 int8_t* e_lo, const float* bias, void* out, int out_dtype,
                                 int64_t ldo, void* stream);

/* Block-scaled dual dgrad:
 *   dx[i,k] = sum_n 2^eg[n/block,i] G[i,n] * ( 2^ehi[k/block,n] W_hi[n,k]
 *                                          + 2^elo[k/block,n] W_lo[n,k] )
 * with g [m, d_out] (E5M2 or E4M3, g_fmt), e_g [d_out/block, m],
 * w_hi / w_lo [d_out, d_in] E4M3, e_hi / e_lo [d_in/block, d_out];
 * dx [m, d_in] fp32.  e_lo == -128 marks a zero W_lo block.  w_lo == NULL
 * uses W_hi alone (ABD).  Replaces fused_block_scaled_dual_gemm_backward_dx
 * (tcfp/kernels.py:2428-2469, kernel :1051-1205).  The operands are
 * dequantised exactly into bf16 in `workspace` (G as is, W transposed) and
 * multiplied on the bf16 MFMA with fp32 accumulation.
 *   d_out % block == 0, d_in % block == 0; workspace 16-byte aligned and at
 *   least tcfp_block_dual_gemm_dx_workspace_bytes(m, d_out, d_in) bytes. */
size_t tcfp_block_dual_gemm_dx_workspace_bytes(int64_t m, int64_t d_out, int64_t d_in);
int tcfp_block_dual_gemm_dx(const uint8_t* g, int g_fmt, const int8_t* e_g,
                            const uint8_t* w_hi, const uint8_t* w_lo, const int8_t* e_hi,
                            const int8_t* e_lo, int64_t m, int64_t d_out, int64_t d_in,
                            int block, float* dx, void* workspace, size_t workspace_bytes,
                            void* stream);

/* Block-path weight gradient with an fp32 gradient:
 *   dw[n, k] = sum_i g[i, n] * 2^ex[k/block, i] * x[i, k]
 * g [m, n_out] fp32, x [m, k_in] fp8 (x_fmt) with exponents [k_in/block, m],
 * dw [n_out, k_in] fp32.  Replaces the reference's fp32
 * `grad_2d.t() @ block_dequantize_fp8(act)` (tcfp/nn/__init__.py:743-750).
 * The dequantised activation is exact in bf16 and g is split into
 * g_hi = bf16(g), g_lo = bf16(g - g_hi) (relative representation error
 * <= 2^-17); both products run as one bf16-MFMA GEMM over the
 * concatenated contraction [g_hi | g_lo] x [x | x] with fp32 accumulation.
 *   m % 4 == 0; k_in % block == 0; workspace 16-byte aligned and at least
 *   tcfp_block_wgrad_workspace_bytes(m, n_out, k_in) bytes. */
size_t tcfp_block_wgrad_workspace_bytes(int64_t m, int64_t n_out, int64_t k_in);
int tcfp_block_wgrad(const float* g, int64_t m, int64_t n_out, const uint8_t* x, int x_fmt,
                     const int8_t* e_x, int64_t k_in, int block, float* dw, void* workspace,
                     size_t workspace_bytes, void* stream);

/* Block backward, fused operand preparation (no single reference
 * counterpart: it produces, in one pass over the fp32 gradient g [m, n],
 * what the reference's backward derives from it separately,
 * tcfp/nn/__init__.py:700-761):
 *   g_deq     [m, n] bf16: g block-quantised to E5M2 per (row, n-block of
 *             `block`) with the block_quantize_fp8 rule (tcfp/kernels.py:
 *             1675-1722) and dequantised -- the dgrad's G operand;
 *   g_split_t [n, 2m] bf16: [bf16(g) | bf16(g - bf16(g))] transposed -- the
 *             wgrad's split fp32 gradient (split_lo 1); with split_lo 0
 *             [n, m] bf16: bf16(g) transposed, the single-pass wgrad's
 *             operand;
 *   bias_grad [n] fp32: column sums of g (grad.sum(0)), summed per 64-row
 *             tile and then over tiles in order;
 *   g_fp8 [m, n] E5M2 codes with g_exps [n / block, m] int8: the same block
 *             quantisation as codes (block_quantize_fp8(g, block, e5m2)) --
 *             the FP8 block dgrad's G operand (both or neither).
 * Any output may be NULL.  n % block == 0; bias_grad needs a workspace of
 * tcfp_block_grad_prep_workspace_bytes(m, n) bytes. */
size_t tcfp_block_grad_prep_workspace_bytes(int64_t m, int64_t n);
int tcfp_block_grad_prep(const float* g, int64_t m, int64_t n, int block, uint16_t* g_deq,
                         uint16_t* g_split_t, int split_lo, float* bias_grad, uint8_t* g_fp8,
                         int8_t* g_exps, void* workspace, size_t workspace_bytes, void* stream);

/* tcfp_block_dual_gemm_dx with the gradient already dequantised to bf16
 * (g_deq from tcfp_block_grad_prep): same result bit for bit.  Workspace:
 * tcfp_block_dual_gemm_dx_bf16_workspace_bytes(d_out, d_in). */
size_t tcfp_block_dual_gemm_dx_bf16_workspace_bytes(int64_t d_out, int64_t d_in);
int tcfp_block_dual_gemm_dx_bf16(const uint16_t* g_deq, const uint8_t* w_hi, const uint8_t* w_lo,
                                 const int8_t* e_hi, const int8_t* e_lo, int64_t m, int64_t d_out,
                                 int64_t d_in, int block, float* dx, void* workspace,
                                 size_t workspace_bytes, void* stream);

/* tcfp_block_wgrad with the gradient already split and transposed
 * (g_split_t [n_out, 2m] from tcfp_block_grad_prep with split_lo 1): same
 * result bit for bit.  With split_lo 0, g_split_t is [n_out, m] (bf16(g)
 * transposed) and dW = bf16(g)^T deq(x): one bf16 pass instead of two,
 * relative error ~2^-9 per gradient element (the reference's wgrad
 * contract is 1e-2 relative; m % 64 == 0).  Workspace:
 * tcfp_block_wgrad_presplit_workspace_bytes(m, n_out, k_in, split_lo). */
size_t tcfp_block_wgrad_presplit_workspace_bytes(int64_t m, int64_t n_out, int64_t k_in,
                                                 int split_lo);
int tcfp_block_wgrad_presplit(const uint16_t* g_split_t, int split_lo, int64_t m,
                              int64_t n_out, const uint8_t* x, int x_fmt, const int8_t* e_x,
                              int64_t k_in, int block, float* dw, void* workspace,
                              size_t workspace_bytes, void* stream);

/* ---- layout helpers ---------------------------------------------------- */

/* dst[c, r] = src[r, c] for a [rows, cols] byte matrix (ld = cols / rows).
 * Used where the reference calls ensure_column_major / .t().contiguous()
 * (tcfp/core.py:196-213, tcfp/nn/__init__.py:546-555). */
int tcfp_transpose_u8(const uint8_t* src, int64_t rows, int64_t cols, uint8_t* dst,
                      void* stream);

/* ---- tuning hooks (no reference counterpart) --------------------------- */

/* GEMM tile selection for all later calls in the process: 0 automatic (the
 * 256 x 128 tile unless it would leave CUs idle; FP8 dual GEMMs with more
 * full tiles than CUs run one persistent workgroup per CU; block-scaled
 * single GEMMs with at least as many full 256 x 256 tiles as CUs take that
 * tile; per-tensor dual GEMMs with bf16 output and K >= 8192 the persistent
 * 256 x 128 tile with four waves, one per SIMD), 1 always 256 x 128, 2 always
 * 128 x 64, 3 128 x 64 with eight waves where the
 * small-tile grid fits in one round (FP8 operands; bf16 ones keep four
 * waves), 4 256 x 128 with one workgroup per tile (no persistent launch),
 * 5 the four-wave persistent 256 x 128 tile for per-tensor dual GEMMs with
 * bf16 output (the others as 0).  Results do not depend on the policy. */
int tcfp_gemm_set_tile_policy(int policy);

/* ---- self-test hooks (no reference counterpart) ------------------------ */

/* Converts every float32 whose bit pattern lies in [lo_bits, hi_bits] (and
 * its negation) with both the hardware and the software FP8 encoder, and
 * decodes all 256 codes with both the hardware and the software decoder
 * (NaN codes must decode to NaN in both); counts mismatches into
 * *mismatches (device uint64, accumulated). */
int tcfp_selftest_fp8_cvt(uint32_t lo_bits, uint32_t hi_bits, int fp8_fmt,
                          unsigned long long* mismatches, void* stream);

/* Runs the block stochastic-rounding candidate rule with software FP8
 * converts and with the hardware converts the kernels use, on every float32
 * whose bit pattern lies in [lo_bits, hi_bits] (at most 448.0's) and its
 * negation, at uniform u; counts disagreements into *mismatches. */
int tcfp_selftest_sr_block(uint32_t lo_bits, uint32_t hi_bits, float u,
                           unsigned long long* mismatches, void* stream);

/* Fills out[4*i .. 4*i+3] with Philox4x32-10 of counter (i + ctr0, ctr1,
 * ctr2, ctr3) under key (k0, k1), for i < n. */
int tcfp_selftest_philox(uint32_t ctr0, uint32_t ctr1, uint32_t ctr2, uint32_t ctr3,
                         uint32_t k0, uint32_t k1, int64_t n, uint32_t* out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TCFP_HIP_H_ */
