/*
 * nc_hip.h -- the thin C-ABI layer of hand-written HIP kernels (gfx950) under the newch engine.
 *
 * The engine (include/nc.h, newch_amd/libnc.so) calls these from its op forward/backward functions
 * in place of the reference engine's CPU kernel table and row loops; they are exported from the same
 * libnc.so so tests and benchmarks can drive them directly on device buffers.
 *
 * Conventions
 *   - every pointer is a device pointer (HBM) unless named host_*; sizes and strides are in elements;
 *   - `stream` is a hipStream_t (NULL = the legacy default stream); every call only enqueues work;
 *   - calls return NC_HIP_OK or an error code and never abort; nc_hip_last_error() has the detail;
 *   - float arithmetic follows the reference's evaluation order op for op (IEEE fp32, fused only
 *     where the reference's AVX2 tier fuses), so elementwise results are bit-identical to it;
 *     reductions accumulate in fp64 with a fixed partition, so they are deterministic;
 *   - functions that need scratch take (ws, ws_bytes): device memory of at least the size the
 *     matching *_workspace() query returns (0 = none needed).
 */
#ifndef NC_HIP_H
#define NC_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NC_HIP_API __attribute__((visibility("default")))

enum { NC_HIP_OK = 0, NC_HIP_ERR_ARG = 4, NC_HIP_ERR_DEVICE = 5, NC_HIP_ERR_WORKSPACE = 6 };

/* activation kinds */
enum {
    NC_HIP_UN_RELU = 0, NC_HIP_UN_LEAKY_RELU, NC_HIP_UN_RELU6, NC_HIP_UN_HARDSIGMOID, NC_HIP_UN_HARDSWISH,
    NC_HIP_UN_SILU, NC_HIP_UN_GELU, NC_HIP_UN_GELU_TANH, NC_HIP_UN_SIGMOID, NC_HIP_UN_TANH, NC_HIP_UN_EXP,
    NC_HIP_UN_NEG, NC_HIP_UN_SCALE, NC_HIP_UN_ADD_SCALAR, NC_HIP_UN_LOG, NC_HIP_UN_SQRT, NC_HIP_UN_POW,
    NC_HIP_UN_COUNT
};
enum { NC_HIP_BIN_ADD = 0, NC_HIP_BIN_SUB, NC_HIP_BIN_MUL, NC_HIP_BIN_DIV };
enum { NC_HIP_RED_SUM = 0, NC_HIP_RED_MEAN, NC_HIP_RED_MAX, NC_HIP_RED_ARGMAX };
/* element types (same codes as nc_dtype) */
enum { NC_HIP_F32 = 0, NC_HIP_I32 = 1, NC_HIP_I8 = 3, NC_HIP_U8 = 4 };

#define NC_HIP_MAX_DIMS 6

NC_HIP_API const char *nc_hip_last_error(void);
NC_HIP_API int nc_hip_device_count(void);
/* Test hook (host only, no device work): how many (d, n) pairs the kernels' multiply-high index
 * divider gets wrong against n / d, over every d in divs and n in nums. */
NC_HIP_API uint64_t nc_hip_check_intdiv(const uint32_t *divs, int ndivs, const uint32_t *nums, int nnums);
/* Test hook: size the grids of grid-stride kernels for n compute units instead of the device's own
 * count (n <= 0 restores it; the NC_HIP_CUS environment variable sets the same at start-up).  Every
 * split of a reduction into partials depends on the problem shape only, so results are bit-identical
 * for any n: the GPU counterpart of the reference's thread-count determinism (threadpool.c:182-186,
 * engine/tests/test_main.c:1169-1246). */
NC_HIP_API void nc_hip_set_grid_cus(int n);

/* Activation forward over n contiguous floats: y = f(x).  `s` is the leaky_relu slope / scale
 * factor / added scalar / exponent.  Replaces unary_fwd_span, ops_elementwise.c:229-266 (with the
 * exp8/sigmoid8/tanh8/erf8 maps of kernels_avx2.c:96-178). */
NC_HIP_API int nc_hip_unary_fwd(int kind, float s, const float *x, float *y, int64_t n, void *stream);

/* Activation backward: gi[i] (+)= f'(x[i]) * g[i].  Reads x (relu family, silu, gelu, log, pow),
 * y (sigmoid, tanh, exp, sqrt) or neither (neg, scale, add_scalar); pass NULL for the unread one.
 * accumulate = 1: gi += term (the reference contract); 0: gi = 0 + term (a fresh zeroed buffer,
 * same bits without reading gi).  Replaces unary_bwd_span, ops_elementwise.c:289-338. */
NC_HIP_API int nc_hip_unary_bwd(int kind, float s, const float *x, const float *y, const float *g, float *gi,
                                int64_t n, int accumulate, void *stream);

/* Broadcast binary forward o = a op b over an nd-d output `shape` (nd <= 6) with element strides
 * sa/sb (0 on broadcast dims) and so.  Replaces binary_fwd + row_add..row_div + nc__iterate,
 * ops_elementwise.c:19-30,108-127 and tensor.c:313-345. */
NC_HIP_API int nc_hip_binary_fwd(int op, int nd, const int64_t *shape, const float *a, const int64_t *sa,
                                 const float *b, const int64_t *sb, float *o, const int64_t *so, void *stream);

/* Gradient of one operand of o = a op b (sum-to-shape): for every output index i,
 *     gx[i . sgx] (+)= term(g[i . sg], a[i . sa], b[i . sb])
 * with term = g (add, sub wrt a), -g (sub wrt b), g*other (mul), g/b (div wrt a),
 * -(g*a)/(b*b) (div wrt b); dims where sgx is 0 are summed.  which = 0 (wrt a) or 1 (wrt b).
 * accumulate as in nc_hip_unary_bwd.  Unreduced grads are bit-identical to the reference's
 * row_acc/axpy; reduced ones are summed in fp64 in a fixed order.  Replaces binary_bwd and
 * row_acc*, ops_elementwise.c:33-54,129-186. */
NC_HIP_API size_t nc_hip_binary_bwd_workspace(int nd, const int64_t *shape, const int64_t *sgx);
NC_HIP_API int nc_hip_binary_bwd(int op, int which, int nd, const int64_t *shape, const float *g,
                                 const int64_t *sg, const float *a, const int64_t *sa, const float *b,
                                 const int64_t *sb, float *gx, const int64_t *sgx, int accumulate, void *ws,
                                 size_t ws_bytes, void *stream);

/* Both operand grads of o = a op b from one pass over g (the broadcast-binary backward when a and
 * b are both reduced).  Same terms and contract as two nc_hip_binary_bwd calls; ga or gb may be
 * NULL.  Workspace from nc_hip_binary_bwd2_workspace. */
NC_HIP_API size_t nc_hip_binary_bwd2_workspace(int nd, const int64_t *shape, const int64_t *sga,
                                               const int64_t *sgb);
NC_HIP_API int nc_hip_binary_bwd2(int op, int nd, const int64_t *shape, const float *g, const int64_t *sg,
                                  const float *a, const int64_t *sa, const float *b, const int64_t *sb, float *ga,
                                  const int64_t *sga, float *gb, const int64_t *sgb, int accumulate, void *ws,
                                  size_t ws_bytes, void *stream);

/* Strided gather into contiguous dst (elem_bytes 1, 2, 4 or 8).  Replaces nc__copy_strided /
 * nc__contig_f32, tensor.c:347-373. */
NC_HIP_API int nc_hip_copy_strided(int elem_bytes, int nd, const int64_t *shape, const void *src,
                                   const int64_t *ss, void *dst, void *stream);
/* dst[i . sd] += src[i] for contiguous src over `shape` (the strided grad scatter of transpose /
 * slice backward, ops_shape.c:169-184,254-267). */
NC_HIP_API int nc_hip_accumulate_strided(int nd, const int64_t *shape, const float *src, float *dst,
                                         const int64_t *sd, void *stream);

/* y[i] += alpha * x[i] (fused, as axpy_f32 kernels_avx2.c:39-45). */
NC_HIP_API int nc_hip_axpy(int64_t n, float alpha, const float *x, float *y, void *stream);
/* Fill n elements of elem_bytes (1, 2, 4, 8) with the low bytes of `pattern`. */
NC_HIP_API int nc_hip_fill(void *dst, int elem_bytes, uint64_t pattern, int64_t n, void *stream);
/* dtype conversion with the reference's rules (ops_shape.c:474-504): float -> int truncates toward
 * zero, saturates, NaN -> 0; int -> float exact. */
NC_HIP_API int nc_hip_convert(int from, int to, int64_t n, const void *src, void *dst, void *stream);
/* *p += v for one float (the loss-grad seed of backward, autograd.c:156-158). */
NC_HIP_API int nc_hip_add_scalar_at(float *p, float v, void *stream);

/* Reductions over contiguous x viewed as [outer, R, inner].  kind SUM/MEAN write y; MAX writes y and
 * arg; ARGMAX writes arg.  Sums accumulate in fp64 (deterministic); max/argmax follow the
 * reference's strict-greater scan (first index wins, a NaN at r = 0 wins, later NaNs are skipped).
 * Replaces get_dims/reduce_fwd, ops_reduce.c:13-116. */
NC_HIP_API size_t nc_hip_reduce_workspace(int kind, int64_t outer, int64_t R, int64_t inner);
NC_HIP_API int nc_hip_reduce_fwd(int kind, int64_t outer, int64_t R, int64_t inner, const float *x, float *y,
                                 int32_t *arg, void *ws, size_t ws_bytes, void *stream);
/* nc_hip_reduce_fwd without a workspace argument and without allocating: no counterpart in the
 * reference.  For callers that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc).  The partials live in a static device array of
 * 8 MiB per GPU, held until the process ends, whose address is looked up (hipGetSymbolAddress) on
 * the first call on each device; every shape nc_hip_reduce_fwd takes fits, and a plan that would not
 * is refused with NC_HIP_ERR_WORKSPACE.  Same results, bit for bit, as nc_hip_reduce_fwd.  All calls
 * on one GPU share that array: calls that overlap on one GPU (on different streams, or from
 * different threads) race and must be serialized by the caller. */
NC_HIP_API int nc_hip_reduce_fwd_noalloc(int kind, int64_t outer, int64_t R, int64_t inner, const float *x,
                                         float *y, int32_t *arg, void *stream);
/* gi (+)= broadcast-back of g (sum, mean) or scatter to arg (max).  ops_reduce.c:118-163. */
NC_HIP_API int nc_hip_reduce_bwd(int kind, int64_t outer, int64_t R, int64_t inner, const float *g,
                                 const int32_t *arg, float *gi, int accumulate, void *stream);
/* Sum of int32 over [outer, R, inner] in int64, stored as int32 (ops_reduce.c:63-75). */
NC_HIP_API int nc_hip_reduce_sum_i32(int64_t outer, int64_t R, int64_t inner, const int32_t *x, int32_t *y,
                                     void *stream);

/* Row softmax / log_softmax over the last dim (rows x C, contiguous).  softmax_row,
 * ops_nn.c:22-46; backward ops_nn.c:48-71 (gi (+)= ...). */
NC_HIP_API int nc_hip_softmax_fwd(int log_form, int64_t rows, int64_t C, const float *x, float *y, void *stream);
NC_HIP_API int nc_hip_softmax_bwd(int log_form, int64_t rows, int64_t C, const float *y, const float *g,
                                  float *gi, int accumulate, void *stream);

/* LayerNorm over rows of D (w, b may be NULL); stats = [rows][2] {mean, rstd}, fp64 row statistics
 * rounded to fp32 as layer_norm_fwd, ops_nn.c:463-490.  Backward ops_nn.c:492-522: gx (+)= ...
 * (may be NULL); gw, gb += column sums (may be NULL), deterministic via per-block partials. */
NC_HIP_API int nc_hip_layer_norm_fwd(int64_t rows, int64_t D, const float *x, const float *w, const float *b,
                                     float eps, float *y, float *stats, void *stream);
NC_HIP_API size_t nc_hip_layer_norm_bwd_workspace(int64_t rows, int64_t D);
NC_HIP_API int nc_hip_layer_norm_bwd(int64_t rows, int64_t D, const float *x, const float *w,
                                     const float *stats, const float *g, float *gx, float *gw, float *gb,
                                     int accumulate, void *ws, size_t ws_bytes, void *stream);

/* Symmetric per-row int8 quantization of w [rows, cols]: scale = absmax/127 (1 for a zero row),
 * q = clamp(rne(w / scale), -127, 127).  quantize_row / nc_quantize_rows, ops_quant.c:11-39.
 * Several matrices stacked along rows are one call. */
NC_HIP_API int nc_hip_quantize_rows(int64_t rows, int64_t cols, const float *w, int8_t *q, float *scale,
                                    void *stream);
/* w = (float)q * scale[row]: to_dtype i8->f32 (ops_shape.c:491-504) then the row-broadcast mul. */
NC_HIP_API int nc_hip_dequantize_rows(int64_t rows, int64_t cols, const int8_t *q, const float *scale, float *w,
                                      void *stream);

/* Losses over rows [N, C] (contiguous) with i32 labels [N].  `loss` and `gout` are one float in
 * device memory.  `bad` (8 bytes, device) receives all ones, or the first row whose label is outside
 * [0, C) as (row << 32) | (uint32)label — that row contributes nothing; the caller reads it back to
 * raise the reference's "label %d at row %lld outside [0, %lld)" error.  Loss sums are fp64 in a
 * fixed order.  Workspace of both forwards: nc_hip_loss_workspace(N, C) bytes. */
NC_HIP_API size_t nc_hip_loss_workspace(int64_t N, int64_t C);
/* Cross entropy (fused log-softmax + NLL, mean over rows; NaN for N = 0): ce_fwd, ops_nn.c:107-131.
 * stats (8-byte aligned, [N][2] floats) receives each row's {max m, ls = logf(sum exp8(x - m))}: the
 * reference's saved probabilities are exp8((x - m) - ls), which the backward recomputes from x. */
NC_HIP_API int nc_hip_cross_entropy_fwd(int64_t N, int64_t C, const float *x, const int32_t *lab, float *stats,
                                        float *loss, uint64_t *bad, void *ws, size_t ws_bytes, void *stream);
/* gi (+)= s * prob, then gi[i, lab_i] -= s, with s = gout / N and prob = exp8((x - m) - ls) from the
 * forward's stats: ce_bwd, ops_nn.c:133-147, with the reference's fp32 operations (bit for bit given
 * the stats; the stats' ls is an fp64 row sum, so prob is within the reductions' tolerance of the
 * probabilities the reference's forward saves).  x must hold the values the forward read. */
NC_HIP_API int nc_hip_cross_entropy_bwd(int64_t N, int64_t C, const float *x, const float *stats,
                                        const int32_t *lab, const float *gout, float *gi, int accumulate,
                                        void *stream);
/* NLL over log-probabilities: loss = -sum_i x[i, lab_i] (sum != 0), or that / N (NaN for N = 0):
 * nll_fwd, ops_nn.c:391-410. */
NC_HIP_API int nc_hip_nll_loss_fwd(int64_t N, int64_t C, const float *x, const int32_t *lab, int sum,
                                   float *loss, uint64_t *bad, void *ws, size_t ws_bytes, void *stream);
/* gi[i, lab_i] -= s, s = gout (sum) or gout / N; gi is read and written: nll_bwd, ops_nn.c:412-420. */
NC_HIP_API int nc_hip_nll_loss_bwd(int64_t N, int64_t C, const int32_t *lab, const float *gout, int sum,
                                   float *gi, void *stream);

/* One optimizer update of a parameter w [n] with gradient g (optim.c:161-216): the reference's fp32
 * expression per element, in its order, without fused multiply-adds.  kind: NC_HIP_OPT_*.  s1 is
 * the momentum buffer (SGD, RMSprop; NULL without momentum) or Adam's m, s2 Adam's v or RMSprop's
 * square average.  gs = 1 / accumulation steps; bc1, bc2 = Adam's 1 - beta^t (1 otherwise). */
enum { NC_HIP_OPT_SGD = 0, NC_HIP_OPT_ADAM = 1, NC_HIP_OPT_ADAMW = 2, NC_HIP_OPT_RMSPROP = 3 };
NC_HIP_API int nc_hip_optim_step(int kind, int64_t n, float *w, const float *g, float *s1, float *s2, float lr,
                                 float momentum, float weight_decay, float beta1, float beta2, float eps, float gs,
                                 float bc1, float bc2, int eps_inside_sqrt, void *stream);
/* The same update for up to NC_HIP_OPT_MULTI_MAX parameters in one launch (no counterpart in the
 * reference, whose step loops over its parameters one call each; for models with many small
 * parameters, where one launch per parameter dominates the step).  Every parameter's n is a multiple
 * of 4 and its arrays 16-byte aligned; s1 and s2 are present for every parameter or for none, as in
 * one optimizer.  Bit-identical to one nc_hip_optim_step per parameter.  The parameters are updated
 * concurrently: no parameter's w may share memory with another's w or g. */
#define NC_HIP_OPT_MULTI_MAX 32
typedef struct {
    float *w;
    const float *g;
    float *s1;
    float *s2;
    int64_t n;
} nc_hip_opt_param;
NC_HIP_API int nc_hip_optim_step_multi(int kind, int count, const nc_hip_opt_param *params, float lr, float momentum,
                                       float weight_decay, float beta1, float beta2, float eps, float gs, float bc1,
                                       float bc2, int eps_inside_sqrt, void *stream);
/* ss (+)= sum of x[i]^2 in fp64 (one double in device memory), clip_grad_norm's sum
 * (optim.c:217-223); fixed order.  Workspace: nc_hip_sumsq_workspace(n). */
NC_HIP_API size_t nc_hip_sumsq_workspace(int64_t n);
NC_HIP_API int nc_hip_sumsq(int64_t n, const float *x, double *ss, int accumulate, void *ws, size_t ws_bytes,
                            void *stream);
/* The same sum over up to NC_HIP_OPT_MULTI_MAX tensors x[t] of n[t] floats in two launches (no
 * counterpart in the reference, whose clip_grad_norm calls one sum per gradient; for models with
 * many small gradients).  Bit-identical to one nc_hip_sumsq per tensor in turn, the first with the
 * given accumulate and the others accumulating.  The tables are host memory.  Workspace:
 * nc_hip_sumsq_multi_workspace(count, n) = the sum of the tensors' nc_hip_sumsq_workspace. */
NC_HIP_API size_t nc_hip_sumsq_multi_workspace(int count, const int64_t *n);
NC_HIP_API int nc_hip_sumsq_multi(int count, const float *const *x, const int64_t *n, double *ss, int accumulate,
                                  void *ws, size_t ws_bytes, void *stream);
/* x[t] = coef * x[t] in place for up to NC_HIP_OPT_MULTI_MAX tensors in one launch (no counterpart
 * in the reference: clip_grad_norm's rescale of every gradient, scale_f32 at optim.c:226-231); the
 * bits of nc_hip_unary_fwd(NC_HIP_UN_SCALE, coef) per tensor. */
NC_HIP_API int nc_hip_scale_multi(int count, float *const *x, const int64_t *n, float coef, void *stream);

/* Row-major fp32 GEMM: C = alpha * op(A) op(B) + beta * C, op(X) = X^T when its flag is set; op(A) is
 * M x K, op(B) K x N, leading dims in elements.  The reference's gemm_f32 (kernels.h:36-41) as used by
 * matmul / linear (ops_linalg.c:64-99,296-330); hand-written fp32 matrix-core kernels, each output
 * summing its K products in one fixed order (the same for every tile size, grid and device).  The
 * batched form takes device arrays of `count` matrix pointers. */
NC_HIP_API int nc_hip_gemm_f32(int ta, int tb, int64_t M, int64_t N, int64_t K, float alpha, const float *A,
                               int64_t lda, const float *B, int64_t ldb, float beta, float *C, int64_t ldc,
                               void *stream);
/* C = alpha * op(A) op(B) + bias, bias[N] added to every row (NULL: none): the bits of nc_hip_gemm_f32
 * with beta 0 followed by a broadcast add of the bias, in one pass over C.  linear's forward
 * (ops_linalg.c:296-330, x W^T then the bias) uses it. */
NC_HIP_API int nc_hip_gemm_f32_bias(int ta, int tb, int64_t M, int64_t N, int64_t K, float alpha, const float *A,
                                    int64_t lda, const float *B, int64_t ldb, const float *bias, float *C, int64_t ldc,
                                    void *stream);
NC_HIP_API int nc_hip_gemm_f32_batched(int ta, int tb, int64_t M, int64_t N, int64_t K, float alpha,
                                       const float *const *A, int64_t lda, const float *const *B, int64_t ldb,
                                       float beta, float *const *C, int64_t ldc, int64_t count, void *stream);
/* Batched matmul with broadcast batch dims (the reference's bmm, ops_linalg.c:89-252): for every index
 * of the batch shape bshape[nb], C_i = op(A_i) op(B_i) + beta C_i with A_i = A + sum_d idx_d sa[d]
 * (likewise B, C; stride 0 = broadcast).  When several batch indices share one C block (sc has a 0 on
 * a dim > 1, a broadcast operand's gradient) they run in batch order, each adding into the block; the
 * others run as one launch that decodes the batch strides per workgroup.  Workspace: none
 * (nc_hip_gemm_f32_bmm_workspace returns 0; the argument pair is kept for callers that pass one). */
NC_HIP_API size_t nc_hip_gemm_f32_bmm_workspace(int64_t count);
NC_HIP_API int nc_hip_gemm_f32_bmm(int ta, int tb, int64_t M, int64_t N, int64_t K, const float *A, int64_t lda,
                                   const float *B, int64_t ldb, float beta, float *C, int64_t ldc, int nb,
                                   const int64_t *bshape, const int64_t *sa, const int64_t *sb, const int64_t *sc,
                                   void *ws, size_t ws_bytes, void *stream);

/* int8 GEMM, C[m][n] = sum_k A[m][k] B[n][k] in int32 (A [M, K], B [N, K], both K-contiguous with
 * leading dims lda / ldb; C leading dim ldc).  Exact, so bit-identical to the reference's gemm_s8_nt
 * (kernels.h:42-43, kernels_ref.c:117-128) for K <= 133143.  Matrix cores (MFMA int8). */
NC_HIP_API int nc_hip_gemm_s8_nt(int64_t M, int64_t N, int64_t K, const int8_t *A, int64_t lda, const int8_t *B,
                                 int64_t ldb, int32_t *C, int64_t ldc, void *stream);
/* linear_int8 forward (ops_quant.c:41-113): rows of x [M, K] quantized as quantize_rows does, the
 * int8 product with wq [N, K] on the matrix cores, and the epilogue
 * y = (float)acc * xs[m] * wscale[n] + (bias ? bias[n] : 0) fused into it; bit-identical to the
 * reference.  Workspace: the quantized rows and their scales. */
NC_HIP_API size_t nc_hip_linear_int8_workspace(int64_t M, int64_t K);
NC_HIP_API int nc_hip_linear_int8(int64_t M, int64_t K, int64_t N, const float *x, const int8_t *wq,
                                  const float *wscale, const float *bias, float *y, void *ws, size_t ws_bytes,
                                  void *stream);

#ifdef __cplusplus
}
#endif
#endif /* NC_HIP_H */
