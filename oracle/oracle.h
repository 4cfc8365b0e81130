/* CPU oracle for the newch hot path -- TEST INFRASTRUCTURE ONLY.
 *
 * A from-scratch C restatement of the reference engine's arithmetic on this path, used by tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg to check results against.  The product library
 * (newch_amd/libnc.so) never links or calls it.
 *
 * Every function follows the reference's evaluation order op for op (file:line cited at each
 * definition in oracle.c), so on the same inputs it reproduces the reference bit for bit,
 * including its sequential fp32 summation orders.  Pinning: tests/test_oracle.py checks each
 * function against the fixtures in tests/golden/ (written by the compiled reference), against
 * oracle/_ref/libnc_ref.so when it is built, against the reference's own known-answer tests and
 * against closed forms / fp64 brute force.
 *
 * Layout conventions: all tensors are float32 unless noted; strides are in elements; "contiguous"
 * means row-major.
 */
#ifndef NC_ORACLE_H
#define NC_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* unary kinds (same numbering as the HIP layer's NC_HIP_UN_*) */
enum {
    OR_UN_RELU = 0, OR_UN_LEAKY_RELU, OR_UN_RELU6, OR_UN_HARDSIGMOID, OR_UN_HARDSWISH,
    OR_UN_SILU, OR_UN_GELU, OR_UN_GELU_TANH, OR_UN_SIGMOID, OR_UN_TANH, OR_UN_EXP,
    OR_UN_NEG, OR_UN_SCALE, OR_UN_ADD_SCALAR, OR_UN_LOG, OR_UN_SQRT, OR_UN_POW, OR_UN_COUNT
};
enum { OR_BIN_ADD = 0, OR_BIN_SUB, OR_BIN_MUL, OR_BIN_DIV };
enum { OR_RED_SUM = 0, OR_RED_MEAN, OR_RED_MAX, OR_RED_ARGMAX };

/* vector-tier transcendentals, one element at a time */
float or_exp(float x);
float or_sigmoid(float x);
float or_tanh(float x);
float or_erf(float x);
void or_map(int fn, int64_t n, const float *x, float *y); /* fn: 0 exp, 1 sigmoid, 2 tanh, 3 erf */

float or_sum_f32(int64_t n, const float *x);
void or_axpy(int64_t n, float alpha, const float *x, float *y);

/* activations: y = f(x); gi += f'(x) * g  (x and y both given; each kind reads what it needs) */
void or_unary_fwd(int kind, float s, const float *x, float *y, int64_t n);
void or_unary_bwd(int kind, float s, const float *x, const float *y, const float *g, float *gi, int64_t n);

/* broadcast binary forward over an output of `nd` dims; sa/sb are broadcast strides (0 on
 * broadcast dims), so = output strides */
void or_binary_fwd(int op, int nd, const int64_t *shape, const float *a, const int64_t *sa, const float *b,
                   const int64_t *sb, float *o, const int64_t *so);

/* binary backward (sum-to-shape).  a/b are given by data + ndim + shape + strides (a view may be
 * strided); g is the contiguous output grad; ga/gb are contiguous grads of a's and b's shapes,
 * accumulated into (NULL = not needed). */
void or_binary_bwd(int op, int a_nd, const int64_t *a_shape, const int64_t *a_stride, const float *a, int b_nd,
                   const int64_t *b_shape, const int64_t *b_stride, const float *b, const float *g, float *ga,
                   float *gb);

/* reductions over x viewed as [outer, R, inner] (contiguous); arg may be NULL for sum/mean */
void or_reduce_fwd(int kind, int64_t outer, int64_t R, int64_t inner, const float *x, float *y, int32_t *arg);
void or_reduce_bwd(int kind, int64_t outer, int64_t R, int64_t inner, const float *g, const int32_t *arg,
                   float *gi);

void or_softmax_fwd(int log_form, int64_t rows, int64_t C, const float *x, float *y);
void or_softmax_bwd(int log_form, int64_t rows, int64_t C, const float *y, const float *g, float *gi);

/* stats: [rows][2] = {mean, rstd}; w/b may be NULL; gx/gw/gb may be NULL and accumulate */
void or_layer_norm_fwd(int64_t rows, int64_t D, const float *x, const float *w, const float *b, float eps,
                       float *y, float *stats);
void or_layer_norm_bwd(int64_t rows, int64_t D, const float *x, const float *w, const float *stats,
                       const float *g, float *gx, float *gw, float *gb);

void or_quantize_rows(int64_t rows, int64_t cols, const float *w, int8_t *q, float *scale);
void or_dequantize_rows(int64_t rows, int64_t cols, const int8_t *q, const float *scale, float *w);

/* int8 GEMM C[m][n] = sum_k A[m][k] B[n][k] in int32 (A [M, K] lda, B [N, K] ldb, C ldc) */
void or_gemm_s8_nt(int64_t M, int64_t N, int64_t K, const int8_t *A, int64_t lda, const int8_t *B, int64_t ldb,
                   int32_t *C, int64_t ldc);
/* linear_int8 forward: x [M, K] f32, wq [N, K] i8, ws [N], bias [N] or NULL -> y [M, N] */
void or_linear_int8(int64_t M, int64_t K, int64_t N, const float *x, const int8_t *wq, const float *ws,
                    const float *bias, float *y);

/* cross entropy over logits [N, C] with labels [N] (mean over rows): prob [N, C] receives
 * exp(log_softmax(x)), *loss the mean; returns -1, or the first row whose label is outside [0, C). */
int64_t or_cross_entropy_fwd(int64_t N, int64_t C, const float *x, const int32_t *lab, float *prob, float *loss);
/* gi (accumulated) += (gout / N) * prob; gi[i, lab_i] -= gout / N */
void or_cross_entropy_bwd(int64_t N, int64_t C, const float *prob, const int32_t *lab, float gout, float *gi);
/* nll loss over log-probabilities [N, C]: -sum of x[i, lab_i], or its mean (sum == 0); returns -1 or
 * the first row with an out-of-range label */
int64_t or_nll_loss_fwd(int64_t N, int64_t C, const float *x, const int32_t *lab, int sum, float *loss);
void or_nll_loss_bwd(int64_t N, int64_t C, const int32_t *lab, float gout, int sum, float *gi);

/* One optimizer update of one parameter (optim.c:161-216), the reference's fp32 expressions in its
 * order without fused multiply-adds.  kind: 0 SGD, 1 Adam, 2 AdamW, 3 RMSprop (OR_OPT_*); s1 / s2
 * may be NULL when that state does not exist; gs = 1 / accumulation steps; bc1 / bc2 = Adam's
 * 1 - beta^t. */
enum { OR_OPT_SGD = 0, OR_OPT_ADAM = 1, OR_OPT_ADAMW = 2, OR_OPT_RMSPROP = 3 };
void or_optim_step(int kind, int64_t n, float *w, const float *g, float *s1, float *s2, float lr, float momentum,
                   float weight_decay, float beta1, float beta2, float eps, float gs, float bc1, float bc2,
                   int eps_inside_sqrt);
/* sum of squares in double, as clip_grad_norm accumulates it (optim.c:217-223) */
double or_sumsq(int64_t n, const float *x);

#ifdef __cplusplus
}
#endif
#endif
