/* Test-only probe compiled together with the reference engine sources into
 * oracle/_ref/libnc_ref.so (see oracle/Makefile).  It exposes the reference's
 * internal kernel-table entries, which the public nc.h API only reaches
 * inside composite ops, so the oracle's transcendental and summation
 * restatements can be compared with them directly.
 *
 * Reference interfaces used (read-only, compiled in place):
 *   engine/src/kernels/kernels.h:9-44      nc_kernels table
 *   engine/src/kernels/dispatch.c:35-47    nc__select_kernels (avx2 tier on x86 with AVX2+FMA)
 *   engine/src/kernels/x86/kernels_avx2.c  exp8/sigmoid8/tanh8/erf8/sum_f32/axpy_f32,
 *                                          gemm_f32 (:298-303), gemm_s8_nt (:314-340)
 */
#include "kernels.h"
#include "../core/nc_internal.h"

#include <stdint.h>

static const nc_kernels *probe_table(void) {
    static const nc_kernels *k;
    if (!k) {
        nc_cpu_info cpu;
        nc__detect_cpu(&cpu);
        k = nc__select_kernels(&cpu, 0);
    }
    return k;
}

const char *ncref_backend(void) { return probe_table()->name; }
void ncref_exp_f32(int64_t n, const float *x, float *y) { probe_table()->exp_f32(n, x, y); }
void ncref_sigmoid_f32(int64_t n, const float *x, float *y) { probe_table()->sigmoid_f32(n, x, y); }
void ncref_tanh_f32(int64_t n, const float *x, float *y) { probe_table()->tanh_f32(n, x, y); }
void ncref_erf_f32(int64_t n, const float *x, float *y) { probe_table()->erf_f32(n, x, y); }
float ncref_sum_f32(int64_t n, const float *x) { return probe_table()->sum_f32(n, x); }
void ncref_axpy_f32(int64_t n, float alpha, const float *x, float *y) { probe_table()->axpy_f32(n, alpha, x, y); }
void ncref_gemm_f32(int ta, int tb, int64_t M, int64_t N, int64_t K, float alpha, const float *A, int64_t lda,
                    const float *B, int64_t ldb, float beta, float *C, int64_t ldc) {
    probe_table()->gemm_f32(ta, tb, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc);
}
void ncref_gemm_s8_nt(int64_t M, int64_t N, int64_t K, const int8_t *A, int64_t lda, const int8_t *B, int64_t ldb,
                      int32_t *C, int64_t ldc) {
    probe_table()->gemm_s8_nt(M, N, K, A, lda, B, ldb, C, ldc);
}

/* ---- per-op timing of the reference engine (the CPU baseline of the benchmark) ------------------
 * The public API times an op together with its dispatch and its output allocation (a fresh large
 * block is first-touched page by page).  These re-run the forward or backward function of the op
 * that produced `out` -- the reference's own code path, engine/src/ops/*.c -- on buffers that already
 * exist, and return the mean wall time of `reps` runs in seconds.  `out` must have been produced with
 * grad enabled and an input requiring grad, so its node is on the tape (autograd.c:55-64).
 * Reference interfaces used: nc_node / nc_op_def (nc_internal.h), nc__grad_buf (tensor.c:375-388). */
#include <string.h>
#include <time.h>

static double probe_now(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double)ts.tv_sec + 1e-9 * (double)ts.tv_nsec;
}

/* Temporaries an op allocates in one run (arena blocks logged as nc_backward_ex logs them,
 * autograd.c:160-168) go back to the arena after the run, so the next run reuses them instead of
 * first-touching new memory; `keep` leaves the last run's blocks (the forward's saved values) live. */
static void run_begin(nc_ctx *ctx) {
    ctx->bwd_logging = 1;
    ctx->bwd_tmp_n = 0;
}

static void run_end(nc_ctx *ctx, int keep) {
    ctx->bwd_logging = 0;
    if (!keep)
        for (int i = 0; i < ctx->bwd_tmp_n; i++) nc__arena_free(ctx, ctx->bwd_tmp[i], ctx->bwd_tmp_size[i]);
    ctx->bwd_tmp_n = 0;
}

/* One untimed run first (it sizes the arena's blocks), then `reps` timed runs. */
double ncref_time_forward(nc_tensor *out, int reps) {
    if (!out || !out->node || reps < 1) return -1.0;
    nc_node *n = out->node;
    nc_ctx *ctx = out->ctx;
    double t = 0.0;
    for (int r = -1; r < reps; r++) {
        run_begin(ctx);
        const double t0 = probe_now();
        const nc_status st = n->op->forward(n);
        const double t1 = probe_now();
        run_end(ctx, r == reps - 1);
        if (st != NC_OK) return -1.0;
        if (r >= 0) t += t1 - t0;
    }
    return t / reps;
}

/* out's gradient is set to g; every input gradient is zero-filled before each run (outside the
 * timed region, as nc_backward_ex clears intermediate grads, autograd.c:151-154), so each run is one
 * backward of the op into zeroed buffers. */
double ncref_time_backward(nc_tensor *out, const float *g, int reps) {
    if (!out || !out->node || !out->node->op->backward || reps < 1) return -1.0;
    nc_node *n = out->node;
    nc_ctx *ctx = out->ctx;
    nc_tensor *go = nc__grad_buf(out);
    if (!go) return -1.0;
    memcpy(go->data, g, (size_t)nc_numel(out) * sizeof(float));
    for (int i = 0; i < n->n_in; i++)
        if ((n->in[i]->flags & NC_TF_REQUIRES_GRAD) && !nc__grad_buf(n->in[i])) return -1.0;
    double t = 0.0;
    for (int r = -1; r < reps; r++) {
        for (int i = 0; i < n->n_in; i++) {
            nc_tensor *x = n->in[i];
            if (x->flags & NC_TF_REQUIRES_GRAD) memset(x->grad->data, 0, (size_t)nc_numel(x) * sizeof(float));
        }
        run_begin(ctx);
        const double t0 = probe_now();
        n->op->backward(n);
        const double t1 = probe_now();
        run_end(ctx, 0);
        if (r >= 0) t += t1 - t0;
    }
    return t / reps;
}
