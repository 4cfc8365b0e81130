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
