/* Test-only probe compiled together with the reference engine sources into
 * oracle/_ref/libnc_ref.so (see oracle/Makefile).  It exposes the reference's
 * internal kernel-table entries, which the public nc.h API only reaches
 * inside composite ops, so the oracle's transcendental and summation
 * restatements can be compared with them directly.
 *
 * Reference interfaces used (read-only, compiled in place):
 *   engine/src/kernels/kernels.h:9-44      nc_kernels table
 *   engine/src/kernels/dispatch.c:35-47    nc__select_kernels (avx2 tier on x86 with AVX2+FMA)
 *   engine/src/kernels/x86/kernels_avx2.c  exp8/sigmoid8/tanh8/erf8/sum_f32/axpy_f32
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
