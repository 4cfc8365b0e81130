// Shared pieces of the HIP kernel layer: vector types, the reference's transcendental
// approximations as device functions, wave/block reductions, launch and error helpers.
//
// Built for gfx950 only (wave64, 256 CUs in 8 XCDs, 160 KiB LDS/CU) with -ffp-contract=off:
// every fused multiply-add below is an explicit __builtin_fmaf placed where the reference's AVX2
// tier uses _mm256_fmadd_ps / _mm256_fnmadd_ps (kernels_avx2.c), so elementwise results match the
// reference bit for bit.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

#include "nc_hip.h"

namespace nchip {

typedef float f4 __attribute__((ext_vector_type(4)));
typedef float f2 __attribute__((ext_vector_type(2)));
typedef int i4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;

// Every split of a reduction into partial sums -- and so every rounding of its result -- is a
// function of the problem shape alone, planned for the 256 CUs of an MI355X whatever device runs
// it: the same inputs give the same bits on a part with another CU count or partition mode.  The
// device's own count (num_cus) sizes only the grids of grid-stride kernels whose partials do not
// depend on the grid.
constexpr int kPlanCUs = 256;

// ------------------------------------------------------------------------------------------------
// errors (thread-local detail string, nc_hip_last_error)
// ------------------------------------------------------------------------------------------------
int set_error(int code, const char *fmt, ...);
int check_launch(const char *what);
// Compute units that grids are sized for: the current device's count (cached per device), or the
// override set by nc_hip_set_grid_cus / the NC_HIP_CUS environment variable.  Grid size only:
// nothing that fixes a summation order may depend on it (see kPlanCUs).
int num_cus();
hipStream_t as_stream(void *s);

// ------------------------------------------------------------------------------------------------
// transcendental maps of the reference's AVX2 tier (kernels_avx2.c:74-178).  Constants are the
// reference's published-method coefficients: Cephes expf degree-6 polynomial with Cody-Waite
// ln2 split, an odd Taylor tanh series below |x| < 0.25, Abramowitz & Stegun 7.1.26 for erf.
// ------------------------------------------------------------------------------------------------
#define NC_K_EXP_HI 88.8f
#define NC_K_EXP_LO -87.3365448f
#define NC_K_LOG2E 1.44269504088896341f
#define NC_K_LN2_HI 0.693359375f
#define NC_K_LN2_LO -2.12194440e-4f
#define NC_K_TANH_SMALL 0.25f
#define NC_K_SQRT1_2 0.70710678118654752f
#define NC_K_INV_SQRT_2PI 0.39894228040143268f
#define NC_K_SQRT_2_PI 0.79788456080286536f
#define NC_K_GELU_C 0.044715f

__device__ __forceinline__ float fma_(float a, float b, float c) { return __builtin_fmaf(a, b, c); }

// exp8: clamp (NaN -> LO through the compare-select), n = floor(x log2e + 1/2), r = x - n ln2 in two
// fused steps, degree-6 polynomial, 2^n assembled in the exponent field (n = 128 as 2^127 * 2),
// zero below LO, NaN passed through.
__device__ __forceinline__ float exp8_poly(float xc, int &n) {  // p(r) for a clamped argument; n
    const float fx = __builtin_floorf(fma_(xc, NC_K_LOG2E, 0.5f));
    float r = fma_(-fx, NC_K_LN2_HI, xc);
    r = fma_(-fx, NC_K_LN2_LO, r);
    float y = 1.9875691500e-4f;
    y = fma_(y, r, 1.3981999507e-3f);
    y = fma_(y, r, 8.3334519073e-3f);
    y = fma_(y, r, 4.1665795894e-2f);
    y = fma_(y, r, 1.6666665459e-1f);
    y = fma_(y, r, 5.0000001201e-1f);
    y = fma_(y, r * r, r + 1.0f);
    n = (int)fx;
    return y;
}

__device__ __forceinline__ float exp8(float x) {
    const float x0 = x;
    float xc = x > NC_K_EXP_LO ? x : NC_K_EXP_LO;
    xc = xc < NC_K_EXP_HI ? xc : NC_K_EXP_HI;
    int n;
    const float y = exp8_poly(xc, n);
    const int big = n > 127;
    n -= big;
    float res = y * __int_as_float((n + 127) << 23);
    res = res * (big ? 2.0f : 1.0f);
    res = x0 < NC_K_EXP_LO ? 0.0f : res;
    return x0 != x0 ? x0 : res;
}

// exp8 for arguments that are <= 0 or NaN (x minus its row maximum, log-probabilities): there the
// upper clamp is inactive and n <= 0, so the 2^128 split multiplies by 1; both are dropped, and the
// result is bit-identical to exp8 on that domain.
__device__ __forceinline__ float exp8_nonpos(float x) {
    const float x0 = x;
    const float xc = x > NC_K_EXP_LO ? x : NC_K_EXP_LO;
    int n;
    const float y = exp8_poly(xc, n);
    float res = y * __int_as_float((n + 127) << 23);
    res = x0 < NC_K_EXP_LO ? 0.0f : res;
    return x0 != x0 ? x0 : res;
}

__device__ __forceinline__ float sigmoid8(float x) { return 1.0f / (1.0f + exp8(0.0f - x)); }

__device__ __forceinline__ float tanh8(float x) {
    const unsigned sign = __float_as_uint(x) & 0x80000000u;
    const float ax = __uint_as_float(__float_as_uint(x) & 0x7fffffffu);
    const float e = exp8(ax * -2.0f);
    float big = (1.0f - e) / (1.0f + e);
    big = __uint_as_float(__float_as_uint(big) | sign);
    const float z = x * x;
    float p = fma_(0.021869489f, z, -0.053968254f);
    p = fma_(p, z, 0.133333333f);
    p = fma_(p, z, -0.333333333f);
    p = fma_(p * z, x, x);
    return ax < NC_K_TANH_SMALL ? p : big;
}

__device__ __forceinline__ float erf8(float x) {
    const unsigned sign = __float_as_uint(x) & 0x80000000u;
    const float ax = __uint_as_float(__float_as_uint(x) & 0x7fffffffu);
    const float t = 1.0f / fma_(ax, 0.3275911f, 1.0f);
    float p = fma_(1.061405429f, t, -1.453152027f);
    p = fma_(p, t, 1.421413741f);
    p = fma_(p, t, -0.284496736f);
    p = fma_(p, t, 0.254829592f);
    const float e = exp8(0.0f - ax * ax);
    const float r = fma_(-(p * t), e, 1.0f);
    return __uint_as_float(__float_as_uint(r) | sign);
}

// fminf/fmaxf as the reference's glibc calls behave on x86-64 (NaN operand ignored; for equal
// operands, including -0 vs +0, the second argument).  Pinned by the special-value golden vectors.
__device__ __forceinline__ float ref_fmaxf(float a, float b) {
    if (a != a) return b;
    if (b != b) return a;
    return a > b ? a : b;
}
__device__ __forceinline__ float ref_fminf(float a, float b) {
    if (a != a) return b;
    if (b != b) return a;
    return a < b ? a : b;
}

// ------------------------------------------------------------------------------------------------
// wave64 reductions (__shfl_xor: ds_bpermute / DPP lane exchanges)
// ------------------------------------------------------------------------------------------------
// max of a row with the reference's scan semantics (ops_nn.c:23-25): NaN at index 0 wins, later
// NaNs are skipped (fmaxf ignores them, order-free), otherwise the plain maximum.
__device__ __forceinline__ float row_max_finish(float m_nonnan, float x0) { return x0 != x0 ? x0 : m_nonnan; }

// Workgroup barrier for LDS traffic only: waits for this wave's LDS operations, then meets the
// other waves.  Unlike __syncthreads(), whose fence also waits for every outstanding global load,
// it leaves prefetched global loads in flight.  The memory clobber keeps the compiler from moving
// memory accesses across it.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

__device__ __forceinline__ double wave_sum(double v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
    return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
    return v;
}
__device__ __forceinline__ float wave_max_nan_skip(float v) {  // fmaxf semantics, order-free
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = __builtin_fmaxf(v, __shfl_xor(v, o, kWave));
    return v;
}

// ------------------------------------------------------------------------------------------------
// 64-bit strided index decomposition for up to 6 dims (row-major, last dim fastest)
// ------------------------------------------------------------------------------------------------
struct Dims {
    int nd;
    int64_t shape[NC_HIP_MAX_DIMS];
};

template <int NOPS>
struct Strides {
    int64_t s[NOPS][NC_HIP_MAX_DIMS];
};

// Merges adjacent dims that are contiguous with each other for every operand, drops size-1 dims.
// Returns the new dim count; shape/strides are rewritten in place (nops operands).
int coalesce(int nd, int64_t *shape, int nops, int64_t (*st)[NC_HIP_MAX_DIMS]);

inline bool aligned16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

// grid size for a grid-stride streaming kernel: enough blocks to fill every CU `per_cu` times
inline unsigned stream_grid(int64_t work_items, int block, int per_cu = 8) {
    int64_t need = (work_items + block - 1) / block;
    int64_t cap = (int64_t)num_cus() * per_cu;
    if (need < 1) need = 1;
    return (unsigned)(need < cap ? need : cap);
}

}  // namespace nchip
