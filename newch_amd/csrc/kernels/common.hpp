// Shared pieces of the HIP kernel layer: vector types, the reference's transcendental
// approximations as device functions, wave/block reductions, launch and error helpers.
//
// Built for gfx950 only (wave64, 256 CUs in 8 XCDs, 160 KiB LDS/CU) with -ffp-contract=off:
// every fused multiply-add below is an explicit __builtin_fmaf placed where the reference's AVX2
// tier uses _mm256_fmadd_ps / _mm256_fnmadd_ps (kernels_avx2.c), so elementwise results match the
// reference bit for bit.
#pragma once

#include <hip/hip_runtime.h>
#include <type_traits>
#include <stdint.h>
#include <stddef.h>
#include <stdlib.h>

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

// exp8 for arguments that are <= 0 or NaN (x minus its row maximum, log-probabilities, erf's and
// tanh's exponentials, GELU's Gaussian): there the
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

// exp(x) for x <= 0 (or NaN) through the hardware base-2 exponential: within a few ulp of exp8 on
// that domain, at a fraction of its instructions.  Only for terms of a row sum whose total is
// compared at the reductions' tolerance (the log-sum-exp of log_softmax and cross entropy); every
// value that is an output, or is recomputed bit for bit later, uses exp8.
__device__ __forceinline__ float exp_sum_term(float x) { return __builtin_amdgcn_exp2f(x * NC_K_LOG2E); }

__device__ __forceinline__ float tanh8(float x) {
    const unsigned sign = __float_as_uint(x) & 0x80000000u;
    const float ax = __uint_as_float(__float_as_uint(x) & 0x7fffffffu);
    const float e = exp8_nonpos(ax * -2.0f);  // ax * -2 <= 0 (or NaN)
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
    const float e = exp8_nonpos(0.0f - ax * ax);  // <= 0 (or NaN)
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
// wave64 reductions
// ------------------------------------------------------------------------------------------------
// max of a row with the reference's scan semantics (ops_nn.c:23-25): NaN at index 0 wins, later
// NaNs are skipped (fmaxf ignores them, order-free), otherwise the plain maximum.
__device__ __forceinline__ float row_max_finish(float m_nonnan, float x0) { return x0 != x0 ? x0 : m_nonnan; }

// Workgroup barrier for LDS traffic only: waits for this wave's LDS operations, then meets the
// other waves.  Unlike __syncthreads(), whose fence also waits for every outstanding global load,
// it leaves prefetched global loads in flight.  The memory clobber keeps the compiler from moving
// memory accesses across it.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Reductions over all 64 lanes by DPP lane moves, with no LDS crossbar (ds_bpermute) round trips:
// pairs (lane xor 1, xor 2) within quads, the half-row and row mirrors leave every lane of a 16-lane
// row with the row's result, then row 15 -> rows 1, 3 and lane 31 -> rows 2, 3 leave the wave's
// result in lane 63, which is broadcast (readlane) to every lane.  A fixed order, so deterministic.
// Every lane of the wave must be active (the kernels call these in wave-uniform control flow).
template <int CTRL, int ROWMASK = 0xf>
__device__ __forceinline__ int dpp_i32(int v, int old) {
    return __builtin_amdgcn_update_dpp(old, v, CTRL, ROWMASK, 0xf, false);
}
template <int CTRL, int ROWMASK = 0xf>
__device__ __forceinline__ float dpp_f32(float v, float old) {
    return __int_as_float(dpp_i32<CTRL, ROWMASK>(__float_as_int(v), __float_as_int(old)));
}
template <int CTRL, int ROWMASK = 0xf>
__device__ __forceinline__ double dpp_f64(double v, double old) {
    union { double d; int i[2]; } a, o, r;
    a.d = v;
    o.d = old;
    r.i[0] = dpp_i32<CTRL, ROWMASK>(a.i[0], o.i[0]);
    r.i[1] = dpp_i32<CTRL, ROWMASK>(a.i[1], o.i[1]);
    return r.d;
}
__device__ __forceinline__ int lane63_i32(int v) { return __builtin_amdgcn_readlane(v, 63); }
__device__ __forceinline__ float lane63_f32(float v) { return __int_as_float(lane63_i32(__float_as_int(v))); }
__device__ __forceinline__ double lane63_f64(double v) {
    union { double d; int i[2]; } a;
    a.d = v;
    a.i[0] = lane63_i32(a.i[0]);
    a.i[1] = lane63_i32(a.i[1]);
    return a.d;
}
// DPP steps: quad_perm [1,0,3,2], quad_perm [2,3,0,1], row_half_mirror, row_mirror, then
// row_bcast:15 into rows 1 and 3 and row_bcast:31 into rows 2 and 3
enum : int { kDppXor1 = 0xB1, kDppXor2 = 0x4E, kDppHalfMirror = 0x141, kDppMirror = 0x140, kDppBcast15 = 0x142,
             kDppBcast31 = 0x143 };

__device__ __forceinline__ double wave_sum(double v) {
    v += dpp_f64<kDppXor1>(v, 0.0);
    v += dpp_f64<kDppXor2>(v, 0.0);
    v += dpp_f64<kDppHalfMirror>(v, 0.0);
    v += dpp_f64<kDppMirror>(v, 0.0);
    v += dpp_f64<kDppBcast15, 0xa>(v, 0.0);
    v += dpp_f64<kDppBcast31, 0xc>(v, 0.0);
    return lane63_f64(v);
}
__device__ __forceinline__ float wave_sum(float v) {
    v += dpp_f32<kDppXor1>(v, 0.0f);
    v += dpp_f32<kDppXor2>(v, 0.0f);
    v += dpp_f32<kDppHalfMirror>(v, 0.0f);
    v += dpp_f32<kDppMirror>(v, 0.0f);
    v += dpp_f32<kDppBcast15, 0xa>(v, 0.0f);
    v += dpp_f32<kDppBcast31, 0xc>(v, 0.0f);
    return lane63_f32(v);
}
__device__ __forceinline__ float wave_max_nan_skip(float v) {  // fmaxf semantics, order-free
    v = __builtin_fmaxf(v, dpp_f32<kDppXor1>(v, v));
    v = __builtin_fmaxf(v, dpp_f32<kDppXor2>(v, v));
    v = __builtin_fmaxf(v, dpp_f32<kDppHalfMirror>(v, v));
    v = __builtin_fmaxf(v, dpp_f32<kDppMirror>(v, v));
    v = __builtin_fmaxf(v, dpp_f32<kDppBcast15, 0xa>(v, v));
    v = __builtin_fmaxf(v, dpp_f32<kDppBcast31, 0xc>(v, v));
    return lane63_f32(v);
}
__device__ __forceinline__ unsigned long long wave_min_u64(unsigned long long v) {  // order-free
    auto step = [](unsigned long long a, unsigned long long moved) { return moved < a ? moved : a; };
    auto dpp = [](auto ctrl, unsigned long long x) {
        constexpr int C = decltype(ctrl)::value;
        constexpr int M = C == kDppBcast15 ? 0xa : C == kDppBcast31 ? 0xc : 0xf;
        const int lo = dpp_i32<C, M>((int)(uint32_t)x, (int)(uint32_t)x);
        const int hi = dpp_i32<C, M>((int)(uint32_t)(x >> 32), (int)(uint32_t)(x >> 32));
        return ((unsigned long long)(uint32_t)hi << 32) | (uint32_t)lo;
    };
    v = step(v, dpp(std::integral_constant<int, kDppXor1>{}, v));
    v = step(v, dpp(std::integral_constant<int, kDppXor2>{}, v));
    v = step(v, dpp(std::integral_constant<int, kDppHalfMirror>{}, v));
    v = step(v, dpp(std::integral_constant<int, kDppMirror>{}, v));
    v = step(v, dpp(std::integral_constant<int, kDppBcast15>{}, v));
    v = step(v, dpp(std::integral_constant<int, kDppBcast31>{}, v));
    const uint32_t lo = (uint32_t)lane63_i32((int)(uint32_t)v), hi = (uint32_t)lane63_i32((int)(uint32_t)(v >> 32));
    return ((unsigned long long)hi << 32) | lo;
}
// lane 0's value in every lane (the row's first element for the reference's NaN rule)
__device__ __forceinline__ float lane0_f32(float v) { return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(v))); }

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

// global_load_lds_dwordx4: each lane's 16 bytes at g land in LDS at M0 + 16 * lane (M0 = lds, the
// wave's destination; one wait state separates its write from the load).  Issued from inline assembly
// so the compiler does not wait for these loads before every LDS read: callers wait with explicit
// vmcnt counts.  The compiler treats M0 as reserved and does not honour the clobber: a kernel using
// this must touch M0 nowhere else (checked in its compiled code).
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma16(const void *g, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(lds), "v"(g) : "memory", "m0");
}
#pragma clang diagnostic pop

inline bool aligned16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

// ------------------------------------------------------------------------------------------------
// Problems past the 32-bit kernels' reach, cut into runs.  A problem of `nd` dims over `nops`
// operands (element strides st[o][d]) is tiled in index order by runs of at most `limit` elements:
// slabs of the outermost dim where a whole index of it fits, else, for each index of the outermost
// dim, the same cut one dim further in.  fn(run_shape, off, first) is called per run with the run's
// shape (the dims outside the cut dim become 1), each operand's element offset of the run's first
// element, and per operand whether the run is the first, in index order, to touch the elements that
// operand maps it to: false exactly when an earlier run differs from it only along dims where the
// operand's stride is 0 (an output reduced over a cut dim, which later runs add into).  Returns the
// first nonzero return of fn.
// ------------------------------------------------------------------------------------------------
constexpr int64_t kRunLimit = int64_t(1) << 30;

// When a problem runs as runs: above `above` elements, in runs of at most `limit`.  By default problems
// of 2^32 elements or more (past the 32-bit index kernels) run as runs of at most 2^30.  The test hook
// NC_HIP_RUN_LIMIT=n (0 < n < 2^30) lowers both to n, so that small problems take the split path.
struct RunSplit {
    int64_t above, limit;
};
inline RunSplit run_split() {
    if (const char *e = getenv("NC_HIP_RUN_LIMIT")) {
        const long long v = atoll(e);
        if (v > 0 && v < kRunLimit) return {(int64_t)v, (int64_t)v};
    }
    return {(int64_t)UINT32_MAX - 1, kRunLimit};
}

template <class F>
int for_each_run_from(int nd, const int64_t *shape, int nops, const int64_t *const *st, int64_t limit, int d,
                      const int64_t *off, const bool *first, F &fn) {
    int64_t inner = 1;
    for (int e = d + 1; e < nd; e++) inner *= shape[e];
    int64_t rs[NC_HIP_MAX_DIMS];
    for (int e = 0; e < nd; e++) rs[e] = e < d ? 1 : shape[e];
    int64_t o2[8];
    bool f2[8];
    if (inner <= limit || d == nd - 1) {
        const int64_t L = inner <= limit ? limit / inner : 1;
        for (int64_t r0 = 0; r0 < shape[d]; r0 += L) {
            rs[d] = shape[d] - r0 < L ? shape[d] - r0 : L;
            for (int o = 0; o < nops; o++) {
                o2[o] = off[o] + r0 * st[o][d];
                f2[o] = first[o] && (st[o][d] != 0 || r0 == 0);
            }
            const int rc = fn((const int64_t *)rs, (const int64_t *)o2, (const bool *)f2);
            if (rc) return rc;
        }
        return 0;
    }
    for (int64_t i = 0; i < shape[d]; i++) {
        for (int o = 0; o < nops; o++) {
            o2[o] = off[o] + i * st[o][d];
            f2[o] = first[o] && (st[o][d] != 0 || i == 0);
        }
        const int rc = for_each_run_from(nd, shape, nops, st, limit, d + 1, o2, f2, fn);
        if (rc) return rc;
    }
    return 0;
}

template <class F>
int for_each_run(int nd, const int64_t *shape, int nops, const int64_t *const *st, int64_t limit, F &&fn) {
    const int64_t off[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    const bool first[8] = {true, true, true, true, true, true, true, true};
    return nd > 0 ? for_each_run_from(nd, shape, nops, st, limit, 0, off, first, fn) : fn(shape, off, first);
}

inline int64_t numel_of(int nd, const int64_t *shape) {
    int64_t n = 1;
    for (int d = 0; d < nd; d++) n *= shape[d];
    return n;
}

// p advanced by off elements (NULL stays NULL)
template <typename T>
inline T *adv(T *p, int64_t off) { return p ? p + off : p; }

// grid size for a grid-stride streaming kernel: enough blocks to fill every CU `per_cu` times
inline unsigned stream_grid(int64_t work_items, int block, int per_cu = 8) {
    int64_t need = (work_items + block - 1) / block;
    int64_t cap = (int64_t)num_cus() * per_cu;
    if (need < 1) need = 1;
    return (unsigned)(need < cap ? need : cap);
}

}  // namespace nchip
