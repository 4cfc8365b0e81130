// Activation forward / backward over contiguous fp32 (the reference's unary_fwd_span /
// unary_bwd_span, ops_elementwise.c:229-338).
//
// HBM-bound streaming maps: 128-bit vector loads/stores (4 floats per lane), non-temporal hints so
// the 2^28-element streams do not thrash L2/MALL.  Launch shape: one wave64 per workgroup and one
// float4 per lane, with a grid that covers the whole array (one pass; the grid-stride loop only runs
// again past 2^24 workgroups per 256 CUs).  Measured on MI355X this moves 6.4-6.6 TB/s where a grid
// sized to the CUs with 4 vectors per lane looping over the array moved 5.5-5.8.  One template
// instance per activation so the per-element arithmetic is straight-line code.
#include "common.hpp"

namespace nchip {

// log and pow, which the reference takes from the host libm (logf, powf: errors under one ulp, nearly
// always the correctly rounded result), are evaluated here in double precision and rounded once to
// float: the correctly rounded result except where the exact value lies within ~2^-29 of a rounding
// boundary, so they agree with the host libm wherever it rounds correctly.  The single-precision
// device functions differ from it by 1-2 ulp on 15-47% of inputs.  Special values (negative, zero,
// infinite and NaN arguments) follow the C rules of the double functions, which match the float ones.
__device__ __forceinline__ float log_cr(float v) { return (float)log((double)v); }
__device__ __forceinline__ float pow_cr(float v, float s) { return (float)pow((double)v, (double)s); }

template <int K>
__device__ __forceinline__ float act_fwd(float v, float s) {
    constexpr float sixth = 1.0f / 6.0f;
    if constexpr (K == NC_HIP_UN_RELU) return v > 0.0f ? v : 0.0f;
    else if constexpr (K == NC_HIP_UN_LEAKY_RELU) return v > 0.0f ? v : s * v;
    else if constexpr (K == NC_HIP_UN_RELU6) return ref_fminf(ref_fmaxf(v, 0.0f), 6.0f);
    else if constexpr (K == NC_HIP_UN_HARDSIGMOID) return ref_fminf(ref_fmaxf(v * sixth + 0.5f, 0.0f), 1.0f);
    else if constexpr (K == NC_HIP_UN_HARDSWISH) return (v * ref_fminf(ref_fmaxf(v + 3.0f, 0.0f), 6.0f)) * sixth;
    else if constexpr (K == NC_HIP_UN_SILU) return sigmoid8(v) * v;
    else if constexpr (K == NC_HIP_UN_GELU) return (0.5f * v) * (1.0f + erf8(NC_K_SQRT1_2 * v));
    else if constexpr (K == NC_HIP_UN_GELU_TANH) {
        const float u = NC_K_SQRT_2_PI * (v + ((NC_K_GELU_C * v) * v) * v);
        return (0.5f * v) * (1.0f + tanh8(u));
    } else if constexpr (K == NC_HIP_UN_SIGMOID) return sigmoid8(v);
    else if constexpr (K == NC_HIP_UN_TANH) return tanh8(v);
    else if constexpr (K == NC_HIP_UN_EXP) return exp8(v);
    else if constexpr (K == NC_HIP_UN_NEG) return -1.0f * v;
    else if constexpr (K == NC_HIP_UN_SCALE) return s * v;
    else if constexpr (K == NC_HIP_UN_ADD_SCALAR) return v + s;
    else if constexpr (K == NC_HIP_UN_LOG) return log_cr(v);
    else if constexpr (K == NC_HIP_UN_SQRT) return sqrtf(v);
    else return pow_cr(v, s);
}

// What each backward kind reads besides g.
template <int K>
struct BwdReads {
    static constexpr bool y = K == NC_HIP_UN_SIGMOID || K == NC_HIP_UN_TANH || K == NC_HIP_UN_EXP ||
                              K == NC_HIP_UN_SQRT;
    static constexpr bool x = !y && K != NC_HIP_UN_NEG && K != NC_HIP_UN_SCALE && K != NC_HIP_UN_ADD_SCALAR;
};

// gi_new from gi_old; the fused kinds are the reference's axpy_f32 (neg, scale, add_scalar).
template <int K>
__device__ __forceinline__ float act_bwd(float gi, float v, float y, float g, float s) {
    constexpr float sixth = 1.0f / 6.0f, third = 1.0f / 3.0f;
    if constexpr (K == NC_HIP_UN_NEG) return fma_(-1.0f, g, gi);
    else if constexpr (K == NC_HIP_UN_SCALE) return fma_(s, g, gi);
    else if constexpr (K == NC_HIP_UN_ADD_SCALAR) return fma_(1.0f, g, gi);
    else {
        float t;
        if constexpr (K == NC_HIP_UN_RELU) t = v > 0.0f ? g : 0.0f;
        else if constexpr (K == NC_HIP_UN_LEAKY_RELU) t = v > 0.0f ? g : s * g;
        else if constexpr (K == NC_HIP_UN_RELU6) t = (v > 0.0f && v < 6.0f) ? g : 0.0f;
        else if constexpr (K == NC_HIP_UN_HARDSIGMOID) t = (v > -3.0f && v < 3.0f) ? g * sixth : 0.0f;
        else if constexpr (K == NC_HIP_UN_HARDSWISH) t = v < -3.0f ? 0.0f : v <= 3.0f ? g * (v * third + 0.5f) : g;
        else if constexpr (K == NC_HIP_UN_SILU) {
            const float sg = sigmoid8(v);
            t = (g * sg) * (1.0f + v * (1.0f - sg));
        } else if constexpr (K == NC_HIP_UN_GELU) {
            const float e = erf8(NC_K_SQRT1_2 * v);
            const float q = exp8_nonpos((-0.5f * v) * v);  // -v^2 / 2 <= 0 (or NaN)
            t = g * (0.5f * (1.0f + e) + (v * NC_K_INV_SQRT_2PI) * q);
        } else if constexpr (K == NC_HIP_UN_GELU_TANH) {
            const float th = tanh8(NC_K_SQRT_2_PI * (v + ((NC_K_GELU_C * v) * v) * v));
            const float dt = ((1.0f - th * th) * NC_K_SQRT_2_PI) * (1.0f + ((3.0f * NC_K_GELU_C) * v) * v);
            t = g * (0.5f * (1.0f + th) + (0.5f * v) * dt);
        } else if constexpr (K == NC_HIP_UN_SIGMOID) t = (g * y) * (1.0f - y);
        else if constexpr (K == NC_HIP_UN_TANH) t = g * (1.0f - y * y);
        else if constexpr (K == NC_HIP_UN_EXP) t = g * y;
        else if constexpr (K == NC_HIP_UN_LOG) t = g / v;
        else if constexpr (K == NC_HIP_UN_SQRT) t = (g * 0.5f) / y;
        else t = (g * s) * pow_cr(v, s - 1.0f);
        return gi + t;
    }
}

// Launch shape: NC_UNARY_BLOCK-lane workgroups, NC_UNARY_UNROLL 128-bit vectors per lane,
// NC_UNARY_GRID_PER_CU workgroups per CU at most (grid-stride beyond that); non-temporal hints on the
// streamed loads / stores.  Defaults chosen by sweeping them on MI355X (64 / 1 / whole array).
#ifndef NC_UNARY_UNROLL
#define NC_UNARY_UNROLL 1
#endif
#ifndef NC_UNARY_GRID_PER_CU
#define NC_UNARY_GRID_PER_CU 65536
#endif
#ifndef NC_UNARY_NT_LOAD
#define NC_UNARY_NT_LOAD 1
#endif
#ifndef NC_UNARY_NT_STORE
#define NC_UNARY_NT_STORE 1
#endif

#ifndef NC_UNARY_BLOCK
#define NC_UNARY_BLOCK 64
#endif
constexpr int kBlock = NC_UNARY_BLOCK;
constexpr int kUnroll = NC_UNARY_UNROLL;

template <typename T>
__device__ __forceinline__ T ld_nt(const T *p) {
    if constexpr (NC_UNARY_NT_LOAD) return __builtin_nontemporal_load(p);
    else return *p;
}
template <typename T>
__device__ __forceinline__ void st_nt(T v, T *p) {
    if constexpr (NC_UNARY_NT_STORE) __builtin_nontemporal_store(v, p);
    else *p = v;
}

template <int K>
__global__ __launch_bounds__(kBlock) void k_unary_fwd(const f4 *__restrict__ x, f4 *__restrict__ y, int64_t nvec,
                                                      float s) {
    const int64_t step = (int64_t)gridDim.x * kBlock * kUnroll;
    for (int64_t base = (int64_t)blockIdx.x * kBlock * kUnroll + threadIdx.x; base < nvec; base += step) {
        f4 v[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; u++) {
            const int64_t j = base + u * kBlock;
            if (j < nvec) v[u] = ld_nt(x + j);
        }
#pragma unroll
        for (int u = 0; u < kUnroll; u++) {
            const int64_t j = base + u * kBlock;
            if (j < nvec) {
                f4 r;
                r.x = act_fwd<K>(v[u].x, s);
                r.y = act_fwd<K>(v[u].y, s);
                r.z = act_fwd<K>(v[u].z, s);
                r.w = act_fwd<K>(v[u].w, s);
                st_nt(r, y + j);
            }
        }
    }
}

template <int K>
__global__ __launch_bounds__(kBlock) void k_unary_fwd_scalar(const float *__restrict__ x, float *__restrict__ y,
                                                             int64_t n, float s) {
    const int64_t step = (int64_t)gridDim.x * kBlock;
    for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += step) y[i] = act_fwd<K>(x[i], s);
}

template <int K, bool ACC>
__global__ __launch_bounds__(kBlock) void k_unary_bwd(const f4 *__restrict__ x, const f4 *__restrict__ y,
                                                      const f4 *__restrict__ g, f4 *__restrict__ gi, int64_t nvec,
                                                      float s) {
    constexpr bool RX = BwdReads<K>::x, RY = BwdReads<K>::y;
    const int64_t step = (int64_t)gridDim.x * kBlock * kUnroll;
    for (int64_t base = (int64_t)blockIdx.x * kBlock * kUnroll + threadIdx.x; base < nvec; base += step) {
        f4 vx[kUnroll], vy[kUnroll], vg[kUnroll], vo[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; u++) {
            const int64_t j = base + u * kBlock;
            if (j < nvec) {
                if constexpr (RX) vx[u] = ld_nt(x + j);
                else vx[u] = f4{0.f, 0.f, 0.f, 0.f};
                if constexpr (RY) vy[u] = ld_nt(y + j);
                else vy[u] = f4{0.f, 0.f, 0.f, 0.f};
                vg[u] = ld_nt(g + j);
                if constexpr (ACC) vo[u] = ld_nt(gi + j);
                else vo[u] = f4{0.f, 0.f, 0.f, 0.f};
            }
        }
#pragma unroll
        for (int u = 0; u < kUnroll; u++) {
            const int64_t j = base + u * kBlock;
            if (j < nvec) {
                f4 r;
                r.x = act_bwd<K>(vo[u].x, vx[u].x, vy[u].x, vg[u].x, s);
                r.y = act_bwd<K>(vo[u].y, vx[u].y, vy[u].y, vg[u].y, s);
                r.z = act_bwd<K>(vo[u].z, vx[u].z, vy[u].z, vg[u].z, s);
                r.w = act_bwd<K>(vo[u].w, vx[u].w, vy[u].w, vg[u].w, s);
                // an opaque value: the compiler otherwise folds hardswish's selects into the store and
                // drops its non-temporal hint (686 against 655 us for the other 2^28 backward maps)
                asm volatile("" : "+v"(r));
                st_nt(r, gi + j);
            }
        }
    }
}

template <int K, bool ACC>
__global__ __launch_bounds__(kBlock) void k_unary_bwd_scalar(const float *__restrict__ x, const float *__restrict__ y,
                                                             const float *__restrict__ g, float *__restrict__ gi,
                                                             int64_t n, float s) {
    constexpr bool RX = BwdReads<K>::x, RY = BwdReads<K>::y;
    const int64_t step = (int64_t)gridDim.x * kBlock;
    for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += step) {
        const float vx = RX ? x[i] : 0.0f, vy = RY ? y[i] : 0.0f;
        gi[i] = act_bwd<K>(ACC ? gi[i] : 0.0f, vx, vy, g[i], s);
    }
}

template <int K>
static int launch_fwd(float s, const float *x, float *y, int64_t n, hipStream_t st) {
    const int64_t nvec = (aligned16(x) && aligned16(y)) ? n / 4 : 0;
    if (nvec > 0) {
        hipLaunchKernelGGL(k_unary_fwd<K>, dim3(stream_grid((nvec + kUnroll - 1) / kUnroll, kBlock, NC_UNARY_GRID_PER_CU)), dim3(kBlock), 0,
                           st, (const f4 *)x, (f4 *)y, nvec, s);
    }
    const int64_t done = nvec * 4;
    if (done < n) {
        hipLaunchKernelGGL(k_unary_fwd_scalar<K>, dim3(stream_grid(n - done, kBlock)), dim3(kBlock), 0, st, x + done,
                           y + done, n - done, s);
    }
    return check_launch("nc_hip_unary_fwd");
}

template <int K, bool ACC>
static int launch_bwd2(float s, const float *x, const float *y, const float *g, float *gi, int64_t n, hipStream_t st) {
    const bool al = (!x || aligned16(x)) && (!y || aligned16(y)) && aligned16(g) && aligned16(gi);
    const int64_t nvec = al ? n / 4 : 0;
    if (nvec > 0) {
        hipLaunchKernelGGL((k_unary_bwd<K, ACC>), dim3(stream_grid((nvec + kUnroll - 1) / kUnroll, kBlock, NC_UNARY_GRID_PER_CU)),
                           dim3(kBlock), 0, st, (const f4 *)x, (const f4 *)y, (const f4 *)g, (f4 *)gi, nvec, s);
    }
    const int64_t done = nvec * 4;
    if (done < n) {
        hipLaunchKernelGGL((k_unary_bwd_scalar<K, ACC>), dim3(stream_grid(n - done, kBlock)), dim3(kBlock), 0, st,
                           x ? x + done : nullptr, y ? y + done : nullptr, g + done, gi + done, n - done, s);
    }
    return check_launch("nc_hip_unary_bwd");
}

template <int K>
static int launch_bwd(float s, const float *x, const float *y, const float *g, float *gi, int64_t n, int acc,
                      hipStream_t st) {
    if (BwdReads<K>::x && !x) return set_error(NC_HIP_ERR_ARG, "nc_hip_unary_bwd: kind %d needs x", K);
    if (BwdReads<K>::y && !y) return set_error(NC_HIP_ERR_ARG, "nc_hip_unary_bwd: kind %d needs y", K);
    const float *xx = BwdReads<K>::x ? x : nullptr, *yy = BwdReads<K>::y ? y : nullptr;
    return acc ? launch_bwd2<K, true>(s, xx, yy, g, gi, n, st) : launch_bwd2<K, false>(s, xx, yy, g, gi, n, st);
}

}  // namespace nchip

using namespace nchip;

#define NC_UNARY_DISPATCH(FN, ...)                                      \
    switch (kind) {                                                     \
    case NC_HIP_UN_RELU: return FN<NC_HIP_UN_RELU>(__VA_ARGS__);         \
    case NC_HIP_UN_LEAKY_RELU: return FN<NC_HIP_UN_LEAKY_RELU>(__VA_ARGS__); \
    case NC_HIP_UN_RELU6: return FN<NC_HIP_UN_RELU6>(__VA_ARGS__);       \
    case NC_HIP_UN_HARDSIGMOID: return FN<NC_HIP_UN_HARDSIGMOID>(__VA_ARGS__); \
    case NC_HIP_UN_HARDSWISH: return FN<NC_HIP_UN_HARDSWISH>(__VA_ARGS__); \
    case NC_HIP_UN_SILU: return FN<NC_HIP_UN_SILU>(__VA_ARGS__);         \
    case NC_HIP_UN_GELU: return FN<NC_HIP_UN_GELU>(__VA_ARGS__);         \
    case NC_HIP_UN_GELU_TANH: return FN<NC_HIP_UN_GELU_TANH>(__VA_ARGS__); \
    case NC_HIP_UN_SIGMOID: return FN<NC_HIP_UN_SIGMOID>(__VA_ARGS__);   \
    case NC_HIP_UN_TANH: return FN<NC_HIP_UN_TANH>(__VA_ARGS__);         \
    case NC_HIP_UN_EXP: return FN<NC_HIP_UN_EXP>(__VA_ARGS__);           \
    case NC_HIP_UN_NEG: return FN<NC_HIP_UN_NEG>(__VA_ARGS__);           \
    case NC_HIP_UN_SCALE: return FN<NC_HIP_UN_SCALE>(__VA_ARGS__);       \
    case NC_HIP_UN_ADD_SCALAR: return FN<NC_HIP_UN_ADD_SCALAR>(__VA_ARGS__); \
    case NC_HIP_UN_LOG: return FN<NC_HIP_UN_LOG>(__VA_ARGS__);           \
    case NC_HIP_UN_SQRT: return FN<NC_HIP_UN_SQRT>(__VA_ARGS__);         \
    case NC_HIP_UN_POW: return FN<NC_HIP_UN_POW>(__VA_ARGS__);           \
    default: return set_error(NC_HIP_ERR_ARG, "unknown activation kind %d", kind); \
    }

extern "C" NC_HIP_API int nc_hip_unary_fwd(int kind, float s, const float *x, float *y, int64_t n, void *stream) {
    if (n < 0 || (n > 0 && (!x || !y))) return set_error(NC_HIP_ERR_ARG, "nc_hip_unary_fwd: bad arguments");
    if (n == 0) return NC_HIP_OK;
    NC_UNARY_DISPATCH(launch_fwd, s, x, y, n, as_stream(stream))
}

extern "C" NC_HIP_API int nc_hip_unary_bwd(int kind, float s, const float *x, const float *y, const float *g,
                                           float *gi, int64_t n, int accumulate, void *stream) {
    if (n < 0 || (n > 0 && (!g || !gi))) return set_error(NC_HIP_ERR_ARG, "nc_hip_unary_bwd: bad arguments");
    if (n == 0) return NC_HIP_OK;
    NC_UNARY_DISPATCH(launch_bwd, s, x, y, g, gi, n, accumulate, as_stream(stream))
}
