// Optimizer updates and the gradient norm (optim.c:161-233).
//
// k_optim<KIND, ...>: one streaming pass over a parameter: w, g and the state the optimizer keeps
// read once, w and the state written once, 128-bit accesses (4 items in flight per lane) when every
// array is 16-byte aligned, one float per lane for the rest.  Per element the reference's scalar
// expression is evaluated in fp32, left to right, without fused multiply-adds (this file is compiled
// with -ffp-contract=off), with correctly rounded division and square root: updates are
// bit-identical to the reference's.  Constants the reference recomputes per element (1 - beta,
// AdamW's 1 - lr * wd) are computed once on the host with the same fp32 operations.
//
// k_sumsq + k_sumsq_finish: fp64 sum of squares (each square exact in fp64), workgroup partials in
// order and one ordered combine into a double that several tensors accumulate into.
#include "common.hpp"

#include <math.h>

#include <algorithm>

namespace nchip {

#ifndef NC_OPT_BLOCK
#define NC_OPT_BLOCK 64
#endif
#ifndef NC_OPT_GRID_PER_CU
#define NC_OPT_GRID_PER_CU 65536
#endif
constexpr int kOB = NC_OPT_BLOCK;

struct OptArgs {
    float lr, momentum, wd, b1, b2, eps, gs, bc1, bc2;
    float one_m_b1, one_m_b2;  // 1 - beta1, 1 - beta2 (RMSprop: 1 - alpha)
    float decay, l2;           // AdamW: w *= 1 - lr * wd; Adam: L2 term wd
    int inside;                // RMSprop: sqrt(v + eps) instead of sqrt(v) + eps
};

enum { K_SGD = 0, K_ADAM = 1, K_RMS = 3 };

template <int KIND, bool S1>
__device__ __forceinline__ void opt1(float &w, float g, float &s1, float &s2, const OptArgs &a) {
    if constexpr (KIND == K_SGD) {
        float gj = a.gs * g + a.wd * w;
        if constexpr (S1) {
            s1 = a.momentum * s1 + gj;
            gj = s1;
        }
        w = w - a.lr * gj;
    } else if constexpr (KIND == K_RMS) {
        const float gj = a.gs * g + a.wd * w;
        s2 = a.b2 * s2 + a.one_m_b2 * gj * gj;
        const float den = a.inside ? sqrtf(s2 + a.eps) : sqrtf(s2) + a.eps;
        float step = gj / den;
        if constexpr (S1) {
            s1 = a.momentum * s1 + step;
            step = s1;
        }
        w = w - a.lr * step;
    } else {
        w = w * a.decay;
        const float gj = a.gs * g + a.l2 * w;
        s1 = a.b1 * s1 + a.one_m_b1 * gj;
        s2 = a.b2 * s2 + a.one_m_b2 * gj * gj;
        w = w - a.lr * (s1 / a.bc1) / (sqrtf(s2 / a.bc2) + a.eps);
    }
}

#ifndef NC_OPT_NT
#define NC_OPT_NT 1
#endif
// the parameter and state streams: plain or non-temporal accesses
__device__ __forceinline__ f4 opt_ld(const f4 *p) {
    if constexpr (NC_OPT_NT) return __builtin_nontemporal_load(p);
    else return *p;
}
__device__ __forceinline__ void opt_st(f4 v, f4 *p) {
    if constexpr (NC_OPT_NT) __builtin_nontemporal_store(v, p);
    else *p = v;
}

// One float4 of every stream: a single load-compute-store body (with the loads and the stores in two
// separate unrolled loops, the optimizer rebuilt the stores and dropped their non-temporal hint:
// plain stores, 18% slower at 2^26 parameters).
template <int KIND, bool S1, bool S2>
__device__ __forceinline__ void opt_item4(f4 *__restrict__ w, const f4 *__restrict__ g, f4 *__restrict__ s1,
                                          f4 *__restrict__ s2, int64_t e, const OptArgs &a) {
    const f4 W = opt_ld(w + e), G = __builtin_nontemporal_load(g + e);
    const f4 A = S1 ? opt_ld(s1 + e) : f4{0.f, 0.f, 0.f, 0.f};
    const f4 B = S2 ? opt_ld(s2 + e) : f4{0.f, 0.f, 0.f, 0.f};
    float wv[4] = {W.x, W.y, W.z, W.w}, av[4] = {A.x, A.y, A.z, A.w}, bv[4] = {B.x, B.y, B.z, B.w};
    const float gv[4] = {G.x, G.y, G.z, G.w};
#pragma unroll
    for (int c = 0; c < 4; c++) opt1<KIND, S1>(wv[c], gv[c], av[c], bv[c], a);
    opt_st(f4{wv[0], wv[1], wv[2], wv[3]}, w + e);
    if constexpr (S1) opt_st(f4{av[0], av[1], av[2], av[3]}, s1 + e);
    if constexpr (S2) opt_st(f4{bv[0], bv[1], bv[2], bv[3]}, s2 + e);
}

template <int KIND, bool S1, bool S2>
__global__ __launch_bounds__(kOB) void k_optim4(f4 *__restrict__ w, const f4 *__restrict__ g, f4 *__restrict__ s1,
                                                f4 *__restrict__ s2, int64_t n4, OptArgs a) {
    const int64_t step = (int64_t)gridDim.x * kOB;
    for (int64_t e = (int64_t)blockIdx.x * kOB + threadIdx.x; e < n4; e += step) opt_item4<KIND, S1, S2>(w, g, s1, s2, e, a);
}

// Several parameters in one launch: parameter t owns workgroups first[t] .. first[t + 1] - 1, one
// float4 per lane, so a workgroup finds its parameter with a wave-uniform scan of the (at most
// NC_HIP_OPT_MULTI_MAX) boundaries and every element gets the single-parameter kernel's arithmetic.
struct OptMulti {
    f4 *w[NC_HIP_OPT_MULTI_MAX];
    const f4 *g[NC_HIP_OPT_MULTI_MAX];
    f4 *s1[NC_HIP_OPT_MULTI_MAX];
    f4 *s2[NC_HIP_OPT_MULTI_MAX];
    int64_t n4[NC_HIP_OPT_MULTI_MAX];
    int64_t first[NC_HIP_OPT_MULTI_MAX + 1];
    int count;
};

template <int KIND, bool S1, bool S2>
__global__ __launch_bounds__(kOB) void k_optim4_multi(OptMulti m, OptArgs a) {
    const int64_t b = blockIdx.x;
    int t = 0;
    while (t + 1 < m.count && m.first[t + 1] <= b) t++;
    const int64_t e = (b - m.first[t]) * kOB + threadIdx.x;
    if (e < m.n4[t]) opt_item4<KIND, S1, S2>(m.w[t], m.g[t], S1 ? m.s1[t] : nullptr, S2 ? m.s2[t] : nullptr, e, a);
}

template <int KIND, bool S1, bool S2>
__global__ __launch_bounds__(kOB) void k_optim1(float *__restrict__ w, const float *__restrict__ g,
                                                float *__restrict__ s1, float *__restrict__ s2, int64_t n, OptArgs a) {
    for (int64_t e = (int64_t)blockIdx.x * kOB + threadIdx.x; e < n; e += (int64_t)gridDim.x * kOB) {
        float W = w[e], A = S1 ? s1[e] : 0.0f, B = S2 ? s2[e] : 0.0f;
        opt1<KIND, S1>(W, g[e], A, B, a);
        w[e] = W;
        if (S1) s1[e] = A;
        if (S2) s2[e] = B;
    }
}

template <int KIND, bool S1, bool S2>
static void launch_opt(float *w, const float *g, float *s1, float *s2, int64_t n, const OptArgs &a, hipStream_t st) {
    const bool vec = aligned16(w) && aligned16(g) && (!S1 || aligned16(s1)) && (!S2 || aligned16(s2));
    const int64_t n4 = vec ? n / 4 : 0;
    if (n4 > 0)
        hipLaunchKernelGGL((k_optim4<KIND, S1, S2>), dim3(stream_grid(n4, kOB, NC_OPT_GRID_PER_CU)), dim3(kOB), 0, st,
                           (f4 *)w, (const f4 *)g, (f4 *)s1, (f4 *)s2, n4, a);
    const int64_t done = n4 * 4;
    if (done < n)
        hipLaunchKernelGGL((k_optim1<KIND, S1, S2>), dim3(stream_grid(n - done, kOB)), dim3(kOB), 0, st, w + done,
                           g + done, S1 ? s1 + done : nullptr, S2 ? s2 + done : nullptr, n - done, a);
}

constexpr int kSB = 256;  // sum of squares: workgroup size
constexpr int kSU = 4;    // float4 items per lane in flight (and fp64 accumulators per lane)

// sum of squares: fp64 per thread, workgroup partials in wave order, then an ordered combine
__device__ __forceinline__ double block_sum_waves(double v) {
    __shared__ double sh[kSB / kWave];
    v = wave_sum(v);
    if ((threadIdx.x & (kWave - 1)) == 0) sh[threadIdx.x / kWave] = v;
    __syncthreads();
    double t = 0.0;
    if (threadIdx.x == 0)
        for (int i = 0; i < kSB / kWave; i++) t += sh[i];
    return t;
}

// float4 items (kSU per lane in flight) into four fp64 accumulators per lane, one per item slot,
// added in slot order at the end; the scalar tail (n % 4, or an unaligned x) goes to slot 0.
// Workgroup blk of nblk; thread 0 gets the workgroup's partial.
__device__ __forceinline__ double sumsq_block(const float *__restrict__ x, int64_t n, int64_t n4, int64_t blk,
                                              int64_t nblk) {
    double acc[kSU] = {0.0, 0.0, 0.0, 0.0};
    const f4 *x4 = (const f4 *)x;
    const int64_t step = nblk * kSB * kSU;
    for (int64_t base = blk * kSB * kSU + threadIdx.x; base < n4; base += step) {
        f4 v[kSU];
#pragma unroll
        for (int u = 0; u < kSU; u++)
            if (base + (int64_t)u * kSB < n4) v[u] = __builtin_nontemporal_load(x4 + base + (int64_t)u * kSB);
#pragma unroll
        for (int u = 0; u < kSU; u++) {
            if (base + (int64_t)u * kSB < n4) {
                const double a = v[u].x, b = v[u].y, c = v[u].z, d = v[u].w;
                acc[u] += (a * a + b * b) + (c * c + d * d);
            }
        }
    }
    for (int64_t e = n4 * 4 + blk * kSB + threadIdx.x; e < n; e += nblk * kSB) {
        const double v = (double)x[e];
        acc[0] += v * v;
    }
    return block_sum_waves((acc[0] + acc[1]) + (acc[2] + acc[3]));
}

__global__ __launch_bounds__(kSB) void k_sumsq(const float *__restrict__ x, int64_t n, int64_t n4,
                                               double *__restrict__ part) {
    const double t = sumsq_block(x, n, n4, blockIdx.x, gridDim.x);
    if (threadIdx.x == 0) part[blockIdx.x] = t;
}

// partials threadIdx.x, + kSB, ... of part[0, nparts) added in that order, their loads issued kU at a
// time; the workgroup total comes back in thread 0
__device__ __forceinline__ double sum_parts(const double *__restrict__ part, int nparts) {
    constexpr int kU = 8;
    double t = 0.0;
    for (int base = threadIdx.x; base < nparts; base += kSB * kU) {
        double v[kU];
#pragma unroll
        for (int u = 0; u < kU; u++) v[u] = base + u * kSB < nparts ? part[base + u * kSB] : 0.0;
#pragma unroll
        for (int u = 0; u < kU; u++)
            if (base + u * kSB < nparts) t += v[u];
    }
    return block_sum_waves(t);
}

__global__ __launch_bounds__(kSB) void k_sumsq_finish(const double *__restrict__ part, int nparts, double *ss,
                                                      int accumulate) {
    const double s = sum_parts(part, nparts);
    if (threadIdx.x == 0) *ss = (accumulate ? *ss : 0.0) + s;
}

// Up to NC_HIP_OPT_MULTI_MAX tensors in one launch: workgroups [first[t], first[t + 1]) are the grid
// k_sumsq would launch for tensor t alone (workgroup b plays workgroup b - first[t]), so every
// partial is the one-tensor partial.
struct SumsqMulti {
    const float *x[NC_HIP_OPT_MULTI_MAX];
    int64_t n[NC_HIP_OPT_MULTI_MAX], n4[NC_HIP_OPT_MULTI_MAX];
    int first[NC_HIP_OPT_MULTI_MAX + 1];
    int count;
};

__global__ __launch_bounds__(kSB) void k_sumsq_multi(SumsqMulti m, double *__restrict__ part) {
    const int b = blockIdx.x;
    int t = 0;  // workgroup-uniform
    while (t + 1 < m.count && m.first[t + 1] <= b) t++;
    const double s = sumsq_block(m.x[t], m.n[t], m.n4[t], b - m.first[t], m.first[t + 1] - m.first[t]);
    if (threadIdx.x == 0) part[b] = s;
}

// ss = (((ss or 0) + S_0) + S_1) + ..., S_t tensor t's partials summed as k_sumsq_finish sums them:
// the bits of one nc_hip_sumsq per tensor in turn.  ONE: every tensor has at most kSB partials (one
// per thread), so the loads of all tensors go out at once and their wave sums interleave (the
// tensor-by-tensor loop waited for each tensor's loads and barrier in turn: 20 us for 32 tensors);
// per tensor the arithmetic is sum_parts' (the thread's partial added to 0, the wave sum, the waves
// added in order).
template <bool ONE>
__global__ __launch_bounds__(kSB) void k_sumsq_multi_finish(const double *__restrict__ part, SumsqMulti m, double *ss,
                                                            int accumulate) {
    double acc = accumulate ? *ss : 0.0;
    if constexpr (ONE) {
        __shared__ double sh[NC_HIP_OPT_MULTI_MAX][kSB / kWave];
        double v[NC_HIP_OPT_MULTI_MAX];
#pragma unroll
        for (int t = 0; t < NC_HIP_OPT_MULTI_MAX; t++) {
            const int i = m.first[t] + (int)threadIdx.x;
            v[t] = t < m.count && i < m.first[t + 1] ? part[i] : 0.0;
        }
#pragma unroll
        for (int t = 0; t < NC_HIP_OPT_MULTI_MAX; t++) {
            if (t < m.count) {
                const double w = wave_sum(0.0 + v[t]);
                if ((threadIdx.x & (kWave - 1)) == 0) sh[t][threadIdx.x / kWave] = w;
            }
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            for (int t = 0; t < m.count; t++) {
                double s = 0.0;
                for (int w = 0; w < kSB / kWave; w++) s += sh[t][w];
                acc = acc + s;
            }
            *ss = acc;
        }
        return;
    }
    for (int t = 0; t < m.count; t++) {
        const double s = sum_parts(part + m.first[t], m.first[t + 1] - m.first[t]);
        if (threadIdx.x == 0) acc = acc + s;
        __syncthreads();  // the wave sums' LDS slots are written again for the next tensor
    }
    if (threadIdx.x == 0) *ss = acc;
}

// x[t] = coef * x[t] for up to NC_HIP_OPT_MULTI_MAX tensors, the unary scale kernel's expression;
// a workgroup scales kSB float4 items of one tensor (kSB floats of a tensor not 16-byte aligned)
struct ScaleMulti {
    float *x[NC_HIP_OPT_MULTI_MAX];
    int64_t n[NC_HIP_OPT_MULTI_MAX];
    int first[NC_HIP_OPT_MULTI_MAX + 1];
    int vec[NC_HIP_OPT_MULTI_MAX];
    int count;
};

__global__ __launch_bounds__(kSB) void k_scale_multi(ScaleMulti m, float coef) {
    const int b = blockIdx.x;
    int t = 0;
    while (t + 1 < m.count && m.first[t + 1] <= b) t++;
    float *x = m.x[t];
    const int64_t n = m.n[t], i = (int64_t)(b - m.first[t]) * kSB + threadIdx.x;
    if (m.vec[t]) {
        if (4 * i + 3 < n) {
            f4 v = ((f4 *)x)[i];
            v.x = coef * v.x;
            v.y = coef * v.y;
            v.z = coef * v.z;
            v.w = coef * v.w;
            ((f4 *)x)[i] = v;
        } else {
            for (int64_t e = 4 * i; e < n; e++) x[e] = coef * x[e];
        }
    } else if (i < n) {
        x[i] = coef * x[i];
    }
}

#ifndef NC_SUMSQ_GRID_PER_CU
#define NC_SUMSQ_GRID_PER_CU 8
#endif
// one fp64 partial per workgroup: the grid is part of the summation order, so it is planned from the
// shape alone (kPlanCUs), never from the device's CU count
static unsigned sumsq_grid(int64_t n) {
    const int64_t blocks = (n + 4 * kSB * kSU - 1) / (4 * kSB * kSU), cap = (int64_t)kPlanCUs * NC_SUMSQ_GRID_PER_CU;
    return (unsigned)std::max<int64_t>(1, std::min(blocks, cap));
}

}  // namespace nchip

using namespace nchip;

static OptArgs opt_args(int kind, float lr, float momentum, float weight_decay, float beta1, float beta2, float eps,
                        float gs, float bc1, float bc2, int eps_inside_sqrt) {
    OptArgs a{};
    a.lr = lr;
    a.momentum = momentum;
    a.wd = weight_decay;
    a.b1 = beta1;
    a.b2 = beta2;
    a.eps = eps;
    a.gs = gs;
    a.bc1 = bc1;
    a.bc2 = bc2;
    a.one_m_b1 = 1.0f - beta1;
    a.one_m_b2 = 1.0f - beta2;
    a.inside = eps_inside_sqrt ? 1 : 0;
    a.l2 = kind == NC_HIP_OPT_ADAM ? weight_decay : 0.0f;
    a.decay = kind == NC_HIP_OPT_ADAMW ? 1.0f - lr * weight_decay : 1.0f;
    return a;
}

extern "C" NC_HIP_API int nc_hip_optim_step(int kind, int64_t n, float *w, const float *g, float *s1, float *s2,
                                            float lr, float momentum, float weight_decay, float beta1, float beta2,
                                            float eps, float gs, float bc1, float bc2, int eps_inside_sqrt,
                                            void *stream) {
    if (n < 0) return set_error(NC_HIP_ERR_ARG, "nc_hip_optim_step: negative size");
    if (n == 0) return NC_HIP_OK;
    if (!w || !g) return set_error(NC_HIP_ERR_ARG, "nc_hip_optim_step: NULL parameter or gradient");
    OptArgs a = opt_args(kind, lr, momentum, weight_decay, beta1, beta2, eps, gs, bc1, bc2, eps_inside_sqrt);
    hipStream_t st = as_stream(stream);
    switch (kind) {
    case NC_HIP_OPT_SGD:
        if (s1) launch_opt<K_SGD, true, false>(w, g, s1, nullptr, n, a, st);
        else launch_opt<K_SGD, false, false>(w, g, nullptr, nullptr, n, a, st);
        break;
    case NC_HIP_OPT_ADAM:
    case NC_HIP_OPT_ADAMW:
        if (!s1 || !s2) return set_error(NC_HIP_ERR_ARG, "nc_hip_optim_step: Adam needs both state buffers");
        launch_opt<K_ADAM, true, true>(w, g, s1, s2, n, a, st);
        break;
    case NC_HIP_OPT_RMSPROP:
        if (!s2) return set_error(NC_HIP_ERR_ARG, "nc_hip_optim_step: RMSprop needs its square average");
        if (s1) launch_opt<K_RMS, true, true>(w, g, s1, s2, n, a, st);
        else launch_opt<K_RMS, false, true>(w, g, nullptr, s2, n, a, st);
        break;
    default: return set_error(NC_HIP_ERR_ARG, "nc_hip_optim_step: unknown optimizer %d", kind);
    }
    return check_launch("nc_hip_optim_step");
}

extern "C" NC_HIP_API int nc_hip_optim_step_multi(int kind, int count, const nc_hip_opt_param *params, float lr,
                                                  float momentum, float weight_decay, float beta1, float beta2,
                                                  float eps, float gs, float bc1, float bc2, int eps_inside_sqrt,
                                                  void *stream) {
    if (count < 0 || count > NC_HIP_OPT_MULTI_MAX)
        return set_error(NC_HIP_ERR_ARG, "nc_hip_optim_step_multi: %d parameters (1 to %d per call)", count,
                         NC_HIP_OPT_MULTI_MAX);
    if (count == 0) return NC_HIP_OK;
    if (!params) return set_error(NC_HIP_ERR_ARG, "nc_hip_optim_step_multi: NULL parameter list");
    const bool with1 = params[0].s1 != nullptr, with2 = params[0].s2 != nullptr;
    OptMulti m{};
    m.count = count;
    m.first[0] = 0;
    for (int t = 0; t < count; t++) {
        const nc_hip_opt_param &q = params[t];
        if (q.n == 0) {  // nothing to update: no workgroups
            m.first[t + 1] = m.first[t];
            continue;
        }
        if (q.n < 0 || q.n % 4 != 0 || !q.w || !q.g || !aligned16(q.w) || !aligned16(q.g) ||
            (q.s1 != nullptr) != with1 || (q.s2 != nullptr) != with2 || (q.s1 && !aligned16(q.s1)) ||
            (q.s2 && !aligned16(q.s2)))
            return set_error(NC_HIP_ERR_ARG,
                             "nc_hip_optim_step_multi: parameter %d needs n a multiple of 4, 16-byte aligned arrays "
                             "and the same state buffers as parameter 0",
                             t);
        m.w[t] = (f4 *)q.w;
        m.g[t] = (const f4 *)q.g;
        m.s1[t] = (f4 *)q.s1;
        m.s2[t] = (f4 *)q.s2;
        m.n4[t] = q.n / 4;
        m.first[t + 1] = m.first[t] + (m.n4[t] + kOB - 1) / kOB;
    }
    const int64_t blocks = m.first[count];
    if (blocks == 0) return NC_HIP_OK;
    if (blocks > INT32_MAX) return set_error(NC_HIP_ERR_ARG, "nc_hip_optim_step_multi: too many elements for one launch");
    const OptArgs a = opt_args(kind, lr, momentum, weight_decay, beta1, beta2, eps, gs, bc1, bc2, eps_inside_sqrt);
    hipStream_t st = as_stream(stream);
    const dim3 grid((unsigned)blocks), block(kOB);
    switch (kind) {
    case NC_HIP_OPT_SGD:
        if (with1) hipLaunchKernelGGL((k_optim4_multi<K_SGD, true, false>), grid, block, 0, st, m, a);
        else hipLaunchKernelGGL((k_optim4_multi<K_SGD, false, false>), grid, block, 0, st, m, a);
        break;
    case NC_HIP_OPT_ADAM:
    case NC_HIP_OPT_ADAMW:
        if (!with1 || !with2) return set_error(NC_HIP_ERR_ARG, "nc_hip_optim_step_multi: Adam needs both state buffers");
        hipLaunchKernelGGL((k_optim4_multi<K_ADAM, true, true>), grid, block, 0, st, m, a);
        break;
    case NC_HIP_OPT_RMSPROP:
        if (!with2) return set_error(NC_HIP_ERR_ARG, "nc_hip_optim_step_multi: RMSprop needs its square average");
        if (with1) hipLaunchKernelGGL((k_optim4_multi<K_RMS, true, true>), grid, block, 0, st, m, a);
        else hipLaunchKernelGGL((k_optim4_multi<K_RMS, false, true>), grid, block, 0, st, m, a);
        break;
    default: return set_error(NC_HIP_ERR_ARG, "nc_hip_optim_step_multi: unknown optimizer %d", kind);
    }
    return check_launch("nc_hip_optim_step_multi");
}

extern "C" NC_HIP_API size_t nc_hip_sumsq_workspace(int64_t n) {
    return n > 0 ? (size_t)sumsq_grid(n) * sizeof(double) : 0;
}

extern "C" NC_HIP_API int nc_hip_sumsq(int64_t n, const float *x, double *ss, int accumulate, void *ws,
                                       size_t ws_bytes, void *stream) {
    if (n < 0 || !ss) return set_error(NC_HIP_ERR_ARG, "nc_hip_sumsq: bad arguments");
    hipStream_t st = as_stream(stream);
    int nparts = 0;
    if (n > 0) {
        if (!x || !ws || ws_bytes < nc_hip_sumsq_workspace(n))
            return set_error(NC_HIP_ERR_WORKSPACE, "nc_hip_sumsq: workspace of %zu bytes needed",
                             nc_hip_sumsq_workspace(n));
        const unsigned grid = sumsq_grid(n);
        const int64_t n4 = aligned16(x) ? n / 4 : 0;  // float4 items; the rest one float per lane
        hipLaunchKernelGGL(k_sumsq, grid, kSB, 0, st, x, n, n4, (double *)ws);
        nparts = (int)grid;
    }
    hipLaunchKernelGGL(k_sumsq_finish, 1, kSB, 0, st, (const double *)ws, nparts, ss, accumulate ? 1 : 0);
    return check_launch("nc_hip_sumsq");
}

// checks a multi-tensor table and lays the tensors' workgroup ranges end to end: tensor t gets
// blocks(t) workgroups from first[t] (false, with the error set, when the table is bad)
template <class Blocks>
static bool multi_spans(const char *fn, int count, const int64_t *n, const void *const *x, int *first, Blocks blocks) {
    if (count < 0 || count > NC_HIP_OPT_MULTI_MAX || (count && (!n || !x)))
        return set_error(NC_HIP_ERR_ARG, "%s: count %d outside [0, %d] or NULL table", fn, count,
                         NC_HIP_OPT_MULTI_MAX), false;
    int64_t total = 0;
    for (int t = 0; t < count; t++) {
        if (n[t] < 0 || (n[t] > 0 && !x[t]))
            return set_error(NC_HIP_ERR_ARG, "%s: tensor %d: negative size or NULL pointer", fn, t), false;
        first[t] = (int)total;
        total += n[t] > 0 ? blocks(t) : 0;
        if (total > INT32_MAX) return set_error(NC_HIP_ERR_ARG, "%s: more than 2^31 - 1 workgroups", fn), false;
    }
    first[count] = (int)total;
    return true;
}

extern "C" NC_HIP_API size_t nc_hip_sumsq_multi_workspace(int count, const int64_t *n) {
    size_t b = 0;
    for (int t = 0; n && t < count && t < NC_HIP_OPT_MULTI_MAX; t++) b += nc_hip_sumsq_workspace(n[t]);
    return b;
}

extern "C" NC_HIP_API int nc_hip_sumsq_multi(int count, const float *const *x, const int64_t *n, double *ss,
                                             int accumulate, void *ws, size_t ws_bytes, void *stream) {
    SumsqMulti m{};
    if (!ss) return set_error(NC_HIP_ERR_ARG, "nc_hip_sumsq_multi: NULL ss");
    if (!multi_spans("nc_hip_sumsq_multi", count, n, (const void *const *)x, m.first,
                     [&](int t) { return (int64_t)sumsq_grid(n[t]); }))
        return NC_HIP_ERR_ARG;
    const size_t need = nc_hip_sumsq_multi_workspace(count, n);
    if (need && (!ws || ws_bytes < need))
        return set_error(NC_HIP_ERR_WORKSPACE, "nc_hip_sumsq_multi: workspace of %zu bytes needed", need);
    m.count = count;
    for (int t = 0; t < count; t++) {
        m.x[t] = x[t];
        m.n[t] = n[t];
        m.n4[t] = n[t] > 0 && aligned16(x[t]) ? n[t] / 4 : 0;  // as nc_hip_sumsq
    }
    hipStream_t st = as_stream(stream);
    if (m.first[count] > 0) hipLaunchKernelGGL(k_sumsq_multi, m.first[count], kSB, 0, st, m, (double *)ws);
    bool one = true;
    for (int t = 0; t < count; t++) one = one && m.first[t + 1] - m.first[t] <= kSB;
    if (one) hipLaunchKernelGGL(k_sumsq_multi_finish<true>, 1, kSB, 0, st, (const double *)ws, m, ss, accumulate ? 1 : 0);
    else hipLaunchKernelGGL(k_sumsq_multi_finish<false>, 1, kSB, 0, st, (const double *)ws, m, ss, accumulate ? 1 : 0);
    return check_launch("nc_hip_sumsq_multi");
}

extern "C" NC_HIP_API int nc_hip_scale_multi(int count, float *const *x, const int64_t *n, float coef, void *stream) {
    ScaleMulti m{};
    // a workgroup per kSB float4 items (kSB floats for a tensor that is not 16-byte aligned)
    if (!multi_spans("nc_hip_scale_multi", count, n, (const void *const *)x, m.first, [&](int t) {
            m.vec[t] = aligned16(x[t]) ? 1 : 0;
            const int64_t items = m.vec[t] ? (n[t] + 3) / 4 : n[t];
            return (items + kSB - 1) / kSB;
        }))
        return NC_HIP_ERR_ARG;
    m.count = count;
    for (int t = 0; t < count; t++) {
        m.x[t] = x[t];
        m.n[t] = n[t];
    }
    if (m.first[count] > 0) hipLaunchKernelGGL(k_scale_multi, m.first[count], kSB, 0, as_stream(stream), m, coef);
    return check_launch("nc_hip_scale_multi");
}
