// Cross entropy and NLL loss over [N, C] rows with i32 labels (ce_fwd / ce_bwd, ops_nn.c:107-147;
// nll_fwd / nll_bwd, ops_nn.c:391-420).
//
// cross entropy forward, one wave per row with the row in registers (C % 4 == 0, C <= 4096, 16-byte
// aligned): the log-softmax of nc_hip_softmax_fwd (the reference's max/NaN rule, exp8 terms, fp64
// row sum, logf), the label's log-probability added to the holding lane's fp64 accumulator, and
// prob = exp8(logp) stored for the backward: one read of x, one write of prob.  The next row is
// loaded before the current one is reduced.  Other shapes: nc_hip_softmax_fwd (log form) into
// prob, the per-row gather below, then exp8 over prob in place.
//
// Loss sums: fp64 per lane (or per thread), wave sums, workgroup partials added in wave order, and
// one ordered combine (k_loss_finish): loss = -S / N (mean; NaN for N = 0, 0/0 as the reference) or
// -S (sum).  A label outside [0, C) contributes nothing; the first such row is reported in *bad as
// (row << 32) | (uint32)label, each workgroup's minimum key written beside its loss partial and the
// minimum taken in the final combine (all ones when every label is valid: no separate initialising launch),
// for the caller to raise the reference's error.
#include "common.hpp"
#include "intdiv.hpp"

#include <algorithm>

namespace nchip {

constexpr int kLB = 256;  // 4 waves
constexpr int kLWaves = kLB / kWave;
constexpr unsigned long long kNoBad = ~0ull;

__device__ __forceinline__ unsigned long long bad_key(int64_t row, int32_t lab) {
    return ((unsigned long long)row << 32) | (uint32_t)lab;
}

// minimum over the workgroup of the lanes' first-bad-row keys; thread 0 returns it
__device__ __forceinline__ unsigned long long block_min_key(unsigned long long v) {
    __shared__ unsigned long long shk[kLWaves];
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const unsigned long long u = __shfl_xor(v, o, kWave);
        v = u < v ? u : v;
    }
    if ((threadIdx.x & (kWave - 1)) == 0) shk[threadIdx.x / kWave] = v;
    __syncthreads();
    unsigned long long t = kNoBad;
    if (threadIdx.x == 0)
        for (int i = 0; i < kLWaves; i++) t = shk[i] < t ? shk[i] : t;
    return t;
}

// sum of this workgroup's per-thread fp64 values, waves added in order; thread 0 returns it
__device__ __forceinline__ double block_sum_ordered(double v) {
    __shared__ double sh[kLWaves];
    v = wave_sum(v);
    if ((threadIdx.x & (kWave - 1)) == 0) sh[threadIdx.x / kWave] = v;
    __syncthreads();
    double t = 0.0;
    if (threadIdx.x == 0)
        for (int i = 0; i < kLWaves; i++) t += sh[i];
    return t;
}

template <int VPL>
__global__ __launch_bounds__(kLB) void k_ce_fwd_reg(const float *__restrict__ x, const int32_t *__restrict__ lab,
                                                    float *__restrict__ prob, double *__restrict__ part,
                                                    unsigned long long *__restrict__ badpart, int64_t N, int C) {
    const int lane = threadIdx.x & (kWave - 1);
    const int nv = C / 4;
    const int64_t stride = (int64_t)gridDim.x * kLWaves;
    auto load = [&](int64_t r, f4 *v) {
        const f4 *xr = (const f4 *)(x + r * C);
#pragma unroll
        for (int k = 0; k < VPL; k++)
            if (lane + k * kWave < nv) v[k] = __builtin_nontemporal_load(xr + lane + k * kWave);
    };
    double acc = 0.0;  // log-probabilities of the labels this lane holds
    unsigned long long mybad = kNoBad;  // first row with an out-of-range label among this wave's
    const int64_t r0 = ((int64_t)blockIdx.x * kLB + threadIdx.x) / kWave;
    f4 v[VPL], vn[VPL];
    int32_t L = 0, Ln = 0;
    if (r0 < N) {
        load(r0, v);
        L = lab[r0];
    }
    for (int64_t r = r0; r < N; r += stride) {
        if (r + stride < N) {
            load(r + stride, vn);
            Ln = lab[r + stride];
        }
        const bool ok = L >= 0 && L < C;
        if (!ok) mybad = bad_key(r, L) < mybad ? bad_key(r, L) : mybad;
        float m = -__builtin_inff();
#pragma unroll
        for (int k = 0; k < VPL; k++) {
            if (lane + k * kWave < nv)
                m = __builtin_fmaxf(m, __builtin_fmaxf(__builtin_fmaxf(v[k].x, v[k].y), __builtin_fmaxf(v[k].z, v[k].w)));
        }
        m = wave_max_nan_skip(m);
        m = row_max_finish(m, __shfl(v[0].x, 0, kWave));  // lane 0 holds the row's first element
        double s = 0.0;
#pragma unroll
        for (int k = 0; k < VPL; k++) {
            if (lane + k * kWave < nv)
                s += ((double)exp8_nonpos(v[k].x - m) + (double)exp8_nonpos(v[k].y - m)) +
                     ((double)exp8_nonpos(v[k].z - m) + (double)exp8_nonpos(v[k].w - m));
        }
        const float ls = logf((float)wave_sum(s));
        f4 *pr = (f4 *)(prob + r * C);
#pragma unroll
        for (int k = 0; k < VPL; k++) {
            const int j = lane + k * kWave;
            if (j < nv) {
                const float lp[4] = {(v[k].x - m) - ls, (v[k].y - m) - ls, (v[k].z - m) - ls, (v[k].w - m) - ls};
                if (ok && (L >> 2) == j) acc -= (double)lp[L & 3];
                __builtin_nontemporal_store(f4{exp8_nonpos(lp[0]), exp8_nonpos(lp[1]), exp8_nonpos(lp[2]), exp8_nonpos(lp[3])}, pr + j);
            }
        }
#pragma unroll
        for (int k = 0; k < VPL; k++) v[k] = vn[k];
        L = Ln;
    }
    const double t = block_sum_ordered(acc);
    const unsigned long long kb = block_min_key(mybad);
    if (threadIdx.x == 0) {
        part[blockIdx.x] = t;
        badpart[blockIdx.x] = kb;
    }
}

// one thread per row: -x[i, lab_i] into fp64 per-thread sums, workgroup partials
__global__ __launch_bounds__(kLB) void k_label_gather(const float *__restrict__ x, const int32_t *__restrict__ lab,
                                                      double *__restrict__ part, unsigned long long *__restrict__ badpart,
                                                      int64_t N, int64_t C) {
    double acc = 0.0;
    unsigned long long mybad = kNoBad;
    for (int64_t r = (int64_t)blockIdx.x * kLB + threadIdx.x; r < N; r += (int64_t)gridDim.x * kLB) {
        const int32_t L = lab[r];
        if (L >= 0 && L < C) acc -= (double)x[r * C + L];
        else mybad = bad_key(r, L) < mybad ? bad_key(r, L) : mybad;
    }
    const double t = block_sum_ordered(acc);
    const unsigned long long kb = block_min_key(mybad);
    if (threadIdx.x == 0) {
        part[blockIdx.x] = t;
        badpart[blockIdx.x] = kb;
    }
}

// loss from the ordered partials: S = sum (already negated terms); mean -> S / N (NaN for N = 0)
__global__ __launch_bounds__(kLB) void k_loss_finish(const double *__restrict__ part,
                                                     const unsigned long long *__restrict__ badpart, int nparts,
                                                     int64_t N, int sum, float *__restrict__ loss,
                                                     unsigned long long *__restrict__ bad) {
    double t = 0.0;
    unsigned long long kb = kNoBad;
    for (int i = threadIdx.x; i < nparts; i += kLB) {
        t += part[i];
        kb = badpart[i] < kb ? badpart[i] : kb;
    }
    const double S = block_sum_ordered(t);
    kb = block_min_key(kb);
    if (threadIdx.x == 0) {
        *loss = sum ? (float)S : N ? (float)(S / (double)N) : __builtin_nanf("");
        *bad = kb;
    }
}

// gi (+)= s * prob; gi[i, lab_i] -= s, s = gout / N.  A lane owns float4 items (four consecutive
// floats of a row), kCeU of them loaded before any is stored.
#ifndef NC_CEB_UNROLL
#define NC_CEB_UNROLL 1
#endif
#ifndef NC_CEB_BLOCK
#define NC_CEB_BLOCK 64
#endif
#ifndef NC_CEB_GRID_PER_CU
#define NC_CEB_GRID_PER_CU 65536
#endif
constexpr int kCeU = NC_CEB_UNROLL;
constexpr int kCeB = NC_CEB_BLOCK;
template <bool ACC>
__global__ __launch_bounds__(kCeB) void k_ce_bwd4(const f4 *__restrict__ prob, const int32_t *__restrict__ lab,
                                                 const float *__restrict__ gout, f4 *__restrict__ gi, int64_t N,
                                                 uint32_t n4, IntDiv row4) {
    const float s = gout[0] / (float)(N ? N : 1);
    const uint32_t per_row = row4.d;
    const uint64_t step = (uint64_t)gridDim.x * kCeB * kCeU;
    for (uint64_t base = (uint64_t)blockIdx.x * kCeB * kCeU + threadIdx.x; base < n4; base += step) {
        f4 p[kCeU], o[kCeU];
        int32_t rel[kCeU];  // label column relative to the item's first column
#pragma unroll
        for (int u = 0; u < kCeU; u++) {
            const uint64_t e = base + (uint64_t)u * kCeB;
            if (e < n4) {
                const uint32_t r = row4.div((uint32_t)e);
                rel[u] = lab[r] - 4 * (int32_t)((uint32_t)e - r * per_row);
                p[u] = __builtin_nontemporal_load(prob + e);
                o[u] = ACC ? __builtin_nontemporal_load(gi + e) : f4{0.f, 0.f, 0.f, 0.f};
            }
        }
#pragma unroll
        for (int u = 0; u < kCeU; u++) {
            const uint64_t e = base + (uint64_t)u * kCeB;
            if (e < n4) {
                f4 v = o[u];
                v.x = v.x + s * p[u].x;
                v.y = v.y + s * p[u].y;
                v.z = v.z + s * p[u].z;
                v.w = v.w + s * p[u].w;
                if (rel[u] == 0) v.x = v.x - s;
                if (rel[u] == 1) v.y = v.y - s;
                if (rel[u] == 2) v.z = v.z - s;
                if (rel[u] == 3) v.w = v.w - s;
                __builtin_nontemporal_store(v, gi + e);
            }
        }
    }
}

template <bool ACC>
__global__ __launch_bounds__(kLB) void k_ce_bwd1(const float *__restrict__ prob, const int32_t *__restrict__ lab,
                                                 const float *__restrict__ gout, float *__restrict__ gi, int64_t N,
                                                 int64_t C) {
    const float s = gout[0] / (float)(N ? N : 1);
    const int64_t n = N * C;
    for (int64_t e = (int64_t)blockIdx.x * kLB + threadIdx.x; e < n; e += (int64_t)gridDim.x * kLB) {
        const int64_t r = e / C;
        float o = (ACC ? gi[e] : 0.0f) + s * prob[e];
        if ((int64_t)lab[r] == e - r * C) o = o - s;
        gi[e] = o;
    }
}

__global__ __launch_bounds__(kLB) void k_nll_bwd(const int32_t *__restrict__ lab, const float *__restrict__ gout,
                                                 int sum, float *__restrict__ gi, int64_t N, int64_t C) {
    const float g = gout[0];
    const float s = sum ? g : g / (float)(N ? N : 1);
    for (int64_t r = (int64_t)blockIdx.x * kLB + threadIdx.x; r < N; r += (int64_t)gridDim.x * kLB) {
        const int32_t L = lab[r];
        if (L >= 0 && L < C) gi[r * C + L] = gi[r * C + L] - s;
    }
}

static int vpl_for_row(int64_t C) {
    const int64_t nv = C / 4;
    return nv <= 64 ? 1 : nv <= 128 ? 2 : nv <= 256 ? 4 : nv <= 512 ? 8 : nv <= 1024 ? 16 : 0;
}

#ifndef NC_CE_GRID_PER_CU
#define NC_CE_GRID_PER_CU 16
#endif
// Both forwards write one fp64 loss partial per workgroup, so their grids are part of the summation
// order: planned from the shape alone (kPlanCUs), never from the device's CU count.
static unsigned ce_grid(int64_t N) {
    const int64_t blocks = (N + kLWaves - 1) / kLWaves, cap = (int64_t)kPlanCUs * NC_CE_GRID_PER_CU;
    return (unsigned)std::max<int64_t>(1, std::min(blocks, cap));
}

static unsigned gather_grid(int64_t N) {
    const int64_t blocks = (N + kLB - 1) / kLB, cap = (int64_t)kPlanCUs * 4;
    return (unsigned)std::max<int64_t>(1, std::min(blocks, cap));
}

// workgroup partials of either forward: fp64 loss sums, then first-bad-row keys
static int64_t loss_parts(int64_t N) { return std::max(ce_grid(N), gather_grid(N)); }

}  // namespace nchip

using namespace nchip;

extern "C" NC_HIP_API size_t nc_hip_loss_workspace(int64_t N, int64_t C) {
    (void)C;
    if (N < 0) return 0;
    return (size_t)loss_parts(N) * (sizeof(double) + sizeof(unsigned long long));
}

extern "C" NC_HIP_API int nc_hip_cross_entropy_fwd(int64_t N, int64_t C, const float *x, const int32_t *lab,
                                                   float *prob, float *loss, uint64_t *bad, void *ws,
                                                   size_t ws_bytes, void *stream) {
    if (N < 0 || C < 1) return set_error(NC_HIP_ERR_ARG, "nc_hip_cross_entropy_fwd: bad size [%lld, %lld]",
                                         (long long)N, (long long)C);
    if (!loss || !bad || (N > 0 && (!x || !lab || !prob)))
        return set_error(NC_HIP_ERR_ARG, "nc_hip_cross_entropy_fwd: NULL pointer");
    if (ws_bytes < nc_hip_loss_workspace(N, C) || !ws)
        return set_error(NC_HIP_ERR_WORKSPACE, "nc_hip_cross_entropy_fwd: workspace of %zu bytes needed",
                         nc_hip_loss_workspace(N, C));
    hipStream_t st = as_stream(stream);
    unsigned long long *b = (unsigned long long *)bad;
    double *part = (double *)ws;
    unsigned long long *bp = (unsigned long long *)(part + loss_parts(N));
    int nparts = 0;
    if (N > 0) {
        const int vpl = (C % 4 == 0 && aligned16(x) && aligned16(prob)) ? vpl_for_row(C) : 0;
        if (vpl) {
            const unsigned grid = ce_grid(N);
            switch (vpl) {
            case 1: hipLaunchKernelGGL(k_ce_fwd_reg<1>, grid, kLB, 0, st, x, lab, prob, part, bp, N, (int)C); break;
            case 2: hipLaunchKernelGGL(k_ce_fwd_reg<2>, grid, kLB, 0, st, x, lab, prob, part, bp, N, (int)C); break;
            case 4: hipLaunchKernelGGL(k_ce_fwd_reg<4>, grid, kLB, 0, st, x, lab, prob, part, bp, N, (int)C); break;
            case 8: hipLaunchKernelGGL(k_ce_fwd_reg<8>, grid, kLB, 0, st, x, lab, prob, part, bp, N, (int)C); break;
            default: hipLaunchKernelGGL(k_ce_fwd_reg<16>, grid, kLB, 0, st, x, lab, prob, part, bp, N, (int)C); break;
            }
            nparts = (int)grid;
        } else {
            // log-softmax into prob, gather the labels' terms, then prob = exp8(logp) in place
            int rc = nc_hip_softmax_fwd(1, N, C, x, prob, stream);
            if (rc) return rc;
            const unsigned grid = gather_grid(N);
            hipLaunchKernelGGL(k_label_gather, grid, kLB, 0, st, prob, lab, part, bp, N, C);
            nparts = (int)grid;
            rc = nc_hip_unary_fwd(NC_HIP_UN_EXP, 0.0f, prob, prob, N * C, stream);
            if (rc) return rc;
        }
    }
    hipLaunchKernelGGL(k_loss_finish, 1, kLB, 0, st, part, bp, nparts, N, 0, loss, b);
    return check_launch("nc_hip_cross_entropy_fwd");
}

extern "C" NC_HIP_API int nc_hip_cross_entropy_bwd(int64_t N, int64_t C, const float *prob, const int32_t *lab,
                                                   const float *gout, float *gi, int accumulate, void *stream) {
    if (N < 0 || C < 1) return set_error(NC_HIP_ERR_ARG, "nc_hip_cross_entropy_bwd: bad size");
    const int64_t n = N * C;
    if (n == 0) return NC_HIP_OK;
    if (!prob || !lab || !gout || !gi) return set_error(NC_HIP_ERR_ARG, "nc_hip_cross_entropy_bwd: NULL pointer");
    hipStream_t st = as_stream(stream);
    if (C % 4 == 0 && aligned16(prob) && aligned16(gi) && n / 4 < (int64_t)UINT32_MAX) {
        const uint32_t n4 = (uint32_t)(n / 4);
        const unsigned grid = stream_grid((n4 + kCeU - 1) / kCeU, kCeB, NC_CEB_GRID_PER_CU);
        const IntDiv row4((uint32_t)(C / 4));
        if (accumulate)
            hipLaunchKernelGGL(k_ce_bwd4<true>, grid, kCeB, 0, st, (const f4 *)prob, lab, gout, (f4 *)gi, N, n4, row4);
        else
            hipLaunchKernelGGL(k_ce_bwd4<false>, grid, kCeB, 0, st, (const f4 *)prob, lab, gout, (f4 *)gi, N, n4, row4);
    } else {
        const unsigned grid = stream_grid(n, kLB);
        if (accumulate) hipLaunchKernelGGL(k_ce_bwd1<true>, grid, kLB, 0, st, prob, lab, gout, gi, N, C);
        else hipLaunchKernelGGL(k_ce_bwd1<false>, grid, kLB, 0, st, prob, lab, gout, gi, N, C);
    }
    return check_launch("nc_hip_cross_entropy_bwd");
}

extern "C" NC_HIP_API int nc_hip_nll_loss_fwd(int64_t N, int64_t C, const float *x, const int32_t *lab, int sum,
                                              float *loss, uint64_t *bad, void *ws, size_t ws_bytes,
                                              void *stream) {
    if (N < 0 || C < 0) return set_error(NC_HIP_ERR_ARG, "nc_hip_nll_loss_fwd: bad size");
    if (!loss || !bad || (N > 0 && (!x || !lab))) return set_error(NC_HIP_ERR_ARG, "nc_hip_nll_loss_fwd: NULL pointer");
    if (ws_bytes < nc_hip_loss_workspace(N, C) || !ws)
        return set_error(NC_HIP_ERR_WORKSPACE, "nc_hip_nll_loss_fwd: workspace of %zu bytes needed",
                         nc_hip_loss_workspace(N, C));
    hipStream_t st = as_stream(stream);
    unsigned long long *b = (unsigned long long *)bad;
    double *part = (double *)ws;
    unsigned long long *bp = (unsigned long long *)(part + loss_parts(N));
    int nparts = 0;
    if (N > 0) {
        const unsigned grid = gather_grid(N);
        hipLaunchKernelGGL(k_label_gather, grid, kLB, 0, st, x, lab, part, bp, N, C);
        nparts = (int)grid;
    }
    hipLaunchKernelGGL(k_loss_finish, 1, kLB, 0, st, part, bp, nparts, N, sum ? 1 : 0, loss, b);
    return check_launch("nc_hip_nll_loss_fwd");
}

extern "C" NC_HIP_API int nc_hip_nll_loss_bwd(int64_t N, int64_t C, const int32_t *lab, const float *gout, int sum,
                                              float *gi, void *stream) {
    if (N < 0 || C < 0) return set_error(NC_HIP_ERR_ARG, "nc_hip_nll_loss_bwd: bad size");
    if (N == 0 || C == 0) return NC_HIP_OK;
    if (!lab || !gout || !gi) return set_error(NC_HIP_ERR_ARG, "nc_hip_nll_loss_bwd: NULL pointer");
    hipLaunchKernelGGL(k_nll_bwd, gather_grid(N), kLB, 0, as_stream(stream), lab, gout, sum ? 1 : 0, gi, N, C);
    return check_launch("nc_hip_nll_loss_bwd");
}
