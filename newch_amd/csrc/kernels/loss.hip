// Cross entropy and NLL loss over [N, C] rows with i32 labels (ce_fwd / ce_bwd, ops_nn.c:107-147;
// nll_fwd / nll_bwd, ops_nn.c:391-420).
//
// The reference's forward stores prob = exp(log_softmax(x)) for its backward, one float per
// element.  prob is a function of x and two numbers per row: logp = (x - m) - ls with m the row
// maximum (the reference's scan rule) and ls = logf(sum exp8(x - m)), and prob = exp8(logp).  So
// the forward here reads x once and writes only stats = [N][2] {m, ls}; the backward recomputes
// prob = exp8((x - m) - ls) from x with the reference's fp32 operations and reads x where the
// reference reads prob: the forward moves 4 B/element instead of 8, the backward the same 12.  Given
// the stats, prob is bit for bit that expression.  ls itself comes from an fp64 sum of hardware
// exponentials (the reductions' tolerance), where the reference takes logf of an fp32 sum of exp8
// terms, so the recomputed prob can differ from the probabilities the reference saves in its last
// bits: the gradient matches the reference's at the reductions' tolerance, not bit for bit.
//
// cross entropy forward, one wave per row with the row in registers (C % 4 == 0, C <= 4096, 16-byte
// aligned): the max, the row sum of exp(x - m) (hardware exponential: the sum is only compared at the
// reductions' tolerance), logf, and the label's log-probability (its logit read back as one uniform
// load rather than picked out of the registers) added to lane 0's fp64 accumulator.  The next row is
// loaded before the current one is reduced.  Other
// shapes: one workgroup per row, the same arithmetic over the (L2-resident) row.
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

// the workgroup's loss sum (wave sums, then the waves added in order) and its minimum first-bad-row
// key, both by DPP within each wave and one LDS exchange; thread 0 holds the results
__device__ __forceinline__ void block_sum_min(double v, unsigned long long k, double &sum,
                                              unsigned long long &key) {
    __shared__ double shs[kLWaves];
    __shared__ unsigned long long shk[kLWaves];
    v = wave_sum(v);
    k = wave_min_u64(k);
    if ((threadIdx.x & (kWave - 1)) == 0) {
        shs[threadIdx.x / kWave] = v;
        shk[threadIdx.x / kWave] = k;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        double t = 0.0;
        unsigned long long m = kNoBad;
        for (int i = 0; i < kLWaves; i++) {
            t += shs[i];
            m = shk[i] < m ? shk[i] : m;
        }
        sum = t;
        key = m;
    }
}

template <int VPL>
__device__ __forceinline__ void ce_fwd_rows(const float *__restrict__ x, const int32_t *__restrict__ lab,
                                            f2 *__restrict__ stats, double *__restrict__ part,
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
    // the label's logit, one wave-uniform 4-byte load (the row is in cache); an out-of-range label
    // reads column 0 and is not used
    auto label_logit = [&](int64_t r, int32_t L) {
        return x[r * C + (L >= 0 && L < C ? L : 0)];
    };
    double acc = 0.0;  // lane 0: the negated log-probabilities of this wave's labels
    unsigned long long mybad = kNoBad;  // first row with an out-of-range label among this wave's
    auto row = [&](int64_t r, const f4 *v, int32_t L, float xl) {
        const bool ok = L >= 0 && L < C;
        if (!ok) mybad = bad_key(r, L) < mybad ? bad_key(r, L) : mybad;
        float m = -__builtin_inff();
#pragma unroll
        for (int k = 0; k < VPL; k++) {
            if (lane + k * kWave < nv)
                m = __builtin_fmaxf(m, __builtin_fmaxf(__builtin_fmaxf(v[k].x, v[k].y), __builtin_fmaxf(v[k].z, v[k].w)));
        }
        m = wave_max_nan_skip(m);
        m = row_max_finish(m, lane0_f32(v[0].x));  // lane 0 holds the row's first element
        // exp(x - m) as exp2((x - m) log2e): the difference first, so the exponent's error is relative
        // to x - m, not to m (x log2e - m log2e would carry m log2e's rounding, 1e-4 at |m| = 1e3); each
        // lane's terms (at most 64, each in (0, 1]) in fp32, the 64 lane sums in fp64
        float s = 0.0f;
#pragma unroll
        for (int k = 0; k < VPL; k++) {
            if (lane + k * kWave < nv)
                s += (exp_sum_term(v[k].x - m) + exp_sum_term(v[k].y - m)) +
                     (exp_sum_term(v[k].z - m) + exp_sum_term(v[k].w - m));
        }
        const float ls = logf((float)wave_sum((double)s));
        if (lane == 0) {
            stats[r] = f2{m, ls};
            if (ok) acc -= (double)((xl - m) - ls);
        }
    };
    // rows r0, r0 + stride, ... through two register sets in turn.  In the steady state every load is
    // unconditional and issued in this order: the current row's label logit, then the next row and its
    // label, so the waits for the current row never cover the next row's loads.  Where the workgroup's
    // four waves run the steady-state loop the same number of times (every workgroup unless N ends
    // inside its last stride), they meet at a barrier before each row: waves kept in step read
    // neighbouring rows together (over X[65536, 1024]: 45.9 -> 45.3 us with a barrier before every
    // second row, 0.1-0.9 us less again with one before every row).
    auto trips = [&](int64_t r) { return r < N ? (N - r - 1) / (2 * stride) : (int64_t)0; };
    const int64_t rw = (int64_t)blockIdx.x * kLWaves;  // the workgroup's first row
    const bool lock = trips(rw) == trips(rw + kLWaves - 1);  // uniform over the workgroup
    int64_t r = ((int64_t)blockIdx.x * kLB + threadIdx.x) / kWave;
    f4 va[VPL], vb[VPL];
    int32_t la = 0, lb = 0;
    if (r < N) {
        load(r, va);
        la = lab[r];
    }
    while (r + 2 * stride < N) {
        if (lock) __syncthreads();
        const float xa = label_logit(r, la);
        load(r + stride, vb);
        lb = lab[r + stride];
        row(r, va, la, xa);
        if (lock) __syncthreads();
        const float xb = label_logit(r + stride, lb);
        load(r + 2 * stride, va);
        la = lab[r + 2 * stride];
        row(r + stride, vb, lb, xb);
        r += 2 * stride;
    }
    if (r < N) {
        const float xa = label_logit(r, la);
        const bool more = r + stride < N;
        if (more) {
            load(r + stride, vb);
            lb = lab[r + stride];
        }
        row(r, va, la, xa);
        if (more) row(r + stride, vb, lb, label_logit(r + stride, lb));
    }
    double t = 0.0;
    unsigned long long kb = kNoBad;
    block_sum_min(acc, mybad, t, kb);
    if (threadIdx.x == 0) {
        part[blockIdx.x] = t;
        badpart[blockIdx.x] = kb;
    }
}

// rows of up to 1024 floats: at most 64 VGPRs (8 waves per SIMD), so the grid of 8 workgroups per CU
// is resident at once; longer rows keep the compiler's allocation
template <int VPL>
__global__ __attribute__((amdgpu_waves_per_eu(8, 8))) __launch_bounds__(kLB) void k_ce_fwd_reg(
    const float *__restrict__ x, const int32_t *__restrict__ lab, f2 *__restrict__ stats, double *__restrict__ part,
    unsigned long long *__restrict__ badpart, int64_t N, int C) {
    ce_fwd_rows<VPL>(x, lab, stats, part, badpart, N, C);
}

template <int VPL>
__global__ __launch_bounds__(kLB) void k_ce_fwd_reg_long(const float *__restrict__ x, const int32_t *__restrict__ lab,
                                                         f2 *__restrict__ stats, double *__restrict__ part,
                                                         unsigned long long *__restrict__ badpart, int64_t N, int C) {
    ce_fwd_rows<VPL>(x, lab, stats, part, badpart, N, C);
}

// Any row length / alignment: one workgroup per row (rows in a grid-stride loop), the same
// statistics and label term; the row is re-read from L2 for the exp sum.
__device__ __forceinline__ float block_max_nan_skip(float v, float *sh) {
    v = wave_max_nan_skip(v);
    if ((threadIdx.x & (kWave - 1)) == 0) sh[threadIdx.x / kWave] = v;
    __syncthreads();
    float t = sh[0];
#pragma unroll
    for (int i = 1; i < kLWaves; i++) t = __builtin_fmaxf(t, sh[i]);
    __syncthreads();
    return t;
}

__device__ __forceinline__ double block_sum_all(double v, double *sh) {
    v = wave_sum(v);
    if ((threadIdx.x & (kWave - 1)) == 0) sh[threadIdx.x / kWave] = v;
    __syncthreads();
    double t = 0.0;
#pragma unroll
    for (int i = 0; i < kLWaves; i++) t += sh[i];
    __syncthreads();
    return t;
}

__global__ __launch_bounds__(kLB) void k_ce_fwd_blk(const float *__restrict__ x, const int32_t *__restrict__ lab,
                                                    f2 *__restrict__ stats, double *__restrict__ part,
                                                    unsigned long long *__restrict__ badpart, int64_t N, int64_t C) {
    __shared__ float shm[kLWaves];
    __shared__ double shs[kLWaves];
    double acc = 0.0;
    unsigned long long mybad = kNoBad;
    for (int64_t r = blockIdx.x; r < N; r += gridDim.x) {
        const float *xr = x + r * C;
        float m = -__builtin_inff();
        for (int64_t c = threadIdx.x; c < C; c += kLB) m = __builtin_fmaxf(m, xr[c]);
        m = row_max_finish(block_max_nan_skip(m, shm), xr[0]);
        double s = 0.0;
        for (int64_t c = threadIdx.x; c < C; c += kLB) s += (double)exp_sum_term(xr[c] - m);
        const float ls = logf((float)block_sum_all(s, shs));
        if (threadIdx.x == 0) {
            const int32_t L = lab[r];
            if (L >= 0 && L < C) acc -= (double)((xr[L] - m) - ls);
            else mybad = bad_key(r, L) < mybad ? bad_key(r, L) : mybad;
            stats[r] = f2{m, ls};
        }
    }
    double t = 0.0;
    unsigned long long kb = kNoBad;
    block_sum_min(acc, mybad, t, kb);
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
    double t = 0.0;
    unsigned long long kb = kNoBad;
    block_sum_min(acc, mybad, t, kb);
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
    // each thread adds partials threadIdx.x, + kLB, + 2 kLB, ... in that order; their loads are issued
    // kU at a time, so the chain of dependent memory latencies is nparts / (kLB kU) long, not
    // nparts / kLB (4096 partials: 5.8 -> ~1 us)
    constexpr int kU = 16;
    double t = 0.0;
    unsigned long long kb = kNoBad;
    for (int base = threadIdx.x; base < nparts; base += kLB * kU) {
        double v[kU];
        unsigned long long key[kU];
#pragma unroll
        for (int u = 0; u < kU; u++) {
            const int i = base + u * kLB;
            v[u] = i < nparts ? part[i] : 0.0;
            key[u] = i < nparts ? badpart[i] : kNoBad;
        }
#pragma unroll
        for (int u = 0; u < kU; u++) {
            if (base + u * kLB < nparts) t += v[u];
            kb = key[u] < kb ? key[u] : kb;
        }
    }
    double S = 0.0;
    block_sum_min(t, kb, S, kb);
    if (threadIdx.x == 0) {
        *loss = sum ? (float)S : N ? (float)(S / (double)N) : __builtin_nanf("");
        *bad = kb;
    }
}

// gi (+)= s * prob; gi[i, lab_i] -= s, s = gout / N, with prob = exp8((x - m) - ls) recomputed from
// x and the row's statistics.  A lane owns float4 items (four consecutive floats of a row), kCeU of
// them loaded before any is stored.
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

__device__ __forceinline__ float ce_prob(float x, f2 st) { return exp8_nonpos((x - st.x) - st.y); }

template <bool ACC>
__global__ __launch_bounds__(kCeB) void k_ce_bwd4(const f4 *__restrict__ x, const f2 *__restrict__ stats,
                                                 const int32_t *__restrict__ lab, const float *__restrict__ gout,
                                                 f4 *__restrict__ gi, int64_t N, uint32_t n4, IntDiv row4) {
    const float s = gout[0] / (float)(N ? N : 1);
    const uint32_t per_row = row4.d;
    const uint64_t step = (uint64_t)gridDim.x * kCeB * kCeU;
    for (uint64_t base = (uint64_t)blockIdx.x * kCeB * kCeU + threadIdx.x; base < n4; base += step) {
        f4 p[kCeU], o[kCeU];
        f2 st[kCeU];
        int32_t rel[kCeU];  // label column relative to the item's first column
#pragma unroll
        for (int u = 0; u < kCeU; u++) {
            const uint64_t e = base + (uint64_t)u * kCeB;
            if (e < n4) {
                const uint32_t r = row4.div((uint32_t)e);
                rel[u] = lab[r] - 4 * (int32_t)((uint32_t)e - r * per_row);
                st[u] = stats[r];
                p[u] = __builtin_nontemporal_load(x + e);
                o[u] = ACC ? __builtin_nontemporal_load(gi + e) : f4{0.f, 0.f, 0.f, 0.f};
            }
        }
#pragma unroll
        for (int u = 0; u < kCeU; u++) {
            const uint64_t e = base + (uint64_t)u * kCeB;
            if (e < n4) {
                f4 v = o[u];
                v.x = v.x + s * ce_prob(p[u].x, st[u]);
                v.y = v.y + s * ce_prob(p[u].y, st[u]);
                v.z = v.z + s * ce_prob(p[u].z, st[u]);
                v.w = v.w + s * ce_prob(p[u].w, st[u]);
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
__global__ __launch_bounds__(kLB) void k_ce_bwd1(const float *__restrict__ x, const f2 *__restrict__ stats,
                                                 const int32_t *__restrict__ lab, const float *__restrict__ gout,
                                                 float *__restrict__ gi, int64_t N, int64_t C) {
    const float s = gout[0] / (float)(N ? N : 1);
    const int64_t n = N * C;
    for (int64_t e = (int64_t)blockIdx.x * kLB + threadIdx.x; e < n; e += (int64_t)gridDim.x * kLB) {
        const int64_t r = e / C;
        float o = (ACC ? gi[e] : 0.0f) + s * ce_prob(x[e], stats[r]);
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
#define NC_CE_GRID_PER_CU 8
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
                                                   float *stats, float *loss, uint64_t *bad, void *ws,
                                                   size_t ws_bytes, void *stream) {
    if (N < 0 || C < 1) return set_error(NC_HIP_ERR_ARG, "nc_hip_cross_entropy_fwd: bad size [%lld, %lld]",
                                         (long long)N, (long long)C);
    if (!loss || !bad || (N > 0 && (!x || !lab || !stats)))
        return set_error(NC_HIP_ERR_ARG, "nc_hip_cross_entropy_fwd: NULL pointer");
    if (((uintptr_t)stats & 7u) != 0) return set_error(NC_HIP_ERR_ARG, "nc_hip_cross_entropy_fwd: stats not 8-byte aligned");
    if (ws_bytes < nc_hip_loss_workspace(N, C) || !ws)
        return set_error(NC_HIP_ERR_WORKSPACE, "nc_hip_cross_entropy_fwd: workspace of %zu bytes needed",
                         nc_hip_loss_workspace(N, C));
    hipStream_t st = as_stream(stream);
    unsigned long long *b = (unsigned long long *)bad;
    double *part = (double *)ws;
    unsigned long long *bp = (unsigned long long *)(part + loss_parts(N));
    f2 *sv = (f2 *)stats;
    int nparts = 0;
    if (N > 0) {
        const int vpl = (C % 4 == 0 && aligned16(x)) ? vpl_for_row(C) : 0;
        const unsigned grid = ce_grid(N);
        switch (vpl) {
        case 1: hipLaunchKernelGGL(k_ce_fwd_reg<1>, grid, kLB, 0, st, x, lab, sv, part, bp, N, (int)C); break;
        case 2: hipLaunchKernelGGL(k_ce_fwd_reg<2>, grid, kLB, 0, st, x, lab, sv, part, bp, N, (int)C); break;
        case 4: hipLaunchKernelGGL(k_ce_fwd_reg<4>, grid, kLB, 0, st, x, lab, sv, part, bp, N, (int)C); break;
        case 8: hipLaunchKernelGGL(k_ce_fwd_reg_long<8>, grid, kLB, 0, st, x, lab, sv, part, bp, N, (int)C); break;
        case 16: hipLaunchKernelGGL(k_ce_fwd_reg_long<16>, grid, kLB, 0, st, x, lab, sv, part, bp, N, (int)C); break;
        default: hipLaunchKernelGGL(k_ce_fwd_blk, grid, kLB, 0, st, x, lab, sv, part, bp, N, C); break;
        }
        nparts = (int)grid;
    }
    hipLaunchKernelGGL(k_loss_finish, 1, kLB, 0, st, part, bp, nparts, N, 0, loss, b);
    return check_launch("nc_hip_cross_entropy_fwd");
}

extern "C" NC_HIP_API int nc_hip_cross_entropy_bwd(int64_t N, int64_t C, const float *x, const float *stats,
                                                   const int32_t *lab, const float *gout, float *gi, int accumulate,
                                                   void *stream) {
    if (N < 0 || C < 1) return set_error(NC_HIP_ERR_ARG, "nc_hip_cross_entropy_bwd: bad size");
    const int64_t n = N * C;
    if (n == 0) return NC_HIP_OK;
    if (!x || !stats || !lab || !gout || !gi) return set_error(NC_HIP_ERR_ARG, "nc_hip_cross_entropy_bwd: NULL pointer");
    if (((uintptr_t)stats & 7u) != 0) return set_error(NC_HIP_ERR_ARG, "nc_hip_cross_entropy_bwd: stats not 8-byte aligned");
    hipStream_t st = as_stream(stream);
    const f2 *sv = (const f2 *)stats;
    if (C % 4 == 0 && aligned16(x) && aligned16(gi) && n / 4 < (int64_t)UINT32_MAX) {
        const uint32_t n4 = (uint32_t)(n / 4);
        const unsigned grid = stream_grid((n4 + kCeU - 1) / kCeU, kCeB, NC_CEB_GRID_PER_CU);
        const IntDiv row4((uint32_t)(C / 4));
        if (accumulate)
            hipLaunchKernelGGL(k_ce_bwd4<true>, grid, kCeB, 0, st, (const f4 *)x, sv, lab, gout, (f4 *)gi, N, n4, row4);
        else
            hipLaunchKernelGGL(k_ce_bwd4<false>, grid, kCeB, 0, st, (const f4 *)x, sv, lab, gout, (f4 *)gi, N, n4, row4);
    } else {
        const unsigned grid = stream_grid(n, kLB);
        if (accumulate) hipLaunchKernelGGL(k_ce_bwd1<true>, grid, kLB, 0, st, x, sv, lab, gout, gi, N, C);
        else hipLaunchKernelGGL(k_ce_bwd1<false>, grid, kLB, 0, st, x, sv, lab, gout, gi, N, C);
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
