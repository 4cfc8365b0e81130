// Reductions over one axis or all (the reference's ops_reduce.c:13-163): x is viewed as
// [outer, R, inner] and reduced over R.
//
// Layout-driven kernels:
//   * inner == 1, many rows: one wave per row, 128-bit loads along the row, wave64 shuffle reduce;
//   * inner == 1, few long rows (a full reduction is outer = 1): each row is split into fixed
//     chunks, one workgroup per (row, chunk) writes an fp64 partial, a second kernel combines the
//     partials of each row in chunk order (two-pass, deterministic);
//   * inner > 1: lanes run along the contiguous inner dim (coalesced), each lane scans R (split into
//     fixed chunks with a combine pass when outer * inner is too small to fill the GPU).
// Sums accumulate in fp64.  max / argmax reproduce the reference's sequential strict-greater scan
// exactly: the first maximal index wins, a NaN at r = 0 is sticky, any later NaN is skipped.
#include "common.hpp"
#include "intdiv.hpp"

#include <float.h>

#include <mutex>

#ifndef NC_RED_ROWS_GRID_PER_CU
#define NC_RED_ROWS_GRID_PER_CU 65536
#endif

namespace nchip {

constexpr int kRB = 256;
constexpr int kEmpty = 0x7fffffff;  // argmax state "no element yet"

// (value, index) state of the sequential scan restricted to non-NaN elements
struct ArgState {
    float v;
    int i;
};

__device__ __forceinline__ void arg_push(ArgState &s, float v, int i) {
    // elements arrive in increasing index order within one lane
    if (v != v) return;
    if (s.i == kEmpty || v > s.v) {
        s.v = v;
        s.i = i;
    }
}

__device__ __forceinline__ ArgState arg_combine(ArgState a, ArgState b) {
    if (a.i == kEmpty) return b;
    if (b.i == kEmpty) return a;
    if (b.v > a.v) return b;
    if (a.v > b.v) return a;
    return a.i <= b.i ? a : b;  // equal (including -0 == +0): first index
}

// arg_combine is a total order (larger value, then smaller index), so any combine order gives the
// same state: the DPP steps of wave_sum, each moving the value and the index
template <int CTRL, int ROWMASK = 0xf>
__device__ __forceinline__ ArgState dpp_arg(ArgState s) {
    return ArgState{dpp_f32<CTRL, ROWMASK>(s.v, s.v), dpp_i32<CTRL, ROWMASK>(s.i, s.i)};
}
__device__ __forceinline__ ArgState wave_arg(ArgState s) {
    s = arg_combine(s, dpp_arg<kDppXor1>(s));
    s = arg_combine(s, dpp_arg<kDppXor2>(s));
    s = arg_combine(s, dpp_arg<kDppHalfMirror>(s));
    s = arg_combine(s, dpp_arg<kDppMirror>(s));
    s = arg_combine(s, dpp_arg<kDppBcast15, 0xa>(s));
    s = arg_combine(s, dpp_arg<kDppBcast31, 0xc>(s));
    return ArgState{lane63_f32(s.v), lane63_i32(s.i)};
}

template <int KIND>
struct Acc {
    double sum;
    ArgState a;
    __device__ __forceinline__ void init() {
        sum = 0.0;
        a = ArgState{0.0f, kEmpty};
    }
    __device__ __forceinline__ void push(float v, int i) {
        if constexpr (KIND == NC_HIP_RED_SUM || KIND == NC_HIP_RED_MEAN) sum += (double)v;
        else arg_push(a, v, i);
    }
    __device__ __forceinline__ void combine(const Acc &o) {
        if constexpr (KIND == NC_HIP_RED_SUM || KIND == NC_HIP_RED_MEAN) sum += o.sum;
        else a = arg_combine(a, o.a);
    }
    __device__ __forceinline__ void wave() {
        if constexpr (KIND == NC_HIP_RED_SUM || KIND == NC_HIP_RED_MEAN) sum = wave_sum(sum);
        else a = wave_arg(a);
    }
};

// writes the result of row `o` (column `i`) given the row's first element x0 (NaN rule)
template <int KIND>
__device__ __forceinline__ void emit(const Acc<KIND> &acc, float x0, float scale, float *y, int32_t *arg,
                                     int64_t at) {
    if constexpr (KIND == NC_HIP_RED_SUM || KIND == NC_HIP_RED_MEAN) {
        y[at] = scale * (float)acc.sum;
    } else {
        ArgState s = acc.a;
        if (x0 != x0 || s.i == kEmpty) s = ArgState{x0, 0};
        if (KIND == NC_HIP_RED_MAX) y[at] = s.v;
        arg[at] = s.i;
    }
}

// --- inner == 1, one wave per row --------------------------------------------------------------------
template <int KIND, bool VEC>
__global__ __launch_bounds__(kRB) void k_rows_wave(const float *__restrict__ x, float *__restrict__ y,
                                                   int32_t *__restrict__ arg, int64_t outer, int64_t R, float scale) {
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t wave = ((int64_t)blockIdx.x * kRB + threadIdx.x) / kWave;
    const int64_t nwaves = (int64_t)gridDim.x * (kRB / kWave);
    if constexpr (VEC) {
        if (R <= 16 * kWave) {
            // a row is at most 4 vectors per lane: the next row's loads are issued before the current
            // row is reduced; lane 0 holds the row's first element (the NaN rule's x0) in q[0].x
            const int64_t nv = R / 4;
            auto load = [&](int64_t o, f4 *q) {
                const f4 *row = (const f4 *)(x + o * R);
#pragma unroll
                for (int k = 0; k < 4; k++)
                    if (lane + k * kWave < nv) q[k] = __builtin_nontemporal_load(row + lane + k * kWave);
            };
            auto process = [&](int64_t o, const f4 *q) {
                Acc<KIND> acc;
                acc.init();
                if constexpr (KIND == NC_HIP_RED_SUM || KIND == NC_HIP_RED_MEAN) {
#pragma unroll
                    for (int k = 0; k < 4; k++) {
                        const int v = lane + k * kWave;
                        if (v < nv) {
                            acc.push(q[k].x, 4 * v);
                            acc.push(q[k].y, 4 * v + 1);
                            acc.push(q[k].z, 4 * v + 2);
                            acc.push(q[k].w, 4 * v + 3);
                        }
                    }
                } else {
                    // the lane's elements arrive in increasing index order, so its scan state is the
                    // first element equal to their NaN-skipping maximum (-0 and +0 compare equal, and
                    // the first of them is the one kept, with its sign): one max pass, then one
                    // compare-and-select pass from the last element down, instead of a compare, a NaN
                    // test and two selects per element
                    float m = __builtin_nanf("");
#pragma unroll
                    for (int k = 0; k < 4; k++)
                        if (lane + k * kWave < nv)
                            m = __builtin_fmaxf(m, __builtin_fmaxf(__builtin_fmaxf(q[k].x, q[k].y),
                                                                   __builtin_fmaxf(q[k].z, q[k].w)));
                    int hit = 16;  // position 4 k + c of that element (16: every element is NaN)
                    float hv = 0.0f;
#pragma unroll
                    for (int k = 3; k >= 0; k--) {
                        if (lane + k * kWave < nv) {
#pragma unroll
                            for (int c = 3; c >= 0; c--) {
                                const float e = c == 0 ? q[k].x : c == 1 ? q[k].y : c == 2 ? q[k].z : q[k].w;
                                if (e == m) {
                                    hit = 4 * k + c;
                                    hv = e;
                                }
                            }
                        }
                    }
                    if (hit < 16) acc.a = ArgState{hv, 4 * (lane + (hit >> 2) * kWave) + (hit & 3)};
                }
                acc.wave();
                if (lane == 0) emit<KIND>(acc, q[0].x, scale, y, arg, o);
            };
            // two register bundles in turn, every steady-state load unconditional
            int64_t o = wave;
            f4 A[4], B[4];
            if (o < outer) load(o, A);
            while (o + 2 * nwaves < outer) {
                load(o + nwaves, B);
                process(o, A);
                load(o + 2 * nwaves, A);
                process(o + nwaves, B);
                o += 2 * nwaves;
            }
            if (o < outer) {
                const bool hb = o + nwaves < outer;
                if (hb) load(o + nwaves, B);
                process(o, A);
                if (hb) process(o + nwaves, B);
            }
            return;
        }
    }
    for (int64_t o = wave; o < outer; o += nwaves) {
        const float *row = x + o * R;
        Acc<KIND> acc;
        acc.init();
        if constexpr (VEC) {
            // 4 vectors per lane in flight, pushed in increasing index order (argmax tie rule)
            const int64_t nv = R / 4;
            for (int64_t v0 = lane; v0 < nv; v0 += 4 * kWave) {
                f4 q[4];
#pragma unroll
                for (int k = 0; k < 4; k++)
                    if (v0 + k * kWave < nv) q[k] = __builtin_nontemporal_load((const f4 *)row + v0 + k * kWave);
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    const int64_t v = v0 + k * kWave;
                    if (v < nv) {
                        acc.push(q[k].x, (int)(4 * v));
                        acc.push(q[k].y, (int)(4 * v + 1));
                        acc.push(q[k].z, (int)(4 * v + 2));
                        acc.push(q[k].w, (int)(4 * v + 3));
                    }
                }
            }
        } else {
            for (int64_t r = lane; r < R; r += kWave) acc.push(row[r], (int)r);
        }
        acc.wave();
        if (lane == 0) emit<KIND>(acc, row[0], scale, y, arg, o);
    }
}

// --- inner == 1, few long rows: chunk partials then combine -------------------------------------------
template <int KIND>
__global__ __launch_bounds__(kRB) void k_rows_chunk(const float *__restrict__ x, int64_t R, int64_t chunk, int P,
                                                    double *__restrict__ psum, ArgState *__restrict__ parg,
                                                    bool vec) {
    const int64_t o = blockIdx.y;
    const int p = blockIdx.x;
    const float *row = x + o * R;
    const int64_t r0 = (int64_t)p * chunk, r1 = min(R, r0 + chunk);
    Acc<KIND> acc;
    acc.init();
    if (vec) {  // chunk is a multiple of 4 and the row is 16-byte aligned
        const f4 *v4 = (const f4 *)(row + r0);
        const int64_t nv = (r1 - r0) / 4;
        for (int64_t v = threadIdx.x; v < nv; v += kRB) {
            const f4 q = __builtin_nontemporal_load(v4 + v);
            const int base = (int)(r0 + 4 * v);
            acc.push(q.x, base);
            acc.push(q.y, base + 1);
            acc.push(q.z, base + 2);
            acc.push(q.w, base + 3);
        }
        for (int64_t r = r0 + nv * 4 + threadIdx.x; r < r1; r += kRB) acc.push(row[r], (int)r);
    } else {
        for (int64_t r = r0 + threadIdx.x; r < r1; r += kRB) acc.push(row[r], (int)r);
    }
    acc.wave();
    __shared__ Acc<KIND> sh[kRB / kWave];
    if ((threadIdx.x & (kWave - 1)) == 0) sh[threadIdx.x / kWave] = acc;
    __syncthreads();
    if (threadIdx.x == 0) {
        Acc<KIND> t = sh[0];
#pragma unroll
        for (int i = 1; i < kRB / kWave; i++) t.combine(sh[i]);
        if constexpr (KIND == NC_HIP_RED_SUM || KIND == NC_HIP_RED_MEAN) psum[o * P + p] = t.sum;
        else parg[o * P + p] = t.a;
    }
}

template <int KIND>
__global__ __launch_bounds__(kRB) void k_rows_combine(const float *__restrict__ x, int64_t R, int P,
                                                      const double *__restrict__ psum,
                                                      const ArgState *__restrict__ parg, float *__restrict__ y,
                                                      int32_t *__restrict__ arg, float scale) {
    const int64_t o = blockIdx.x;
    // fixed tree: each lane folds a strided subset of partials in order, then a fixed wave/block tree
    Acc<KIND> acc;
    acc.init();
    for (int p = threadIdx.x; p < P; p += kRB) {
        Acc<KIND> t;
        t.init();
        if constexpr (KIND == NC_HIP_RED_SUM || KIND == NC_HIP_RED_MEAN) t.sum = psum[o * P + p];
        else t.a = parg[o * P + p];
        acc.combine(t);
    }
    acc.wave();
    __shared__ Acc<KIND> sh[kRB / kWave];
    if ((threadIdx.x & (kWave - 1)) == 0) sh[threadIdx.x / kWave] = acc;
    __syncthreads();
    if (threadIdx.x == 0) {
        Acc<KIND> t = sh[0];
#pragma unroll
        for (int i = 1; i < kRB / kWave; i++) t.combine(sh[i]);
        emit<KIND>(t, x[o * R], scale, y, arg, o);
    }
}

// --- inner > 1: lanes along inner, scan over R (optionally chunked) -------------------------------------
template <int KIND>
__global__ __launch_bounds__(kRB) void k_cols(const float *__restrict__ x, int64_t outer, int64_t R, int64_t inner,
                                              int64_t chunk, int P, double *__restrict__ psum,
                                              ArgState *__restrict__ parg, float *__restrict__ y,
                                              int32_t *__restrict__ arg, float scale) {
    const int64_t cols = outer * inner;
    const int64_t total = cols * P;
    for (int64_t t = (int64_t)blockIdx.x * kRB + threadIdx.x; t < total; t += (int64_t)gridDim.x * kRB) {
        const int64_t c = t % cols;  // (o, i), i fastest
        const int p = (int)(t / cols);
        const int64_t o = c / inner, i = c % inner;
        const float *base = x + o * R * inner + i;
        const int64_t r0 = (int64_t)p * chunk, r1 = min(R, r0 + chunk);
        Acc<KIND> acc;
        acc.init();
        for (int64_t r = r0; r < r1; r++) acc.push(base[r * inner], (int)r);
        if (P == 1) {
            emit<KIND>(acc, base[0], scale, y, arg, c);
        } else {
            if constexpr (KIND == NC_HIP_RED_SUM || KIND == NC_HIP_RED_MEAN) psum[(int64_t)p * cols + c] = acc.sum;
            else parg[(int64_t)p * cols + c] = acc.a;
        }
    }
}

template <int KIND>
__global__ __launch_bounds__(kRB) void k_cols_combine(const float *__restrict__ x, int64_t outer, int64_t R,
                                                      int64_t inner, int P, const double *__restrict__ psum,
                                                      const ArgState *__restrict__ parg, float *__restrict__ y,
                                                      int32_t *__restrict__ arg, float scale) {
    const int64_t cols = outer * inner;
    for (int64_t c = (int64_t)blockIdx.x * kRB + threadIdx.x; c < cols; c += (int64_t)gridDim.x * kRB) {
        Acc<KIND> acc;
        acc.init();
        // the partials in order, their loads issued kU at a time
        constexpr int kU = 8;
        for (int p0 = 0; p0 < P; p0 += kU) {
            Acc<KIND> t[kU];
#pragma unroll
            for (int u = 0; u < kU; u++) {
                t[u].init();
                if (p0 + u < P) {
                    if constexpr (KIND == NC_HIP_RED_SUM || KIND == NC_HIP_RED_MEAN)
                        t[u].sum = psum[(int64_t)(p0 + u) * cols + c];
                    else
                        t[u].a = parg[(int64_t)(p0 + u) * cols + c];
                }
            }
#pragma unroll
            for (int u = 0; u < kU; u++)
                if (p0 + u < P) acc.combine(t[u]);
        }
        const int64_t o = c / inner, i = c % inner;
        emit<KIND>(acc, x[o * R * inner + i], scale, y, arg, c);
    }
}

__global__ void k_fill_f32(float *y, float v, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * kRB + threadIdx.x; i < n; i += (int64_t)gridDim.x * kRB) y[i] = v;
}

// Plan shared by the workspace query and the launch.
struct RedShape {
    int mode;  // 0 rows_wave, 1 rows_chunk, 2 cols
    int64_t chunk;
    int P;
    size_t ws;
};

static RedShape plan(int kind, int64_t outer, int64_t R, int64_t inner) {
    RedShape s{0, R, 1, 0};
    const int64_t cus = kPlanCUs;  // the partition depends on the shape only
    const size_t elt = (kind == NC_HIP_RED_SUM || kind == NC_HIP_RED_MEAN) ? sizeof(double) : sizeof(ArgState);
    if (inner == 1) {
        if (outer >= cus * 16 || R <= 4096) {
            s.mode = 0;
            return s;
        }
        s.mode = 1;
        int64_t want = (cus * 8 + outer - 1) / outer;       // workgroups per row
        int64_t maxp = (R + 4 * 4 * kRB - 1) / (4 * 4 * kRB); // >= 4 vectors per lane
        int64_t P = want < maxp ? want : maxp;
        if (P < 1) P = 1;
        if (P > 65535) P = 65535;
        int64_t chunk = (R + P - 1) / P;
        chunk = (chunk + 3) / 4 * 4;
        s.chunk = chunk;
        s.P = (int)((R + chunk - 1) / chunk);
        s.ws = (size_t)outer * s.P * elt;
        return s;
    }
    s.mode = 2;
    const int64_t cols = outer * inner;
    const int64_t target = cus * 2048;
    int64_t P = cols >= target ? 1 : (target + cols - 1) / cols;
    const int64_t maxp = (R + 31) / 32;
    if (P > maxp) P = maxp;
    if (P < 1) P = 1;
    s.chunk = (R + P - 1) / P;
    s.P = (int)((R + s.chunk - 1) / s.chunk);
    s.ws = s.P > 1 ? (size_t)cols * s.P * elt : 0;
    return s;
}

template <int KIND>
static int launch(int64_t outer, int64_t R, int64_t inner, const float *x, float *y, int32_t *arg, void *ws,
                  size_t ws_bytes, hipStream_t st) {
    const float scale = KIND == NC_HIP_RED_MEAN ? 1.0f / (float)(R ? R : 1) : 1.0f;
    const RedShape s = plan(KIND, outer, R, inner);
    if (s.ws && (ws_bytes < s.ws || !ws))
        return set_error(NC_HIP_ERR_WORKSPACE, "nc_hip_reduce_fwd: workspace of %zu bytes needed", s.ws);
    double *psum = (double *)ws;
    ArgState *parg = (ArgState *)ws;
    if (s.mode == 0) {
        const bool vec = R % 4 == 0 && aligned16(x);
        const int64_t waves = outer;
        const int64_t blocks64 = (waves + (kRB / kWave) - 1) / (kRB / kWave);
        const int64_t cap = (int64_t)num_cus() * NC_RED_ROWS_GRID_PER_CU;
        const unsigned grid = (unsigned)(blocks64 < cap ? blocks64 : cap);
        if (vec)
            hipLaunchKernelGGL((k_rows_wave<KIND, true>), grid, kRB, 0, st, x, y, arg, outer, R, scale);
        else
            hipLaunchKernelGGL((k_rows_wave<KIND, false>), grid, kRB, 0, st, x, y, arg, outer, R, scale);
    } else if (s.mode == 1) {
        if (outer > 65535) return set_error(NC_HIP_ERR_ARG, "nc_hip_reduce_fwd: too many long rows");
        const bool vec = R % 4 == 0 && aligned16(x);
        hipLaunchKernelGGL(k_rows_chunk<KIND>, dim3(s.P, outer), kRB, 0, st, x, R, s.chunk, s.P, psum, parg, vec);
        hipLaunchKernelGGL(k_rows_combine<KIND>, dim3(outer), kRB, 0, st, x, R, s.P, psum, parg, y, arg, scale);
    } else {
        const int64_t cols = outer * inner;
        const int64_t items = cols * s.P;
        const unsigned grid = stream_grid(items, kRB, 16);
        hipLaunchKernelGGL(k_cols<KIND>, grid, kRB, 0, st, x, outer, R, inner, s.chunk, s.P, psum, parg, y, arg,
                           scale);
        if (s.P > 1)
            hipLaunchKernelGGL(k_cols_combine<KIND>, stream_grid(cols, kRB, 16), kRB, 0, st, x, outer, R, inner, s.P,
                               psum, parg, y, arg, scale);
    }
    return check_launch("nc_hip_reduce_fwd");
}

// --- backward ------------------------------------------------------------------------------------------
// sum / mean: gi[o, r, i] (+)= scale * g[o, i].  inner == 1 follows the reference's `p[r] += v` with
// v = scale * g (ops_reduce.c:136-138); inner > 1 its axpy (one fused rounding, :139).
template <bool INNER1, bool ACC>
__global__ __launch_bounds__(kRB) void k_red_bwd(const float *__restrict__ g, float *__restrict__ gi, int64_t n,
                                                 uint32_t Rinner, IntDiv divRI, uint32_t inner, IntDiv divI,
                                                 float scale) {
    // n < 2^32 here; e = (o * R + r) * inner + i
    const uint32_t step = gridDim.x * kRB;
    for (uint32_t e = blockIdx.x * kRB + threadIdx.x; e < (uint32_t)n; e += step) {
        const uint32_t o = divRI.div(e);
        float gv;
        if (INNER1) {
            gv = g[o];
            const float v = scale * gv;
            gi[e] = (ACC ? gi[e] : 0.0f) + v;
        } else {
            const uint32_t i = e - divI.div(e) * inner;
            gv = g[(int64_t)o * inner + i];
            gi[e] = fma_(scale, gv, ACC ? gi[e] : 0.0f);
        }
    }
}

__global__ __launch_bounds__(kRB) void k_max_bwd(const float *__restrict__ g, const int32_t *__restrict__ arg,
                                                 float *__restrict__ gi, int64_t outer, int64_t R, int64_t inner) {
    const int64_t cols = outer * inner;
    for (int64_t c = (int64_t)blockIdx.x * kRB + threadIdx.x; c < cols; c += (int64_t)gridDim.x * kRB) {
        const int64_t o = c / inner, i = c % inner;
        float *p = gi + (o * R + arg[c]) * inner + i;
        *p = *p + g[c];
    }
}

__global__ __launch_bounds__(kRB) void k_sum_i32(const int32_t *__restrict__ x, int32_t *__restrict__ y, int64_t outer,
                                                 int64_t R, int64_t inner) {
    const int64_t cols = outer * inner;
    for (int64_t c = (int64_t)blockIdx.x * kRB + threadIdx.x; c < cols; c += (int64_t)gridDim.x * kRB) {
        const int64_t o = c / inner, i = c % inner;
        int64_t s = 0;
        for (int64_t r = 0; r < R; r++) s += x[(o * R + r) * inner + i];
        y[c] = (int32_t)s;
    }
}

}  // namespace nchip

using namespace nchip;

extern "C" NC_HIP_API size_t nc_hip_reduce_workspace(int kind, int64_t outer, int64_t R, int64_t inner) {
    if (outer <= 0 || R <= 0 || inner <= 0) return 0;
    if (kind == NC_HIP_RED_ARGMAX) kind = NC_HIP_RED_MAX;
    return plan(kind, outer, R, inner).ws;
}

extern "C" NC_HIP_API int nc_hip_reduce_fwd(int kind, int64_t outer, int64_t R, int64_t inner, const float *x,
                                            float *y, int32_t *arg, void *ws, size_t ws_bytes, void *stream) {
    if (outer < 0 || R < 0 || inner < 0) return set_error(NC_HIP_ERR_ARG, "nc_hip_reduce_fwd: negative size");
    hipStream_t st = as_stream(stream);
    const int64_t nout = outer * inner;
    if (nout == 0) return NC_HIP_OK;
    if (R == 0) {
        if (kind == NC_HIP_RED_MAX || kind == NC_HIP_RED_ARGMAX)
            return set_error(NC_HIP_ERR_ARG, "nc_hip_reduce_fwd: max of an empty axis");
        hipLaunchKernelGGL(k_fill_f32, stream_grid(nout, kRB), kRB, 0, st, y,
                           kind == NC_HIP_RED_MEAN ? __builtin_nanf("") : 0.0f, nout);
        return check_launch("nc_hip_reduce_fwd");
    }
    if ((kind == NC_HIP_RED_SUM || kind == NC_HIP_RED_MEAN || kind == NC_HIP_RED_MAX) && !y)
        return set_error(NC_HIP_ERR_ARG, "nc_hip_reduce_fwd: y is NULL");
    if ((kind == NC_HIP_RED_MAX || kind == NC_HIP_RED_ARGMAX) && !arg)
        return set_error(NC_HIP_ERR_ARG, "nc_hip_reduce_fwd: arg is NULL");
    if (R > INT32_MAX && (kind == NC_HIP_RED_MAX || kind == NC_HIP_RED_ARGMAX))
        return set_error(NC_HIP_ERR_ARG, "nc_hip_reduce_fwd: argmax over more than 2^31 elements");
    switch (kind) {
    case NC_HIP_RED_SUM: return launch<NC_HIP_RED_SUM>(outer, R, inner, x, y, arg, ws, ws_bytes, st);
    case NC_HIP_RED_MEAN: return launch<NC_HIP_RED_MEAN>(outer, R, inner, x, y, arg, ws, ws_bytes, st);
    case NC_HIP_RED_MAX: return launch<NC_HIP_RED_MAX>(outer, R, inner, x, y, arg, ws, ws_bytes, st);
    case NC_HIP_RED_ARGMAX: return launch<NC_HIP_RED_ARGMAX>(outer, R, inner, x, y, arg, ws, ws_bytes, st);
    default: return set_error(NC_HIP_ERR_ARG, "nc_hip_reduce_fwd: unknown kind %d", kind);
    }
}

// ---- allocation-free variant ---------------------------------------------------------------------------
// Partials of nc_hip_reduce_fwd_noalloc: one array per GPU in the code object's device memory, held
// until the process ends.  Host code never passes `scratch` itself to a kernel (in host code the name
// is a stand-in, not a device address): the first call on a device looks its address up with
// hipGetSymbolAddress, with that device current, and every later call on the device uses that
// address.  The largest workspace any reduction plan asks for is below 8 MiB (column scans:
// (cols * P) < 2 * 2^19 partials of 8 bytes), so every shape nc_hip_reduce_fwd takes fits.
constexpr size_t kNoAllocScratchBytes = size_t(8) << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

static void *g_scratch_ptr[64];
static std::mutex g_scratch_mu;

static void *scratch_ptr() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void *p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) {
            (void)hipGetLastError();
            return nullptr;
        }
        g_scratch_ptr[dev] = p;
    }
    return g_scratch_ptr[dev];
}

extern "C" NC_HIP_API int nc_hip_reduce_fwd_noalloc(int kind, int64_t outer, int64_t R, int64_t inner,
                                                    const float *x, float *y, int32_t *arg, void *stream) {
    if (outer < 0 || R < 0 || inner < 0)
        return set_error(NC_HIP_ERR_ARG, "nc_hip_reduce_fwd_noalloc: negative size");
    const size_t need = nc_hip_reduce_workspace(kind, outer, R, inner);
    if (need > kNoAllocScratchBytes)
        return set_error(NC_HIP_ERR_WORKSPACE,
                         "nc_hip_reduce_fwd_noalloc: this shape needs %zu bytes of partials, more than the %zu "
                         "bytes of the static scratch; use nc_hip_reduce_fwd with a workspace",
                         need, kNoAllocScratchBytes);
    void *ws = nullptr;
    if (need) {
        ws = scratch_ptr();
        if (!ws) return set_error(NC_HIP_ERR_DEVICE, "nc_hip_reduce_fwd_noalloc: scratch address lookup failed");
    }
    return nc_hip_reduce_fwd(kind, outer, R, inner, x, y, arg, ws, need, stream);
}

// inner1: the whole problem's inner extent is 1, where the reference adds scale * g (rounded) to gi
// instead of its axpy's fused multiply-add.  A run cut from a longer inner dim keeps the fused form even
// where it is one element wide.
static int reduce_bwd_sum_run(int64_t outer, int64_t R, int64_t inner, const float *g, float *gi, float scale,
                              int accumulate, bool inner1, hipStream_t st) {
    const int64_t n = outer * R * inner;
    const uint32_t RI = (uint32_t)(R * inner);
    const IntDiv dRI(RI), dI((uint32_t)inner);
    const unsigned grid = stream_grid(n, kRB, 16);
    if (inner1) {
        if (accumulate)
            hipLaunchKernelGGL((k_red_bwd<true, true>), grid, kRB, 0, st, g, gi, n, RI, dRI, (uint32_t)inner, dI, scale);
        else
            hipLaunchKernelGGL((k_red_bwd<true, false>), grid, kRB, 0, st, g, gi, n, RI, dRI, (uint32_t)inner, dI, scale);
    } else {
        if (accumulate)
            hipLaunchKernelGGL((k_red_bwd<false, true>), grid, kRB, 0, st, g, gi, n, RI, dRI, (uint32_t)inner, dI, scale);
        else
            hipLaunchKernelGGL((k_red_bwd<false, false>), grid, kRB, 0, st, g, gi, n, RI, dRI, (uint32_t)inner, dI, scale);
    }
    return check_launch("nc_hip_reduce_bwd");
}

// sum / mean gradients of 2^32 elements or more run as runs of at most 2^30 elements of gi
// (for_each_run over [outer, R, inner]), each a broadcast-back launch with mean's 1/R of the whole R.
extern "C" NC_HIP_API int nc_hip_reduce_bwd(int kind, int64_t outer, int64_t R, int64_t inner, const float *g,
                                            const int32_t *arg, float *gi, int accumulate, void *stream) {
    hipStream_t st = as_stream(stream);
    if (outer < 0 || R < 0 || inner < 0) return set_error(NC_HIP_ERR_ARG, "nc_hip_reduce_bwd: negative size");
    const int64_t n = outer * R * inner;
    if (n <= 0) return NC_HIP_OK;
    if (kind == NC_HIP_RED_MAX) {
        if (!accumulate) hipLaunchKernelGGL(k_fill_f32, stream_grid(n, kRB, 16), kRB, 0, st, gi, 0.0f, n);
        hipLaunchKernelGGL(k_max_bwd, stream_grid(outer * inner, kRB, 16), kRB, 0, st, g, arg, gi, outer, R, inner);
        return check_launch("nc_hip_reduce_bwd");
    }
    if (kind != NC_HIP_RED_SUM && kind != NC_HIP_RED_MEAN)
        return set_error(NC_HIP_ERR_ARG, "nc_hip_reduce_bwd: kind %d has no gradient", kind);
    const float scale = kind == NC_HIP_RED_MEAN ? 1.0f / (float)(R ? R : 1) : 1.0f;
    const RunSplit rsp = run_split();
    if (n <= rsp.above) return reduce_bwd_sum_run(outer, R, inner, g, gi, scale, accumulate, inner == 1, st);
    const int64_t shape[3] = {outer, R, inner}, sgi[3] = {R * inner, inner, 1}, sg[3] = {inner, 0, 1};
    const int64_t *strides[2] = {sg, sgi};
    return for_each_run(3, shape, 2, strides, rsp.limit, [&](const int64_t *rs, const int64_t *off, const bool *) {
        return reduce_bwd_sum_run(rs[0], rs[1], rs[2], g + off[0], gi + off[1], scale, accumulate, inner == 1, st);
    });
}

extern "C" NC_HIP_API int nc_hip_reduce_sum_i32(int64_t outer, int64_t R, int64_t inner, const int32_t *x,
                                                int32_t *y, void *stream) {
    const int64_t cols = outer * inner;
    if (cols <= 0) return NC_HIP_OK;
    hipLaunchKernelGGL(k_sum_i32, stream_grid(cols, kRB, 16), kRB, 0, as_stream(stream), x, y, outer, R, inner);
    return check_launch("nc_hip_reduce_sum_i32");
}
