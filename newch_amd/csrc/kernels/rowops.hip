// Row kernels: softmax / log_softmax (ops_nn.c:22-71) and LayerNorm (ops_nn.c:434-522).
//
// A row of up to 4096 floats is held in registers by one wave64 (VPL 128-bit vectors per lane),
// so each op reads its inputs from HBM exactly once and writes its outputs once; the row
// statistics (max, sums) are wave64 shuffle reductions.  Longer or unaligned rows take a
// workgroup-per-row path that re-reads the row from global memory (L2-resident) per pass.
//
// Per element the fp32 expressions are the reference's (exp8 for the softmax exponentials, the
// same association everywhere), so given the row statistics each output is the reference's
// bit pattern; the statistics are accumulated in fp64 (the reference sums in fp32 for softmax and
// fp64 for LayerNorm), which keeps every result within a few ulp of it.
#include "common.hpp"

namespace nchip {

constexpr int kRowB = 256;             // 4 waves per workgroup, one row per wave
constexpr int kWavesPerBlock = kRowB / kWave;


// ------------------------------------------------------------------------------------------------
// softmax, register-resident rows
// ------------------------------------------------------------------------------------------------
// One wave per row; the next row's loads are issued before the current row is reduced.
template <int VPL, bool LOG>
__global__ __launch_bounds__(kRowB) void k_softmax_fwd_reg(const float *__restrict__ x, float *__restrict__ y,
                                                           int64_t rows, int C) {
    const int lane = threadIdx.x & (kWave - 1);
    const int nv = C / 4;
    const int64_t stride = (int64_t)gridDim.x * kWavesPerBlock;
    auto load = [&](int64_t r, f4 *v) {
        const f4 *xr = (const f4 *)(x + r * C);
#pragma unroll
        for (int k = 0; k < VPL; k++)
            if (lane + k * kWave < nv) v[k] = __builtin_nontemporal_load(xr + lane + k * kWave);
    };
    const int64_t r0 = ((int64_t)blockIdx.x * kRowB + threadIdx.x) / kWave;
    f4 v[VPL], vn[VPL];
    if (r0 < rows) load(r0, v);
    for (int64_t r = r0; r < rows; r += stride) {
        if (r + stride < rows) load(r + stride, vn);
        float m = -__builtin_inff();
#pragma unroll
        for (int k = 0; k < VPL; k++) {
            if (lane + k * kWave < nv)
                m = __builtin_fmaxf(m, __builtin_fmaxf(__builtin_fmaxf(v[k].x, v[k].y), __builtin_fmaxf(v[k].z, v[k].w)));
        }
        m = wave_max_nan_skip(m);
        m = row_max_finish(m, lane0_f32(v[0].x));  // lane 0 holds the row's first element
        // the row sum: plain softmax needs exp8's values themselves (outputs); log_softmax only their
        // sum, whose terms come from the hardware exponential (exp_sum_term)
        double s = 0.0;
#pragma unroll
        for (int k = 0; k < VPL; k++) {
            const int j = lane + k * kWave;
            if (j < nv) {
                f4 e;
                if (LOG) {
                    e.x = exp_sum_term(v[k].x - m);
                    e.y = exp_sum_term(v[k].y - m);
                    e.z = exp_sum_term(v[k].z - m);
                    e.w = exp_sum_term(v[k].w - m);
                } else {
                    e.x = exp8_nonpos(v[k].x - m);
                    e.y = exp8_nonpos(v[k].y - m);
                    e.z = exp8_nonpos(v[k].z - m);
                    e.w = exp8_nonpos(v[k].w - m);
                    v[k] = e;
                }
                s += ((double)e.x + (double)e.y) + ((double)e.z + (double)e.w);
            }
        }
        const float sf = (float)wave_sum(s);
        f4 *yr = (f4 *)(y + r * C);
        if (LOG) {
            const float ls = logf(sf);
#pragma unroll
            for (int k = 0; k < VPL; k++) {
                const int j = lane + k * kWave;
                if (j < nv) {
                    f4 o;
                    o.x = (v[k].x - m) - ls;
                    o.y = (v[k].y - m) - ls;
                    o.z = (v[k].z - m) - ls;
                    o.w = (v[k].w - m) - ls;
                    __builtin_nontemporal_store(o, yr + j);
                }
            }
        } else {
            const float inv = 1.0f / sf;
#pragma unroll
            for (int k = 0; k < VPL; k++) {
                const int j = lane + k * kWave;
                if (j < nv) {
                    f4 o;
                    o.x = inv * v[k].x;
                    o.y = inv * v[k].y;
                    o.z = inv * v[k].z;
                    o.w = inv * v[k].w;
                    __builtin_nontemporal_store(o, yr + j);
                }
            }
        }
#pragma unroll
        for (int k = 0; k < VPL; k++) v[k] = vn[k];
    }
}

// One wave per row; the row's gi (when accumulating) and the next row's y, g are requested before
// the current row is reduced.
template <int VPL, bool LOG, bool ACC>
__global__ __launch_bounds__(kRowB) void k_softmax_bwd_reg(const float *__restrict__ y, const float *__restrict__ g,
                                                           float *__restrict__ gi, int64_t rows, int C) {
    const int lane = threadIdx.x & (kWave - 1);
    const int nv = C / 4;
    const int64_t stride = (int64_t)gridDim.x * kWavesPerBlock;
    auto load = [&](int64_t r, f4 *vy, f4 *vg) {
        const f4 *yr = (const f4 *)(y + r * C), *gr = (const f4 *)(g + r * C);
#pragma unroll
        for (int k = 0; k < VPL; k++) {
            const int j = lane + k * kWave;
            if (j < nv) {
                vy[k] = __builtin_nontemporal_load(yr + j);
                vg[k] = __builtin_nontemporal_load(gr + j);
            }
        }
    };
    const int64_t r0 = ((int64_t)blockIdx.x * kRowB + threadIdx.x) / kWave;
    f4 vy[VPL], vg[VPL], ny[VPL], ng[VPL];
    if (r0 < rows) load(r0, vy, vg);
    for (int64_t r = r0; r < rows; r += stride) {
        f4 *orow = (f4 *)(gi + r * C);
        f4 go[VPL];
        if (ACC) {
#pragma unroll
            for (int k = 0; k < VPL; k++)
                if (lane + k * kWave < nv) go[k] = __builtin_nontemporal_load(orow + lane + k * kWave);
        }
        if (r + stride < rows) load(r + stride, ny, ng);
        double s = 0.0;
#pragma unroll
        for (int k = 0; k < VPL; k++) {
            if (lane + k * kWave < nv) {
                if (LOG) s += ((double)vg[k].x + (double)vg[k].y) + ((double)vg[k].z + (double)vg[k].w);
                else
                    s += ((double)(vg[k].x * vy[k].x) + (double)(vg[k].y * vy[k].y)) +
                         ((double)(vg[k].z * vy[k].z) + (double)(vg[k].w * vy[k].w));
            }
        }
        const float sf = (float)wave_sum(s);
#pragma unroll
        for (int k = 0; k < VPL; k++) {
            const int j = lane + k * kWave;
            if (j < nv) {
                f4 o = ACC ? go[k] : f4{0.f, 0.f, 0.f, 0.f};
                if (LOG) {
                    o.x = o.x + (vg[k].x - expf(vy[k].x) * sf);
                    o.y = o.y + (vg[k].y - expf(vy[k].y) * sf);
                    o.z = o.z + (vg[k].z - expf(vy[k].z) * sf);
                    o.w = o.w + (vg[k].w - expf(vy[k].w) * sf);
                } else {
                    o.x = o.x + vy[k].x * (vg[k].x - sf);
                    o.y = o.y + vy[k].y * (vg[k].y - sf);
                    o.z = o.z + vy[k].z * (vg[k].z - sf);
                    o.w = o.w + vy[k].w * (vg[k].w - sf);
                }
                __builtin_nontemporal_store(o, orow + j);
            }
        }
#pragma unroll
        for (int k = 0; k < VPL; k++) {
            vy[k] = ny[k];
            vg[k] = ng[k];
        }
    }
}

// block-wide reductions for the workgroup-per-row paths
__device__ __forceinline__ double block_sum(double v, double *sh) {
    v = wave_sum(v);
    __syncthreads();
    if ((threadIdx.x & (kWave - 1)) == 0) sh[threadIdx.x / kWave] = v;
    __syncthreads();
    double t = 0.0;
#pragma unroll
    for (int i = 0; i < kWavesPerBlock; i++) t += sh[i];
    return t;
}
__device__ __forceinline__ float block_max(float v, float *sh) {
    v = wave_max_nan_skip(v);
    __syncthreads();
    if ((threadIdx.x & (kWave - 1)) == 0) sh[threadIdx.x / kWave] = v;
    __syncthreads();
    float t = sh[0];
#pragma unroll
    for (int i = 1; i < kWavesPerBlock; i++) t = __builtin_fmaxf(t, sh[i]);
    return t;
}

template <bool LOG>
__global__ __launch_bounds__(kRowB) void k_softmax_fwd_blk(const float *__restrict__ x, float *__restrict__ y,
                                                           int64_t rows, int64_t C) {
    __shared__ double shd[kWavesPerBlock];
    __shared__ float shf[kWavesPerBlock];
    for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
        const float *xr = x + r * C;
        float *yr = y + r * C;
        float m = -__builtin_inff();
        for (int64_t c = threadIdx.x; c < C; c += kRowB) m = __builtin_fmaxf(m, xr[c]);
        m = row_max_finish(block_max(m, shf), xr[0]);
        double s = 0.0;
        for (int64_t c = threadIdx.x; c < C; c += kRowB) s += (double)exp8_nonpos(xr[c] - m);
        const float sf = (float)block_sum(s, shd);
        if (LOG) {
            const float ls = logf(sf);
            for (int64_t c = threadIdx.x; c < C; c += kRowB) yr[c] = (xr[c] - m) - ls;
        } else {
            const float inv = 1.0f / sf;
            for (int64_t c = threadIdx.x; c < C; c += kRowB) yr[c] = inv * exp8_nonpos(xr[c] - m);
        }
        __syncthreads();
    }
}

template <bool LOG, bool ACC>
__global__ __launch_bounds__(kRowB) void k_softmax_bwd_blk(const float *__restrict__ y, const float *__restrict__ g,
                                                           float *__restrict__ gi, int64_t rows, int64_t C) {
    __shared__ double shd[kWavesPerBlock];
    for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
        const float *yr = y + r * C, *gr = g + r * C;
        float *o = gi + r * C;
        double s = 0.0;
        for (int64_t c = threadIdx.x; c < C; c += kRowB) s += LOG ? (double)gr[c] : (double)(gr[c] * yr[c]);
        const float sf = (float)block_sum(s, shd);
        for (int64_t c = threadIdx.x; c < C; c += kRowB) {
            const float old = ACC ? o[c] : 0.0f;
            o[c] = LOG ? old + (gr[c] - expf(yr[c]) * sf) : old + yr[c] * (gr[c] - sf);
        }
        __syncthreads();
    }
}

// ------------------------------------------------------------------------------------------------
// LayerNorm
// ------------------------------------------------------------------------------------------------
// One wave per row; gamma / beta are held in registers and the next row's loads are issued before
// the current row is reduced.
template <int VPL>
__global__ __launch_bounds__(kRowB) void k_ln_fwd_reg(const float *__restrict__ x, const float *__restrict__ w,
                                                      const float *__restrict__ b, float eps, float *__restrict__ y,
                                                      float *__restrict__ stats, int64_t rows, int D) {
    const int lane = threadIdx.x & (kWave - 1);
    const int nv = D / 4;
    const int64_t stride = (int64_t)gridDim.x * kWavesPerBlock;
    f4 ww[VPL], bv[VPL];
#pragma unroll
    for (int k = 0; k < VPL; k++) {
        const int j = lane + k * kWave;
        ww[k] = (w && j < nv) ? ((const f4 *)w)[j] : f4{0.f, 0.f, 0.f, 0.f};
        bv[k] = (b && j < nv) ? ((const f4 *)b)[j] : f4{0.f, 0.f, 0.f, 0.f};
    }
    auto load = [&](int64_t r, f4 *v) {
        const f4 *xr = (const f4 *)(x + r * D);
#pragma unroll
        for (int k = 0; k < VPL; k++)
            if (lane + k * kWave < nv) v[k] = __builtin_nontemporal_load(xr + lane + k * kWave);
    };
    const int64_t r0 = ((int64_t)blockIdx.x * kRowB + threadIdx.x) / kWave;
    f4 v[VPL], vn[VPL];
    if (r0 < rows) load(r0, v);
    for (int64_t r = r0; r < rows; r += stride) {
        if (r + stride < rows) load(r + stride, vn);
        double s = 0.0;
#pragma unroll
        for (int k = 0; k < VPL; k++) {
            if (lane + k * kWave < nv) s += ((double)v[k].x + (double)v[k].y) + ((double)v[k].z + (double)v[k].w);
        }
        const double mean = wave_sum(s) / (double)D;
        double ss = 0.0;
#pragma unroll
        for (int k = 0; k < VPL; k++) {
            if (lane + k * kWave < nv) {
                const double a = (double)v[k].x - mean, bb = (double)v[k].y - mean, c = (double)v[k].z - mean,
                             d = (double)v[k].w - mean;
                ss += (a * a + bb * bb) + (c * c + d * d);
            }
        }
        ss = wave_sum(ss);
        const float rstd = (float)(1.0 / sqrt(ss / (double)D + (double)eps));
        const float mf = (float)mean;
        if (lane == 0) {
            stats[2 * r] = mf;
            stats[2 * r + 1] = rstd;
        }
        f4 *yr = (f4 *)(y + r * D);
#pragma unroll
        for (int k = 0; k < VPL; k++) {
            const int j = lane + k * kWave;
            if (j < nv) {
                f4 o;
                float t;
                t = (v[k].x - mf) * rstd; o.x = (w ? t * ww[k].x : t) + bv[k].x;
                t = (v[k].y - mf) * rstd; o.y = (w ? t * ww[k].y : t) + bv[k].y;
                t = (v[k].z - mf) * rstd; o.z = (w ? t * ww[k].z : t) + bv[k].z;
                t = (v[k].w - mf) * rstd; o.w = (w ? t * ww[k].w : t) + bv[k].w;
                __builtin_nontemporal_store(o, yr + j);
            }
        }
#pragma unroll
        for (int k = 0; k < VPL; k++) v[k] = vn[k];
    }
}

__global__ __launch_bounds__(kRowB) void k_ln_fwd_blk(const float *__restrict__ x, const float *__restrict__ w,
                                                      const float *__restrict__ b, float eps, float *__restrict__ y,
                                                      float *__restrict__ stats, int64_t rows, int64_t D) {
    __shared__ double shd[kWavesPerBlock];
    for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
        const float *xr = x + r * D;
        double s = 0.0;
        for (int64_t i = threadIdx.x; i < D; i += kRowB) s += (double)xr[i];
        const double mean = block_sum(s, shd) / (double)D;
        double ss = 0.0;
        for (int64_t i = threadIdx.x; i < D; i += kRowB) {
            const double d = (double)xr[i] - mean;
            ss += d * d;
        }
        ss = block_sum(ss, shd);
        const float rstd = (float)(1.0 / sqrt(ss / (double)D + (double)eps));
        const float mf = (float)mean;
        if (threadIdx.x == 0) {
            stats[2 * r] = mf;
            stats[2 * r + 1] = rstd;
        }
        for (int64_t i = threadIdx.x; i < D; i += kRowB) {
            const float t = (xr[i] - mf) * rstd;
            y[r * D + i] = (w ? t * w[i] : t) + (b ? b[i] : 0.0f);
        }
        __syncthreads();
    }
}

// Backward, register rows.  Each workgroup (8 waves) owns a contiguous range of rows; its waves take
// rows round-robin.  Per row, the gx loads (when accumulating) and then the next row's x and g are
// requested before the row is reduced.  The gw / gb column partials of a wave's rows accumulate in
// fp32 in that wave's own LDS slice (rows up to 1024 floats; registers for longer rows), in row
// order; at the end each column's 8 wave partials are added in wave order in fp64 and written as
// the workgroup's partial, which k_ln_cols_combine adds up in a fixed order.
constexpr int kLnB = 512;
constexpr int kLnWaves = kLnB / kWave;

template <int VPL>
constexpr bool ln_cols_in_lds() { return VPL <= 4; }

// bytes of dynamic LDS k_ln_bwd_reg needs for gw / gb
static size_t ln_bwd_lds(int vpl, int64_t D, bool cols) {
    if (!cols) return 0;
    return vpl <= 4 ? (size_t)kLnWaves * 2 * D * sizeof(float) : (size_t)2 * D * sizeof(double);
}

// rows up to 1024 floats: two workgroups per CU (at most 128 VGPRs); longer rows: one
template <int VPL, bool ACC>
__global__ __launch_bounds__(kLnB, VPL <= 4 ? 4 : 2) void k_ln_bwd_reg(const float *__restrict__ x, const float *__restrict__ w,
                                                     const float *__restrict__ stats, const float *__restrict__ g,
                                                     float *__restrict__ gx, double *__restrict__ part, int64_t rows,
                                                     int D, int64_t rows_per_block) {
    extern __shared__ char ln_lds[];
    // gamma staged in LDS: its reads then wait on the LDS counter, not behind the prefetched row
    __shared__ f4 wsh[VPL * kWave];
    constexpr bool kLdsCols = ln_cols_in_lds<VPL>();
    const int lane = threadIdx.x & (kWave - 1);
    const int wv = threadIdx.x / kWave;
    const int nv = D / 4;
    const int64_t r0 = (int64_t)blockIdx.x * rows_per_block;
    const int64_t r1 = min(rows, r0 + rows_per_block);
    const bool cols = part != nullptr;
    if (w) {
        for (int j = threadIdx.x; j < nv; j += kLnB) wsh[j] = ((const f4 *)w)[j];
        __syncthreads();
    }
    // column accumulators: this wave's LDS slice [2][D] floats, or registers
    f4 *accw = (f4 *)ln_lds + (size_t)wv * 2 * nv, *accb = accw + nv;
    f4 aw[kLdsCols ? 1 : VPL], ab[kLdsCols ? 1 : VPL];
    if constexpr (kLdsCols) {
        if (cols) {
#pragma unroll
            for (int k = 0; k < VPL; k++) {
                const int j = lane + k * kWave;
                if (j < nv) accw[j] = accb[j] = f4{0.f, 0.f, 0.f, 0.f};
            }
        }
    } else {
#pragma unroll
        for (int k = 0; k < VPL; k++) aw[k] = ab[k] = f4{0.f, 0.f, 0.f, 0.f};
    }
    auto load = [&](int64_t r, f4 *xv, f4 *gv) {
        const f4 *xr = (const f4 *)(x + r * D), *gr = (const f4 *)(g + r * D);
#pragma unroll
        for (int k = 0; k < VPL; k++) {
            const int j = lane + k * kWave;
            if (j < nv) {
                xv[k] = __builtin_nontemporal_load(xr + j);
                gv[k] = __builtin_nontemporal_load(gr + j);
            }
        }
    };
    constexpr bool kPrefetch = VPL <= 4;  // longer rows have no registers for the next row
    f4 xv4[VPL], gg[VPL], xn[kPrefetch ? VPL : 1], gn[kPrefetch ? VPL : 1];
    if (kPrefetch && r0 + wv < r1) load(r0 + wv, xv4, gg);
    for (int64_t r = r0 + wv; r < r1; r += kLnWaves) {
        f4 *dx = gx ? (f4 *)(gx + r * D) : nullptr;
        // the row's statistics, then its gx, then the next row: waits for the first two do not
        // wait for the prefetch
        const float mean = stats[2 * r], rstd = stats[2 * r + 1];
        if (!kPrefetch) load(r, xv4, gg);
        f4 go[VPL];
        if (ACC && dx) {
#pragma unroll
            for (int k = 0; k < VPL; k++)
                if (lane + k * kWave < nv) go[k] = __builtin_nontemporal_load(dx + lane + k * kWave);
        }
        if (kPrefetch && r + kLnWaves < r1) load(r + kLnWaves, xn, gn);
        // xhat = (x - mean) * rstd and gw = g * w, recomputed (same fp32 operations) in the second
        // pass rather than held live across the row reductions
        auto terms = [&](int k, int j, f4 &xh, f4 &gw) {
            const f4 ww = w ? wsh[j] : f4{1.f, 1.f, 1.f, 1.f};
            xh.x = (xv4[k].x - mean) * rstd;
            xh.y = (xv4[k].y - mean) * rstd;
            xh.z = (xv4[k].z - mean) * rstd;
            xh.w = (xv4[k].w - mean) * rstd;
            gw.x = w ? gg[k].x * ww.x : gg[k].x;
            gw.y = w ? gg[k].y * ww.y : gg[k].y;
            gw.z = w ? gg[k].z * ww.z : gg[k].z;
            gw.w = w ? gg[k].w * ww.w : gg[k].w;
        };
        double sg = 0.0, sgx = 0.0;
#pragma unroll
        for (int k = 0; k < VPL; k++) {
            const int j = lane + k * kWave;
            if (j < nv) {
                f4 xh, gw4;
                terms(k, j, xh, gw4);
                sg += ((double)gw4.x + (double)gw4.y) + ((double)gw4.z + (double)gw4.w);
                sgx += ((double)(gw4.x * xh.x) + (double)(gw4.y * xh.y)) +
                       ((double)(gw4.z * xh.z) + (double)(gw4.w * xh.w));
                if (cols) {
                    f4 t = kLdsCols ? accw[j] : aw[k], u = kLdsCols ? accb[j] : ab[k];
                    t.x += gg[k].x * xh.x;
                    t.y += gg[k].y * xh.y;
                    t.z += gg[k].z * xh.z;
                    t.w += gg[k].w * xh.w;
                    u += gg[k];
                    if constexpr (kLdsCols) {
                        accw[j] = t;
                        accb[j] = u;
                    } else {
                        aw[k] = t;
                        ab[k] = u;
                    }
                }
            }
        }
        if (dx) {
            sg = wave_sum(sg);
            sgx = wave_sum(sgx);
            const float mg = (float)(sg / (double)D), mgx = (float)(sgx / (double)D);
#pragma unroll
            for (int k = 0; k < VPL; k++) {
                const int j = lane + k * kWave;
                if (j < nv) {
                    f4 xh, gw4;
                    terms(k, j, xh, gw4);
                    f4 o = ACC ? go[k] : f4{0.f, 0.f, 0.f, 0.f};
                    o.x = o.x + rstd * ((gw4.x - mg) - xh.x * mgx);
                    o.y = o.y + rstd * ((gw4.y - mg) - xh.y * mgx);
                    o.z = o.z + rstd * ((gw4.z - mg) - xh.z * mgx);
                    o.w = o.w + rstd * ((gw4.w - mg) - xh.w * mgx);
                    __builtin_nontemporal_store(o, dx + j);
                }
            }
        }
        if constexpr (kPrefetch) {
#pragma unroll
            for (int k = 0; k < VPL; k++) {
                xv4[k] = xn[k];
                gg[k] = gn[k];
            }
        }
    }
    if (!cols) return;
    double *out = part + (size_t)blockIdx.x * 2 * D;
    if constexpr (kLdsCols) {
        // column i of [gw | gb]: the 8 wave slices added in wave order
        __syncthreads();
        const float *acc = (const float *)ln_lds;
        for (int i = threadIdx.x; i < 2 * D; i += kLnB) {
            double t = 0.0;
#pragma unroll
            for (int w8 = 0; w8 < kLnWaves; w8++) t += (double)acc[(size_t)w8 * 2 * D + i];
            out[i] = t;
        }
    } else {
        // combine the waves' register partials in LDS (wave order)
        double *lds = (double *)ln_lds;  // [2][D]
        for (int i = threadIdx.x; i < 2 * D; i += kLnB) lds[i] = 0.0;
        __syncthreads();
        for (int wsel = 0; wsel < kLnWaves; wsel++) {
            if (wv == wsel) {
#pragma unroll
                for (int k = 0; k < VPL; k++) {
                    const int j = lane + k * kWave;
                    if (j < nv) {
                        lds[4 * j + 0] += aw[k].x;
                        lds[4 * j + 1] += aw[k].y;
                        lds[4 * j + 2] += aw[k].z;
                        lds[4 * j + 3] += aw[k].w;
                        lds[D + 4 * j + 0] += ab[k].x;
                        lds[D + 4 * j + 1] += ab[k].y;
                        lds[D + 4 * j + 2] += ab[k].z;
                        lds[D + 4 * j + 3] += ab[k].w;
                    }
                }
            }
            __syncthreads();
        }
        for (int i = threadIdx.x; i < 2 * D; i += kLnB) out[i] = lds[i];
    }
}

// Backward for full rows (D = 256 VPL floats, VPL <= 4) that write gx: the same arithmetic and
// column partials as k_ln_bwd_reg, with the rows streamed through two register bundles (x, g and
// the old gx of a row) in turn: the loads of row r + 8 are issued, then row r is reduced and
// stored, then row r + 16 is loaded into the first bundle and row r + 8 reduced.  Every load in the
// steady-state loop is unconditional, so the compiler's in-order memory-counter waits for a row's
// bundle never cover the other bundle's loads (a single prefetch buffer copied forward at the end
// of each row makes it wait for the prefetched row before moving on).  Rows are dealt to the
// waves of the whole grid in turn (wave w of workgroup b takes rows 8 b + w, 8 b + w + 8 G, ...),
// so the chip sweeps the four row streams together instead of one contiguous range per workgroup
// (65536 x 1024: 197 -> 190 us).  At 160-210 VGPRs one workgroup is resident per CU.
#ifndef NC_LN_BWD_INTERLEAVE
#define NC_LN_BWD_INTERLEAVE 1
#endif
#ifndef NC_LN_BWD_WAVES_PER_EU
#define NC_LN_BWD_WAVES_PER_EU 2
#endif
template <int VPL, bool ACC, bool HW>
__global__ __launch_bounds__(kLnB, NC_LN_BWD_WAVES_PER_EU) void k_ln_bwd_pp(const float *__restrict__ x, const float *__restrict__ w,
                                                      const float *__restrict__ stats, const float *__restrict__ g,
                                                      float *__restrict__ gx, double *__restrict__ part,
                                                      int64_t rows, int D, int64_t rows_per_block) {
    extern __shared__ char ln_lds[];
    __shared__ f4 wsh[VPL * kWave];
    constexpr int nv = VPL * kWave;
    const int lane = threadIdx.x & (kWave - 1);
    const int wv = threadIdx.x / kWave;
    const int64_t r0 = (int64_t)blockIdx.x * rows_per_block;
    const int64_t r1 = min(rows, r0 + rows_per_block);
    const bool cols = part != nullptr;
    if constexpr (HW) {  // HW: w is given (the kernel is specialised so no per-element test remains)
        for (int j = threadIdx.x; j < nv; j += kLnB) wsh[j] = ((const f4 *)w)[j];
        __syncthreads();
    }
    // column partials of this wave's rows, fp32 in row order, in registers (the LDS slice layout of
    // k_ln_bwd_reg is filled once at the end, so the sums are the same)
    f4 aw[VPL], ab[VPL];
#pragma unroll
    for (int k = 0; k < VPL; k++) aw[k] = ab[k] = f4{0.f, 0.f, 0.f, 0.f};
    struct Bundle {
        f4 x[VPL], g[VPL], o[VPL];
        f2 st;  // mean, rstd
    };
    auto load = [&](int64_t r, Bundle &b) {
        const f4 *xr = (const f4 *)(x + r * D), *gr = (const f4 *)(g + r * D), *orow = (const f4 *)(gx + r * D);
#pragma unroll
        for (int k = 0; k < VPL; k++) {
            const int j = lane + k * kWave;
            b.x[k] = __builtin_nontemporal_load(xr + j);
            b.g[k] = __builtin_nontemporal_load(gr + j);
            if (ACC) b.o[k] = __builtin_nontemporal_load(orow + j);
        }
        b.st = *(const f2 *)(stats + 2 * r);  // with the row: a later load would be waited for with the other bundle
    };
    auto process = [&](int64_t r, const Bundle &b) {
        const float mean = b.st.x, rstd = b.st.y;
        auto terms = [&](int k, f4 &xh, f4 &gw) {
            const f4 ww = HW ? wsh[lane + k * kWave] : f4{1.f, 1.f, 1.f, 1.f};
            xh.x = (b.x[k].x - mean) * rstd;
            xh.y = (b.x[k].y - mean) * rstd;
            xh.z = (b.x[k].z - mean) * rstd;
            xh.w = (b.x[k].w - mean) * rstd;
            gw.x = HW ? b.g[k].x * ww.x : b.g[k].x;
            gw.y = HW ? b.g[k].y * ww.y : b.g[k].y;
            gw.z = HW ? b.g[k].z * ww.z : b.g[k].z;
            gw.w = HW ? b.g[k].w * ww.w : b.g[k].w;
        };
        double sg = 0.0, sgx = 0.0;
#pragma unroll
        for (int k = 0; k < VPL; k++) {
            f4 xh, gw4;
            terms(k, xh, gw4);
            sg += ((double)gw4.x + (double)gw4.y) + ((double)gw4.z + (double)gw4.w);
            sgx += ((double)(gw4.x * xh.x) + (double)(gw4.y * xh.y)) + ((double)(gw4.z * xh.z) + (double)(gw4.w * xh.w));
            if (cols) {
                aw[k].x += b.g[k].x * xh.x;
                aw[k].y += b.g[k].y * xh.y;
                aw[k].z += b.g[k].z * xh.z;
                aw[k].w += b.g[k].w * xh.w;
                ab[k] += b.g[k];
            }
        }
        sg = wave_sum(sg);
        sgx = wave_sum(sgx);
        const float mg = (float)(sg / (double)D), mgx = (float)(sgx / (double)D);
        f4 *dx = (f4 *)(gx + r * D);
#pragma unroll
        for (int k = 0; k < VPL; k++) {
            f4 xh, gw4;
            terms(k, xh, gw4);
            f4 o = ACC ? b.o[k] : f4{0.f, 0.f, 0.f, 0.f};
            o.x = o.x + rstd * ((gw4.x - mg) - xh.x * mgx);
            o.y = o.y + rstd * ((gw4.y - mg) - xh.y * mgx);
            o.z = o.z + rstd * ((gw4.z - mg) - xh.z * mgx);
            o.w = o.w + rstd * ((gw4.w - mg) - xh.w * mgx);
            __builtin_nontemporal_store(o, dx + lane + k * kWave);
        }
    };
    // rows of this wave: r, r + step, r + 2 step, ...
    int64_t r = NC_LN_BWD_INTERLEAVE ? (int64_t)blockIdx.x * kLnWaves + wv : r0 + wv;
    const int64_t step = NC_LN_BWD_INTERLEAVE ? (int64_t)gridDim.x * kLnWaves : kLnWaves;
    const int64_t rend = NC_LN_BWD_INTERLEAVE ? rows : r1;
    Bundle A, B;
    if (r < rend) load(r, A);
    // steady state: rows r and r + step exist, and row r + 2 step too for the next first bundle
    while (r + 2 * step < rend) {
        load(r + step, B);
        process(r, A);
        load(r + 2 * step, A);
        process(r + step, B);
        r += 2 * step;
    }
    if (r < rend) {
        const bool hb = r + step < rend;
        if (hb) load(r + step, B);
        process(r, A);
        if (hb) process(r + step, B);
    }
    if (!cols) return;
    // column i of [gw | gb]: the 8 wave slices added in wave order
    f4 *accw = (f4 *)ln_lds + (size_t)wv * 2 * nv, *accb = accw + nv;
#pragma unroll
    for (int k = 0; k < VPL; k++) {
        accw[lane + k * kWave] = aw[k];
        accb[lane + k * kWave] = ab[k];
    }
    __syncthreads();
    double *out = part + (size_t)blockIdx.x * 2 * D;
    const float *acc = (const float *)ln_lds;
    for (int i = threadIdx.x; i < 2 * D; i += kLnB) {
        double t = 0.0;
#pragma unroll
        for (int w8 = 0; w8 < kLnWaves; w8++) t += (double)acc[(size_t)w8 * 2 * D + i];
        out[i] = t;
    }
}

// Backward for full rows of 512 VH floats (VH = 1, 2) that write gx, each row split between the two
// waves of a pair: wave 2p + h of the workgroup holds columns [h D / 2, (h + 1) D / 2) of the pair's
// rows, so a wave's bundle (x, g and the old gx) is half a row and two bundles fit in 128 VGPRs: four
// waves per SIMD instead of the two of k_ln_bwd_pp.  Per row the two halves' fp64 sums (sum of g w,
// sum of g w xhat) meet in LDS: each wave writes its wave sum, one barrier, and both waves add half 0
// then half 1.  The workgroup's pairs step through their rows together (pair p of workgroup b takes
// rows P b + p, P b + p + P G, ...), so every wave meets the same barriers; the sum slots alternate
// between two sets, since a set is rewritten only after the next barrier, which every wave reaches
// after reading it.  Rows stream through two bundles as in k_ln_bwd_pp.  gw / gb: each wave's column
// partials in fp32 in row order; at the end a column's partials of the workgroup's pairs are added in
// pair order in fp64 (the workgroup's partial, added up by k_ln_cols_combine).
constexpr int kLnPairWaves = 16;  // one 1024-lane workgroup per CU
constexpr int kLnPairs = kLnPairWaves / 2;
template <int VH, bool ACC, bool HW>
__global__ __launch_bounds__(kLnPairWaves *kWave, 4) void k_ln_bwd_pair(const float *__restrict__ x,
                                                                        const float *__restrict__ w,
                                                                        const float *__restrict__ stats,
                                                                        const float *__restrict__ g,
                                                                        float *__restrict__ gx,
                                                                        double *__restrict__ part, int64_t rows) {
    constexpr int D = 512 * VH, nh = VH * kWave;  // row length, float4 per half row
    __shared__ f4 wsh[2 * nh];
    __shared__ double xch[2][kLnPairWaves][2];
    __shared__ float colp[kLnPairWaves][2][4 * nh];  // each wave's gw / gb column partials
    const int lane = threadIdx.x & (kWave - 1);
    const int wv = threadIdx.x / kWave, h = wv & 1, pr = wv >> 1;
    const bool cols = part != nullptr;
    if constexpr (HW) {
        for (int j = threadIdx.x; j < 2 * nh; j += kLnPairWaves * kWave) wsh[j] = ((const f4 *)w)[j];
        __syncthreads();
    }
    const int c0 = h * nh;  // this wave's first float4 of a row
    f4 aw[VH], ab[VH];
#pragma unroll
    for (int k = 0; k < VH; k++) aw[k] = ab[k] = f4{0.f, 0.f, 0.f, 0.f};
    struct Bundle {
        f4 x[VH], g[VH], o[VH];
        f2 st;
    };
    auto load = [&](int64_t r, Bundle &b) {
        const f4 *xr = (const f4 *)(x + r * D) + c0, *gr = (const f4 *)(g + r * D) + c0;
        const f4 *orow = (const f4 *)(gx + r * D) + c0;
#pragma unroll
        for (int k = 0; k < VH; k++) {
            b.x[k] = __builtin_nontemporal_load(xr + lane + k * kWave);
            b.g[k] = __builtin_nontemporal_load(gr + lane + k * kWave);
            if (ACC) b.o[k] = __builtin_nontemporal_load(orow + lane + k * kWave);
        }
        b.st = *(const f2 *)(stats + 2 * r);
    };
    auto terms = [&](const Bundle &b, int k, f4 &xh, f4 &gw) {
        const float mean = b.st.x, rstd = b.st.y;
        const f4 ww = HW ? wsh[c0 + lane + k * kWave] : f4{1.f, 1.f, 1.f, 1.f};
        xh.x = (b.x[k].x - mean) * rstd;
        xh.y = (b.x[k].y - mean) * rstd;
        xh.z = (b.x[k].z - mean) * rstd;
        xh.w = (b.x[k].w - mean) * rstd;
        gw.x = HW ? b.g[k].x * ww.x : b.g[k].x;
        gw.y = HW ? b.g[k].y * ww.y : b.g[k].y;
        gw.z = HW ? b.g[k].z * ww.z : b.g[k].z;
        gw.w = HW ? b.g[k].w * ww.w : b.g[k].w;
    };
    // one row of the pair: called by every wave of the workgroup at the same step (one barrier)
    auto step = [&](int64_t r, const Bundle &b, int par) {
        const bool valid = r < rows;
        double sg = 0.0, sgx = 0.0;
        if (valid) {
#pragma unroll
            for (int k = 0; k < VH; k++) {
                f4 xh, gw4;
                terms(b, k, xh, gw4);
                sg += ((double)gw4.x + (double)gw4.y) + ((double)gw4.z + (double)gw4.w);
                sgx += ((double)(gw4.x * xh.x) + (double)(gw4.y * xh.y)) + ((double)(gw4.z * xh.z) + (double)(gw4.w * xh.w));
                if (cols) {
                    aw[k].x += b.g[k].x * xh.x;
                    aw[k].y += b.g[k].y * xh.y;
                    aw[k].z += b.g[k].z * xh.z;
                    aw[k].w += b.g[k].w * xh.w;
                    ab[k] += b.g[k];
                }
            }
        }
        sg = wave_sum(sg);
        sgx = wave_sum(sgx);
        if (lane == 0) {
            xch[par][wv][0] = sg;
            xch[par][wv][1] = sgx;
        }
        __syncthreads();
        if (!valid) return;
        const double tg = xch[par][2 * pr][0] + xch[par][2 * pr + 1][0];
        const double tgx = xch[par][2 * pr][1] + xch[par][2 * pr + 1][1];
        const float mg = (float)(tg / (double)D), mgx = (float)(tgx / (double)D);
        const float rstd = b.st.y;
        f4 *dx = (f4 *)(gx + r * D) + c0;
#pragma unroll
        for (int k = 0; k < VH; k++) {
            f4 xh, gw4;
            terms(b, k, xh, gw4);
            f4 o = ACC ? b.o[k] : f4{0.f, 0.f, 0.f, 0.f};
            o.x = o.x + rstd * ((gw4.x - mg) - xh.x * mgx);
            o.y = o.y + rstd * ((gw4.y - mg) - xh.y * mgx);
            o.z = o.z + rstd * ((gw4.z - mg) - xh.z * mgx);
            o.w = o.w + rstd * ((gw4.w - mg) - xh.w * mgx);
            __builtin_nontemporal_store(o, dx + lane + k * kWave);
        }
    };
    const int64_t Q = (int64_t)gridDim.x * kLnPairs;       // rows per step over the grid
    const int64_t q0 = (int64_t)blockIdx.x * kLnPairs;     // this workgroup's first pair
    const int64_t nsteps = q0 < rows ? (rows - q0 + Q - 1) / Q : 0;  // pair 0 has the most rows
    const int64_t myq = q0 + pr;
    Bundle A, B;
    if (nsteps > 0 && myq < rows) load(myq, A);
    for (int64_t k = 0; k < nsteps; k += 2) {
        const int64_t ra = myq + k * Q, rb = ra + Q, ra2 = rb + Q;
        const bool has_b = k + 1 < nsteps;  // uniform over the workgroup
        if (has_b && rb < rows) load(rb, B);
        step(ra, A, 0);
        if (k + 2 < nsteps && ra2 < rows) load(ra2, A);
        if (has_b) step(rb, B, 1);
    }
    if (!cols) return;
#pragma unroll
    for (int k = 0; k < VH; k++) {
        ((f4 *)colp[wv][0])[lane + k * kWave] = aw[k];
        ((f4 *)colp[wv][1])[lane + k * kWave] = ab[k];
    }
    __syncthreads();
    double *out = part + (size_t)blockIdx.x * 2 * D;
    for (int i = threadIdx.x; i < 2 * D; i += kLnPairWaves * kWave) {
        const int which = i / D, c = i % D, hh = c / (4 * nh), cc = c % (4 * nh);
        double t = 0.0;
#pragma unroll
        for (int p = 0; p < kLnPairs; p++) t += (double)colp[2 * p + hh][which][cc];
        out[i] = t;
    }
}

// Generic backward: one workgroup per row for gx, and column partials for gw/gb.
template <bool ACC>
__global__ __launch_bounds__(kRowB) void k_ln_bwd_blk(const float *__restrict__ x, const float *__restrict__ w,
                                                      const float *__restrict__ stats, const float *__restrict__ g,
                                                      float *__restrict__ gx, int64_t rows, int64_t D) {
    __shared__ double shd[kWavesPerBlock];
    for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
        const float *xr = x + r * D, *gr = g + r * D;
        const float mean = stats[2 * r], rstd = stats[2 * r + 1];
        double sg = 0.0, sgx = 0.0;
        for (int64_t i = threadIdx.x; i < D; i += kRowB) {
            const float xhat = (xr[i] - mean) * rstd, gi = w ? gr[i] * w[i] : gr[i];
            sg += (double)gi;
            sgx += (double)(gi * xhat);
        }
        sg = block_sum(sg, shd);
        sgx = block_sum(sgx, shd);
        const float mg = (float)(sg / (double)D), mgx = (float)(sgx / (double)D);
        for (int64_t i = threadIdx.x; i < D; i += kRowB) {
            const float xhat = (xr[i] - mean) * rstd, gi = w ? gr[i] * w[i] : gr[i];
            const float old = ACC ? gx[r * D + i] : 0.0f;
            gx[r * D + i] = old + rstd * ((gi - mg) - xhat * mgx);
        }
        __syncthreads();
    }
}

// column partials for the generic path: part[p][2][D] over row chunk p
__global__ __launch_bounds__(kRowB) void k_ln_cols_part(const float *__restrict__ x, const float *__restrict__ stats,
                                                        const float *__restrict__ g, double *__restrict__ part,
                                                        int64_t rows, int64_t D, int64_t chunk, int P) {
    const int64_t total = D * P;
    for (int64_t t = (int64_t)blockIdx.x * kRowB + threadIdx.x; t < total; t += (int64_t)gridDim.x * kRowB) {
        const int64_t i = t % D;
        const int p = (int)(t / D);
        const int64_t r0 = (int64_t)p * chunk, r1 = min(rows, r0 + chunk);
        double sw = 0.0, sb = 0.0;
        for (int64_t r = r0; r < r1; r++) {
            const float xhat = (x[r * D + i] - stats[2 * r]) * stats[2 * r + 1];
            const float gv = g[r * D + i];
            sw += (double)(gv * xhat);
            sb += (double)gv;
        }
        part[(size_t)p * 2 * D + i] = sw;
        part[(size_t)p * 2 * D + D + i] = sb;
    }
}

// gw[i] (+)= sum_p part[p][0][i], gb[i] (+)= sum_p part[p][1][i] in a fixed order: a 16 x 64 thread
// block covers 16 columns of one of the two (blockIdx.y: 0 gw, 1 gb); slice y sums partials y,
// y + 64, y + 128, ... in order, then slice 0 adds the 64 slice sums in slice order.  Narrow column
// tiles give D/16 x 2 workgroups, so the few MiB of partials are read by many CUs at once (64 x 16
// tiles over both outputs: 16 workgroups at D = 1024, 10 us for 512 partials).
constexpr int kCombCols = 16, kCombSlices = 64;
__global__ __launch_bounds__(kCombCols *kCombSlices) void k_ln_cols_combine(const double *__restrict__ part,
                                                                            float *__restrict__ gw,
                                                                            float *__restrict__ gb, int64_t D, int P) {
    __shared__ double sh[kCombSlices][kCombCols];
    const int x = threadIdx.x % kCombCols, y = threadIdx.x / kCombCols;
    const int64_t i = (int64_t)blockIdx.x * kCombCols + x;
    const int which = blockIdx.y;
    float *out = which == 0 ? gw : gb;
    if (!out) return;  // uniform over the workgroup
    const double *src = part + (size_t)which * D;
    // the gradient being added into, loaded beside the partials rather than after their sum
    const float o = y == 0 && i < D ? out[i] : 0.0f;
    double t = 0.0;
    if (i < D) {
#pragma unroll 4
        for (int p = y; p < P; p += kCombSlices) t += src[(size_t)p * 2 * D + i];
    }
    sh[y][x] = t;
    __syncthreads();
    if (y == 0 && i < D) {
        double s = 0.0;
#pragma unroll
        for (int k = 0; k < kCombSlices; k++) s += sh[k][x];
        out[i] = (float)((double)o + s);
    }
}

static int vpl_for(int64_t C) {
    const int64_t nv = C / 4;
    if (nv <= 64) return 1;
    if (nv <= 128) return 2;
    if (nv <= 256) return 4;
    if (nv <= 512) return 8;
    if (nv <= 1024) return 16;
    return 0;
}

#ifndef NC_LN_BWD_BLOCKS_PER_CU
#define NC_LN_BWD_BLOCKS_PER_CU 2  // k_ln_bwd_reg, rows up to 1024 floats
#endif
#ifndef NC_LN_BWD_PP_BLOCKS_PER_CU
#define NC_LN_BWD_PP_BLOCKS_PER_CU 1  // k_ln_bwd_pp
#endif
#ifndef NC_LN_BWD_PAIR
#define NC_LN_BWD_PAIR 1  // k_ln_bwd_pair for rows of 512 and 1024 floats
#endif
#ifndef NC_ROWS_GRID_PER_CU
#define NC_ROWS_GRID_PER_CU 65536
#endif
static unsigned rows_grid(int64_t rows) {
    const int64_t blocks = (rows + kWavesPerBlock - 1) / kWavesPerBlock;
    const int64_t cap = (int64_t)num_cus() * NC_ROWS_GRID_PER_CU;
    return (unsigned)(blocks < cap ? blocks : cap);
}

#define NC_VPL_SWITCH(V, CALL)                      \
    switch (V) {                                    \
    case 1: { constexpr int VP = 1; CALL; } break;  \
    case 2: { constexpr int VP = 2; CALL; } break;  \
    case 4: { constexpr int VP = 4; CALL; } break;  \
    case 8: { constexpr int VP = 8; CALL; } break;  \
    default: { constexpr int VP = 16; CALL; } break; \
    }

#define NC_VPL_SWITCH4(V, CALL)                     \
    switch (V) {                                    \
    case 1: { constexpr int VP = 1; CALL; } break;  \
    case 2: { constexpr int VP = 2; CALL; } break;  \
    default: { constexpr int VP = 4; CALL; } break; \
    }

#define NC_VPL_SWITCH8(V, CALL)                     \
    switch (V) {                                    \
    case 1: { constexpr int VP = 1; CALL; } break;  \
    case 2: { constexpr int VP = 2; CALL; } break;  \
    case 4: { constexpr int VP = 4; CALL; } break;  \
    default: { constexpr int VP = 8; CALL; } break; \
    }

// LayerNorm backward plan (shared by the workspace query and the launch)
struct LnPlan {
    bool reg;
    int vpl;
    bool full;                       // k_ln_bwd_pp (full rows of up to 1024 floats, gx written)
    bool pair;                       // k_ln_bwd_pair (rows of 512 or 1024 floats, gx written)
    int64_t blocks, rows_per_block;  // register path
    int64_t chunk;
    int P;                           // generic path
    size_t ws;
};

static LnPlan ln_plan(int64_t rows, int64_t D, bool aligned, bool has_gx) {
    LnPlan p{};
    p.vpl = (D % 4 == 0 && aligned) ? vpl_for(D) : 0;
    if (p.vpl > 8) p.vpl = 0;  // rows beyond 2048 floats would spill registers: generic path
    p.reg = p.vpl != 0;
    if (p.reg) {
        p.full = has_gx && p.vpl <= 4 && D == (int64_t)p.vpl * 4 * kWave;
        p.pair = NC_LN_BWD_PAIR && p.full && (p.vpl == 2 || p.vpl == 4);
        if (p.pair) {  // one workgroup per CU of a 256-CU part, rows dealt to its pairs in turn
            p.blocks = std::min<int64_t>(kPlanCUs, (rows + kLnPairs - 1) / kLnPairs);
            if (p.blocks < 1) p.blocks = 1;
            p.rows_per_block = 0;
            p.ws = (size_t)p.blocks * 2 * D * sizeof(double);
            return p;
        }
        const int per_cu = p.full ? NC_LN_BWD_PP_BLOCKS_PER_CU : p.vpl <= 4 ? NC_LN_BWD_BLOCKS_PER_CU : 1;
        // the resident workgroups of a 256-CU part: rows_per_block fixes which rows each gw/gb
        // partial holds, so it depends on the shape only
        int64_t want = (int64_t)kPlanCUs * per_cu;
        int64_t rpb = (rows + want - 1) / want;
        if (rpb < kLnWaves) rpb = kLnWaves;
        p.rows_per_block = rpb;
        p.blocks = (rows + rpb - 1) / rpb;
        p.ws = (size_t)p.blocks * 2 * D * sizeof(double);
    } else {
        const int64_t target = (int64_t)kPlanCUs * 1024;  // shape-only partition
        int64_t P = (target + D - 1) / D;
        if (P > rows) P = rows;
        if (P < 1) P = 1;
        p.chunk = (rows + P - 1) / P;
        p.P = (int)((rows + p.chunk - 1) / p.chunk);
        p.ws = (size_t)p.P * 2 * D * sizeof(double);
    }
    return p;
}

}  // namespace nchip

using namespace nchip;

extern "C" NC_HIP_API int nc_hip_softmax_fwd(int log_form, int64_t rows, int64_t C, const float *x, float *y,
                                             void *stream) {
    if (rows < 0 || C < 0) return set_error(NC_HIP_ERR_ARG, "nc_hip_softmax_fwd: negative size");
    if (rows == 0 || C == 0) return NC_HIP_OK;
    hipStream_t st = as_stream(stream);
    const int v = (C % 4 == 0 && aligned16(x) && aligned16(y)) ? vpl_for(C) : 0;
    if (v) {
        if (log_form) NC_VPL_SWITCH(v, hipLaunchKernelGGL((k_softmax_fwd_reg<VP, true>), rows_grid(rows), kRowB, 0, st, x, y, rows, (int)C))
        else NC_VPL_SWITCH(v, hipLaunchKernelGGL((k_softmax_fwd_reg<VP, false>), rows_grid(rows), kRowB, 0, st, x, y, rows, (int)C))
    } else {
        const unsigned grid = (unsigned)(rows < num_cus() * 8 ? rows : num_cus() * 8);
        if (log_form) hipLaunchKernelGGL(k_softmax_fwd_blk<true>, grid, kRowB, 0, st, x, y, rows, C);
        else hipLaunchKernelGGL(k_softmax_fwd_blk<false>, grid, kRowB, 0, st, x, y, rows, C);
    }
    return check_launch("nc_hip_softmax_fwd");
}

extern "C" NC_HIP_API int nc_hip_softmax_bwd(int log_form, int64_t rows, int64_t C, const float *y, const float *g,
                                             float *gi, int accumulate, void *stream) {
    if (rows < 0 || C < 0) return set_error(NC_HIP_ERR_ARG, "nc_hip_softmax_bwd: negative size");
    if (rows == 0 || C == 0) return NC_HIP_OK;
    hipStream_t st = as_stream(stream);
    const int v = (C % 4 == 0 && aligned16(y) && aligned16(g) && aligned16(gi)) ? vpl_for(C) : 0;
    const unsigned rg = rows_grid(rows);
    if (v) {
        if (log_form && accumulate) NC_VPL_SWITCH(v, hipLaunchKernelGGL((k_softmax_bwd_reg<VP, true, true>), rg, kRowB, 0, st, y, g, gi, rows, (int)C))
        else if (log_form) NC_VPL_SWITCH(v, hipLaunchKernelGGL((k_softmax_bwd_reg<VP, true, false>), rg, kRowB, 0, st, y, g, gi, rows, (int)C))
        else if (accumulate) NC_VPL_SWITCH(v, hipLaunchKernelGGL((k_softmax_bwd_reg<VP, false, true>), rg, kRowB, 0, st, y, g, gi, rows, (int)C))
        else NC_VPL_SWITCH(v, hipLaunchKernelGGL((k_softmax_bwd_reg<VP, false, false>), rg, kRowB, 0, st, y, g, gi, rows, (int)C))
    } else {
        const unsigned grid = (unsigned)(rows < num_cus() * 8 ? rows : num_cus() * 8);
        if (log_form && accumulate) hipLaunchKernelGGL((k_softmax_bwd_blk<true, true>), grid, kRowB, 0, st, y, g, gi, rows, C);
        else if (log_form) hipLaunchKernelGGL((k_softmax_bwd_blk<true, false>), grid, kRowB, 0, st, y, g, gi, rows, C);
        else if (accumulate) hipLaunchKernelGGL((k_softmax_bwd_blk<false, true>), grid, kRowB, 0, st, y, g, gi, rows, C);
        else hipLaunchKernelGGL((k_softmax_bwd_blk<false, false>), grid, kRowB, 0, st, y, g, gi, rows, C);
    }
    return check_launch("nc_hip_softmax_bwd");
}

extern "C" NC_HIP_API int nc_hip_layer_norm_fwd(int64_t rows, int64_t D, const float *x, const float *w,
                                                const float *b, float eps, float *y, float *stats, void *stream) {
    if (rows < 0 || D <= 0) return set_error(NC_HIP_ERR_ARG, "nc_hip_layer_norm_fwd: bad size");
    if (rows == 0) return NC_HIP_OK;
    hipStream_t st = as_stream(stream);
    const bool al = aligned16(x) && aligned16(y) && (!w || aligned16(w)) && (!b || aligned16(b));
    const int v = (D % 4 == 0 && al) ? vpl_for(D) : 0;
    if (v) {
        NC_VPL_SWITCH(v, hipLaunchKernelGGL(k_ln_fwd_reg<VP>, rows_grid(rows), kRowB, 0, st, x, w, b, eps, y, stats, rows, (int)D))
    } else {
        const unsigned grid = (unsigned)(rows < num_cus() * 8 ? rows : num_cus() * 8);
        hipLaunchKernelGGL(k_ln_fwd_blk, grid, kRowB, 0, st, x, w, b, eps, y, stats, rows, D);
    }
    return check_launch("nc_hip_layer_norm_fwd");
}

extern "C" NC_HIP_API size_t nc_hip_layer_norm_bwd_workspace(int64_t rows, int64_t D) {
    if (rows <= 0 || D <= 0) return 0;
    // the plans without gx have at least as many workgroups (partials) as those with it
    const size_t a = ln_plan(rows, D, true, false).ws, b = ln_plan(rows, D, false, false).ws;
    return a > b ? a : b;
}

extern "C" NC_HIP_API int nc_hip_layer_norm_bwd(int64_t rows, int64_t D, const float *x, const float *w,
                                                const float *stats, const float *g, float *gx, float *gw, float *gb,
                                                int accumulate, void *ws, size_t ws_bytes, void *stream) {
    if (rows < 0 || D <= 0) return set_error(NC_HIP_ERR_ARG, "nc_hip_layer_norm_bwd: bad size");
    if (rows == 0) return NC_HIP_OK;
    hipStream_t st = as_stream(stream);
    const bool al = aligned16(x) && aligned16(g) && (!gx || aligned16(gx)) && (!w || aligned16(w));
    const LnPlan p = ln_plan(rows, D, al, gx != nullptr);
    const bool cols = gw || gb;
    if (cols && (ws_bytes < p.ws || !ws))
        return set_error(NC_HIP_ERR_WORKSPACE, "nc_hip_layer_norm_bwd: workspace of %zu bytes needed", p.ws);
    double *part = cols ? (double *)ws : nullptr;
    if (p.pair) {
        const dim3 grid((unsigned)p.blocks), block(kLnPairWaves * kWave);
#define NC_LN_PAIR(VH_, ACC_)                                                                                     \
    do {                                                                                                          \
        if (w) hipLaunchKernelGGL((k_ln_bwd_pair<VH_, ACC_, true>), grid, block, 0, st, x, w, stats, g, gx, part, rows); \
        else hipLaunchKernelGGL((k_ln_bwd_pair<VH_, ACC_, false>), grid, block, 0, st, x, w, stats, g, gx, part, rows); \
    } while (0)
        if (p.vpl == 4 && accumulate) NC_LN_PAIR(2, true);
        else if (p.vpl == 4) NC_LN_PAIR(2, false);
        else if (accumulate) NC_LN_PAIR(1, true);
        else NC_LN_PAIR(1, false);
#undef NC_LN_PAIR
        if (cols)
            hipLaunchKernelGGL(k_ln_cols_combine, dim3((unsigned)((D + kCombCols - 1) / kCombCols), 2), kCombCols * kCombSlices, 0, st, part, gw, gb, D, (int)p.blocks);
    } else if (p.reg) {
        const size_t lds = ln_bwd_lds(p.vpl, D, cols);
        if (lds > 65536) return set_error(NC_HIP_ERR_ARG, "nc_hip_layer_norm_bwd: D too large for LDS combine");
        const bool full = p.full;
        if (full && accumulate)
            NC_VPL_SWITCH4(p.vpl, if (w) hipLaunchKernelGGL((k_ln_bwd_pp<VP, true, true>), dim3(p.blocks), kLnB, lds, st, x, w, stats, g, gx, part, rows, (int)D, p.rows_per_block); else hipLaunchKernelGGL((k_ln_bwd_pp<VP, true, false>), dim3(p.blocks), kLnB, lds, st, x, w, stats, g, gx, part, rows, (int)D, p.rows_per_block))
        else if (full)
            NC_VPL_SWITCH4(p.vpl, if (w) hipLaunchKernelGGL((k_ln_bwd_pp<VP, false, true>), dim3(p.blocks), kLnB, lds, st, x, w, stats, g, gx, part, rows, (int)D, p.rows_per_block); else hipLaunchKernelGGL((k_ln_bwd_pp<VP, false, false>), dim3(p.blocks), kLnB, lds, st, x, w, stats, g, gx, part, rows, (int)D, p.rows_per_block))
        else if (accumulate)
            NC_VPL_SWITCH8(p.vpl, hipLaunchKernelGGL((k_ln_bwd_reg<VP, true>), dim3(p.blocks), kLnB, lds, st, x, w, stats, g, gx, part, rows, (int)D, p.rows_per_block))
        else
            NC_VPL_SWITCH8(p.vpl, hipLaunchKernelGGL((k_ln_bwd_reg<VP, false>), dim3(p.blocks), kLnB, lds, st, x, w, stats, g, gx, part, rows, (int)D, p.rows_per_block))
        if (cols)
            hipLaunchKernelGGL(k_ln_cols_combine, dim3((unsigned)((D + kCombCols - 1) / kCombCols), 2), kCombCols * kCombSlices, 0, st, part, gw, gb, D, (int)p.blocks);
    } else {
        const unsigned grid = (unsigned)(rows < num_cus() * 8 ? rows : num_cus() * 8);
        if (gx) {
            if (accumulate) hipLaunchKernelGGL(k_ln_bwd_blk<true>, grid, kRowB, 0, st, x, w, stats, g, gx, rows, D);
            else hipLaunchKernelGGL(k_ln_bwd_blk<false>, grid, kRowB, 0, st, x, w, stats, g, gx, rows, D);
        }
        if (cols) {
            hipLaunchKernelGGL(k_ln_cols_part, stream_grid(D * p.P, kRowB), kRowB, 0, st, x, stats, g, part, rows, D,
                               p.chunk, p.P);
            hipLaunchKernelGGL(k_ln_cols_combine, dim3((unsigned)((D + kCombCols - 1) / kCombCols), 2), kCombCols * kCombSlices, 0, st, part, gw, gb, D, p.P);
        }
    }
    return check_launch("nc_hip_layer_norm_bwd");
}
