// int8 absmax quantization and dequantization (quantize_row / nc_quantize_rows, ops_quant.c:11-39;
// dequantize = to_dtype i8 -> f32 then a row-broadcast multiply, ops_shape.c:491-504 and
// ops_elementwise.c:22).
//
// quantize: a row of up to 8192 floats stays in registers -- spread over a workgroup of 4 waves when
// its length is a multiple of 1024, else in one wave64 (VPL 128-bit vectors per lane) -- so w is read
// once (4 B/el) and q written once (1 B/el, four int8 packed per 32-bit store).  Rows are
// independent, so 48 stacked 4096x4096 matrices are a single launch.
// dequantize: a streaming map, each lane reading 4 int8 (one 32-bit load) and writing one 128-bit
// float vector, lane-contiguous so loads and stores coalesce.
//
// Arithmetic is the reference's exactly: amax = max |x| (fmaxf, NaN ignored, order-free),
// s = amax / 127 (1 for a zero row), inv = 1 / s, q = clamp(rne(x * inv), -127, 127); the
// float -> int8 conversion maps NaN to 0 as the reference's truncating conversion does.
#include "common.hpp"
#include "intdiv.hpp"

#ifndef NC_QUANT_GRID_PER_CU
#define NC_QUANT_GRID_PER_CU 16
#endif

namespace nchip {

constexpr int kQB = 256;

__device__ __forceinline__ int quant1(float x, float inv) {
    const float v = __builtin_rintf(x * inv);
    const float c = v > 127.0f ? 127.0f : v < -127.0f ? -127.0f : v;
    return c != c ? 0 : (int)c;
}

__device__ __forceinline__ uint32_t pack4(int a, int b, int c, int d) {
    return (uint32_t)(a & 0xff) | ((uint32_t)(b & 0xff) << 8) | ((uint32_t)(c & 0xff) << 16) |
           ((uint32_t)(d & 0xff) << 24);
}

template <int VPL>
__global__ __launch_bounds__(kQB) void k_quant_reg(const float *__restrict__ w, int8_t *__restrict__ q,
                                                   float *__restrict__ scale, int64_t rows, int cols) {
    const int lane = threadIdx.x & (kWave - 1);
    const int nv = cols / 4;
    for (int64_t r = ((int64_t)blockIdx.x * kQB + threadIdx.x) / kWave; r < rows;
         r += (int64_t)gridDim.x * (kQB / kWave)) {
        const f4 *wr = (const f4 *)(w + r * cols);
        f4 v[VPL];
        float amax = 0.0f;
#pragma unroll
        for (int k = 0; k < VPL; k++) {
            const int j = lane + k * kWave;
            if (j < nv) {
                v[k] = __builtin_nontemporal_load(wr + j);
                amax = __builtin_fmaxf(amax, __builtin_fmaxf(__builtin_fmaxf(__builtin_fabsf(v[k].x), __builtin_fabsf(v[k].y)),
                                                             __builtin_fmaxf(__builtin_fabsf(v[k].z), __builtin_fabsf(v[k].w))));
            }
        }
        amax = wave_max_nan_skip(amax);
        const float s = amax > 0.0f ? amax / 127.0f : 1.0f;
        const float inv = 1.0f / s;
        uint32_t *qr = (uint32_t *)(q + r * cols);
#pragma unroll
        for (int k = 0; k < VPL; k++) {
            const int j = lane + k * kWave;
            if (j < nv)
                __builtin_nontemporal_store(pack4(quant1(v[k].x, inv), quant1(v[k].y, inv), quant1(v[k].z, inv),
                                                  quant1(v[k].w, inv)),
                                            qr + j);
        }
        if (lane == 0) scale[r] = s;
    }
}

// Rows of VPLW * 1024 floats (1024 .. 8192): a workgroup of 4 waves per row, each lane holding VPLW
// float4 of it, the waves' maxima meeting in LDS, and a grid with a workgroup for every row.  A wave
// then has a quarter of a row in flight and many rows are resident at once: the 48 x 4096 x 4096
// quantization runs at 665-673 us where one wave per 16 KiB row (k_quant_reg) took 712-723, and the
// same workgroups looping over rows took 790-804.
template <int VPLW>
__global__ __launch_bounds__(kQB) void k_quant_wg(const float *__restrict__ w, int8_t *__restrict__ q,
                                                  float *__restrict__ scale, int cols) {
    __shared__ float sh[kQB / kWave];
    const int tid = threadIdx.x;
    const int64_t r = blockIdx.x;
    const f4 *wr = (const f4 *)(w + r * cols);
    f4 v[VPLW];
    float amax = 0.0f;
#pragma unroll
    for (int k = 0; k < VPLW; k++) {
        v[k] = __builtin_nontemporal_load(wr + tid + k * kQB);
        amax = __builtin_fmaxf(amax, __builtin_fmaxf(__builtin_fmaxf(__builtin_fabsf(v[k].x), __builtin_fabsf(v[k].y)),
                                                     __builtin_fmaxf(__builtin_fabsf(v[k].z), __builtin_fabsf(v[k].w))));
    }
    amax = wave_max_nan_skip(amax);
    if ((tid & (kWave - 1)) == 0) sh[tid / kWave] = amax;
    __syncthreads();
    amax = __builtin_fmaxf(__builtin_fmaxf(sh[0], sh[1]), __builtin_fmaxf(sh[2], sh[3]));
    const float s = amax > 0.0f ? amax / 127.0f : 1.0f;
    const float inv = 1.0f / s;
    uint32_t *qr = (uint32_t *)(q + r * cols);
#pragma unroll
    for (int k = 0; k < VPLW; k++)
        __builtin_nontemporal_store(pack4(quant1(v[k].x, inv), quant1(v[k].y, inv), quant1(v[k].z, inv),
                                          quant1(v[k].w, inv)),
                                    qr + tid + k * kQB);
    if (tid == 0) scale[r] = s;
}

// any row length / alignment: one workgroup per row, two passes over the (L2-resident) row
__global__ __launch_bounds__(kQB) void k_quant_blk(const float *__restrict__ w, int8_t *__restrict__ q,
                                                   float *__restrict__ scale, int64_t rows, int64_t cols) {
    __shared__ float sh[kQB / kWave];
    for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
        const float *wr = w + r * cols;
        float amax = 0.0f;
        for (int64_t i = threadIdx.x; i < cols; i += kQB) amax = __builtin_fmaxf(amax, __builtin_fabsf(wr[i]));
        amax = wave_max_nan_skip(amax);
        __syncthreads();
        if ((threadIdx.x & (kWave - 1)) == 0) sh[threadIdx.x / kWave] = amax;
        __syncthreads();
        amax = sh[0];
#pragma unroll
        for (int i = 1; i < kQB / kWave; i++) amax = __builtin_fmaxf(amax, sh[i]);
        const float s = amax > 0.0f ? amax / 127.0f : 1.0f;
        const float inv = 1.0f / s;
        for (int64_t i = threadIdx.x; i < cols; i += kQB) q[r * cols + i] = (int8_t)quant1(wr[i], inv);
        if (threadIdx.x == 0) scale[r] = s;
    }
}

// Lane-contiguous dequantization: lane j reads 4 int8 as one 32-bit word and writes one 128-bit
// float vector, so a wave reads 256 contiguous bytes and writes 1 KiB contiguous; U words in
// flight per lane.  Requires cols % 4 == 0, q 4-byte and w 16-byte aligned, rows * cols / 4 < 2^32.
#ifndef NC_DQ_UNROLL
#define NC_DQ_UNROLL 2
#endif
#ifndef NC_DQ_BLOCK
#define NC_DQ_BLOCK 128
#endif
#ifndef NC_DQ_GRID_PER_CU
#define NC_DQ_GRID_PER_CU 65536
#endif
constexpr int kDqU = NC_DQ_UNROLL;
constexpr int kDqB = NC_DQ_BLOCK;
__global__ __launch_bounds__(kDqB) void k_dequant4(const uint32_t *__restrict__ q, const float *__restrict__ scale,
                                                  f4 *__restrict__ w, uint32_t n4, IntDiv per_row4) {
    const uint64_t step = (uint64_t)gridDim.x * kDqB * kDqU;
    for (uint64_t base = (uint64_t)blockIdx.x * kDqB * kDqU + threadIdx.x; base < n4; base += step) {
        uint32_t v[kDqU];
#pragma unroll
        for (int u = 0; u < kDqU; u++) {
            const uint64_t j = base + (uint64_t)u * kDqB;
            if (j < n4) v[u] = __builtin_nontemporal_load(q + j);
        }
#pragma unroll
        for (int u = 0; u < kDqU; u++) {
            const uint64_t j = base + (uint64_t)u * kDqB;
            if (j < n4) {
                const float s = scale[per_row4.div((uint32_t)j)];
                const uint32_t x = v[u];
                f4 r;
                r.x = (float)(int8_t)(x & 0xffu) * s;
                r.y = (float)(int8_t)((x >> 8) & 0xffu) * s;
                r.z = (float)(int8_t)((x >> 16) & 0xffu) * s;
                r.w = (float)(int8_t)(x >> 24) * s;
                __builtin_nontemporal_store(r, w + j);
            }
        }
    }
}

__global__ __launch_bounds__(kQB) void k_dequant1(const int8_t *__restrict__ q, const float *__restrict__ scale,
                                                  float *__restrict__ w, int64_t n, int64_t cols) {
    const int64_t step = (int64_t)gridDim.x * kQB;
    for (int64_t i = (int64_t)blockIdx.x * kQB + threadIdx.x; i < n; i += step) w[i] = (float)q[i] * scale[i / cols];
}

}  // namespace nchip

using namespace nchip;

extern "C" NC_HIP_API int nc_hip_quantize_rows(int64_t rows, int64_t cols, const float *w, int8_t *q, float *scale,
                                               void *stream) {
    if (rows < 0 || cols < 0) return set_error(NC_HIP_ERR_ARG, "nc_hip_quantize_rows: negative size");
    if (rows == 0) return NC_HIP_OK;
    hipStream_t st = as_stream(stream);
    if (cols == 0) {  // empty rows: scale 1
        nc_hip_fill(scale, 4, 0x3f800000u, rows, stream);
        return check_launch("nc_hip_quantize_rows");
    }
    const bool al = aligned16(w) && ((uintptr_t)q & 3u) == 0;
    const int64_t nv = cols / 4;
    int vpl = 0;
    if (cols % 4 == 0 && al) vpl = nv <= 64 ? 1 : nv <= 128 ? 2 : nv <= 256 ? 4 : nv <= 512 ? 8 : nv <= 1024 ? 16 : nv <= 2048 ? 32 : 0;
    if (cols % 4 == 0 && al && cols % (4 * kQB) == 0 && cols <= 8 * 4 * kQB && rows <= INT32_MAX) {
        const unsigned g = (unsigned)rows;
        switch (cols / (4 * kQB)) {
        case 1: hipLaunchKernelGGL(k_quant_wg<1>, g, kQB, 0, st, w, q, scale, (int)cols); break;
        case 2: hipLaunchKernelGGL(k_quant_wg<2>, g, kQB, 0, st, w, q, scale, (int)cols); break;
        case 3: hipLaunchKernelGGL(k_quant_wg<3>, g, kQB, 0, st, w, q, scale, (int)cols); break;
        case 4: hipLaunchKernelGGL(k_quant_wg<4>, g, kQB, 0, st, w, q, scale, (int)cols); break;
        case 5: hipLaunchKernelGGL(k_quant_wg<5>, g, kQB, 0, st, w, q, scale, (int)cols); break;
        case 6: hipLaunchKernelGGL(k_quant_wg<6>, g, kQB, 0, st, w, q, scale, (int)cols); break;
        case 7: hipLaunchKernelGGL(k_quant_wg<7>, g, kQB, 0, st, w, q, scale, (int)cols); break;
        default: hipLaunchKernelGGL(k_quant_wg<8>, g, kQB, 0, st, w, q, scale, (int)cols); break;
        }
        return check_launch("nc_hip_quantize_rows");
    }
    const int64_t blocks = (rows + (kQB / kWave) - 1) / (kQB / kWave);
    const int64_t cap = (int64_t)num_cus() * NC_QUANT_GRID_PER_CU;
    const unsigned grid = (unsigned)(blocks < cap ? blocks : cap);
    switch (vpl) {
    case 1: hipLaunchKernelGGL(k_quant_reg<1>, grid, kQB, 0, st, w, q, scale, rows, (int)cols); break;
    case 2: hipLaunchKernelGGL(k_quant_reg<2>, grid, kQB, 0, st, w, q, scale, rows, (int)cols); break;
    case 4: hipLaunchKernelGGL(k_quant_reg<4>, grid, kQB, 0, st, w, q, scale, rows, (int)cols); break;
    case 8: hipLaunchKernelGGL(k_quant_reg<8>, grid, kQB, 0, st, w, q, scale, rows, (int)cols); break;
    case 16: hipLaunchKernelGGL(k_quant_reg<16>, grid, kQB, 0, st, w, q, scale, rows, (int)cols); break;
    case 32: hipLaunchKernelGGL(k_quant_reg<32>, grid, kQB, 0, st, w, q, scale, rows, (int)cols); break;
    default: {
        const unsigned g2 = (unsigned)(rows < num_cus() * 8 ? rows : num_cus() * 8);
        hipLaunchKernelGGL(k_quant_blk, g2, kQB, 0, st, w, q, scale, rows, cols);
    }
    }
    return check_launch("nc_hip_quantize_rows");
}

extern "C" NC_HIP_API int nc_hip_dequantize_rows(int64_t rows, int64_t cols, const int8_t *q, const float *scale,
                                                 float *w, void *stream) {
    if (rows < 0 || cols < 0) return set_error(NC_HIP_ERR_ARG, "nc_hip_dequantize_rows: negative size");
    const int64_t n = rows * cols;
    if (n == 0) return NC_HIP_OK;
    hipStream_t st = as_stream(stream);
    if (cols % 4 == 0 && ((uintptr_t)q & 3u) == 0 && aligned16(w) && n / 4 < (int64_t)UINT32_MAX) {
        const int64_t n4 = n / 4;
        hipLaunchKernelGGL(k_dequant4, stream_grid((n4 + kDqU - 1) / kDqU, kDqB, NC_DQ_GRID_PER_CU), kDqB, 0, st, (const uint32_t *)q,
                           scale, (f4 *)w, (uint32_t)n4, IntDiv((uint32_t)(cols / 4)));
    } else {
        hipLaunchKernelGGL(k_dequant1, stream_grid(n, kQB, 16), kQB, 0, st, q, scale, w, n, cols);
    }
    return check_launch("nc_hip_dequantize_rows");
}
