// int8 GEMM on the matrix cores and the fused int8 linear (the reference's gemm_s8_nt kernel-table
// entry, kernels.h:42-43 / kernels_ref.c:117-128, and linear_int8, ops_quant.c:41-113).
//
// C[m][n] = sum_k A[m][k] * B[n][k] with A [M, K] and B [N, K] both K-contiguous ("NT"), exact in
// int32 (|C| <= K * 127 * 127 stays below 2^31 for K <= 133143, the range the reference's int32
// accumulation is exact in).  Integer sums do not depend on order, so every tiling gives the
// reference's bits.
//
// Tiling: a 256-thread workgroup (4 wave64, 2 x 2) owns a 128 x 128 tile of C; each wave a 64 x 64
// quarter as 2 x 2 v_mfma_i32_32x32x32_i8 accumulators (16 int32 per lane each).  K advances 64 bytes
// at a time: the workgroup stages the A and B panels (128 x 64 bytes each) in LDS with rows padded to
// 80 bytes (16-byte reads of 16 consecutive rows then hit distinct banks), and loads the next panels
// into registers while the matrix cores work on the current one.  Each lane feeds the MFMA 16
// consecutive k bytes of its row (lanes 0-31 rows 0-31 with k 0-15, lanes 32-63 the same rows with
// k 16-31) for A and for B alike, so whatever order the instruction sums a lane's bytes in, A and B
// pair the same k.
// Blocks are remapped so each XCD (blocks b with b % 8 equal) works a contiguous run of tiles, and
// tiles run in groups of 8 tile-rows so neighbouring blocks share panels in L2.
//
// linear_int8 epilogue (ops_quant.c:75-79): y = (float)acc * xs[m] * ws[n] + (bias ? bias[n] : 0),
// evaluated left to right in fp32 without contraction (the reference's scalar glue), so the fused
// result is bit-identical to the reference's.
#include "common.hpp"

namespace nchip {

typedef int i16v __attribute__((ext_vector_type(16)));

constexpr int kQgB = 256;
constexpr int kQgBM = 128, kQgBN = 128, kQgBK = 64;
constexpr int kQgPitch = kQgBK + 16;
constexpr int kQgGroupM = 8;

struct QgArgs {
    const int8_t *A;
    const int8_t *B;
    int64_t lda, ldb, ldc;
    int M, N, K;
    int tiles_m, tiles_n;
    int32_t *C;        // int32 output (gemm_s8_nt)
    float *Y;          // fp32 output (linear_int8), ld = ldc
    const float *xs;   // [M] row scales of A
    const float *ws;   // [N] row scales of B
    const float *bias; // [N] or null
};

// 16 k-bytes of row `row` starting at column k (zeros past the matrix)
template <bool ALIGNED>
__device__ __forceinline__ i4 load16(const int8_t *p, int64_t ld, int row, int rows, int k, int K) {
    i4 v = {0, 0, 0, 0};
    if (row >= rows) return v;
    const int8_t *r = p + (int64_t)row * ld + k;
    if (ALIGNED) {
        if (k < K) v = *(const i4 *)r;
    } else {
        uint32_t w[4] = {0, 0, 0, 0};
#pragma unroll
        for (int b = 0; b < 16; b++)
            if (k + b < K) w[b >> 2] |= (uint32_t)(uint8_t)r[b] << (8 * (b & 3));
        v = i4{(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
    }
    return v;
}

template <bool ALIGNED, bool OUT_F32>
__global__ __launch_bounds__(kQgB, 2) void k_qgemm(QgArgs p) {
    __shared__ __attribute__((aligned(16))) int8_t sa[kQgBM * kQgPitch];
    __shared__ __attribute__((aligned(16))) int8_t sb[kQgBN * kQgPitch];

    int id = blockIdx.x;
    const int nblk = gridDim.x;
    if ((nblk & 7) == 0) id = (id & 7) * (nblk >> 3) + (id >> 3);
    const int per_group = kQgGroupM * p.tiles_n;
    const int first_m = (id / per_group) * kQgGroupM;
    const int gsize = min(p.tiles_m - first_m, kQgGroupM);
    const int tm = first_m + (id % per_group) % gsize;
    const int tn = (id % per_group) / gsize;
    const int m0 = tm * kQgBM, n0 = tn * kQgBN;

    const int t = threadIdx.x, lane = t & (kWave - 1), wid = t / kWave;
    const int wm = wid >> 1, wn = wid & 1;

    // staging: thread t moves 16-byte chunks c = t and t + 256 of each panel (row c / 4, chunk c % 4)
    const int r0 = t >> 2, r1 = r0 + kQgB / 4, kc = (t & 3) * 16;
    i4 ra0, ra1, rb0, rb1;
    auto gload = [&](int k0) {
        ra0 = load16<ALIGNED>(p.A, p.lda, m0 + r0, p.M, k0 + kc, p.K);
        ra1 = load16<ALIGNED>(p.A, p.lda, m0 + r1, p.M, k0 + kc, p.K);
        rb0 = load16<ALIGNED>(p.B, p.ldb, n0 + r0, p.N, k0 + kc, p.K);
        rb1 = load16<ALIGNED>(p.B, p.ldb, n0 + r1, p.N, k0 + kc, p.K);
    };

    i16v acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) acc[i][j] = i16v{};

    const int frow = lane & 31, fk = (lane >> 5) * 16;
    gload(0);
    for (int k0 = 0; k0 < p.K; k0 += kQgBK) {
        *(i4 *)(sa + r0 * kQgPitch + kc) = ra0;
        *(i4 *)(sa + r1 * kQgPitch + kc) = ra1;
        *(i4 *)(sb + r0 * kQgPitch + kc) = rb0;
        *(i4 *)(sb + r1 * kQgPitch + kc) = rb1;
        __syncthreads();
        if (k0 + kQgBK < p.K) gload(k0 + kQgBK);
#pragma unroll
        for (int s = 0; s < kQgBK / 32; s++) {
            i4 fa[2], fb[2];
#pragma unroll
            for (int i = 0; i < 2; i++)
                fa[i] = *(const i4 *)(sa + (wm * 64 + i * 32 + frow) * kQgPitch + s * 32 + fk);
#pragma unroll
            for (int j = 0; j < 2; j++)
                fb[j] = *(const i4 *)(sb + (wn * 64 + j * 32 + frow) * kQgPitch + s * 32 + fk);
#pragma unroll
            for (int i = 0; i < 2; i++)
#pragma unroll
                for (int j = 0; j < 2; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[i], fb[j], acc[i][j], 0, 0, 0);
        }
        __syncthreads();
    }

    // accumulator layout of a 32 x 32 MFMA tile: lane l, element v holds row 8*(v/4) + 4*(l/32) + v%4,
    // column l % 32
#pragma unroll
    for (int i = 0; i < 2; i++) {
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int n = n0 + wn * 64 + j * 32 + (lane & 31);
            if (n >= p.N) continue;
            float wsn = 0.0f, bn = 0.0f;
            if (OUT_F32) {
                wsn = p.ws[n];
                bn = p.bias ? p.bias[n] : 0.0f;
            }
#pragma unroll
            for (int v = 0; v < 16; v++) {
                const int m = m0 + wm * 64 + i * 32 + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
                if (m >= p.M) continue;
                if (OUT_F32)
                    p.Y[(int64_t)m * p.ldc + n] = (float)acc[i][j][v] * p.xs[m] * wsn + bn;
                else
                    p.C[(int64_t)m * p.ldc + n] = acc[i][j][v];
            }
        }
    }
}

static int launch_qgemm(QgArgs p, bool out_f32, hipStream_t st, const char *what) {
    p.tiles_m = (p.M + kQgBM - 1) / kQgBM;
    p.tiles_n = (p.N + kQgBN - 1) / kQgBN;
    const int64_t blocks = (int64_t)p.tiles_m * p.tiles_n;
    if (blocks > INT32_MAX) return set_error(NC_HIP_ERR_ARG, "%s: %lld tiles exceed one launch", what, (long long)blocks);
    const bool aligned = p.K % 16 == 0 && p.lda % 16 == 0 && p.ldb % 16 == 0 && aligned16(p.A) && aligned16(p.B);
    const dim3 grid((unsigned)blocks), block(kQgB);
    if (aligned && out_f32) hipLaunchKernelGGL((k_qgemm<true, true>), grid, block, 0, st, p);
    else if (aligned) hipLaunchKernelGGL((k_qgemm<true, false>), grid, block, 0, st, p);
    else if (out_f32) hipLaunchKernelGGL((k_qgemm<false, true>), grid, block, 0, st, p);
    else hipLaunchKernelGGL((k_qgemm<false, false>), grid, block, 0, st, p);
    return check_launch(what);
}

static bool fits_int(int64_t v) { return v >= 0 && v <= INT32_MAX; }

}  // namespace nchip

using namespace nchip;

extern "C" NC_HIP_API int nc_hip_gemm_s8_nt(int64_t M, int64_t N, int64_t K, const int8_t *A, int64_t lda,
                                            const int8_t *B, int64_t ldb, int32_t *C, int64_t ldc, void *stream) {
    if (!fits_int(M) || !fits_int(N) || !fits_int(K)) return set_error(NC_HIP_ERR_ARG, "nc_hip_gemm_s8_nt: bad sizes");
    if (lda < K || ldb < K || ldc < N) return set_error(NC_HIP_ERR_ARG, "nc_hip_gemm_s8_nt: leading dim too small");
    if (M == 0 || N == 0) return NC_HIP_OK;
    QgArgs p{};
    p.A = A, p.B = B, p.lda = lda, p.ldb = ldb, p.ldc = ldc;
    p.M = (int)M, p.N = (int)N, p.K = (int)K;
    p.C = C;
    return launch_qgemm(p, false, as_stream(stream), "nc_hip_gemm_s8_nt");
}

// workspace: the quantized activations [M, K] and their row scales [M]
static size_t qlin_xs_offset(int64_t M, int64_t K) { return (size_t)(M * K + 255) / 256 * 256; }

extern "C" NC_HIP_API size_t nc_hip_linear_int8_workspace(int64_t M, int64_t K) {
    if (M <= 0 || K < 0) return 0;
    return qlin_xs_offset(M, K) + (size_t)M * sizeof(float);
}

extern "C" NC_HIP_API int nc_hip_linear_int8(int64_t M, int64_t K, int64_t N, const float *x, const int8_t *wq,
                                             const float *wscale, const float *bias, float *y, void *ws,
                                             size_t ws_bytes, void *stream) {
    if (!fits_int(M) || !fits_int(N) || !fits_int(K)) return set_error(NC_HIP_ERR_ARG, "nc_hip_linear_int8: bad sizes");
    if (M == 0 || N == 0) return NC_HIP_OK;
    if (!ws || ws_bytes < nc_hip_linear_int8_workspace(M, K))
        return set_error(NC_HIP_ERR_ARG, "nc_hip_linear_int8: workspace of %zu bytes, need %zu", ws_bytes,
                         nc_hip_linear_int8_workspace(M, K));
    int8_t *xq = (int8_t *)ws;
    float *xs = (float *)((char *)ws + qlin_xs_offset(M, K));
    if (int rc = nc_hip_quantize_rows(M, K, x, xq, xs, stream)) return rc;
    QgArgs p{};
    p.A = xq, p.B = wq, p.lda = K, p.ldb = K, p.ldc = N;
    p.M = (int)M, p.N = (int)N, p.K = (int)K;
    p.Y = y, p.xs = xs, p.ws = wscale, p.bias = bias;
    return launch_qgemm(p, true, as_stream(stream), "nc_hip_linear_int8");
}
