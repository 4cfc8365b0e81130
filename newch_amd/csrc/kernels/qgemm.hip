// int8 GEMM on the matrix cores and the fused int8 linear (the reference's gemm_s8_nt kernel-table
// entry, kernels.h:42-43 / kernels_ref.c:117-128, and linear_int8, ops_quant.c:41-113).
//
// C[m][n] = sum_k A[m][k] * B[n][k] with A [M, K] and B [N, K] both K-contiguous ("NT"), exact in
// int32 (|C| <= K * 127 * 127 stays below 2^31 for K <= 133143, the range the reference's int32
// accumulation is exact in).  Integer sums do not depend on order, so every tiling gives the
// reference's bits.
//
// Tiling: a workgroup owns a BM x BN tile of C, each of its waves a (32 TM) x (32 TN) block of it as
// TM x TN v_mfma_i32_32x32x32_i8 accumulators (16 int32 per lane each).  K advances BK bytes per
// step through two LDS stages: the A and B panels (BM and BN rows of BK bytes, rows padded by 16 bytes
// so 16-byte reads of 16 consecutive rows hit distinct banks) of step k+1 are loaded into registers
// while the matrix cores work on step k, stored into the other stage, and one barrier per step
// separates the two.  Each lane feeds the MFMA 16 consecutive k bytes of its row (lanes 0-31 rows
// 0-31 with k 0-15, lanes 32-63 the same rows with k 16-31) for A and for B alike, so whatever order
// the instruction sums a lane's bytes in, A and B pair the same k.  Large problems run 256 x 256
// tiles (8 waves of 4 x 2 MFMA tiles, BK 128, 147 KiB of LDS), smaller ones 128 x 128 (4 waves of
// 2 x 2, BK 64).  Large problems with K a multiple of 128 and 16-byte aligned rows take k_qgemm_dma
// instead: the same tile over 16 waves, its panels loaded straight into LDS one 128-byte k step ahead.
// Blocks are remapped so each XCD (blocks b with b % 8 equal) works a contiguous run of tiles, and
// tiles run in groups of 8 tile-rows so neighbouring blocks share panels in L2.
//
// linear_int8 epilogue (ops_quant.c:75-79): y = (float)acc * xs[m] * ws[n] + (bias ? bias[n] : 0),
// evaluated left to right in fp32 without contraction (the reference's scalar glue), so the fused
// result is bit-identical to the reference's.
#include "common.hpp"

namespace nchip {

typedef int i16v __attribute__((ext_vector_type(16)));

constexpr int kQgGroupM = 8;

// Tile configurations: TM x TN MFMA tiles (32 x 32) per wave, WGM x WGN waves per workgroup, BK
// k-bytes per stage, two LDS stages.  Large problems use a 256 x 256 tile (8 waves, 147 KiB of LDS,
// one workgroup per CU); problems with fewer such tiles than CUs use 128 x 128 (4 waves, 40 KiB).
template <int TM_, int TN_, int WGM_, int WGN_, int BK_, int OCC_>
struct QgCfg {
    static constexpr int TM = TM_, TN = TN_, WGM = WGM_, WGN = WGN_, BK = BK_, OCC = OCC_;
    static constexpr int NT = 64 * WGM * WGN;
    static constexpr int BM = 32 * TM * WGM, BN = 32 * TN * WGN;
    static constexpr int PITCH = BK + 16;  // 16-byte reads of 16 consecutive rows land on distinct banks
    static constexpr int CHUNK_ROW = BK / 16;  // 16-byte chunks per staged row
    static constexpr int CHUNKS = (BM + BN) * CHUNK_ROW / NT;
    static constexpr int STAGE = (BM + BN) * PITCH;  // bytes of one LDS stage (A rows, then B rows)
    static constexpr size_t LDS = 2 * (size_t)STAGE;
    static_assert((BM + BN) * CHUNK_ROW % NT == 0, "staging chunks must divide over the workgroup");
};
using QgBig = QgCfg<4, 2, 2, 4, 128, 1>;
using QgSmall = QgCfg<2, 2, 2, 2, 64, 2>;

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

template <class C, bool ALIGNED, bool OUT_F32>
__global__ __launch_bounds__(C::NT, C::OCC) void k_qgemm(QgArgs p) {
    extern __shared__ __attribute__((aligned(16))) int8_t smem[];
    constexpr int kTM = C::TM, kTN = C::TN, kWGN = C::WGN, kBK = C::BK, kQgB = C::NT;
    constexpr int kQgBM = C::BM, kQgBN = C::BN, kQgPitch = C::PITCH, kChunkRow = C::CHUNK_ROW;
    constexpr int kChunks = C::CHUNKS, kStage = C::STAGE;

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
    const int wm = wid / kWGN, wn = wid % kWGN;

    // staging: thread t moves chunks c = t + i * kQgB; chunk c is row c / kChunkRow of the stacked
    // [A rows; B rows] panel, k offset (c % kChunkRow) * 16
    i4 reg[kChunks];
    auto gload = [&](int k0) {
#pragma unroll
        for (int i = 0; i < kChunks; i++) {
            const int c = t + i * kQgB, row = c / kChunkRow, kc = (c % kChunkRow) * 16;
            reg[i] = row < kQgBM ? load16<ALIGNED>(p.A, p.lda, m0 + row, p.M, k0 + kc, p.K)
                                 : load16<ALIGNED>(p.B, p.ldb, n0 + row - kQgBM, p.N, k0 + kc, p.K);
        }
    };
    auto sstore = [&](int8_t *stage) {
#pragma unroll
        for (int i = 0; i < kChunks; i++) {
            const int c = t + i * kQgB, row = c / kChunkRow, kc = (c % kChunkRow) * 16;
            *(i4 *)(stage + row * kQgPitch + kc) = reg[i];
        }
    };

    i16v acc[kTM][kTN];
#pragma unroll
    for (int i = 0; i < kTM; i++)
#pragma unroll
        for (int j = 0; j < kTN; j++) acc[i][j] = i16v{};

    const int frow = lane & 31, fk = (lane >> 5) * 16;
    const int nk = (p.K + kBK - 1) / kBK;
    if (nk > 0) {
        gload(0);
        sstore(smem);
        __syncthreads();
    }
    for (int kt = 0; kt < nk; kt++) {
        const int8_t *cur = smem + (kt & 1) * kStage;
        if (kt + 1 < nk) gload((kt + 1) * kBK);
#pragma unroll
        for (int s = 0; s < kBK / 32; s++) {
            i4 fa[kTM], fb[kTN];
#pragma unroll
            for (int i = 0; i < kTM; i++)
                fa[i] = *(const i4 *)(cur + ((wm * kTM + i) * 32 + frow) * kQgPitch + s * 32 + fk);
#pragma unroll
            for (int j = 0; j < kTN; j++)
                fb[j] = *(const i4 *)(cur + (kQgBM + (wn * kTN + j) * 32 + frow) * kQgPitch + s * 32 + fk);
#pragma unroll
            for (int i = 0; i < kTM; i++)
#pragma unroll
                for (int j = 0; j < kTN; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[i], fb[j], acc[i][j], 0, 0, 0);
        }
        // the other stage was last read before the previous barrier, so it can be refilled now
        if (kt + 1 < nk) sstore(smem + ((kt + 1) & 1) * kStage);
        __syncthreads();
    }

    // accumulator layout of a 32 x 32 MFMA tile: lane l, element v holds row 8*(v/4) + 4*(l/32) + v%4,
    // column l % 32
#pragma unroll
    for (int i = 0; i < kTM; i++) {
#pragma unroll
        for (int j = 0; j < kTN; j++) {
            const int n = n0 + (wn * kTN + j) * 32 + (lane & 31);
            if (n >= p.N) continue;
            float wsn = 0.0f, bn = 0.0f;
            if (OUT_F32) {
                wsn = p.ws[n];
                bn = p.bias ? p.bias[n] : 0.0f;
            }
#pragma unroll
            for (int v = 0; v < 16; v++) {
                const int m = m0 + (wm * kTM + i) * 32 + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
                if (m >= p.M) continue;
                if (OUT_F32)
                    p.Y[(int64_t)m * p.ldc + n] = (float)acc[i][j][v] * p.xs[m] * wsn + bn;
                else
                    p.C[(int64_t)m * p.ldc + n] = acc[i][j][v];
            }
        }
    }
}

// ------------------------------------------------------------------------------------------------
// Direct-to-LDS variant for large aligned problems (K a multiple of 128, 16-byte aligned rows): the
// same 256 x 256 tile, but over 16 waves of 2 x 2 MFMA tiles (64 x 64 each, 64 accumulator registers,
// four waves per SIMD: a third more fragment reads per MFMA than 8 waves of 4 x 2, but their latency
// hides behind the other waves' MFMAs, 4-10% faster), and the A and B panels go straight from global
// memory into LDS (global_load_lds_dwordx4: lane i's 16 bytes land at M0 + 16 i) one k step ahead,
// through two 64 KiB stages of 128 k-bytes.  No staging registers and no LDS write instructions; one
// barrier per k step.  Rows are 128 bytes (whole cache lines: 64-byte row segments, four 32 KiB
// stages three steps ahead, ran 4-6% slower) without padding; logical 16-byte chunk c of row r sits at
// chunk c ^ ((r >> 1) & 7), so the fragment reads of 16 consecutive rows hit distinct banks and every
// load instruction still fills 1 KiB of consecutive LDS (8 rows).  Rows past M or N load row M-1 / N-1
// (in bounds; those accumulators are never stored).  The loads are issued from inline assembly so
// the compiler does not wait for them before every LDS read; the waits are explicit vmcnt counts.
#ifndef QG_BK
#define QG_BK 128
#endif
constexpr int kDmaBK = QG_BK, kDmaRows = 256, kDmaNT = 1024;
constexpr int kDmaChunks = kDmaBK / 16;        // 16-byte chunks per staged row
constexpr int kDmaRowsPerLoad = 1024 / kDmaBK;  // rows one 1 KiB load instruction fills
constexpr int kDmaStage = 2 * kDmaRows * kDmaBK;  // A rows, then B rows
#ifndef QG_STAGES
#define QG_STAGES 2
#endif
constexpr int kDmaStages = QG_STAGES;  // LDS stages; kDmaStages - 1 in flight ahead of the one in use
constexpr size_t kDmaLds = kDmaStages * (size_t)kDmaStage;

__device__ __forceinline__ int dma_swz(int row, int c) {
    return kDmaChunks == 4 ? (c ^ ((row >> 2) & 3)) * 16 : (c ^ ((row >> 1) & 7)) * 16;
}


template <bool OUT_F32>
__global__ __launch_bounds__(kDmaNT, 1) void k_qgemm_dma(QgArgs p) {
    extern __shared__ __attribute__((aligned(16))) int8_t smem[];
    constexpr int kTM = 2, kTN = 2, kWGN = 4;
    constexpr int kLoads = (2 * kDmaRows / kDmaRowsPerLoad) / (kDmaNT / kWave);  // 1 KiB loads per wave per stage
    static_assert(kTM * 32 * (kDmaNT / kWave / kWGN) == kDmaRows && kTN * 32 * kWGN == kDmaRows,
                  "the waves' MFMA tiles cover the workgroup tile");

    int id = blockIdx.x;
    const int nblk = gridDim.x;
    if ((nblk & 7) == 0) id = (id & 7) * (nblk >> 3) + (id >> 3);
    const int per_group = kQgGroupM * p.tiles_n;
    const int first_m = (id / per_group) * kQgGroupM;
    const int gsize = min(p.tiles_m - first_m, kQgGroupM);
    const int tm = first_m + (id % per_group) % gsize;
    const int tn = (id % per_group) / gsize;
    const int m0 = tm * kDmaRows, n0 = tn * kDmaRows;

    const int t = threadIdx.x, lane = t & (kWave - 1), wid = t / kWave;
    const int wm = wid / kWGN, wn = wid % kWGN;

    // the stage holds 64 blocks of 8 rows (one 1 KiB load each: A rows 0-255, then B rows 0-255);
    // wave wid loads blocks wid * kLoads .. wid * kLoads + kLoads - 1
    const int8_t *src[kLoads];
    uint32_t loff[kLoads];
#pragma unroll
    for (int q = 0; q < kLoads; q++) {
        constexpr int kBlocks = kDmaRows / kDmaRowsPerLoad;  // load blocks per panel
        const int blk = wid * kLoads + q, panel = blk / kBlocks, rb = (blk % kBlocks) * kDmaRowsPerLoad;
        const int row = rb + lane / kDmaChunks;
        const int c = dma_swz(row, lane % kDmaChunks) / 16;  // the chunk that belongs at this lane's place
        const int64_t grow = panel == 0 ? min(m0 + row, p.M - 1) : min(n0 + row, p.N - 1);
        src[q] = (panel == 0 ? p.A + grow * p.lda : p.B + grow * p.ldb) + c * 16;
        loff[q] = (uint32_t)(panel * kDmaRows * kDmaBK + rb * kDmaBK);
    }
    const uint32_t sbase = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) int8_t *)smem;
    auto issue = [&](int kt) {
        const uint32_t st = sbase + (uint32_t)(kt % kDmaStages) * kDmaStage;
#pragma unroll
        for (int q = 0; q < kLoads; q++)
            dma16(src[q] + (int64_t)kt * kDmaBK, __builtin_amdgcn_readfirstlane(st + loff[q]));
    };

    i16v acc[kTM][kTN];
#pragma unroll
    for (int i = 0; i < kTM; i++)
#pragma unroll
        for (int j = 0; j < kTN; j++) acc[i][j] = i16v{};

    const int nk = p.K / kDmaBK;
    for (int kt = 0; kt < kDmaStages - 1 && kt < nk; kt++) issue(kt);
    const int frow = lane & 31, fhalf = lane >> 5;
    for (int kt = 0; kt < nk; kt++) {
        // this wave's loads of step kt are done once at most 4 per later step in flight remain
        const int ahead = min(nk - 1 - kt, kDmaStages - 2);
        if (ahead == 3) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(3 * kLoads) : "memory");
        else if (ahead == 2) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * kLoads) : "memory");
        else if (ahead == 1) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kLoads) : "memory");
        else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __builtin_amdgcn_s_barrier();  // every wave's loads of step kt have landed; step kt-1's reads are done
        asm volatile("" ::: "memory");
        if (kt + kDmaStages - 1 < nk) issue(kt + kDmaStages - 1);  // into the stage step kt-1 used
        const int8_t *cur = smem + (kt % kDmaStages) * kDmaStage;
#pragma unroll
        for (int s = 0; s < kDmaBK / 32; s++) {
            const int c = s * 2 + fhalf;
            i4 fa[kTM], fb[kTN];
#pragma unroll
            for (int i = 0; i < kTM; i++) {
                const int r = (wm * kTM + i) * 32 + frow;
                fa[i] = *(const i4 *)(cur + r * kDmaBK + dma_swz(r, c));
            }
#pragma unroll
            for (int j = 0; j < kTN; j++) {
                const int r = (wn * kTN + j) * 32 + frow;
                fb[j] = *(const i4 *)(cur + kDmaRows * kDmaBK + r * kDmaBK + dma_swz(r, c));
            }
#pragma unroll
            for (int i = 0; i < kTM; i++)
#pragma unroll
                for (int j = 0; j < kTN; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[i], fb[j], acc[i][j], 0, 0, 0);
        }
    }

#pragma unroll
    for (int i = 0; i < kTM; i++) {
#pragma unroll
        for (int j = 0; j < kTN; j++) {
            const int n = n0 + (wn * kTN + j) * 32 + (lane & 31);
            if (n >= p.N) continue;
            float wsn = 0.0f, bn = 0.0f;
            if (OUT_F32) {
                wsn = p.ws[n];
                bn = p.bias ? p.bias[n] : 0.0f;
            }
#pragma unroll
            for (int v = 0; v < 16; v++) {
                const int m = m0 + (wm * kTM + i) * 32 + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
                if (m >= p.M) continue;
                if (OUT_F32)
                    p.Y[(int64_t)m * p.ldc + n] = (float)acc[i][j][v] * p.xs[m] * wsn + bn;
                else
                    p.C[(int64_t)m * p.ldc + n] = acc[i][j][v];
            }
        }
    }
}

static int launch_qgemm_dma(QgArgs p, bool out_f32, hipStream_t st, const char *what) {
    p.tiles_m = (p.M + kDmaRows - 1) / kDmaRows;
    p.tiles_n = (p.N + kDmaRows - 1) / kDmaRows;
    const int64_t blocks = (int64_t)p.tiles_m * p.tiles_n;
    if (blocks > INT32_MAX) return set_error(NC_HIP_ERR_ARG, "%s: %lld tiles exceed one launch", what, (long long)blocks);
    static bool done[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) == hipSuccess && dev >= 0 && dev < 64 && !done[dev]) {
        (void)hipFuncSetAttribute((const void *)k_qgemm_dma<true>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kDmaLds);
        (void)hipFuncSetAttribute((const void *)k_qgemm_dma<false>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kDmaLds);
        done[dev] = true;
    }
    if (out_f32) hipLaunchKernelGGL(k_qgemm_dma<true>, dim3((unsigned)blocks), dim3(kDmaNT), kDmaLds, st, p);
    else hipLaunchKernelGGL(k_qgemm_dma<false>, dim3((unsigned)blocks), dim3(kDmaNT), kDmaLds, st, p);
    return check_launch(what);
}

template <class C>
static void qgemm_lds_attr() {
    // dynamic LDS above 64 KiB has to be allowed per kernel, once per device
    static bool done[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64 || done[dev]) return;
    const int lds = (int)C::LDS;
    (void)hipFuncSetAttribute((const void *)k_qgemm<C, true, true>, hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    (void)hipFuncSetAttribute((const void *)k_qgemm<C, true, false>, hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    (void)hipFuncSetAttribute((const void *)k_qgemm<C, false, true>, hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    (void)hipFuncSetAttribute((const void *)k_qgemm<C, false, false>, hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    done[dev] = true;
}

template <class C>
static int launch_qgemm_cfg(QgArgs p, bool out_f32, hipStream_t st, const char *what) {
    p.tiles_m = (p.M + C::BM - 1) / C::BM;
    p.tiles_n = (p.N + C::BN - 1) / C::BN;
    const int64_t blocks = (int64_t)p.tiles_m * p.tiles_n;
    if (blocks > INT32_MAX) return set_error(NC_HIP_ERR_ARG, "%s: %lld tiles exceed one launch", what, (long long)blocks);
    const bool aligned = p.K % 16 == 0 && p.lda % 16 == 0 && p.ldb % 16 == 0 && aligned16(p.A) && aligned16(p.B);
    const dim3 grid((unsigned)blocks), block(C::NT);
    qgemm_lds_attr<C>();
    if (aligned && out_f32) hipLaunchKernelGGL((k_qgemm<C, true, true>), grid, block, C::LDS, st, p);
    else if (aligned) hipLaunchKernelGGL((k_qgemm<C, true, false>), grid, block, C::LDS, st, p);
    else if (out_f32) hipLaunchKernelGGL((k_qgemm<C, false, true>), grid, block, C::LDS, st, p);
    else hipLaunchKernelGGL((k_qgemm<C, false, false>), grid, block, C::LDS, st, p);
    return check_launch(what);
}

static int launch_qgemm(QgArgs p, bool out_f32, hipStream_t st, const char *what) {
    const int64_t big_tiles = (int64_t)((p.M + QgBig::BM - 1) / QgBig::BM) * ((p.N + QgBig::BN - 1) / QgBig::BN);
    const bool dma_ok = p.K > 0 && p.K % kDmaBK == 0 && p.lda % 16 == 0 && p.ldb % 16 == 0 && aligned16(p.A) &&
                        aligned16(p.B);
    if (big_tiles >= num_cus() && dma_ok) return launch_qgemm_dma(p, out_f32, st, what);
    if (big_tiles >= num_cus()) return launch_qgemm_cfg<QgBig>(p, out_f32, st, what);
    return launch_qgemm_cfg<QgSmall>(p, out_f32, st, what);
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
