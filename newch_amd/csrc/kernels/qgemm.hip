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
// When K is also a multiple of 256, k_qgemm_pipe runs that tile over 8 waves with the k loop written
// as one software-pipelined assembly block (below).  Blocks are remapped so each XCD (blocks b with
// b % 8 equal) works a contiguous run of tiles, and tiles run in groups of 8 tile-rows so neighbouring
// blocks share panels in L2.
//
// linear_int8 epilogue (ops_quant.c:75-79): y = (float)acc * xs[m] * ws[n] + (bias ? bias[n] : 0),
// evaluated left to right in fp32 without contraction (the reference's scalar glue), so the fused
// result is bit-identical to the reference's.
#include "common.hpp"

namespace nchip {

typedef int i16v __attribute__((ext_vector_type(16)));

#ifndef QG_GROUP_M
#define QG_GROUP_M 8
#endif
constexpr int kQgGroupM = QG_GROUP_M;

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


// Epilogue of a wave's TM x TN block of 32 x 32 MFMA tiles whose first row and column are mb and nb:
// lane l, element v of a tile holds row 8 (v / 4) + 4 (l / 32) + v % 4, column l % 32, so each store
// instruction writes two 128-byte row segments.  (Issuing the B fragment first gives C^T tiles whose
// lanes hold four consecutive columns, one 16-byte store each; 32 rows of 32 bytes per instruction
// ran slower.)
template <int TM, int TN, bool OUT_F32>
__device__ __forceinline__ void qg_store(const QgArgs &p, const i16v (&acc)[TM][TN], int mb, int nb, int lane) {
    // the row scales a lane needs for tile row i, xs[mb + 32 i + 8 g + 4 (l / 32) .. + 3], loaded four
    // at a time before the tile row's first store (rows past M read row M - 1; they are not stored)
    const bool xs_vec = OUT_F32 && (((uintptr_t)p.xs) & 15) == 0;
#pragma unroll
    for (int i = 0; i < TM; i++) {
        f4 xs4[4];
        if (OUT_F32) {
#pragma unroll
            for (int g = 0; g < 4; g++) {
                const int m = mb + i * 32 + 8 * g + 4 * (lane >> 5);
                if (xs_vec && m + 4 <= p.M) {
                    xs4[g] = *(const f4 *)(p.xs + m);
                } else {
#pragma unroll
                    for (int e = 0; e < 4; e++) xs4[g][e] = p.xs[min(m + e, p.M - 1)];
                }
            }
        }
#pragma unroll
        for (int j = 0; j < TN; j++) {
            const int n = nb + j * 32 + (lane & 31);
            if (n >= p.N) continue;
            float wsn = 0.0f, bn = 0.0f;
            if (OUT_F32) {
                wsn = p.ws[n];
                bn = p.bias ? p.bias[n] : 0.0f;
            }
#pragma unroll
            for (int v = 0; v < 16; v++) {
                const int m = mb + i * 32 + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
                if (m >= p.M) continue;
                if (OUT_F32)
                    p.Y[(int64_t)m * p.ldc + n] = (float)acc[i][j][v] * xs4[v >> 2][v & 3] * wsn + bn;
                else
                    p.C[(int64_t)m * p.ldc + n] = acc[i][j][v];
            }
        }
    }
}

// qg_store's fp32 epilogue with the scales and bias of the workgroup's 256 rows and columns in LDS
// (sxs[r] = xs[m0 + r], sws[c] = ws[n0 + c], sb[c] = bias or 0); mb, nb relative to the tile
template <int TM, int TN>
__device__ __forceinline__ void qg_store_f32_lds(const QgArgs &p, const i16v (&acc)[TM][TN], int m0, int n0, int mb,
                                                 int nb, const float *sxs, const float *sws, const float *sb,
                                                 int lane) {
#pragma unroll
    for (int i = 0; i < TM; i++) {
        f4 xs4[4];
#pragma unroll
        for (int g = 0; g < 4; g++) xs4[g] = *(const f4 *)(sxs + mb + i * 32 + 8 * g + 4 * (lane >> 5));
#pragma unroll
        for (int j = 0; j < TN; j++) {
            const int c = nb + j * 32 + (lane & 31), n = n0 + c;
            if (n >= p.N) continue;
            const float wsn = sws[c], bn = sb[c];
#pragma unroll
            for (int v = 0; v < 16; v++) {
                const int m = m0 + mb + i * 32 + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
                if (m >= p.M) continue;
                p.Y[(int64_t)m * p.ldc + n] = (float)acc[i][j][v] * xs4[v >> 2][v & 3] * wsn + bn;
            }
        }
    }
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

    qg_store<kTM, kTN, OUT_F32>(p, acc, m0 + wm * kTM * 32, n0 + wn * kTN * 32, lane);
}

// ------------------------------------------------------------------------------------------------
// Software-pipelined variant of the direct-to-LDS kernel: the same 256 x 256 tile and 128-byte k steps
// over 8 waves of 4 x 2 MFMA tiles (128 x 64 each) whose 128 accumulator registers are AGPRs.  The
// whole k loop is one inline-assembly block (so the accumulators stay in place: split into one
// block per substep, the compiler moved them between register files at every block), in which a k
// step is four 32-k substeps: each issues the next substep's six fragment reads into the second of
// two register sets, interleaved with its own eight MFMAs on the first, and ends by waiting for those
// reads, so the LDS latency runs under the matrix work instead of between its instructions.  The
// barrier of a k step sits after the reads of its last substep and before that substep's MFMAs: every
// wave has finished reading the stage the barrier frees, and the MFMAs after it need no LDS; the next
// step's panel loads, into the stage just freed, are issued between those MFMAs.  LDS:
// [A stage 0 | A stage 1 | B stage 0 | B stage 1], 32 KiB each, rows of 128 bytes with logical chunk c
// of row r at c ^ ((r >> 1) & 7); a fragment address is one register per substep and operand (the
// permutation depends on r only through the fragment row's bits 1-3, the same for all of a wave's
// tiles), stage and tile offsets immediate.  Waves 0-3 load A's panels, 4-7 B's, each eight 1 KiB
// loads per step from the tile's first row (a scalar base) at one 32-bit lane offset per load, which
// advances 128 bytes a step.  K is a multiple of 256 (whole pairs of steps, one per stage).  The fp32
// epilogue's row and column scales and bias are loaded before the loop and put in LDS past the stages
// after it.  Against the 16-wave kernel on the same boxes: 136-141 against 160-180 us for the int8
// GEMM of [8192, 4096] x [4096, 4096]^T, 168-179 against 196-214 us for linear_int8 of that shape;
// one wave per SIMD of 4 x 4 MFMA tiles (256 AGPRs) ran 161-177 us.
#ifndef QG_PIPE
#define QG_PIPE 1
#endif
constexpr int kPipeNT = 512;
constexpr int kPipePanel = kDmaRows * kDmaBK;  // bytes of one operand's stage

#define QG_RD(dst, addr, off) "ds_read_b128 %[" #dst "], %[" #addr "] offset:" #off "\n\t"
#define QG_MF(c, a, b) "v_mfma_i32_32x32x32_i8 %[" #c "], %[" #a "], %[" #b "], %[" #c "]\n\t"
// eight MFMAs on register set M while set R is read from substep S at stage offsets O0..O3
#define QG_SUB(R, M, S, O0, O1, O2, O3)                                                                   \
    QG_RD(R##a0, aA##S, O0) QG_RD(R##b0, aB##S, O0) QG_MF(c00, M##a0, M##b0) QG_RD(R##a1, aA##S, O1)      \
    QG_MF(c01, M##a0, M##b1) QG_RD(R##b1, aB##S, O1) QG_MF(c10, M##a1, M##b0) QG_RD(R##a2, aA##S, O2)      \
    QG_MF(c11, M##a1, M##b1) QG_RD(R##a3, aA##S, O3) QG_MF(c20, M##a2, M##b0) QG_MF(c21, M##a2, M##b1)    \
    QG_MF(c30, M##a3, M##b0) QG_MF(c31, M##a3, M##b1) "s_waitcnt lgkmcnt(0)\n\t"
#define QG_SUB0(R, M, S) QG_SUB(R, M, S, 0, 4096, 8192, 12288)
#define QG_SUB1(R, M, S) QG_SUB(R, M, S, 32768, 36864, 40960, 45056)
#define QG_LAST(M)                                                                                         \
    QG_MF(c00, M##a0, M##b0) QG_MF(c01, M##a0, M##b1) QG_MF(c10, M##a1, M##b0) QG_MF(c11, M##a1, M##b1)     \
    QG_MF(c20, M##a2, M##b0) QG_MF(c21, M##a2, M##b1) QG_MF(c30, M##a3, M##b0) QG_MF(c31, M##a3, M##b1)
#define QG_READ0(R)                                                                                        \
    QG_RD(R##a0, aA0, 0) QG_RD(R##b0, aB0, 0) QG_RD(R##a1, aA0, 4096) QG_RD(R##b1, aB0, 4096)            \
    QG_RD(R##a2, aA0, 8192) QG_RD(R##a3, aA0, 12288) "s_waitcnt lgkmcnt(0)\n\t"
// one 1 KiB panel load into LDS at lo + OFF (M0), 16 bytes per lane from tb + V
#define QG_LD(V, OFF) "s_add_u32 m0, %[lo], " #OFF "\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %[" #V "], %[tb]\n\t"
#define QG_ADV(V) "v_add_u32 %[" #V "], 0x80, %[" #V "]\n\t"
#define QG_DMA(O0, O1, O2, O3, O4, O5, O6, O7)                                                           \
    QG_LD(v0, O0) QG_LD(v1, O1) QG_LD(v2, O2) QG_LD(v3, O3) QG_LD(v4, O4) QG_LD(v5, O5) QG_LD(v6, O6)     \
    QG_LD(v7, O7) QG_ADV(v0) QG_ADV(v1) QG_ADV(v2) QG_ADV(v3) QG_ADV(v4) QG_ADV(v5) QG_ADV(v6) QG_ADV(v7)
#define QG_DMA0 QG_DMA(0, 1024, 2048, 3072, 4096, 5120, 6144, 7168)
#define QG_DMA1 QG_DMA(32768, 33792, 34816, 35840, 36864, 37888, 38912, 39936)
// QG_SUB with a step's eight panel loads (LDS offsets D0..D7) issued between its MFMAs
#define QG_SUBD(R, M, S, O0, O1, O2, O3, D0, D1, D2, D3, D4, D5, D6, D7)                                  \
    QG_RD(R##a0, aA##S, O0) QG_RD(R##b0, aB##S, O0) QG_MF(c00, M##a0, M##b0) QG_LD(v0, D0)                \
    QG_RD(R##a1, aA##S, O1) QG_MF(c01, M##a0, M##b1) QG_LD(v1, D1) QG_RD(R##b1, aB##S, O1)               \
    QG_MF(c10, M##a1, M##b0) QG_LD(v2, D2) QG_RD(R##a2, aA##S, O2) QG_MF(c11, M##a1, M##b1)              \
    QG_LD(v3, D3) QG_RD(R##a3, aA##S, O3) QG_MF(c20, M##a2, M##b0) QG_LD(v4, D4)                         \
    QG_MF(c21, M##a2, M##b1) QG_LD(v5, D5) QG_MF(c30, M##a3, M##b0) QG_LD(v6, D6)                        \
    QG_MF(c31, M##a3, M##b1) QG_LD(v7, D7) QG_ADV(v0) QG_ADV(v1) QG_ADV(v2) QG_ADV(v3) QG_ADV(v4)        \
    QG_ADV(v5) QG_ADV(v6) QG_ADV(v7) "s_waitcnt lgkmcnt(0)\n\t"
// substep 0 of stage 1 with the loads of stage 0, and substep 0 of stage 0 with those of stage 1
#define QG_SUBD1(R, M) QG_SUBD(R, M, 0, 32768, 36864, 40960, 45056, 0, 1024, 2048, 3072, 4096, 5120, 6144, 7168)
#define QG_SUBD0(R, M)                                                                                     \
    QG_SUBD(R, M, 0, 0, 4096, 8192, 12288, 32768, 33792, 34816, 35840, 36864, 37888, 38912, 39936)


template <bool OUT_F32>
__global__ __launch_bounds__(kPipeNT, 1) void k_qgemm_pipe(QgArgs p) {
    extern __shared__ __attribute__((aligned(16))) int8_t smem[];
    constexpr int kTM = 4, kTN = 2, kWGN = 4;
    constexpr int kWaves = kPipeNT / kWave;
    constexpr int kLoads = 8;  // 1 KiB loads per wave per step
    static_assert(kDmaBK == 128 && kDmaRowsPerLoad == 8 && kPipePanel == 32768,
                  "the assembly's offsets are written for 128-byte steps of 256 rows");
    static_assert(kLoads * kDmaRowsPerLoad * (kWaves / 2) == kDmaRows, "each half of the waves loads one operand");
    static_assert(kTM * 32 * (kWaves / kWGN) == kDmaRows && kTN * 32 * kWGN == kDmaRows,
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

    const int t = threadIdx.x, lane = t & (kWave - 1), wid = __builtin_amdgcn_readfirstlane(t / kWave);
    const int wm = wid / kWGN, wn = wid % kWGN;

    // panel loads: wave w's load q covers rows 64 (w % 4) + 8 q .. + 7 of its operand's panel; rows
    // past M / N read the last row (in bounds; those accumulators are never stored)
    const bool pb = wid >= kWaves / 2;
    const int r0 = pb ? n0 : m0, rows = pb ? p.N : p.M;
    const int64_t ld = pb ? p.ldb : p.lda;
    const int8_t *tb = (pb ? p.B : p.A) + (int64_t)r0 * ld;  // the tile's first row
    uint32_t vo[kLoads];
#pragma unroll
    for (int q = 0; q < kLoads; q++) {
        const int row = (wid % (kWaves / 2)) * (kLoads * kDmaRowsPerLoad) + q * kDmaRowsPerLoad + lane / kDmaChunks;
        const int c = dma_swz(row, lane % kDmaChunks) / 16;  // the chunk that belongs at this lane's place
        vo[q] = (uint32_t)((int64_t)(min(r0 + row, rows - 1) - r0) * ld) + (uint32_t)(c * 16);
    }
    const uint32_t sbase = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) int8_t *)smem;
    const uint32_t lo = sbase + (pb ? 2 * kPipePanel : 0) + (uint32_t)(wid % (kWaves / 2)) * (kLoads * 1024);

    // fragment addresses (stage 0): lane reads row (tile row) + frow, logical chunk 2 s + fh
    const int frow = lane & 31, fh = lane >> 5, x = (frow >> 1) & 7;
    uint32_t aA[4], aB[4];
#pragma unroll
    for (int s = 0; s < 4; s++) {
        const uint32_t sw = (uint32_t)(((2 * s + fh) ^ x) * 16);
        aA[s] = sbase + (uint32_t)(wm * kTM * 32 + frow) * kDmaBK + sw;
        aB[s] = sbase + (uint32_t)(2 * kPipePanel) + (uint32_t)(wn * kTN * 32 + frow) * kDmaBK + sw;
    }

    i16v acc[kTM][kTN];
#pragma unroll
    for (int i = 0; i < kTM; i++)
#pragma unroll
        for (int j = 0; j < kTN; j++) acc[i][j] = i16v{};

    // fp32 epilogue: the tile's 256 row scales, 256 column scales and 256 biases, loaded now (the k loop
    // hides their latency) and put in LDS past the stages once the loop is done
    float sv[2] = {0.0f, 0.0f};
    if (OUT_F32) {
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const int u = min(t + h * kPipeNT, 3 * kDmaRows - 1);  // unconditional loads: no wait before the loop
            const int which = u / kDmaRows, idx = u % kDmaRows;
            const int m = min(m0 + idx, p.M - 1), n = min(n0 + idx, p.N - 1);
            const float *src = which == 0 ? p.xs + m : which == 1 || !p.bias ? p.ws + n : p.bias + n;
            const float v = *src;
            sv[h] = which == 2 && !p.bias ? 0.0f : v;
        }
    }

    int np = p.K / (2 * kDmaBK);  // pairs of k steps, >= 1
    i4 f0[6], f1[6];              // the two fragment register sets: a0-a3, b0-b1
    // the loop sets M0 for its LDS-DMA loads; the compiler treats M0 as reserved and does not honour the
    // clobber, and this kernel's compiled code touches M0 nowhere outside the assembly (checked)
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
    asm volatile(
        "s_nop 7\n\ts_nop 7\n\t"  // the accumulators' zeroing before the first MFMA
        QG_DMA0 "s_waitcnt vmcnt(0)\n\ts_barrier\n\t" QG_DMA1 QG_READ0(p0)
        "L_top_%=:\n\t"
        "s_sub_u32 %[np], %[np], 1\n\t"
        QG_SUB0(p1, p0, 1) QG_SUB0(p0, p1, 2) QG_SUB0(p1, p0, 3)
        "s_waitcnt vmcnt(0)\n\ts_barrier\n\t"
        "s_cmp_eq_u32 %[np], 0\n\ts_cbranch_scc1 L_nodma_%=\n\t"
        QG_SUBD1(p0, p1)
        "s_branch L_s1_%=\n\t"
        "L_nodma_%=:\n\t"
        QG_SUB1(p0, p1, 0)
        "L_s1_%=:\n\t"
        QG_SUB1(p1, p0, 1) QG_SUB1(p0, p1, 2) QG_SUB1(p1, p0, 3)
        "s_cmp_eq_u32 %[np], 0\n\ts_cbranch_scc1 L_last_%=\n\t"
        "s_waitcnt vmcnt(0)\n\ts_barrier\n\t"
        QG_SUBD0(p0, p1)
        "s_branch L_top_%=\n\t"
        "L_last_%=:\n\t"
        QG_LAST(p1)
        "s_nop 7\n\ts_nop 7\n\ts_nop 7"  // the last MFMAs' results before they are read
        : [c00] "+a"(acc[0][0]), [c01] "+a"(acc[0][1]), [c10] "+a"(acc[1][0]), [c11] "+a"(acc[1][1]),
          [c20] "+a"(acc[2][0]), [c21] "+a"(acc[2][1]), [c30] "+a"(acc[3][0]), [c31] "+a"(acc[3][1]),
          [p0a0] "=&v"(f0[0]), [p0a1] "=&v"(f0[1]), [p0a2] "=&v"(f0[2]), [p0a3] "=&v"(f0[3]), [p0b0] "=&v"(f0[4]),
          [p0b1] "=&v"(f0[5]), [p1a0] "=&v"(f1[0]), [p1a1] "=&v"(f1[1]), [p1a2] "=&v"(f1[2]), [p1a3] "=&v"(f1[3]),
          [p1b0] "=&v"(f1[4]), [p1b1] "=&v"(f1[5]), [v0] "+v"(vo[0]), [v1] "+v"(vo[1]), [v2] "+v"(vo[2]),
          [v3] "+v"(vo[3]), [v4] "+v"(vo[4]), [v5] "+v"(vo[5]), [v6] "+v"(vo[6]), [v7] "+v"(vo[7]), [np] "+s"(np)
        : [aA0] "v"(aA[0]), [aA1] "v"(aA[1]), [aA2] "v"(aA[2]), [aA3] "v"(aA[3]), [aB0] "v"(aB[0]),
          [aB1] "v"(aB[1]), [aB2] "v"(aB[2]), [aB3] "v"(aB[3]), [lo] "s"(lo), [tb] "s"(tb)
        : "memory", "m0", "scc");
#pragma clang diagnostic pop

    if (OUT_F32) {
        float *sc = (float *)(smem + 4 * kPipePanel);
#pragma unroll
        for (int h = 0; h < 2; h++)
            if (t + h * kPipeNT < 3 * kDmaRows) sc[t + h * kPipeNT] = sv[h];
        __syncthreads();
        qg_store_f32_lds<kTM, kTN>(p, acc, m0, n0, wm * kTM * 32, wn * kTN * 32, sc, sc + kDmaRows, sc + 2 * kDmaRows,
                                   lane);
    } else {
        qg_store<kTM, kTN, OUT_F32>(p, acc, m0 + wm * kTM * 32, n0 + wn * kTN * 32, lane);
    }
}

constexpr size_t kPipeLds = 4 * (size_t)kPipePanel + 3 * kDmaRows * sizeof(float);

#if QG_PIPE
static bool done_pipe(int dev) {
    static bool done[64] = {};
    if (dev < 0 || dev >= 64 || done[dev]) return true;
    done[dev] = true;
    return false;
}
#endif

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
#if QG_PIPE
    // whole pairs of k steps, and every lane offset of a tile's panel loads within 32 bits
    const bool pipe = p.K % (2 * kDmaBK) == 0 && 256 * (p.lda > p.ldb ? p.lda : p.ldb) + p.K < ((int64_t)1 << 32);
    if (pipe) {
        if (!done_pipe(dev)) {
            (void)hipFuncSetAttribute((const void *)k_qgemm_pipe<true>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kPipeLds);
            (void)hipFuncSetAttribute((const void *)k_qgemm_pipe<false>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kDmaLds);
        }
        if (out_f32) hipLaunchKernelGGL(k_qgemm_pipe<true>, dim3((unsigned)blocks), dim3(kPipeNT), kPipeLds, st, p);
        else hipLaunchKernelGGL(k_qgemm_pipe<false>, dim3((unsigned)blocks), dim3(kPipeNT), kDmaLds, st, p);
        return check_launch(what);
    }
#endif
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
