// fp32 GEMM on the matrix cores (the reference's gemm_f32 kernel-table entry, kernels.h:36-41, as
// ops_linalg.c:58-330 calls it): hand-written for gfx950 around v_mfma_f32_16x16x4_f32.
//
// C (M x N, row-major, leading dim ldc) = alpha op(A) op(B) + beta C with op(A) M x K and op(B) K x N.
// An operand is stored K-contiguous (A untransposed, B transposed) or M/N-contiguous (A transposed, B
// untransposed), each with its own leading dim; batched forms take per-axis batch strides or pointer
// arrays.  beta = 0 never reads C.
//
// Tiling.  A workgroup owns a BM x BN tile of C and each of its waves a (16 TM) x (16 TN) block of it,
// held as TM x TN 16 x 16 accumulator tiles (4 floats per lane each).  K advances 16 at a time
// through two LDS stages: the next step's panels are loaded into registers while the matrix cores
// work on the current one, stored into the other stage, and one barrier per step separates the two.
// Each operand keeps its global layout in LDS:
//   * K-contiguous panel: BM (BN) rows of 16 floats, four 16-byte chunks per row, logical chunk c of
//     row r stored at chunk c ^ ((r >> 2) & 3), so 16-byte reads of consecutive rows spread over the
//     banks;
//   * M/N-contiguous panel: 16 k-rows of BM (BN) floats, the row pitch padded by 4 floats so the four
//     quarter-waves' reads (k-rows k, k + 4, k + 8, k + 12) land in different banks.
//
// k mapping.  One MFMA multiplies a 16 x 4 slice of A by a 4 x 16 slice of B, quarter-wave q (lanes
// 16 q .. 16 q + 15) holding one k.  In each stage of 16 k, quarter q gives the s-th MFMA (s = 0..3)
// the value at k = 4 q + s, for A and B alike, so a K-contiguous operand feeds four MFMAs from one
// 16-byte LDS read.  Each k enters every output element exactly once, four products per instruction
// (K / 4 roundings into the accumulator), and the order of the sum is a property of the kernel
// alone: the same for every tile size and grid, so results are identical run to run and on any
// device.  It differs from the reference's serial order, so the parity bar is the fp32 error bound of
// a K-term dot product.
//
// Tile sizes: 256 x 256 (8 waves of 8 x 4 tiles) when the problem has at least as many such tiles as
// the device has CUs, else 128 x 128 (4 waves of 4 x 4) or 64 x 64 (4 waves of 2 x 2).  Blocks are
// remapped so each XCD (blocks b with b % 8 equal) works a contiguous run of tiles, and tiles run in
// groups of 8 tile-rows so neighbouring blocks share panels in L2.
#include "common.hpp"

namespace nchip {


constexpr int kSgBK = 16;      // k per stage
constexpr int kSgGroupM = 8;   // tile-rows per group in the block order

template <int TM_, int TN_, int WGM_, int WGN_>
struct SgCfg {
    static constexpr int TM = TM_, TN = TN_, WGM = WGM_, WGN = WGN_;
    static constexpr int NT = 64 * WGM * WGN;
    static constexpr int BM = 16 * TM * WGM, BN = 16 * TN * WGN;
    // bytes of one operand panel in LDS (the larger of the two layouts)
    static constexpr int SLAB_A = 64 * BM + 256, SLAB_B = 64 * BN + 256;
    static constexpr int STAGE = SLAB_A + SLAB_B;
    static constexpr size_t LDS = 2 * (size_t)STAGE;
    static constexpr int CA = 4 * BM / NT, CB = 4 * BN / NT;  // 16-byte chunks per thread per panel
    static_assert(4 * BM % NT == 0 && 4 * BN % NT == 0, "panel chunks must divide over the workgroup");
};
using SgBig = SgCfg<8, 4, 2, 4>;    // 256 x 256
using SgMid = SgCfg<4, 4, 2, 2>;    // 128 x 128
using SgSmall = SgCfg<2, 2, 2, 2>;  // 64 x 64

struct SgBatch {
    int nb;  // 0: one matrix per operand
    int64_t shape[NC_HIP_MAX_DIMS];
    int64_t st[3][NC_HIP_MAX_DIMS];  // element strides of A, B, C per batch axis
};

struct SgArgs {
    const float *A, *B;
    float *C;
    const float *const *pa;  // pointer-array batches (instead of strides) when set
    const float *const *pb;
    float *const *pc;
    int64_t lda, ldb, ldc;
    int M, N, K;
    float alpha, beta;
    int tiles_m, tiles_n;
    SgBatch bat;
};

// Chunk q of an R-row panel starting at (row r0, k k0): its 16-byte LDS position.
template <int R, bool KC>
__device__ __forceinline__ uint32_t chunk_lds(int q) {
    if constexpr (KC) {
        const int row = q >> 2, c = q & 3;
        return (uint32_t)(row * 64 + ((c ^ ((row >> 2) & 3)) << 4));
    } else {
        constexpr int per_row = R / 4;
        return (uint32_t)((q / per_row) * (R + 4) * 4 + (q % per_row) * 16);
    }
}

// Chunk q's four floats from global memory, zero past the matrix.  VEC: the operand's rows start
// 16-byte aligned (aligned base, leading dim a multiple of 4), so a chunk wholly inside is one load.
template <int R, bool KC, bool VEC>
__device__ __forceinline__ f4 chunk_load(const float *p, int64_t ld, int rows, int K, int r0, int k0, int q) {
    f4 v = {0.f, 0.f, 0.f, 0.f};
    if constexpr (KC) {
        const int row = r0 + (q >> 2), k = k0 + (q & 3) * 4;
        if (row >= rows || k >= K) return v;
        const float *s = p + (int64_t)row * ld + k;
        if (VEC && k + 4 <= K) return *(const f4 *)s;
#pragma unroll
        for (int j = 0; j < 4; j++)
            if (k + j < K) v[j] = s[j];
    } else {
        constexpr int per_row = R / 4;
        const int k = k0 + q / per_row, row = r0 + (q % per_row) * 4;
        if (k >= K || row >= rows) return v;
        const float *s = p + (int64_t)k * ld + row;
        if (VEC && row + 4 <= rows) return *(const f4 *)s;
#pragma unroll
        for (int j = 0; j < 4; j++)
            if (row + j < rows) v[j] = s[j];
    }
    return v;
}

// The four values (s = 0..3) of panel row r that quarter-wave q gives the stage's MFMAs.
template <int R, bool KC>
__device__ __forceinline__ f4 fragment(const char *slab, int r, int q) {
    if constexpr (KC) {
        return *(const f4 *)(slab + r * 64 + ((q ^ ((r >> 2) & 3)) << 4));
    } else {
        const float *b = (const float *)slab + 4 * q * (R + 4) + r;
        return f4{b[0], b[R + 4], b[2 * (R + 4)], b[3 * (R + 4)]};
    }
}

// element offset of batch matrix `idx` for operand o (0 A, 1 B, 2 C)
__device__ __forceinline__ int64_t batch_off(const SgBatch &bt, int o, int64_t idx) {
    int64_t off = 0;
    for (int d = bt.nb - 1; d >= 0; d--) {
        const int64_t e = bt.shape[d];
        off += (idx % e) * bt.st[o][d];
        idx /= e;
    }
    return off;
}

template <class Cfg, bool AK, bool BK, bool VEC>
__global__ __launch_bounds__(Cfg::NT, 1) void k_sgemm(SgArgs p) {
    extern __shared__ __attribute__((aligned(16))) char smem[];
    constexpr int kTM = Cfg::TM, kTN = Cfg::TN, kWGN = Cfg::WGN, kNT = Cfg::NT;
    constexpr int kBM = Cfg::BM, kBN = Cfg::BN, kCA = Cfg::CA, kCB = Cfg::CB;

    // block -> (batch matrix, tile): XCD-contiguous runs, then groups of kSgGroupM tile-rows
    int64_t id = blockIdx.x;
    const int64_t nblk = gridDim.x;
    if ((nblk & 7) == 0) id = (id & 7) * (nblk >> 3) + (id >> 3);
    const int64_t per_batch = (int64_t)p.tiles_m * p.tiles_n;
    const int64_t batch = id / per_batch;
    const int tile = (int)(id % per_batch);
    const int per_group = kSgGroupM * p.tiles_n;
    const int first_m = (tile / per_group) * kSgGroupM;
    const int gsize = min(p.tiles_m - first_m, kSgGroupM);
    const int tm = first_m + (tile % per_group) % gsize, tn = (tile % per_group) / gsize;
    const int m0 = tm * kBM, n0 = tn * kBN;

    const float *A, *B;
    float *C;
    if (p.pa) {
        A = p.pa[batch], B = p.pb[batch], C = p.pc[batch];
    } else {
        A = p.A + batch_off(p.bat, 0, batch), B = p.B + batch_off(p.bat, 1, batch), C = p.C + batch_off(p.bat, 2, batch);
    }

    const int t = threadIdx.x, lane = t & (kWave - 1), wid = t / kWave;
    const int wm = wid / kWGN, wn = wid % kWGN;

    f4 ra[kCA], rb[kCB];
    auto gload = [&](int k0) {
#pragma unroll
        for (int i = 0; i < kCA; i++) ra[i] = chunk_load<kBM, AK, VEC>(A, p.lda, p.M, p.K, m0, k0, t + i * kNT);
#pragma unroll
        for (int i = 0; i < kCB; i++) rb[i] = chunk_load<kBN, BK, VEC>(B, p.ldb, p.N, p.K, n0, k0, t + i * kNT);
    };
    auto sstore = [&](char *stage) {
#pragma unroll
        for (int i = 0; i < kCA; i++) *(f4 *)(stage + chunk_lds<kBM, AK>(t + i * kNT)) = ra[i];
#pragma unroll
        for (int i = 0; i < kCB; i++) *(f4 *)(stage + Cfg::SLAB_A + chunk_lds<kBN, BK>(t + i * kNT)) = rb[i];
    };

    f4 acc[kTM][kTN];
#pragma unroll
    for (int i = 0; i < kTM; i++)
#pragma unroll
        for (int j = 0; j < kTN; j++) acc[i][j] = f4{0.f, 0.f, 0.f, 0.f};

    const int fr = lane & 15, fq = lane >> 4;
    const int nk = (p.K + kSgBK - 1) / kSgBK;
    if (nk > 0) {
        gload(0);
        sstore(smem);
        __syncthreads();
    }
    for (int kt = 0; kt < nk; kt++) {
        const char *cur = smem + (kt & 1) * Cfg::STAGE;
        if (kt + 1 < nk) gload((kt + 1) * kSgBK);
        {
            f4 fa[kTM], fb[kTN];
#pragma unroll
            for (int i = 0; i < kTM; i++) fa[i] = fragment<kBM, AK>(cur, (wm * kTM + i) * 16 + fr, fq);
#pragma unroll
            for (int j = 0; j < kTN; j++) fb[j] = fragment<kBN, BK>(cur + Cfg::SLAB_A, (wn * kTN + j) * 16 + fr, fq);
#pragma unroll
            for (int s = 0; s < 4; s++)
#pragma unroll
                for (int i = 0; i < kTM; i++)
#pragma unroll
                    for (int j = 0; j < kTN; j++)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(fa[i][s], fb[j][s], acc[i][j], 0, 0, 0);
        }
        // the other stage was last read before the previous barrier, so it can be refilled now
        if (kt + 1 < nk) sstore(smem + ((kt + 1) & 1) * Cfg::STAGE);
        __syncthreads();
    }

    // accumulator layout of a 16 x 16 tile: lane l, element v holds row 4 (l / 16) + v, column l % 16
#pragma unroll
    for (int i = 0; i < kTM; i++) {
#pragma unroll
        for (int j = 0; j < kTN; j++) {
            const int n = n0 + (wn * kTN + j) * 16 + fr;
            if (n >= p.N) continue;
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const int m = m0 + (wm * kTM + i) * 16 + 4 * fq + v;
                if (m >= p.M) continue;
                float *c = C + (int64_t)m * p.ldc + n;
                const float r = p.alpha * acc[i][j][v];
                *c = p.beta != 0.0f ? r + p.beta * *c : r;
            }
        }
    }
}

template <class Cfg, bool AK, bool BK, bool VEC>
static void sg_attr() {
    // dynamic LDS above 64 KiB has to be allowed per kernel, once per device
    static bool done[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64 || done[dev]) return;
    (void)hipFuncSetAttribute((const void *)k_sgemm<Cfg, AK, BK, VEC>, hipFuncAttributeMaxDynamicSharedMemorySize,
                              (int)Cfg::LDS);
    done[dev] = true;
}

template <class Cfg, bool AK, bool BK, bool VEC>
static int sg_launch(SgArgs &p, int64_t count, hipStream_t st, const char *what) {
    p.tiles_m = (p.M + Cfg::BM - 1) / Cfg::BM;
    p.tiles_n = (p.N + Cfg::BN - 1) / Cfg::BN;
    const int64_t blocks = (int64_t)p.tiles_m * p.tiles_n * count;
    if (blocks > INT32_MAX) return set_error(NC_HIP_ERR_ARG, "%s: %lld tiles exceed one launch", what, (long long)blocks);
    sg_attr<Cfg, AK, BK, VEC>();
    hipLaunchKernelGGL((k_sgemm<Cfg, AK, BK, VEC>), dim3((unsigned)blocks), dim3(Cfg::NT), Cfg::LDS, st, p);
    return check_launch(what);
}

template <class Cfg>
static int sg_layouts(SgArgs &p, int ta, int tb, bool vec, int64_t count, hipStream_t st, const char *what) {
    const bool ak = !ta, bk = tb != 0;
#define NC_SG_CASE(AK_, BK_)                                                                \
    if (ak == AK_ && bk == BK_)                                                             \
        return vec ? sg_launch<Cfg, AK_, BK_, true>(p, count, st, what)                     \
                   : sg_launch<Cfg, AK_, BK_, false>(p, count, st, what);
    NC_SG_CASE(true, true)
    NC_SG_CASE(true, false)
    NC_SG_CASE(false, true)
    NC_SG_CASE(false, false)
#undef NC_SG_CASE
    return NC_HIP_OK;
}

static int64_t tiles_of(int64_t M, int64_t N, int bm, int bn) { return ((M + bm - 1) / bm) * ((N + bn - 1) / bn); }

// the largest tile that still gives every CU a tile, else the smallest
static int sg_run(SgArgs &p, int ta, int tb, int64_t count, hipStream_t st, const char *what) {
    // 16-byte loads need every matrix's rows 16-byte aligned: the matrices behind a pointer array may
    // start anywhere, so those take the scalar loads
    bool vec = !p.pa && aligned16(p.A) && aligned16(p.B) && p.lda % 4 == 0 && p.ldb % 4 == 0;
    for (int d = 0; d < p.bat.nb; d++) vec = vec && p.bat.st[0][d] % 4 == 0 && p.bat.st[1][d] % 4 == 0;
    const int64_t cus = num_cus();
    if (tiles_of(p.M, p.N, SgBig::BM, SgBig::BN) * count >= cus) return sg_layouts<SgBig>(p, ta, tb, vec, count, st, what);
    if (tiles_of(p.M, p.N, SgMid::BM, SgMid::BN) * count >= cus) return sg_layouts<SgMid>(p, ta, tb, vec, count, st, what);
    return sg_layouts<SgSmall>(p, ta, tb, vec, count, st, what);
}

static bool fits_int(int64_t v) { return v >= 0 && v <= INT32_MAX; }

static SgArgs sg_args(int64_t M, int64_t N, int64_t K, float alpha, const float *A, int64_t lda, const float *B,
                      int64_t ldb, float beta, float *C, int64_t ldc) {
    SgArgs p{};
    p.A = A, p.B = B, p.C = C;
    p.lda = lda, p.ldb = ldb, p.ldc = ldc;
    p.M = (int)M, p.N = (int)N, p.K = (int)K;
    p.alpha = alpha, p.beta = beta;
    return p;
}

// ------------------------------------------------------------------------------------------------
// batch axes (ops_linalg.c:89-252): per-operand strides over the output's batch shape (0 = broadcast)
// ------------------------------------------------------------------------------------------------
// drops size-1 batch axes and merges neighbours that step uniformly for all three operands
static void coalesce_batch(SgBatch &bd) {
    int w = 0;
    for (int d = 0; d < bd.nb; d++) {
        if (bd.shape[d] == 1) continue;
        if (w > 0) {
            bool merge = true;
            for (int o = 0; o < 3; o++) merge = merge && bd.st[o][w - 1] == bd.st[o][d] * bd.shape[d];
            if (merge) {
                bd.shape[w - 1] *= bd.shape[d];
                for (int o = 0; o < 3; o++) bd.st[o][w - 1] = bd.st[o][d];
                continue;
            }
        }
        bd.shape[w] = bd.shape[d];
        for (int o = 0; o < 3; o++) bd.st[o][w] = bd.st[o][d];
        w++;
    }
    bd.nb = w;
}

// true when batch index idx is the first (in index order) to write its C block: zero on every axis
// along which C is shared
static bool first_writer(const SgBatch &bd, int64_t idx) {
    for (int d = bd.nb - 1; d >= 0; d--) {
        if (bd.st[2][d] == 0 && idx % bd.shape[d] != 0) return false;
        idx /= bd.shape[d];
    }
    return true;
}

static int64_t host_batch_off(const SgBatch &bd, int o, int64_t idx) {
    int64_t off = 0;
    for (int d = bd.nb - 1; d >= 0; d--) {
        off += (idx % bd.shape[d]) * bd.st[o][d];
        idx /= bd.shape[d];
    }
    return off;
}

}  // namespace nchip

using namespace nchip;

extern "C" NC_HIP_API int nc_hip_gemm_f32(int ta, int tb, int64_t M, int64_t N, int64_t K, float alpha, const float *A,
                                          int64_t lda, const float *B, int64_t ldb, float beta, float *C, int64_t ldc,
                                          void *stream) {
    if (!fits_int(M) || !fits_int(N) || !fits_int(K)) return set_error(NC_HIP_ERR_ARG, "nc_hip_gemm_f32: bad size");
    if (M == 0 || N == 0) return NC_HIP_OK;
    if (ldc < N) return set_error(NC_HIP_ERR_ARG, "nc_hip_gemm_f32: ldc %lld < N %lld", (long long)ldc, (long long)N);
    if (K > 0 && (lda < (ta ? M : K) || ldb < (tb ? K : N)))
        return set_error(NC_HIP_ERR_ARG, "nc_hip_gemm_f32: leading dim too small");
    SgArgs p = sg_args(M, N, K, alpha, A, lda, B, ldb, beta, C, ldc);
    return sg_run(p, ta, tb, 1, as_stream(stream), "nc_hip_gemm_f32");
}

extern "C" NC_HIP_API int nc_hip_gemm_f32_batched(int ta, int tb, int64_t M, int64_t N, int64_t K, float alpha,
                                                  const float *const *A, int64_t lda, const float *const *B,
                                                  int64_t ldb, float beta, float *const *C, int64_t ldc, int64_t count,
                                                  void *stream) {
    if (!fits_int(M) || !fits_int(N) || !fits_int(K) || count < 0)
        return set_error(NC_HIP_ERR_ARG, "nc_hip_gemm_f32_batched: bad size");
    if (M == 0 || N == 0 || count == 0) return NC_HIP_OK;
    if (!A || !B || !C) return set_error(NC_HIP_ERR_ARG, "nc_hip_gemm_f32_batched: NULL pointer array");
    if (ldc < N || (K > 0 && (lda < (ta ? M : K) || ldb < (tb ? K : N))))
        return set_error(NC_HIP_ERR_ARG, "nc_hip_gemm_f32_batched: leading dim too small");
    SgArgs p = sg_args(M, N, K, alpha, nullptr, lda, nullptr, ldb, beta, nullptr, ldc);
    p.pa = A, p.pb = B, p.pc = C;
    return sg_run(p, ta, tb, count, as_stream(stream), "nc_hip_gemm_f32_batched");
}

extern "C" NC_HIP_API size_t nc_hip_gemm_f32_bmm_workspace(int64_t count) {
    (void)count;
    return 0;
}

extern "C" NC_HIP_API int nc_hip_gemm_f32_bmm(int ta, int tb, int64_t M, int64_t N, int64_t K, const float *A,
                                              int64_t lda, const float *B, int64_t ldb, float beta, float *C,
                                              int64_t ldc, int nb, const int64_t *bshape, const int64_t *sa,
                                              const int64_t *sb, const int64_t *sc, void *ws, size_t ws_bytes,
                                              void *stream) {
    (void)ws, (void)ws_bytes;
    if (!fits_int(M) || !fits_int(N) || !fits_int(K) || nb < 0 || nb > NC_HIP_MAX_DIMS)
        return set_error(NC_HIP_ERR_ARG, "nc_hip_gemm_f32_bmm: bad sizes");
    SgBatch bd{};
    bd.nb = nb;
    int64_t count = 1;
    for (int d = 0; d < nb; d++) {
        if (bshape[d] < 0) return set_error(NC_HIP_ERR_ARG, "nc_hip_gemm_f32_bmm: negative batch dim");
        bd.shape[d] = bshape[d];
        bd.st[0][d] = sa[d];
        bd.st[1][d] = sb[d];
        bd.st[2][d] = sc[d];
        count *= bshape[d];
    }
    if (M == 0 || N == 0 || count == 0) return NC_HIP_OK;
    if (ldc < N || (K > 0 && (lda < (ta ? M : K) || ldb < (tb ? K : N))))
        return set_error(NC_HIP_ERR_ARG, "nc_hip_gemm_f32_bmm: leading dim too small");
    coalesce_batch(bd);
    bool c_shared = false;  // several batch matrices add into one C block
    for (int d = 0; d < bd.nb; d++) c_shared = c_shared || bd.st[2][d] == 0;
    if (c_shared) {
        // in batch index order, every GEMM after a block's first adding into what the earlier ones wrote
        for (int64_t i = 0; i < count; i++) {
            const int rc = nc_hip_gemm_f32(ta, tb, M, N, K, 1.0f, A + host_batch_off(bd, 0, i), lda,
                                           B + host_batch_off(bd, 1, i), ldb, first_writer(bd, i) ? beta : 1.0f,
                                           C + host_batch_off(bd, 2, i), ldc, stream);
            if (rc != NC_HIP_OK) return rc;
        }
        return NC_HIP_OK;
    }
    SgArgs p = sg_args(M, N, K, 1.0f, A, lda, B, ldb, beta, C, ldc);
    p.bat = bd;
    return sg_run(p, ta, tb, count, as_stream(stream), "nc_hip_gemm_f32_bmm");
}
