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
// Each operand keeps its global layout in LDS (layouts at Panel below): a K-contiguous operand's
// fragment is one 16-byte LDS read, an M/N-contiguous one's four 4-byte reads.  The MFMAs take the B
// fragment first and so produce C^T tiles: each lane holds 4 consecutive columns of a row of C, and
// the epilogue writes (and, for beta != 0, reads) C 16 bytes at a time.
//
// k mapping.  One MFMA multiplies a 16 x 4 slice of A by a 4 x 16 slice of B, quarter-wave q (lanes
// 16 q .. 16 q + 15) holding one k.  In each stage of 16 k, quarter q gives the s-th MFMA (s = 0..3)
// the value at k = 4 q + s, for A and B alike, so a K-contiguous operand feeds four MFMAs from one
// 16-byte LDS read.
//
// Summation order (blocked, like the reference's register blocks summed from zero and added into C,
// kernels_avx2.c:234-247): K is cut into panels of 32 k (two stages).  A panel's 32 products of an
// output element are summed from zero, four per MFMA (eight MFMAs), and the panel sum is added into the
// element's running total (one fp32 add per 32 k).  A small panel sum is not rounded against the whole
// running total, so the error of a K-term dot product grows like that of a blocked sum rather than like
// K sequential additions.  The order is a property of the kernel alone: the same for every tile size
// and grid, so results are identical run to run and on any device.  It differs from the reference's
// serial order, so the parity bar is the fp32 error bound of a K-term dot product.
//
// Tile sizes: 256 x 256 (8 waves of 8 x 4 tiles) when the problem has at least as many such tiles as
// the device has CUs, else 128 x 128 (4 waves of 4 x 4) or 64 x 64 (4 waves of 2 x 2).  Blocks are
// remapped so each XCD (blocks b with b % 8 equal) works a contiguous run of tiles, and tiles run in
// groups of 8 tile-rows so neighbouring blocks share panels in L2.
#include "common.hpp"

namespace nchip {


constexpr int kSgBK = 16;      // k per stage
constexpr int kSgPanel = 2;    // stages per summation panel (32 k)

constexpr int kSgGroupM = 8;   // tile-rows per group in the block order

// MINB: workgroups per CU the register allocation leaves room for
template <int TM_, int TN_, int WGM_, int WGN_, int MINB_>
struct SgCfg {
    static constexpr int TM = TM_, TN = TN_, WGM = WGM_, WGN = WGN_;
    static constexpr int MINB = MINB_;
    static constexpr int NT = 64 * WGM * WGN;
    static constexpr int BM = 16 * TM * WGM, BN = 16 * TN * WGN;
    // bytes of one stage of an operand panel in LDS (R rows by 16 k, either layout)
    static constexpr int SLAB_A = 64 * BM, SLAB_B = 64 * BN;
    static constexpr int STAGE = SLAB_A + SLAB_B;
    static constexpr size_t LDS = 2 * (size_t)STAGE;
};
using SgBig = SgCfg<8, 4, 2, 4, 1>;    // 256 x 256
using SgMid = SgCfg<4, 4, 2, 2, 2>;    // 128 x 128
using SgSmall = SgCfg<2, 2, 2, 2, 4>;  // 64 x 64

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
    const float *bias;  // N floats added to every row after alpha A B + beta C, or none
    int tiles_m, tiles_n;
    SgBatch bat;
};

// ---- operand panels ------------------------------------------------------------------------------
// One stage of an operand: R rows (M or N) by 16 k, loaded as 16-byte chunks spread over the
// workgroup's threads, kept in registers while the previous stage is multiplied, then stored to LDS.
//   * K-contiguous operand: chunk u is row u / 4, k 4 (u % 4) .. + 3; in LDS rows of 64 bytes, logical
//     chunk c of row r at chunk c ^ kc_swz(r), so the 16-byte fragment reads spread over all banks;
//   * M/N-contiguous operand: chunk u is k-row u / (R / 4), rows 4 (u % (R / 4)) .. + 3; in LDS 16
//     k-rows of R floats (R >= 64), the chunk of rows 4 c .. 4 c + 3 of k-row k at chunk c ^ mn_swz(k),
//     so the four quarter-waves' fragment reads (k-rows k, k + 4, k + 8, k + 12 of 16 consecutive
//     rows) land in different banks.  Either layout is 64 R bytes per stage, with no padding, so a
//     load straight into LDS fills it 1 KiB at a time.
template <int R, bool KC, int NT>
struct Panel {
    static constexpr int UNITS = 4 * R;
    static constexpr int UPT = (UNITS + NT - 1) / NT;  // chunks per thread
    static constexpr bool GUARD = UNITS % NT != 0;     // some threads own fewer chunks
};

// global-memory views, so loads are global_load (counted by vmcnt alone) rather than flat
typedef const __attribute__((address_space(1))) float gfloat;
typedef const __attribute__((address_space(1))) f4 gf4;

// row and k of unit u's first chunk within the stage
template <int R, bool KC>
__device__ __forceinline__ void unit_pos(int u, int &row, int &k) {
    if constexpr (KC) {
        row = u >> 2, k = (u & 3) * 4;
    } else {
        row = (u % (R / 4)) * 4, k = u / (R / 4);
    }
}

// 4 floats at (row .. row + 3 or k .. k + 3), zero past the matrix; VEC: 16-byte aligned rows, so a
// chunk wholly inside is one load
template <bool KC, bool VEC>
__device__ __forceinline__ f4 load4(const float *p, int64_t ld, int rows, int K, int row, int k) {
    f4 v = {0.f, 0.f, 0.f, 0.f};
    if constexpr (KC) {
        if (row >= rows || k >= K) return v;
        gfloat *s = (gfloat *)(p + (int64_t)row * ld + k);
        if (VEC && k + 4 <= K) return *(gf4 *)s;
#pragma unroll
        for (int j = 0; j < 4; j++)
            if (k + j < K) v[j] = s[j];
    } else {
        if (k >= K || row >= rows) return v;
        gfloat *s = (gfloat *)(p + (int64_t)k * ld + row);
        if (VEC && row + 4 <= rows) return *(gf4 *)s;
#pragma unroll
        for (int j = 0; j < 4; j++)
            if (row + j < rows) v[j] = s[j];
    }
    return v;
}

// The chunk permutation of K-contiguous panel row r (an XOR mask on its four 16-byte chunks).
// (r >> 1) & 3 leaves the 16-byte fragment reads of the 16 rows and 4 quarter-waves free of bank
// conflicts (SQ_LDS_BANK_CONFLICT reads 0; (r >> 2) & 3 read a third to a half of the LDS cycles).
__device__ __forceinline__ int kc_swz(int r) { return (r >> 1) & 3; }

// The chunk permutation of M/N-contiguous panel k-row k: quarter-wave q reads k-rows 4 q .. 4 q + 3,
// so XOR-ing bits 2-3 of the chunk index with q puts the four quarters' 16 rows in four disjoint
// groups of 16 banks (the 64 banks of 4 bytes, since a k-row's 4 R bytes are a multiple of 256).
__device__ __forceinline__ int mn_swz(int k) { return ((k >> 2) & 3) << 2; }

// LDS store of one chunk
template <int R, bool KC>
__device__ __forceinline__ void unit_store(char *slab, int u, f4 v) {
    int row, k;
    unit_pos<R, KC>(u, row, k);
    if constexpr (KC) {
        const int c = k >> 2;
        *(f4 *)(slab + row * 64 + ((c ^ kc_swz(row)) << 4)) = v;
    } else {
        *(f4 *)(slab + k * R * 4 + (((row >> 2) ^ mn_swz(k)) << 4)) = v;
    }
}

// The four values (s = 0..3) of panel row r that quarter-wave q gives the stage's MFMAs.
template <int R, bool KC>
__device__ __forceinline__ f4 fragment(const char *slab, int r, int q) {
    if constexpr (KC) {
        return *(const f4 *)(slab + r * 64 + ((q ^ kc_swz(r)) << 4));
    } else {
        static_assert(R >= 64, "the k-row permutation needs 16 chunks");
        const float *b = (const float *)slab + 4 * q * R + 4 * ((r >> 2) ^ (q << 2)) + (r & 3);
        return f4{b[0], b[R], b[2 * R], b[3 * R]};
    }
}

// One operand's stage loads: registers, FAST source pointers, load and store.
template <int R, bool KC, int NT, bool VEC, bool FAST>
struct Loader {
    using P = Panel<R, KC, NT>;
    f4 reg[P::UPT];
    gfloat *src[FAST ? P::UPT : 1];
    const float *p;
    int64_t ld;
    int rows, K, r0, t;

    // FAST problems (aligned rows, K a multiple of 16, an M/N-contiguous operand's row count a
    // multiple of 4): rows past the matrix are clamped onto its last row (last 4-row chunk), so every
    // load is in bounds and unconditional; what those rows produce is never stored
    __device__ __forceinline__ void init(const float *p_, int64_t ld_, int rows_, int K_, int r0_, int t_) {
        p = p_, ld = ld_, rows = rows_, K = K_, r0 = r0_, t = t_;
        if constexpr (FAST) {
#pragma unroll
            for (int i = 0; i < P::UPT; i++) {
                int row, k;
                unit_pos<R, KC>(t + i * NT, row, k);
                row = KC ? min(r0 + row, rows - 1) : min(r0 + row, rows - 4);
                src[i] = (gfloat *)(KC ? p + (int64_t)row * ld + k : p + (int64_t)k * ld + row);
            }
        }
    }
    __device__ __forceinline__ bool owns(int i) const { return !P::GUARD || t + i * NT < P::UNITS; }
    __device__ __forceinline__ void load(int k0) {
#pragma unroll
        for (int i = 0; i < P::UPT; i++) {
            if (!owns(i)) continue;
            if constexpr (FAST) {
                reg[i] = *(gf4 *)(src[i] + (KC ? k0 : (int64_t)k0 * ld));
            } else {
                int row, k;
                unit_pos<R, KC>(t + i * NT, row, k);
                reg[i] = load4<KC, VEC>(p, ld, rows, K, r0 + row, k0 + k);
            }
        }
    }
    __device__ __forceinline__ void store(char *slab) const {
#pragma unroll
        for (int i = 0; i < P::UPT; i++)
            if (owns(i)) unit_store<R, KC>(slab, t + i * NT, reg[i]);
    }
};

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

// The workgroup's tile: block -> (batch matrix, tile) with XCD-contiguous runs and groups of
// kSgGroupM tile-rows; the batch matrix's operands.
struct TileAt {
    int m0, n0;
    const float *A, *B;
    float *C;
};

template <int BM, int BN>
__device__ __forceinline__ TileAt locate(const SgArgs &p) {
    int64_t id = blockIdx.x;
    const int64_t nblk = gridDim.x;
    if ((nblk & 7) == 0) id = (id & 7) * (nblk >> 3) + (id >> 3);
    const int64_t per_batch = (int64_t)p.tiles_m * p.tiles_n;
    const int64_t batch = id / per_batch;
    const int tile = (int)(id % per_batch);
    const int per_group = kSgGroupM * p.tiles_n;
    const int first_m = (tile / per_group) * kSgGroupM;
    const int gsize = min(p.tiles_m - first_m, kSgGroupM);
    TileAt at;
    at.m0 = (first_m + (tile % per_group) % gsize) * BM;
    at.n0 = ((tile % per_group) / gsize) * BN;
    if (p.pa) {
        at.A = p.pa[batch], at.B = p.pb[batch], at.C = p.pc[batch];
    } else {
        at.A = p.A + batch_off(p.bat, 0, batch), at.B = p.B + batch_off(p.bat, 1, batch);
        at.C = p.C + batch_off(p.bat, 2, batch);
    }
    return at;
}

// The register-staged kernels keep a panel accumulator per tile beside the running totals: the
// stage's fragments are read, its MFMAs (s = 0..3, the B fragment first: the tile is C^T, so each lane
// ends up holding 4 consecutive columns of a row of C) add into the accumulators, and after a panel's
// last stage the accumulators are added into the totals and cleared.
template <class Cfg, bool AK, bool BK>
__device__ __forceinline__ void stage_acc(const char *cur, f4 (&acc)[Cfg::TM][Cfg::TN], int wm, int wn, int fr, int fq) {
    f4 a[Cfg::TM], b[Cfg::TN];
#pragma unroll
    for (int i = 0; i < Cfg::TM; i++) a[i] = fragment<Cfg::BM, AK>(cur, (wm * Cfg::TM + i) * 16 + fr, fq);
#pragma unroll
    for (int j = 0; j < Cfg::TN; j++) b[j] = fragment<Cfg::BN, BK>(cur + Cfg::SLAB_A, (wn * Cfg::TN + j) * 16 + fr, fq);
#pragma unroll
    for (int s = 0; s < 4; s++)
#pragma unroll
        for (int i = 0; i < Cfg::TM; i++)
#pragma unroll
            for (int j = 0; j < Cfg::TN; j++) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(b[j][s], a[i][s], acc[i][j], 0, 0, 0);
}

template <class Cfg>
__device__ __forceinline__ void fold(f4 (&tot)[Cfg::TM][Cfg::TN], f4 (&acc)[Cfg::TM][Cfg::TN]) {
#pragma unroll
    for (int i = 0; i < Cfg::TM; i++)
#pragma unroll
        for (int j = 0; j < Cfg::TN; j++) {
            tot[i][j] = tot[i][j] + acc[i][j];
            acc[i][j] = f4{0.f, 0.f, 0.f, 0.f};
        }
}

// A wave's stores of one row block's final totals during the last panel: C row (tile row + fr) of row
// block 0 at byte offset `off` from the tile's C (lane's four columns), row block i `rb` bytes further.
struct RbStore {
    const float *base;  // the batch matrix's C (wave-uniform)
    uint32_t off;       // this lane's first element, row block 0, tile column 0, in bytes
    uint32_t rb;        // 16 rows of C, in bytes
    float alpha;
};

// One 16-byte store at a wave-uniform base plus a 32-bit offset.  The store reads its data registers
// after it issues, and a VALU instruction may overwrite them only two wait states later on this
// family; the compiler inserts those after its own stores, not after inline assembly, so the s_nop
// (three wait states) is part of the statement (without it the next value's fourth component reached
// memory now and then).
__device__ __forceinline__ void store16(const float *base, uint32_t off, f4 v) {
    asm volatile("global_store_dwordx4 %0, %1, %2\n\ts_nop 2" ::"v"(off), "v"(v), "s"(base) : "memory");
}

// The direct-to-LDS kernel has a whole panel in LDS and works it row block by row block, so only one
// row block's TN panel sums are live beside the totals: the B fragments of the panel's stages are read
// once; per row block the A fragments are read, each tile sums its panel's products from zero (stage
// 0's four MFMAs, then stage 1's), and the sums are added into the totals.  st (the tile's last panel,
// stored as it completes, through rs): once the next row block's adds have made a row block's totals
// final, its TN tiles are stored between that row block's MFMAs, so a tile's 256 x 256 output leaves
// spread over its last panel instead of all CUs storing at the same moment after it.
template <class Cfg, bool AK, bool BK>
__device__ __forceinline__ void panel_mfma(const char *c0, const char *c1, f4 (&tot)[Cfg::TM][Cfg::TN], int wm, int wn,
                                           int fr, int fq, const RbStore *rs = nullptr, bool st = false) {
    auto store_rb = [&](int i) {
#pragma unroll
        for (int j = 0; j < Cfg::TN; j++) store16(rs->base, rs->off + (uint32_t)i * rs->rb + (uint32_t)(j * 64), rs->alpha * tot[i][j]);
    };
    static_assert(Cfg::TN == 4, "one previous-row-block add per k step");
    f4 b0[Cfg::TN], b1[Cfg::TN];
#pragma unroll
    for (int j = 0; j < Cfg::TN; j++) {
        b0[j] = fragment<Cfg::BN, BK>(c0 + Cfg::SLAB_A, (wn * Cfg::TN + j) * 16 + fr, fq);
        b1[j] = fragment<Cfg::BN, BK>(c1 + Cfg::SLAB_A, (wn * Cfg::TN + j) * 16 + fr, fq);
    }
    f4 a0 = fragment<Cfg::BM, AK>(c0, wm * Cfg::TM * 16 + fr, fq);
    f4 a1 = fragment<Cfg::BM, AK>(c1, wm * Cfg::TM * 16 + fr, fq);
    // Issue order, pinned by scheduling barriers: per row block, 8 k steps of the TN tiles' independent
    // MFMAs; in each of the first TN steps one tile of the previous row block adds its finished sum
    // into its total (the sum's last MFMA was issued at least TN MFMAs earlier, so the add needs no
    // wait states and issues between MFMAs); the next row block's A fragments are read meanwhile.
    f4 tp[Cfg::TN];
#pragma unroll
    for (int i = 0; i < Cfg::TM; i++) {
        f4 na0 = a0, na1 = a1;
        if (i + 1 < Cfg::TM) {
            const int row = (wm * Cfg::TM + i + 1) * 16 + fr;
            na0 = fragment<Cfg::BM, AK>(c0, row, fq);
            na1 = fragment<Cfg::BM, AK>(c1, row, fq);
        }
        f4 t[Cfg::TN];
#pragma unroll
        for (int s = 0; s < 8; s++) {
            const f4 &a = s < 4 ? a0 : a1;
#pragma unroll
            for (int j = 0; j < Cfg::TN; j++) {
                const f4 &b = s < 4 ? b0[j] : b1[j];
                t[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(b[s & 3], a[s & 3], s == 0 ? f4{0.f, 0.f, 0.f, 0.f} : t[j],
                                                            0, 0, 0);
            }
            if (i > 0 && s < Cfg::TN) tot[i - 1][s] = tot[i - 1][s] + tp[s];
            if (st && i > 0 && s == Cfg::TN) store_rb(i - 1);
            __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int j = 0; j < Cfg::TN; j++) tp[j] = t[j];
        a0 = na0, a1 = na1;
    }
#pragma unroll
    for (int j = 0; j < Cfg::TN; j++) tot[Cfg::TM - 1][j] = tot[Cfg::TM - 1][j] + tp[j];
    if (st) store_rb(Cfg::TM - 1);
}

// C = alpha acc + beta C (+ bias[n]) over the wave's tiles.  acc[i][j] is the 16 x 16 tile C^T: lane l,
// element v holds row (tile row + l % 16), column (tile column + 4 (l / 16) + v).  The bias is added to
// the rounded alpha acc + beta C, as a separate broadcast add of it would.
template <class Cfg>
__device__ __forceinline__ void write_tiles(const SgArgs &p, const TileAt &at, const f4 (&acc)[Cfg::TM][Cfg::TN],
                                            int wm, int wn, int fr, int fq) {
    constexpr int kTM = Cfg::TM, kTN = Cfg::TN;
    const bool vec_c = ((uintptr_t)at.C & 15) == 0 && p.ldc % 4 == 0;
    const bool vec_b = ((uintptr_t)p.bias & 15) == 0;
#pragma unroll
    for (int i = 0; i < kTM; i++) {
        const int m = at.m0 + (wm * kTM + i) * 16 + fr;
        if (m >= p.M) continue;
        float *crow = at.C + (int64_t)m * p.ldc;
#pragma unroll
        for (int j = 0; j < kTN; j++) {
            const int n = at.n0 + (wn * kTN + j) * 16 + 4 * fq;
            f4 r = p.alpha * acc[i][j];
            if (vec_c && n + 4 <= p.N) {
                f4 *c = (f4 *)(crow + n);
                if (p.beta != 0.0f) r = r + p.beta * *c;
                if (p.bias) {
                    if (vec_b) r = r + *(const f4 *)(p.bias + n);
                    else r = r + f4{p.bias[n], p.bias[n + 1], p.bias[n + 2], p.bias[n + 3]};
                }
                *c = r;
            } else {
#pragma unroll
                for (int v = 0; v < 4; v++) {
                    if (n + v >= p.N) break;
                    float *c = crow + n + v;
                    const float t = p.beta != 0.0f ? r[v] + p.beta * *c : r[v];
                    *c = p.bias ? t + p.bias[n + v] : t;
                }
            }
        }
    }
}

template <class Cfg, bool AK, bool BK, bool VEC, bool FAST>
__global__ __launch_bounds__(Cfg::NT, Cfg::MINB) void k_sgemm(SgArgs p) {
    extern __shared__ __attribute__((aligned(16))) char smem[];
    const TileAt at = locate<Cfg::BM, Cfg::BN>(p);
    const int t = threadIdx.x, lane = t & (kWave - 1), wid = t / kWave;
    const int wm = wid / Cfg::WGN, wn = wid % Cfg::WGN, fr = lane & 15, fq = lane >> 4;

    Loader<Cfg::BM, AK, Cfg::NT, VEC, FAST> la;
    Loader<Cfg::BN, BK, Cfg::NT, VEC, FAST> lb;
    la.init(at.A, p.lda, p.M, p.K, at.m0, t);
    lb.init(at.B, p.ldb, p.N, p.K, at.n0, t);

    f4 acc[Cfg::TM][Cfg::TN], tot[Cfg::TM][Cfg::TN];  // panel accumulators, running totals
#pragma unroll
    for (int i = 0; i < Cfg::TM; i++)
#pragma unroll
        for (int j = 0; j < Cfg::TN; j++) acc[i][j] = tot[i][j] = f4{0.f, 0.f, 0.f, 0.f};

    const int nk = (p.K + kSgBK - 1) / kSgBK;
    if (nk > 0) {
        la.load(0);
        lb.load(0);
        la.store(smem);
        lb.store(smem + Cfg::SLAB_A);
        __syncthreads();
    }
    for (int kt = 0; kt < nk; kt++) {
        if (kt + 1 < nk) {
            la.load((kt + 1) * kSgBK);
            lb.load((kt + 1) * kSgBK);
        }
        stage_acc<Cfg, AK, BK>(smem + (kt & 1) * Cfg::STAGE, acc, wm, wn, fr, fq);
        if (kt % kSgPanel == kSgPanel - 1 || kt + 1 == nk) fold<Cfg>(tot, acc);
        // the other stage was last read before the previous barrier, so it can be refilled now
        if (kt + 1 < nk) {
            char *next = smem + ((kt + 1) & 1) * Cfg::STAGE;
            la.store(next);
            lb.store(next + Cfg::SLAB_A);
        }
        __syncthreads();
    }
    write_tiles<Cfg>(p, at, tot, wm, wn, fr, fq);
}

// ------------------------------------------------------------------------------------------------
// Large FAST problems with K a multiple of 32: the 256 x 256 tile, its operand panels loaded straight
// from global memory into LDS (global_load_lds_dwordx4) a summation panel (two stages) ahead through
// four LDS stages, with no staging registers and no LDS write instructions; one barrier per summation
// panel.  A stage of an R-row panel is R / 16 load
// instructions of 1 KiB each: 16 rows of a K-contiguous panel (lane l: row l / 4, the chunk that
// belongs at position l % 4 under the row's permutation) or 256 / R k-rows of a M/N-contiguous one
// (lane l: k-row l / (R / 4), position l % (R / 4), loading the rows the k-row's permutation puts
// there).  The 32 instructions of a stage (16 for A, 16 for B) are dealt four to a wave.  Rows past
// the matrix are clamped as in the staged kernel's FAST loads.
constexpr int kSgDmaStages = 4;

template <class Cfg>
struct SgDma {
    static constexpr int NW = Cfg::NT / kWave;
    static constexpr int IA = Cfg::BM / 16, IB = Cfg::BN / 16;  // load instructions per stage
    static constexpr int PER = (IA + IB) / NW;                    // per wave
    static_assert((IA + IB) % NW == 0, "the stage's loads deal evenly over the waves");
    static constexpr size_t LDS = kSgDmaStages * (size_t)Cfg::STAGE;
};

// s_waitcnt vmcnt(N) for a compile-time N
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N <= 15, "vmcnt immediate");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

template <class Cfg, bool AK, bool BK>
__global__ __launch_bounds__(Cfg::NT, 1) void k_sgemm_dma(SgArgs p) {
    using D = SgDma<Cfg>;
    extern __shared__ __attribute__((aligned(16))) char smem[];
    const TileAt at = locate<Cfg::BM, Cfg::BN>(p);
    const int t = threadIdx.x, lane = t & (kWave - 1), wid = t / kWave;
    const int wm = wid / Cfg::WGN, wn = wid % Cfg::WGN, fr = lane & 15, fq = lane >> 4;

    // this wave's load instructions per stage (each one wave-uniform in its panel)
    const float *src[D::PER];
    int64_t kstep[D::PER];  // elements from one stage to the next
    uint32_t loff[D::PER];
#pragma unroll
    for (int i = 0; i < D::PER; i++) {
        const int j = wid * D::PER + i;
        const bool pb = j >= D::IA;
        const int idx = pb ? j - D::IA : j;
        const bool kc = pb ? BK : AK;
        const float *base = pb ? at.B : at.A;
        const int64_t ld = pb ? p.ldb : p.lda;
        const int rows = pb ? p.N : p.M, r0 = pb ? at.n0 : at.m0;
        const int R = pb ? Cfg::BN : Cfg::BM;
        if (kc) {
            const int prow = 16 * idx + (lane >> 2), c = (lane & 3) ^ kc_swz(prow);
            src[i] = base + (int64_t)min(r0 + prow, rows - 1) * ld + 4 * c;
        } else {
            const int per_row = R / 4;  // chunks per k-row
            const int k = idx * (kWave / per_row) + lane / per_row, c = (lane % per_row) ^ mn_swz(k);
            src[i] = base + (int64_t)k * ld + min(r0 + 4 * c, rows - 4);
        }
        kstep[i] = kc ? kSgBK : kSgBK * ld;
        loff[i] = (uint32_t)(idx * 1024) + (pb ? Cfg::SLAB_A : 0);
    }
    const uint32_t sbase = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char *)smem;
    auto issue = [&](int kt) {
        const uint32_t st = sbase + (uint32_t)(kt % kSgDmaStages) * Cfg::STAGE;
#pragma unroll
        for (int i = 0; i < D::PER; i++) dma16(src[i] + kt * kstep[i], __builtin_amdgcn_readfirstlane(st + loff[i]));
    };

    f4 tot[Cfg::TM][Cfg::TN];  // running totals
#pragma unroll
    for (int i = 0; i < Cfg::TM; i++)
#pragma unroll
        for (int j = 0; j < Cfg::TN; j++) tot[i][j] = f4{0.f, 0.f, 0.f, 0.f};

    // LDS stage slots 0-1 and 2-3 alternate between panels: panel q + 1 loads while panel q is worked
    // (K is a multiple of 32: whole panels)
    const int npanel = p.K / (kSgBK * kSgPanel);
    // both operands K-contiguous (the layouts with registers to spare for it), a whole tile, C = alpha A B
    // with 16-byte rows and the tile within 4 GiB of the matrix's start: the last panel stores its row
    // blocks as they complete (uniform over the workgroup).  The 64 x [1024,128] x [128,1024] batched
    // product spent a quarter of its time (185 us against 141 without stores) on its output leaving in one
    // burst per tile round: 185 -> 162-166 us.
    const bool stream_st = AK && BK && p.beta == 0.0f && !p.bias && ((uintptr_t)at.C & 15) == 0 && p.ldc % 4 == 0 &&
                           at.m0 + Cfg::BM <= p.M && at.n0 + Cfg::BN <= p.N &&
                           ((int64_t)at.m0 + Cfg::BM) * p.ldc * 4 < ((int64_t)1 << 32);
    RbStore rs;
    rs.base = at.C;
    rs.off = (uint32_t)(((int64_t)(at.m0 + wm * Cfg::TM * 16 + fr) * p.ldc + at.n0 + wn * Cfg::TN * 16 + 4 * fq) * 4);
    rs.rb = (uint32_t)(16 * p.ldc * 4);
    rs.alpha = p.alpha;
    auto issue_panel = [&](int q) {
        issue(kSgPanel * q);
        issue(kSgPanel * q + 1);
    };
    if (npanel > 0) issue_panel(0);
    for (int q = 0; q < npanel; q++) {
        wait_vmcnt<0>();               // this wave's loads of panel q (the only ones in flight)
        __builtin_amdgcn_s_barrier();  // every wave's loads of panel q have landed; panel q - 1 is read
        asm volatile("" ::: "memory");
        if (q + 1 < npanel) issue_panel(q + 1);  // into the slots panel q - 1 used
        const int k0 = kSgPanel * q;
        panel_mfma<Cfg, AK, BK>(smem + (k0 % kSgDmaStages) * Cfg::STAGE,
                                smem + ((k0 + 1) % kSgDmaStages) * Cfg::STAGE, tot, wm, wn, fr, fq, &rs,
                                stream_st && q + 1 == npanel);
    }
    if (!stream_st) write_tiles<Cfg>(p, at, tot, wm, wn, fr, fq);
}

template <class Cfg, bool AK, bool BK, bool VEC, bool FAST>
static void sg_attr() {
    // dynamic LDS above 64 KiB has to be allowed per kernel, once per device
    static bool done[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64 || done[dev]) return;
    (void)hipFuncSetAttribute((const void *)k_sgemm<Cfg, AK, BK, VEC, FAST>, hipFuncAttributeMaxDynamicSharedMemorySize,
                              (int)Cfg::LDS);
    done[dev] = true;
}

template <class Cfg, bool AK, bool BK, bool VEC, bool FAST>
static int sg_launch(SgArgs &p, int64_t count, hipStream_t st, const char *what) {
    p.tiles_m = (p.M + Cfg::BM - 1) / Cfg::BM;
    p.tiles_n = (p.N + Cfg::BN - 1) / Cfg::BN;
    const int64_t blocks = (int64_t)p.tiles_m * p.tiles_n * count;
    if (blocks > INT32_MAX) return set_error(NC_HIP_ERR_ARG, "%s: %lld tiles exceed one launch", what, (long long)blocks);
    sg_attr<Cfg, AK, BK, VEC, FAST>();
    hipLaunchKernelGGL((k_sgemm<Cfg, AK, BK, VEC, FAST>), dim3((unsigned)blocks), dim3(Cfg::NT), Cfg::LDS, st, p);
    return check_launch(what);
}

#ifndef SG_DMA
#define SG_DMA 1
#endif
template <class Cfg, bool AK, bool BK>
static int sg_launch_dma(SgArgs &p, int64_t count, hipStream_t st, const char *what) {
    p.tiles_m = (p.M + Cfg::BM - 1) / Cfg::BM;
    p.tiles_n = (p.N + Cfg::BN - 1) / Cfg::BN;
    const int64_t blocks = (int64_t)p.tiles_m * p.tiles_n * count;
    if (blocks > INT32_MAX) return set_error(NC_HIP_ERR_ARG, "%s: %lld tiles exceed one launch", what, (long long)blocks);
    static bool done[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) == hipSuccess && dev >= 0 && dev < 64 && !done[dev]) {
        (void)hipFuncSetAttribute((const void *)k_sgemm_dma<Cfg, AK, BK>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                  (int)SgDma<Cfg>::LDS);
        done[dev] = true;
    }
    hipLaunchKernelGGL((k_sgemm_dma<Cfg, AK, BK>), dim3((unsigned)blocks), dim3(Cfg::NT), SgDma<Cfg>::LDS, st, p);
    return check_launch(what);
}

// the register-staged kernels (128 x 128 and 64 x 64 tiles), by operand layout and load width
template <class Cfg>
static int sg_layouts(SgArgs &p, int ta, int tb, bool vec, bool fast, int64_t count, hipStream_t st, const char *what) {
    const bool ak = !ta, bk = tb != 0;
#define NC_SG_CASE(AK_, BK_)                                                                \
    if (ak == AK_ && bk == BK_)                                                             \
        return fast ? sg_launch<Cfg, AK_, BK_, true, true>(p, count, st, what)              \
               : vec  ? sg_launch<Cfg, AK_, BK_, true, false>(p, count, st, what)           \
                      : sg_launch<Cfg, AK_, BK_, false, false>(p, count, st, what);
    NC_SG_CASE(true, true)
    NC_SG_CASE(true, false)
    NC_SG_CASE(false, true)
    NC_SG_CASE(false, false)
#undef NC_SG_CASE
    return NC_HIP_OK;
}

static int64_t tiles_of(int64_t M, int64_t N, int bm, int bn) { return ((M + bm - 1) / bm) * ((N + bn - 1) / bn); }

// The 256 x 256 direct-to-LDS kernel for aligned problems (16-byte rows, K a multiple of 32: whole
// summation panels) with at least a tile per CU; otherwise the largest register-staged tile that still
// gives every CU a tile, else the smallest.
static int sg_run(SgArgs &p, int ta, int tb, int64_t count, hipStream_t st, const char *what) {
    // 16-byte loads need every matrix's rows 16-byte aligned: the matrices behind a pointer array may
    // start anywhere, so those take the scalar loads
    bool vec = !p.pa && aligned16(p.A) && aligned16(p.B) && p.lda % 4 == 0 && p.ldb % 4 == 0;
    for (int d = 0; d < p.bat.nb; d++) vec = vec && p.bat.st[0][d] % 4 == 0 && p.bat.st[1][d] % 4 == 0;
    const bool ak = !ta, bk = tb != 0;
    const bool fast = vec && p.K % kSgBK == 0 && (ak || p.M % 4 == 0) && (bk || p.N % 4 == 0);
    const int64_t cus = num_cus();
    // the DMA kernel clamps M/N-contiguous chunks onto the last 4 rows: at least 4 rows there
    const bool dma = SG_DMA && fast && p.K > 0 && p.K % (kSgBK * kSgPanel) == 0 && (ak || p.M >= 4) && (bk || p.N >= 4);
    if (dma && tiles_of(p.M, p.N, SgBig::BM, SgBig::BN) * count >= cus) {
#define NC_SG_DMA(AK_, BK_) \
    if (ak == AK_ && bk == BK_) return sg_launch_dma<SgBig, AK_, BK_>(p, count, st, what);
        NC_SG_DMA(true, true)
        NC_SG_DMA(true, false)
        NC_SG_DMA(false, true)
        NC_SG_DMA(false, false)
#undef NC_SG_DMA
    }
    if (tiles_of(p.M, p.N, SgMid::BM, SgMid::BN) * count >= cus)
        return sg_layouts<SgMid>(p, ta, tb, vec, fast, count, st, what);
    return sg_layouts<SgSmall>(p, ta, tb, vec, fast, count, st, what);
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

extern "C" NC_HIP_API int nc_hip_gemm_f32_bias(int ta, int tb, int64_t M, int64_t N, int64_t K, float alpha,
                                               const float *A, int64_t lda, const float *B, int64_t ldb,
                                               const float *bias, float *C, int64_t ldc, void *stream) {
    if (!fits_int(M) || !fits_int(N) || !fits_int(K)) return set_error(NC_HIP_ERR_ARG, "nc_hip_gemm_f32_bias: bad size");
    if (M == 0 || N == 0) return NC_HIP_OK;
    if (ldc < N) return set_error(NC_HIP_ERR_ARG, "nc_hip_gemm_f32_bias: ldc %lld < N %lld", (long long)ldc, (long long)N);
    if (K > 0 && (lda < (ta ? M : K) || ldb < (tb ? K : N)))
        return set_error(NC_HIP_ERR_ARG, "nc_hip_gemm_f32_bias: leading dim too small");
    SgArgs p = sg_args(M, N, K, alpha, A, lda, B, ldb, 0.0f, C, ldc);
    p.bias = bias;
    return sg_run(p, ta, tb, 1, as_stream(stream), "nc_hip_gemm_f32_bias");
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
