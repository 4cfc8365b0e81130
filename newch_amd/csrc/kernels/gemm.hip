// fp32 GEMM entry points (the reference's gemm_f32 kernel-table entry, kernels.h:36-41): dense GEMMs
// on the matrix cores through hipBLASLt (rocBLAS for the cases it does not take), row-major interface.
//
// Row-major C (M x N) = op(A) op(B) is column-major C^T = op(B)^T op(A)^T, so the operands are passed
// to the library swapped, each with its own transpose flag.  hipBLASLt runs with no workspace (no
// split-k partial buffers; the same inputs give the same bits run after run) and its first heuristic
// choice, planned once per shape and cached; measured on MI355X it reaches 148-154 TFLOP/s on
// [8192,4096] x [4096,4096] and ~100 on 64 x [1024,128] x [128,1024], where rocBLAS ran 134-139 and
// 46.  rocBLAS (one handle per device, atomics off, host pointer mode) covers K = 0, unaligned
// operands, broadcast batch strides and pointer-array batches.
#include "common.hpp"

#include <hipblaslt/hipblaslt.h>
#include <rocblas/rocblas.h>

#include <mutex>
#include <unordered_map>

namespace nchip {

static rocblas_handle blas_handle() {
    static rocblas_handle handles[64] = {};
    static std::mutex mu;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
    std::lock_guard<std::mutex> lock(mu);
    if (!handles[dev]) {
        rocblas_handle h = nullptr;
        if (rocblas_create_handle(&h) != rocblas_status_success) return nullptr;
        rocblas_set_atomics_mode(h, rocblas_atomics_not_allowed);
        rocblas_set_pointer_mode(h, rocblas_pointer_mode_host);
        handles[dev] = h;
    }
    return handles[dev];
}

static int blas_error(rocblas_status s, const char *what) {
    return set_error(NC_HIP_ERR_DEVICE, "%s: rocBLAS %s", what, rocblas_status_to_string(s));
}

static rocblas_operation op_of(int t) { return t ? rocblas_operation_transpose : rocblas_operation_none; }

// ---- hipBLASLt plans ----------------------------------------------------------------------------
struct LtKey {
    int dev, ta, tb;
    int64_t M, N, K, lda, ldb, ldc, count, sa, sb, sc;
    bool operator==(const LtKey &o) const {
        return dev == o.dev && ta == o.ta && tb == o.tb && M == o.M && N == o.N && K == o.K && lda == o.lda &&
               ldb == o.ldb && ldc == o.ldc && count == o.count && sa == o.sa && sb == o.sb && sc == o.sc;
    }
};
struct LtKeyHash {
    size_t operator()(const LtKey &k) const {
        const int64_t v[] = {k.dev, k.ta, k.tb, k.M, k.N, k.K, k.lda, k.ldb, k.ldc, k.count, k.sa, k.sb, k.sc};
        size_t h = 1469598103934665603ull;
        for (int64_t x : v) h = (h ^ (size_t)x) * 1099511628211ull;
        return h;
    }
};
struct LtPlan {
    bool ok = false;
    hipblasLtMatmulDesc_t desc{};
    hipblasLtMatrixLayout_t la{}, lb{}, lc{};
    hipblasLtMatmulAlgo_t algo{};
};

static std::mutex lt_mu;
static hipblasLtHandle_t lt_handles[64];
static std::unordered_map<LtKey, LtPlan, LtKeyHash> lt_plans;

// The plan for a key (created on first use; ok == false when hipBLASLt offers no algorithm).
static const LtPlan *lt_plan(const LtKey &k) {
    std::lock_guard<std::mutex> lock(lt_mu);
    auto it = lt_plans.find(k);
    if (it != lt_plans.end()) return &it->second;
    LtPlan &p = lt_plans[k];
    if (!lt_handles[k.dev] && hipblasLtCreate(&lt_handles[k.dev]) != HIPBLAS_STATUS_SUCCESS) {
        lt_handles[k.dev] = nullptr;
        return &p;
    }
    hipblasLtHandle_t h = lt_handles[k.dev];
    // column-major D (N x M) = op(B) (N x K) op(A) (K x M)
    const hipblasOperation_t oa = k.tb ? HIPBLAS_OP_T : HIPBLAS_OP_N, ob = k.ta ? HIPBLAS_OP_T : HIPBLAS_OP_N;
    bool ok = hipblasLtMatmulDescCreate(&p.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F) == HIPBLAS_STATUS_SUCCESS;
    ok = ok && hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &oa, sizeof oa) == HIPBLAS_STATUS_SUCCESS;
    ok = ok && hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &ob, sizeof ob) == HIPBLAS_STATUS_SUCCESS;
    ok = ok && hipblasLtMatrixLayoutCreate(&p.la, HIP_R_32F, k.tb ? k.K : k.N, k.tb ? k.N : k.K, k.ldb) == HIPBLAS_STATUS_SUCCESS;
    ok = ok && hipblasLtMatrixLayoutCreate(&p.lb, HIP_R_32F, k.ta ? k.M : k.K, k.ta ? k.K : k.M, k.lda) == HIPBLAS_STATUS_SUCCESS;
    ok = ok && hipblasLtMatrixLayoutCreate(&p.lc, HIP_R_32F, k.N, k.M, k.ldc) == HIPBLAS_STATUS_SUCCESS;
    if (ok && k.count > 1) {
        const int32_t cnt = (int32_t)k.count;
        const int64_t st[3] = {k.sb, k.sa, k.sc};
        hipblasLtMatrixLayout_t ls[3] = {p.la, p.lb, p.lc};
        for (int i = 0; i < 3 && ok; i++) {
            ok = hipblasLtMatrixLayoutSetAttribute(ls[i], HIPBLASLT_MATRIX_LAYOUT_BATCH_COUNT, &cnt, sizeof cnt) ==
                     HIPBLAS_STATUS_SUCCESS &&
                 hipblasLtMatrixLayoutSetAttribute(ls[i], HIPBLASLT_MATRIX_LAYOUT_STRIDED_BATCH_OFFSET, &st[i],
                                                   sizeof st[i]) == HIPBLAS_STATUS_SUCCESS;
        }
    }
    hipblasLtMatmulPreference_t pref{};
    ok = ok && hipblasLtMatmulPreferenceCreate(&pref) == HIPBLAS_STATUS_SUCCESS;
    const uint64_t no_ws = 0;
    ok = ok && hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &no_ws,
                                                     sizeof no_ws) == HIPBLAS_STATUS_SUCCESS;
    hipblasLtMatmulHeuristicResult_t res{};
    int nres = 0;
    ok = ok && hipblasLtMatmulAlgoGetHeuristic(h, p.desc, p.la, p.lb, p.lc, p.lc, pref, 1, &res, &nres) ==
                   HIPBLAS_STATUS_SUCCESS &&
         nres > 0 && res.workspaceSize == 0;
    if (pref) hipblasLtMatmulPreferenceDestroy(pref);
    if (ok) p.algo = res.algo;
    p.ok = ok;
    return &p;
}

// C = alpha op(A) op(B) + beta C through hipBLASLt (count > 1: strided batch).  Returns false when
// the case is left to rocBLAS: K = 0, a zero or negative batch stride, operands not 16-byte aligned or
// leading dims not multiples of 4, or no algorithm.
static bool lt_gemm(int ta, int tb, int64_t M, int64_t N, int64_t K, float alpha, const float *A, int64_t lda,
                    const float *B, int64_t ldb, float beta, float *C, int64_t ldc, int64_t count, int64_t sa,
                    int64_t sb, int64_t sc, hipStream_t st, int *rc) {
    if (K == 0 || count > INT32_MAX || !aligned16(A) || !aligned16(B) || !aligned16(C) || lda % 4 || ldb % 4 || ldc % 4)
        return false;
    if (count > 1 && (sa <= 0 || sb <= 0 || sc <= 0 || sa % 4 || sb % 4 || sc % 4)) return false;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return false;
    const LtKey key{dev, ta ? 1 : 0, tb ? 1 : 0, M, N, K, lda, ldb, ldc, count, count > 1 ? sa : 0,
                    count > 1 ? sb : 0, count > 1 ? sc : 0};
    const LtPlan *p = lt_plan(key);
    if (!p->ok) return false;
    const hipblasStatus_t s = hipblasLtMatmul(lt_handles[dev], p->desc, &alpha, B, p->la, A, p->lb, &beta, C, p->lc,
                                              C, p->lc, &p->algo, nullptr, 0, st);
    *rc = s == HIPBLAS_STATUS_SUCCESS ? NC_HIP_OK
                                      : set_error(NC_HIP_ERR_DEVICE, "hipBLASLt matmul failed (status %d)", (int)s);
    return true;
}

// With K = 0 no element of A or B is read, but rocBLAS still checks their leading dims against the
// stored shapes (row-major A: M x K, or K x M when transposed); a [M, 0] tensor has leading dim 0.
static void k0_leading_dims(int ta, int tb, int64_t M, int64_t N, int64_t K, int64_t *lda, int64_t *ldb) {
    if (K != 0) return;
    const int64_t need_a = ta ? M : K, need_b = tb ? K : N;
    if (*lda < need_a || *lda < 1) *lda = need_a > 1 ? need_a : 1;
    if (*ldb < need_b || *ldb < 1) *ldb = need_b > 1 ? need_b : 1;
}

}  // namespace nchip

using namespace nchip;

extern "C" NC_HIP_API int nc_hip_gemm_f32(int ta, int tb, int64_t M, int64_t N, int64_t K, float alpha, const float *A,
                                          int64_t lda, const float *B, int64_t ldb, float beta, float *C, int64_t ldc,
                                          void *stream) {
    if (M < 0 || N < 0 || K < 0) return set_error(NC_HIP_ERR_ARG, "nc_hip_gemm_f32: negative size");
    if (M == 0 || N == 0) return NC_HIP_OK;
    int rc = NC_HIP_OK;
    if (lt_gemm(ta, tb, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, 1, 0, 0, 0, as_stream(stream), &rc)) return rc;
    rocblas_handle h = blas_handle();
    if (!h) return set_error(NC_HIP_ERR_DEVICE, "nc_hip_gemm_f32: no rocBLAS handle");
    k0_leading_dims(ta, tb, M, N, K, &lda, &ldb);
    rocblas_status s = rocblas_set_stream(h, as_stream(stream));
    if (s == rocblas_status_success)
        s = rocblas_sgemm_64(h, op_of(tb), op_of(ta), N, M, K, &alpha, B, ldb, A, lda, &beta, C, ldc);
    return s == rocblas_status_success ? NC_HIP_OK : blas_error(s, "nc_hip_gemm_f32");
}

extern "C" NC_HIP_API int nc_hip_gemm_f32_batched(int ta, int tb, int64_t M, int64_t N, int64_t K, float alpha,
                                                  const float *const *A, int64_t lda, const float *const *B,
                                                  int64_t ldb, float beta, float *const *C, int64_t ldc, int64_t count,
                                                  void *stream) {
    if (M < 0 || N < 0 || K < 0 || count < 0) return set_error(NC_HIP_ERR_ARG, "nc_hip_gemm_f32_batched: negative size");
    if (M == 0 || N == 0 || count == 0) return NC_HIP_OK;
    rocblas_handle h = blas_handle();
    if (!h) return set_error(NC_HIP_ERR_DEVICE, "nc_hip_gemm_f32_batched: no rocBLAS handle");
    k0_leading_dims(ta, tb, M, N, K, &lda, &ldb);
    rocblas_status s = rocblas_set_stream(h, as_stream(stream));
    if (s == rocblas_status_success)
        s = rocblas_sgemm_batched_64(h, op_of(tb), op_of(ta), N, M, K, &alpha, B, ldb, A, lda, &beta, C, ldc, count);
    return s == rocblas_status_success ? NC_HIP_OK : blas_error(s, "nc_hip_gemm_f32_batched");
}

// ------------------------------------------------------------------------------------------------
// Batched matmul with broadcast batch dims (ops_linalg.c:89-252): one GEMM per batch matrix, batch
// offsets given per operand as strides over the output's batch shape (0 = broadcast).
// ------------------------------------------------------------------------------------------------
namespace nchip {

struct BatchDims {
    int nb;
    int64_t shape[NC_HIP_MAX_DIMS];
    int64_t st[3][NC_HIP_MAX_DIMS];  // A, B, C
};

__global__ void k_batch_ptrs(const float *A, const float *B, float *C, BatchDims bd, int64_t count,
                             const float **pa, const float **pb, float **pc) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= count) return;
    int64_t idx = i, oa = 0, ob = 0, oc = 0;
    for (int d = bd.nb - 1; d >= 0; d--) {
        const int64_t c = idx % bd.shape[d];
        idx /= bd.shape[d];
        oa += c * bd.st[0][d];
        ob += c * bd.st[1][d];
        oc += c * bd.st[2][d];
    }
    pa[i] = A + oa;
    pb[i] = B + ob;
    pc[i] = C + oc;
}

// drops size-1 batch dims and merges neighbours that step uniformly for all three operands
static void coalesce_batch(BatchDims &bd) {
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

// true when batch index idx is the first (in index order) to write its C block: zero on every dim
// along which C is shared
static bool first_writer(const BatchDims &bd, int64_t idx) {
    for (int d = bd.nb - 1; d >= 0; d--) {
        if (bd.st[2][d] == 0 && idx % bd.shape[d] != 0) return false;
        idx /= bd.shape[d];
    }
    return true;
}

static int64_t batch_offset(const BatchDims &bd, int o, int64_t idx) {
    int64_t off = 0;
    for (int d = bd.nb - 1; d >= 0; d--) {
        off += (idx % bd.shape[d]) * bd.st[o][d];
        idx /= bd.shape[d];
    }
    return off;
}

}  // namespace nchip

extern "C" NC_HIP_API size_t nc_hip_gemm_f32_bmm_workspace(int64_t count) {
    return count > 1 ? (size_t)count * 3 * sizeof(void *) : 0;
}

extern "C" NC_HIP_API int nc_hip_gemm_f32_bmm(int ta, int tb, int64_t M, int64_t N, int64_t K, const float *A,
                                              int64_t lda, const float *B, int64_t ldb, float beta, float *C,
                                              int64_t ldc, int nb, const int64_t *bshape, const int64_t *sa,
                                              const int64_t *sb, const int64_t *sc, void *ws, size_t ws_bytes,
                                              void *stream) {
    if (M < 0 || N < 0 || K < 0 || nb < 0 || nb > NC_HIP_MAX_DIMS)
        return set_error(NC_HIP_ERR_ARG, "nc_hip_gemm_f32_bmm: bad sizes");
    BatchDims bd;
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
    coalesce_batch(bd);
    const float one = 1.0f;
    bool c_shared = false;  // several batch matrices accumulate into one C block
    for (int d = 0; d < bd.nb; d++) c_shared = c_shared || bd.st[2][d] == 0;
    if (bd.nb == 0) return nc_hip_gemm_f32(ta, tb, M, N, K, one, A, lda, B, ldb, beta, C, ldc, stream);
    if (c_shared) {
        // ordered: batch index order, each GEMM after a block's first adding into what the earlier ones wrote
        for (int64_t i = 0; i < count; i++) {
            const int rc = nc_hip_gemm_f32(ta, tb, M, N, K, one, A + batch_offset(bd, 0, i), lda,
                                           B + batch_offset(bd, 1, i), ldb, first_writer(bd, i) ? beta : 1.0f,
                                           C + batch_offset(bd, 2, i), ldc, stream);
            if (rc != NC_HIP_OK) return rc;
        }
        return NC_HIP_OK;
    }
    k0_leading_dims(ta, tb, M, N, K, &lda, &ldb);
    if (bd.nb == 1) {
        int rc = NC_HIP_OK;
        if (lt_gemm(ta, tb, M, N, K, one, A, lda, B, ldb, beta, C, ldc, count, bd.st[0][0], bd.st[1][0], bd.st[2][0],
                    as_stream(stream), &rc))
            return rc;
    }
    rocblas_handle h = blas_handle();
    if (!h) return set_error(NC_HIP_ERR_DEVICE, "nc_hip_gemm_f32_bmm: no rocBLAS handle");
    rocblas_status s = rocblas_set_stream(h, as_stream(stream));
    if (s != rocblas_status_success) return blas_error(s, "nc_hip_gemm_f32_bmm");
    if (bd.nb == 1) {
        s = rocblas_sgemm_strided_batched_64(h, op_of(tb), op_of(ta), N, M, K, &one, B, ldb, bd.st[1][0], A, lda,
                                             bd.st[0][0], &beta, C, ldc, bd.st[2][0], count);
        return s == rocblas_status_success ? NC_HIP_OK : blas_error(s, "nc_hip_gemm_f32_bmm");
    }
    if (ws_bytes < nc_hip_gemm_f32_bmm_workspace(count) || !ws)
        return set_error(NC_HIP_ERR_ARG, "nc_hip_gemm_f32_bmm: workspace of %zu bytes, need %zu", ws_bytes,
                         nc_hip_gemm_f32_bmm_workspace(count));
    const float **pa = (const float **)ws;
    const float **pb = pa + count;
    float **pc = (float **)(pb + count);
    hipLaunchKernelGGL(k_batch_ptrs, dim3((unsigned)((count + 255) / 256)), dim3(256), 0, as_stream(stream), A, B, C,
                       bd, count, pa, pb, pc);
    if (int rc = check_launch("nc_hip_gemm_f32_bmm")) return rc;
    s = rocblas_sgemm_batched_64(h, op_of(tb), op_of(ta), N, M, K, &one, pb, ldb, pa, lda, &beta, pc, ldc, count);
    return s == rocblas_status_success ? NC_HIP_OK : blas_error(s, "nc_hip_gemm_f32_bmm");
}
