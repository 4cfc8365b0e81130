// Dense linear algebra: matmul, batched matmul with broadcast batch dims, linear.  Reference:
// engine/src/ops/ops_linalg.c.  Every contraction is an fp32 GEMM on the matrix cores
// (nc_hip_gemm_f32 / nc_hip_gemm_f32_bmm); 2-D operands that are transposed views go to the GEMM as
// transpose flags with their own leading dim instead of being gathered (ops_linalg.c:17-27), anything
// else is gathered once into a contiguous arena copy.  Gradients accumulate through the GEMM's beta
// (0 while a grad buffer is fresh, 1 after), so no zero pass precedes them.
#include "engine.hpp"

using namespace nce;

namespace {

struct GemmOperand {
    const float *p;
    int trans;
    int64_t ld;
};

// rows x cols logical matrix held by a 2-D t (ops_linalg.c:17-27)
bool as_gemm(nc_tensor *t, int64_t rows, int64_t cols, GemmOperand *g) {
    if (t->ndim == 2 && t->stride[1] == 1 && t->stride[0] >= cols) {
        *g = {fptr(t), 0, t->stride[0]};
    } else if (t->ndim == 2 && t->stride[0] == 1 && t->stride[1] >= rows) {
        *g = {fptr(t), 1, t->stride[1]};
    } else {
        *g = {contig_f32(t), 0, cols};
    }
    return g->p != nullptr;
}

// a [..., M, K]: 2-D through as_gemm, otherwise leading dims folded into M (ops_linalg.c:52-56)
bool a_operand(nc_tensor *a, int64_t M, int64_t K, GemmOperand *g) {
    if (a->ndim == 2) return as_gemm(a, M, K, g);
    *g = {contig_f32(a), 0, K};
    return g->p != nullptr;
}

bool gemm(nc_ctx *ctx, int ta, int tb, int64_t M, int64_t N, int64_t K, const float *A, int64_t lda,
          const float *B, int64_t ldb, float beta, float *C, int64_t ldc, const char *what) {
    return hip_layer_ok(ctx, nc_hip_gemm_f32(ta, tb, M, N, K, 1.0f, A, lda, B, ldb, beta, C, ldc, stream(ctx)), what);
}

// ---- matmul: a [..., M, K] @ b [K, N] ------------------------------------------------------------
nc_status matmul_infer(nc_node *n, nc_dtype *dt, int *nd, int64_t *shape) {
    nc_tensor *a = n->in[0], *b = n->in[1];
    if (!expect_f32(n, 0) || !expect_f32(n, 1)) return NC_ERR_DTYPE;
    if (a->ndim < 2 || b->ndim != 2 || a->shape[a->ndim - 1] != b->shape[0]) {
        char sa[96], sb[96];
        error(a->ctx, NC_ERR_SHAPE, "matmul: cannot multiply %s by %s (expected [..., M, K] @ [K, N])",
              shape_str(a->ndim, a->shape, sa, sizeof sa), shape_str(b->ndim, b->shape, sb, sizeof sb));
        return NC_ERR_SHAPE;
    }
    *dt = NC_F32;
    *nd = a->ndim;
    memcpy(shape, a->shape, sizeof(int64_t) * (size_t)a->ndim);
    shape[a->ndim - 1] = b->shape[1];
    return NC_OK;
}

void mm_dims(const nc_node *n, int64_t *M, int64_t *K, int64_t *N) {
    *K = n->in[1]->shape[0];
    *N = n->in[1]->shape[1];
    *M = nc_numel(n->in[0]) / (*K ? *K : 1);
}

nc_status matmul_fwd(nc_node *n) {
    nc_ctx *ctx = n->out->ctx;
    int64_t M, K, N;
    mm_dims(n, &M, &K, &N);
    GemmOperand A, B;
    float *C = fptr(n->out);
    if (!a_operand(n->in[0], M, K, &A) || !as_gemm(n->in[1], K, N, &B) || !C) return NC_ERR_STATE;
    if (!gemm(ctx, A.trans, B.trans, M, N, K, A.p, A.ld, B.p, B.ld, 0.0f, C, N, "matmul")) return NC_ERR_STATE;
    wrote_dev(n->out);
    return NC_OK;
}

void matmul_bwd(nc_node *n) {
    nc_tensor *a = n->in[0], *b = n->in[1];
    nc_ctx *ctx = a->ctx;
    int64_t M, K, N;
    mm_dims(n, &M, &K, &N);
    const float *g = fptr(n->out->grad);  // M x N
    if (!g) return;
    if (needs_grad(a) && grad_buf(a)) {  // dA (M x K) (+)= dC @ B^T
        GemmOperand B;
        const float beta = grad_acc(a) ? 1.0f : 0.0f;
        float *ga = fptr(a->grad);
        if (ga && as_gemm(b, K, N, &B) && gemm(ctx, 0, !B.trans, M, K, N, g, N, B.p, B.ld, beta, ga, K, "matmul"))
            wrote_dev(a->grad);
    }
    if (needs_grad(b) && grad_buf(b)) {  // dB (K x N) (+)= A^T @ dC
        GemmOperand A;
        const float beta = grad_acc(b) ? 1.0f : 0.0f;
        float *gb = fptr(b->grad);
        if (gb && a_operand(a, M, K, &A) && gemm(ctx, !A.trans, 0, K, N, M, A.p, A.ld, g, N, beta, gb, N, "matmul"))
            wrote_dev(b->grad);
    }
}

const OpDef op_matmul = {"matmul", 0, 0, matmul_infer, nullptr, matmul_fwd, matmul_bwd};

// ---- batched matmul: a [..., M, K] @ b [..., K, N], broadcast batch dims (ops_linalg.c:89-252) ----
struct BatchDims {
    int nb;
    int64_t shape[NC_MAX_DIMS];
    int64_t count;
};

bool batch_shape(const nc_tensor *a, const nc_tensor *b, BatchDims *bd) {
    const int na = a->ndim - 2, nb = b->ndim - 2;
    bd->nb = na > nb ? na : nb;
    bd->count = 1;
    for (int i = 0; i < bd->nb; i++) {
        const int ia = i - (bd->nb - na), ib = i - (bd->nb - nb);
        const int64_t da = ia < 0 ? 1 : a->shape[ia], db = ib < 0 ? 1 : b->shape[ib];
        if (da != db && da != 1 && db != 1) return false;
        bd->shape[i] = da == 1 ? db : da;
        bd->count *= bd->shape[i];
    }
    return true;
}

// element stride of t's batch matrices along each output batch dim (0 = broadcast)
void batch_strides(const nc_tensor *t, const int64_t *st, const BatchDims &bd, int64_t *out) {
    const int tb = t->ndim - 2;
    for (int i = 0; i < bd.nb; i++) {
        const int j = i - (bd.nb - tb);
        out[i] = (j < 0 || t->shape[j] == 1) ? 0 : st[j];
    }
}

struct BmmOperand {
    const float *p;
    int trans;
    int64_t ld;
    int64_t bst[NC_MAX_DIMS];
};

bool bmm_operand(nc_tensor *t, const BatchDims &bd, BmmOperand *o) {
    const int nd = t->ndim;
    const int64_t rows = t->shape[nd - 2], cols = t->shape[nd - 1];
    const int64_t *st = t->stride;
    int64_t cs[NC_MAX_DIMS];
    if (t->stride[nd - 1] == 1 && t->stride[nd - 2] >= cols) {
        o->p = fptr(t), o->trans = 0, o->ld = t->stride[nd - 2];
    } else if (t->stride[nd - 2] == 1 && t->stride[nd - 1] >= rows) {
        o->p = fptr(t), o->trans = 1, o->ld = t->stride[nd - 1];
    } else {
        o->p = contig_f32(t), o->trans = 0, o->ld = cols;
        contig_strides(nd, t->shape, cs);
        st = cs;
    }
    batch_strides(t, st, bd, o->bst);
    return o->p != nullptr;
}

nc_status bmm_infer(nc_node *n, nc_dtype *dt, int *nd, int64_t *shape) {
    nc_tensor *a = n->in[0], *b = n->in[1];
    BatchDims bd;
    if (!expect_f32(n, 0) || !expect_f32(n, 1)) return NC_ERR_DTYPE;
    if (a->ndim < 2 || b->ndim < 2 || a->shape[a->ndim - 1] != b->shape[b->ndim - 2] || !batch_shape(a, b, &bd)) {
        char sa[96], sb[96];
        error(a->ctx, NC_ERR_SHAPE, "matmul: cannot multiply %s by %s (expected [..., M, K] @ [..., K, N])",
              shape_str(a->ndim, a->shape, sa, sizeof sa), shape_str(b->ndim, b->shape, sb, sizeof sb));
        return NC_ERR_SHAPE;
    }
    *dt = NC_F32;
    *nd = bd.nb + 2;
    memcpy(shape, bd.shape, sizeof(int64_t) * (size_t)bd.nb);
    shape[bd.nb] = a->shape[a->ndim - 2];
    shape[bd.nb + 1] = b->shape[b->ndim - 1];
    return NC_OK;
}

bool bmm_run(nc_ctx *ctx, const BatchDims &bd, int ta, int tb, int64_t M, int64_t N, int64_t K, const float *A,
             int64_t lda, const int64_t *sa, const float *B, int64_t ldb, const int64_t *sb, float beta, float *C,
             int64_t ldc, const int64_t *sc) {
    const size_t ws_bytes = nc_hip_gemm_f32_bmm_workspace(bd.count);
    char *ws = ws_bytes ? arena_alloc(ctx, ws_bytes) : nullptr;
    if (ws_bytes && !ws) return false;
    return hip_layer_ok(ctx,
                        nc_hip_gemm_f32_bmm(ta, tb, M, N, K, A, lda, B, ldb, beta, C, ldc, bd.nb, bd.shape, sa, sb,
                                            sc, ws, ws_bytes, stream(ctx)),
                        "matmul");
}

nc_status bmm_fwd(nc_node *n) {
    nc_tensor *a = n->in[0], *b = n->in[1], *o = n->out;
    BatchDims bd;
    batch_shape(a, b, &bd);
    BmmOperand A, B;
    float *C = fptr(o);
    if (!bmm_operand(a, bd, &A) || !bmm_operand(b, bd, &B) || !C) return NC_ERR_STATE;
    const int64_t M = o->shape[bd.nb], N = o->shape[bd.nb + 1], K = a->shape[a->ndim - 1];
    int64_t sc[NC_MAX_DIMS];
    batch_strides(o, o->stride, bd, sc);
    if (!bmm_run(o->ctx, bd, A.trans, B.trans, M, N, K, A.p, A.ld, A.bst, B.p, B.ld, B.bst, 0.0f, C, N, sc))
        return NC_ERR_STATE;
    wrote_dev(o);
    return NC_OK;
}

void bmm_bwd(nc_node *n) {
    nc_tensor *a = n->in[0], *b = n->in[1], *o = n->out;
    nc_ctx *ctx = o->ctx;
    BatchDims bd;
    batch_shape(a, b, &bd);
    const int64_t M = o->shape[bd.nb], N = o->shape[bd.nb + 1], K = a->shape[a->ndim - 1];
    const float *g = fptr(o->grad);
    if (!g) return;
    int64_t cs[NC_MAX_DIMS], sg[NC_MAX_DIMS], sgrad[NC_MAX_DIMS];
    contig_strides(o->ndim, o->shape, cs);
    batch_strides(o, cs, bd, sg);
    if (needs_grad(a) && grad_buf(a)) {  // dA_i (M x K) (+)= dC_i @ B_i^T
        BmmOperand B;
        const float beta = grad_acc(a) ? 1.0f : 0.0f;
        float *ga = fptr(a->grad);
        contig_strides(a->ndim, a->shape, cs);
        batch_strides(a, cs, bd, sgrad);
        if (ga && bmm_operand(b, bd, &B) &&
            bmm_run(ctx, bd, 0, !B.trans, M, K, N, g, N, sg, B.p, B.ld, B.bst, beta, ga, K, sgrad))
            wrote_dev(a->grad);
    }
    if (needs_grad(b) && grad_buf(b)) {  // dB_i (K x N) (+)= A_i^T @ dC_i
        BmmOperand A;
        const float beta = grad_acc(b) ? 1.0f : 0.0f;
        float *gb = fptr(b->grad);
        contig_strides(b->ndim, b->shape, cs);
        batch_strides(b, cs, bd, sgrad);
        if (gb && bmm_operand(a, bd, &A) &&
            bmm_run(ctx, bd, !A.trans, 0, K, N, M, A.p, A.ld, A.bst, g, N, sg, beta, gb, N, sgrad))
            wrote_dev(b->grad);
    }
}

const OpDef op_bmm = {"bmm", 0, 0, bmm_infer, nullptr, bmm_fwd, bmm_bwd};

// ---- linear: y = x @ W^T + b, W [out, in] (ops_linalg.c:255-338) ---------------------------------
nc_status linear_infer(nc_node *n, nc_dtype *dt, int *nd, int64_t *shape) {
    nc_tensor *x = n->in[0], *w = n->in[1], *b = n->n_in > 2 ? n->in[2] : nullptr;
    for (int i = 0; i < n->n_in; i++)
        if (!expect_f32(n, i)) return NC_ERR_DTYPE;
    if (x->ndim < 1 || w->ndim != 2 || x->shape[x->ndim - 1] != w->shape[1] ||
        (b && (b->ndim != 1 || b->shape[0] != w->shape[0]))) {
        char sx[96], sw[96], sb[96] = "none";
        if (b) shape_str(b->ndim, b->shape, sb, sizeof sb);
        error(x->ctx, NC_ERR_SHAPE, "linear: expected x [..., in], weight [out, in], bias [out]; got %s, %s, %s",
              shape_str(x->ndim, x->shape, sx, sizeof sx), shape_str(w->ndim, w->shape, sw, sizeof sw), sb);
        return NC_ERR_SHAPE;
    }
    *dt = NC_F32;
    *nd = x->ndim;
    memcpy(shape, x->shape, sizeof(int64_t) * (size_t)x->ndim);
    shape[x->ndim - 1] = w->shape[0];
    return NC_OK;
}

nc_status linear_fwd(nc_node *n) {
    nc_tensor *x = n->in[0], *w = n->in[1], *b = n->n_in > 2 ? n->in[2] : nullptr;
    nc_ctx *ctx = x->ctx;
    const int64_t in = w->shape[1], out = w->shape[0], M = in ? nc_numel(x) / in : 0;
    const float *X = contig_f32(x), *W = contig_f32(w), *B = b ? contig_f32(b) : nullptr;
    float *Y = fptr(n->out);
    if (!X || !W || (b && !B) || !Y) return NC_ERR_STATE;
    if (!gemm(ctx, 0, 1, M, out, in, X, in, W, in, 0.0f, Y, out, "linear")) return NC_ERR_STATE;
    if (B && M > 0 && out > 0) {  // y = (x W^T) + b, one rounding of the sum as the reference's beta = 1 pass
        const int64_t shape[2] = {M, out}, sy[2] = {out, 1}, sbias[2] = {0, 1};
        if (!hip_layer_ok(ctx, nc_hip_binary_fwd(NC_HIP_BIN_ADD, 2, shape, Y, sy, B, sbias, Y, sy, stream(ctx)),
                          "linear"))
            return NC_ERR_STATE;
    }
    wrote_dev(n->out);
    return NC_OK;
}

void linear_bwd(nc_node *n) {
    nc_tensor *x = n->in[0], *w = n->in[1], *b = n->n_in > 2 ? n->in[2] : nullptr;
    nc_ctx *ctx = x->ctx;
    const int64_t in = w->shape[1], out = w->shape[0], M = in ? nc_numel(x) / in : 0;
    const float *g = fptr(n->out->grad);  // M x out
    if (!g) return;
    if (needs_grad(x) && grad_buf(x)) {  // dX (M x in) (+)= dY @ W
        const float beta = grad_acc(x) ? 1.0f : 0.0f;
        const float *W = contig_f32(w);
        float *gx = fptr(x->grad);
        if (W && gx && gemm(ctx, 0, 0, M, in, out, g, out, W, in, beta, gx, in, "linear")) wrote_dev(x->grad);
    }
    if (needs_grad(w) && grad_buf(w)) {  // dW (out x in) (+)= dY^T @ X
        const float beta = grad_acc(w) ? 1.0f : 0.0f;
        const float *X = contig_f32(x);
        float *gw = fptr(w->grad);
        if (X && gw && gemm(ctx, 1, 0, out, in, M, g, out, X, in, beta, gw, in, "linear")) wrote_dev(w->grad);
    }
    if (b && needs_grad(b) && grad_buf(b)) {  // db (+)= column sums of dY, fp64 in a fixed order
        const int acc = grad_acc(b);
        float *gb = fptr(b->grad);
        if (!gb) return;
        const int64_t shape[2] = {M, out}, sg[2] = {out, 1}, sgb[2] = {0, 1};
        const size_t ws_bytes = nc_hip_binary_bwd_workspace(2, shape, sgb);
        char *ws = ws_bytes ? arena_alloc(ctx, ws_bytes) : nullptr;
        if (ws_bytes && !ws) return;
        if (hip_layer_ok(ctx,
                         nc_hip_binary_bwd(NC_HIP_BIN_ADD, 1, 2, shape, g, sg, g, sg, gb, sgb, gb, sgb, acc, ws,
                                           ws_bytes, stream(ctx)),
                         "linear"))
            wrote_dev(b->grad);
    }
}

const OpDef op_linear = {"linear", 0, 0, linear_infer, nullptr, linear_fwd, linear_bwd};

}  // namespace

extern "C" {

nc_tensor *nc_matmul(nc_tensor *a, nc_tensor *b) {
    nc_tensor *in[2] = {a, b};
    return apply(b && b->ndim > 2 ? &op_bmm : &op_matmul, in, 2, nullptr);
}

nc_tensor *nc_linear_fn(nc_tensor *x, nc_tensor *weight, nc_tensor *bias) {
    nc_tensor *in[3] = {x, weight, bias};
    return apply(&op_linear, in, bias ? 3 : 2, nullptr);
}

}  // extern "C"
