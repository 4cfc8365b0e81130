// Dense linear algebra: matmul (2-D right operand), batched matmul with broadcast batch axes, and
// linear.  Reference: engine/src/ops/ops_linalg.c (matmul :40-88, batched :89-252, linear :255-338);
// output shapes and error messages are the reference's.
//
// All three ops, forward and backward, are one thing here: a Product C = A @ B over optional batch
// axes, run as an fp32 GEMM on the device (nc_hip_gemm_f32, or nc_hip_gemm_f32_bmm with per-axis
// batch strides).  Operands go to the GEMM in place whenever their strides allow it -- a transposed
// view is a transpose flag, evenly spaced rows a leading dimension, a broadcast batch axis a zero batch
// stride -- and are packed once into a scratch copy otherwise.  A gradient product is the forward
// product with one operand replaced by the output gradient and the other transposed (its flag flipped,
// no copy); it accumulates through the GEMM's beta (0 while the gradient buffer is fresh, 1 after).
#include "engine.hpp"

namespace nce {
namespace {

// A matrix as the GEMM reads it: element (r, c) at p[r * ld + c], or at p[c * ld + r] when trans.
struct Mat {
    const float *p = nullptr;
    int trans = 0;
    int64_t ld = 0;
    Mat t() const { return {p, trans ^ 1, ld}; }  // the transpose: same memory, other order
};

// One operand of a batched product: its matrix and, per output batch axis, the element step from one
// batch matrix to the next (0 where the operand is broadcast).
struct Operand {
    Mat m;
    int64_t bst[NC_MAX_DIMS] = {};
    Operand transposed() const {
        Operand o = *this;
        o.m = m.t();
        return o;
    }
};

// t's last two axes [rows, cols] in place when one of them is unit-stride and the other steps over
// at least a whole line; packed row-major otherwise.  *strides: the strides the matrix was taken with.
bool last_two(nc_tensor *t, Mat &m, const int64_t **strides, int64_t *packed) {
    const int nd = t->ndim;
    const int64_t rows = t->shape[nd - 2], cols = t->shape[nd - 1];
    const int64_t sr = t->stride[nd - 2], sc = t->stride[nd - 1];
    *strides = t->stride;
    if (sc == 1 && sr >= cols) {
        m = {fptr(t), 0, sr};
    } else if (sr == 1 && sc >= rows) {
        m = {fptr(t), 1, sc};
    } else {
        contig_strides(nd, t->shape, packed);
        *strides = packed;
        m = {contig_f32(t), 0, cols};
    }
    return m.p != nullptr;
}

// t [..., M, K] as one [rows, K] matrix: in place when it is unit-stride along K and each leading axis
// steps over whole blocks of evenly spaced rows, packed otherwise (a 2-D t may be a transposed view).
bool as_rows(nc_tensor *t, Mat &m) {
    const int nd = t->ndim;
    const int64_t K = t->shape[nd - 1];
    if (nd == 1) {
        m = {contig_f32(t), 0, K};
        return m.p != nullptr;
    }
    int64_t packed[NC_MAX_DIMS];
    const int64_t *unused;
    if (nd == 2) return last_two(t, m, &unused, packed);
    const int64_t step = t->stride[nd - 2];
    bool even = (t->stride[nd - 1] == 1 || K <= 1) && step >= K;
    int64_t rows = t->shape[nd - 2];
    for (int i = nd - 3; even && i >= 0; i--) {
        if (t->shape[i] == 1) continue;
        even = t->stride[i] == rows * step;
        rows *= t->shape[i];
    }
    m = even ? Mat{fptr(t), 0, step} : Mat{contig_f32(t), 0, K};
    return m.p != nullptr;
}

// the batch step of a tensor with `strides` along each axis of `batch` (its leading axes aligned at the
// right; an axis of extent 1 against a larger batch axis is broadcast)
void batch_steps(const nc_tensor *t, const int64_t *strides, const Dims &batch, int64_t *out) {
    const int lead = t->ndim - 2;
    for (int i = 0; i < batch.rank; i++) {
        const int j = i - (batch.rank - lead);
        out[i] = (j < 0 || t->shape[j] == 1) ? 0 : strides[j];
    }
}

// a batched-product operand: last two axes as a Mat, leading axes as batch steps
bool batch_operand(nc_tensor *t, const Dims &batch, Operand &o) {
    int64_t packed[NC_MAX_DIMS];
    const int64_t *strides;
    if (!last_two(t, o.m, &strides, packed)) return false;
    batch_steps(t, strides, batch, o.bst);
    return true;
}

// the batch steps of t's (contiguous) gradient buffer: a broadcast axis steps 0, so the GEMM layer
// adds every batch's product into the same gradient matrix
void grad_steps(const nc_tensor *t, const Dims &batch, int64_t *out) {
    int64_t cs[NC_MAX_DIMS];
    contig_strides(t->ndim, t->shape, cs);
    batch_steps(t, cs, batch, out);
}

// C (+)= A @ B, A [M, K], B [K, N], C [M, N] with leading dim ldc; batched when batch has axes.  bias
// (one matrix, beta 0): N floats added to every row of the product in the same pass.
bool product(nc_ctx *ctx, const Dims &batch, int64_t M, int64_t N, int64_t K, const Operand &a, const Operand &b,
             float beta, float *C, int64_t ldc, const int64_t *cst, const char *what, const float *bias = nullptr) {
    if (batch.rank == 0 && bias)
        return hip_layer_ok(ctx,
                            nc_hip_gemm_f32_bias(a.m.trans, b.m.trans, M, N, K, 1.0f, a.m.p, a.m.ld, b.m.p, b.m.ld,
                                                 bias, C, ldc, stream(ctx)),
                            what);
    if (batch.rank == 0)
        return hip_layer_ok(ctx,
                            nc_hip_gemm_f32(a.m.trans, b.m.trans, M, N, K, 1.0f, a.m.p, a.m.ld, b.m.p, b.m.ld, beta, C,
                                            ldc, stream(ctx)),
                            what);
    const size_t ws_bytes = nc_hip_gemm_f32_bmm_workspace(batch.numel());
    char *ws = ws_bytes ? arena_alloc(ctx, ws_bytes) : nullptr;
    if (ws_bytes && !ws) return false;
    return hip_layer_ok(ctx,
                        nc_hip_gemm_f32_bmm(a.m.trans, b.m.trans, M, N, K, a.m.p, a.m.ld, b.m.p, b.m.ld, beta, C, ldc,
                                            batch.rank, batch.e, a.bst, b.bst, cst, ws, ws_bytes, stream(ctx)),
                        what);
}

// the product of all but the last axis
int64_t leading_rows(const nc_tensor *t) {
    int64_t r = 1;
    for (int i = 0; i + 1 < t->ndim; i++) r *= t->shape[i];
    return r;
}

// gradient buffer of x for a product about to write it: its address and the GEMM beta
float *grad_target(nc_tensor *x, float *beta) {
    if (!grad_buf(x)) return nullptr;
    *beta = grad_acc(x) ? 1.0f : 0.0f;
    return fptr(x->grad);
}

// a dense row-major [rows, cols] matrix (an output gradient)
Operand dense(const float *p, int64_t cols) {
    Operand o;
    o.m = {p, 0, cols};
    return o;
}

// ---- matmul: a [..., M, K] @ b [K, N]; a's leading axes fold into M -------------------------------
nc_status matmul_shape(nc_node *n, OutSpec &out) {
    if (!inputs_f32(n, 0, 2)) return NC_ERR_DTYPE;
    const Dims a = Dims::of(n->in[0]), b = Dims::of(n->in[1]);
    if (a.rank < 2 || b.rank != 2 || a.back(0) != b.e[0]) {
        char ta[96], tb[96];
        return reject(n, NC_ERR_SHAPE, "matmul: cannot multiply %s by %s (expected [..., M, K] @ [K, N])",
                      a.text(ta, sizeof ta), b.text(tb, sizeof tb));
    }
    out.dims = a;
    out.dims.e[a.rank - 1] = b.e[1];
    return NC_OK;
}

struct Mnk {
    int64_t M, N, K;
};

Mnk matmul_mnk(const nc_node *n) { return {leading_rows(n->in[0]), n->in[1]->shape[1], n->in[1]->shape[0]}; }

nc_status matmul_fwd(nc_node *n) {
    const Mnk d = matmul_mnk(n);
    Operand a, b;
    const int64_t *unused;
    int64_t packed[NC_MAX_DIMS];
    float *C = fptr(n->out);
    if (!as_rows(n->in[0], a.m) || !last_two(n->in[1], b.m, &unused, packed) || !C) return NC_ERR_STATE;
    if (!product(n->out->ctx, Dims{}, d.M, d.N, d.K, a, b, 0.0f, C, d.N, nullptr, "matmul")) return NC_ERR_STATE;
    wrote_dev(n->out);
    return NC_OK;
}

void matmul_bwd(nc_node *n) {
    nc_tensor *at = n->in[0], *bt = n->in[1];
    nc_ctx *ctx = at->ctx;
    const Mnk d = matmul_mnk(n);
    const float *g = fptr(n->out->grad);  // [M, N]
    if (!g) return;
    float beta;
    const int64_t *unused;
    int64_t packed[NC_MAX_DIMS];
    if (needs_grad(at)) {  // dA [M, K] (+)= G @ B^T
        Operand b;
        float *ga = grad_target(at, &beta);
        if (ga && last_two(bt, b.m, &unused, packed) &&
            product(ctx, Dims{}, d.M, d.K, d.N, dense(g, d.N), b.transposed(), beta, ga, d.K, nullptr, "matmul"))
            wrote_dev(at->grad);
    }
    if (needs_grad(bt)) {  // dB [K, N] (+)= A^T @ G
        Operand a;
        float *gb = grad_target(bt, &beta);
        if (gb && as_rows(at, a.m) &&
            product(ctx, Dims{}, d.K, d.N, d.M, a.transposed(), dense(g, d.N), beta, gb, d.N, nullptr, "matmul"))
            wrote_dev(bt->grad);
    }
}

const OpDef op_matmul = {"matmul", 0, 0, matmul_shape, nullptr, matmul_fwd, matmul_bwd};

// ---- batched matmul: a [..., M, K] @ b [..., K, N], batch axes broadcast ----------------------------
// the broadcast of a's and b's leading axes, false when they do not broadcast
bool batch_of(const nc_tensor *a, const nc_tensor *b, Dims &batch) {
    const int la = a->ndim - 2, lb = b->ndim - 2;
    batch.rank = la > lb ? la : lb;
    for (int k = 0; k < batch.rank; k++) {  // k-th batch axis from the last
        const int64_t ea = k < la ? a->shape[la - 1 - k] : 1, eb = k < lb ? b->shape[lb - 1 - k] : 1;
        if (ea != eb && ea != 1 && eb != 1) return false;
        batch.e[batch.rank - 1 - k] = ea == 1 ? eb : ea;
    }
    return true;
}

nc_status bmm_shape(nc_node *n, OutSpec &out) {
    if (!inputs_f32(n, 0, 2)) return NC_ERR_DTYPE;
    const Dims a = Dims::of(n->in[0]), b = Dims::of(n->in[1]);
    if (a.rank < 2 || b.rank < 2 || a.back(0) != b.back(1) || !batch_of(n->in[0], n->in[1], out.dims)) {
        char ta[96], tb[96];
        return reject(n, NC_ERR_SHAPE, "matmul: cannot multiply %s by %s (expected [..., M, K] @ [..., K, N])",
                      a.text(ta, sizeof ta), b.text(tb, sizeof tb));
    }
    out.dims.push(a.back(1));
    out.dims.push(b.back(0));
    return NC_OK;
}

nc_status bmm_fwd(nc_node *n) {
    nc_tensor *at = n->in[0], *bt = n->in[1], *o = n->out;
    Dims batch;
    batch_of(at, bt, batch);
    const int64_t M = at->shape[at->ndim - 2], K = at->shape[at->ndim - 1], N = bt->shape[bt->ndim - 1];
    Operand a, b;
    int64_t cst[NC_MAX_DIMS];
    batch_steps(o, o->stride, batch, cst);
    float *C = fptr(o);
    if (!batch_operand(at, batch, a) || !batch_operand(bt, batch, b) || !C) return NC_ERR_STATE;
    if (!product(o->ctx, batch, M, N, K, a, b, 0.0f, C, N, cst, "matmul")) return NC_ERR_STATE;
    wrote_dev(o);
    return NC_OK;
}

void bmm_bwd(nc_node *n) {
    nc_tensor *at = n->in[0], *bt = n->in[1], *o = n->out;
    nc_ctx *ctx = o->ctx;
    Dims batch;
    batch_of(at, bt, batch);
    const int64_t M = at->shape[at->ndim - 2], K = at->shape[at->ndim - 1], N = bt->shape[bt->ndim - 1];
    Operand g = dense(fptr(o->grad), N);
    if (!g.m.p) return;
    grad_steps(o, batch, g.bst);
    float beta;
    int64_t gst[NC_MAX_DIMS];
    if (needs_grad(at)) {  // dA_i [M, K] (+)= G_i @ B_i^T
        Operand b;
        float *ga = grad_target(at, &beta);
        grad_steps(at, batch, gst);
        if (ga && batch_operand(bt, batch, b) && product(ctx, batch, M, K, N, g, b.transposed(), beta, ga, K, gst, "matmul"))
            wrote_dev(at->grad);
    }
    if (needs_grad(bt)) {  // dB_i [K, N] (+)= A_i^T @ G_i
        Operand a;
        float *gb = grad_target(bt, &beta);
        grad_steps(bt, batch, gst);
        if (gb && batch_operand(at, batch, a) && product(ctx, batch, K, N, M, a.transposed(), g, beta, gb, N, gst, "matmul"))
            wrote_dev(bt->grad);
    }
}

const OpDef op_bmm = {"bmm", 0, 0, bmm_shape, nullptr, bmm_fwd, bmm_bwd};

// ---- linear: y = x @ W^T + b, x [..., in], W [out, in], b [out] -----------------------------------------
nc_status linear_shape(nc_node *n, OutSpec &out) {
    if (!inputs_f32(n, 0, n->n_in)) return NC_ERR_DTYPE;
    const bool has_b = n->n_in > 2;
    const Dims x = Dims::of(n->in[0]), w = Dims::of(n->in[1]), b = has_b ? Dims::of(n->in[2]) : Dims{};
    if (x.rank < 1 || w.rank != 2 || x.back(0) != w.e[1] || (has_b && (b.rank != 1 || b.e[0] != w.e[0]))) {
        char tx[96], tw[96], tb[96] = "none";
        if (has_b) b.text(tb, sizeof tb);
        return reject(n, NC_ERR_SHAPE, "linear: expected x [..., in], weight [out, in], bias [out]; got %s, %s, %s",
                      x.text(tx, sizeof tx), w.text(tw, sizeof tw), tb);
    }
    out.dims = x;
    out.dims.e[x.rank - 1] = w.e[0];
    return NC_OK;
}

nc_status linear_fwd(nc_node *n) {
    nc_tensor *x = n->in[0], *w = n->in[1], *bias = n->n_in > 2 ? n->in[2] : nullptr;
    nc_ctx *ctx = x->ctx;
    const int64_t M = leading_rows(x), in = w->shape[1], out = w->shape[0];
    Operand a, wt;
    const int64_t *unused;
    int64_t packed[NC_MAX_DIMS];
    const float *B = bias ? contig_f32(bias) : nullptr;
    float *Y = fptr(n->out);
    if (!as_rows(x, a.m) || !last_two(w, wt.m, &unused, packed) || (bias && !B) || !Y) return NC_ERR_STATE;
    // y = (x W^T) + b: the product rounded, then the bias added, in the GEMM's own pass over y
    if (!product(ctx, Dims{}, M, out, in, a, wt.transposed(), 0.0f, Y, out, nullptr, "linear", B)) return NC_ERR_STATE;
    wrote_dev(n->out);
    return NC_OK;
}

void linear_bwd(nc_node *n) {
    nc_tensor *x = n->in[0], *w = n->in[1], *bias = n->n_in > 2 ? n->in[2] : nullptr;
    nc_ctx *ctx = x->ctx;
    const int64_t M = leading_rows(x), in = w->shape[1], out = w->shape[0];
    const float *g = fptr(n->out->grad);  // [M, out]
    if (!g) return;
    float beta;
    const int64_t *unused;
    int64_t packed[NC_MAX_DIMS];
    if (needs_grad(x)) {  // dX [M, in] (+)= G @ W
        Operand wm;
        float *gx = grad_target(x, &beta);
        if (gx && last_two(w, wm.m, &unused, packed) &&
            product(ctx, Dims{}, M, in, out, dense(g, out), wm, beta, gx, in, nullptr, "linear"))
            wrote_dev(x->grad);
    }
    if (needs_grad(w)) {  // dW [out, in] (+)= G^T @ X
        Operand xm;
        float *gw = grad_target(w, &beta);
        if (gw && as_rows(x, xm.m) &&
            product(ctx, Dims{}, out, in, M, dense(g, out).transposed(), xm, beta, gw, in, nullptr, "linear"))
            wrote_dev(w->grad);
    }
    if (bias && needs_grad(bias) && grad_buf(bias)) {  // db (+)= column sums of G, fp64 in a fixed order
        const int acc = grad_acc(bias);
        float *gb = fptr(bias->grad);
        const int64_t shape[2] = {M, out}, sg[2] = {out, 1}, sgb[2] = {0, 1};
        const size_t ws_bytes = nc_hip_binary_bwd_workspace(2, shape, sgb);
        char *ws = ws_bytes ? arena_alloc(ctx, ws_bytes) : nullptr;
        if (!gb || (ws_bytes && !ws)) return;
        if (hip_layer_ok(ctx,
                         nc_hip_binary_bwd(NC_HIP_BIN_ADD, 1, 2, shape, g, sg, g, sg, gb, sgb, gb, sgb, acc, ws,
                                           ws_bytes, stream(ctx)),
                         "linear"))
            wrote_dev(bias->grad);
    }
}

const OpDef op_linear = {"linear", 0, 0, linear_shape, nullptr, linear_fwd, linear_bwd};

}  // namespace
}  // namespace nce

using namespace nce;

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
