// softmax / log_softmax over the last axis and LayerNorm over the last k axes.
// Reference: engine/src/ops/ops_nn.c (:8-77 softmax, :434-538 layer_norm).
#include "engine.hpp"

namespace nce {

enum { SM_LOG = 0, SM_PLAIN = 1 };

static nc_status softmax_infer(nc_node *n, nc_dtype *dt, int *nd, int64_t *shape) {
    nc_tensor *x = n->in[0];
    if (!expect_f32(n, 0)) return NC_ERR_DTYPE;
    if (x->ndim < 1) {
        error(x->ctx, NC_ERR_SHAPE, "%s: input must have at least 1 dimension", n->op->name);
        return NC_ERR_SHAPE;
    }
    *dt = NC_F32;
    *nd = x->ndim;
    memcpy(shape, x->shape, sizeof(int64_t) * (size_t)x->ndim);
    return NC_OK;
}

static void rows_cols(const nc_tensor *t, int64_t *rows, int64_t *C) {
    *C = t->shape[t->ndim - 1];
    *rows = *C ? nc_numel(t) / *C : 0;
}

static nc_status softmax_fwd(nc_node *n) {
    nc_ctx *ctx = n->out->ctx;
    float *x = contig_f32(n->in[0]), *y = fptr(n->out);
    if (!x || !y) return NC_ERR_STATE;
    int64_t rows, C;
    rows_cols(n->out, &rows, &C);
    if (!hip_layer_ok(ctx, nc_hip_softmax_fwd(n->op->kind == SM_LOG, rows, C, x, y, stream(ctx)), n->op->name))
        return NC_ERR_STATE;
    wrote_dev(n->out);
    return NC_OK;
}

static void softmax_bwd(nc_node *n) {
    nc_tensor *in = n->in[0];
    nc_ctx *ctx = in->ctx;
    if (!grad_buf(in)) return;
    float *y = fptr(n->out), *g = fptr(n->out->grad);
    if (!y || !g) return;
    const int acc = grad_acc(in);
    float *gi = fptr(in->grad);
    if (!gi) return;
    int64_t rows, C;
    rows_cols(n->out, &rows, &C);
    if (!hip_layer_ok(ctx, nc_hip_softmax_bwd(n->op->kind == SM_LOG, rows, C, y, g, gi, acc, stream(ctx)),
                      n->op->name))
        return;
    wrote_dev(in->grad);
}

const OpDef op_log_softmax = {"log_softmax", 0, SM_LOG, softmax_infer, nullptr, softmax_fwd, softmax_bwd};
const OpDef op_softmax = {"softmax", 0, SM_PLAIN, softmax_infer, nullptr, softmax_fwd, softmax_bwd};

// ---- layer norm ------------------------------------------------------------------------------------
// inputs: x, then weight and bias [D] when present (p.i[1], p.i[2]); p.i[0] = normalized ndim
static nc_status layer_norm_infer(nc_node *n, nc_dtype *dt, int *nd, int64_t *shape) {
    nc_tensor *x = n->in[0];
    const int k = (int)n->p.i[0];
    for (int i = 0; i < n->n_in; i++)
        if (!expect_f32(n, i)) return NC_ERR_DTYPE;
    if (k < 1 || k > x->ndim) {
        error(x->ctx, NC_ERR_SHAPE, "layer_norm: normalized_shape has %d dims, input only %d", k, x->ndim);
        return NC_ERR_SHAPE;
    }
    const int64_t D = shape_numel(k, x->shape + x->ndim - k);
    for (int i = 1; i < n->n_in; i++) {
        if (nc_numel(n->in[i]) != D) {
            error(x->ctx, NC_ERR_SHAPE, "layer_norm: weight/bias need %lld elements, got %lld", (long long)D,
                  (long long)nc_numel(n->in[i]));
            return NC_ERR_SHAPE;
        }
    }
    *dt = NC_F32;
    *nd = x->ndim;
    memcpy(shape, x->shape, sizeof(int64_t) * (size_t)x->ndim);
    return NC_OK;
}

static int64_t ln_dim(const nc_node *n) {
    const nc_tensor *x = n->in[0];
    const int k = (int)n->p.i[0];
    return shape_numel(k, x->shape + x->ndim - k);
}

static nc_status layer_norm_fwd(nc_node *n) {
    nc_tensor *x = n->in[0];
    nc_ctx *ctx = x->ctx;
    const int has_w = (int)n->p.i[1], has_b = (int)n->p.i[2];
    float *w = has_w ? contig_f32(n->in[1]) : nullptr;
    float *b = has_b ? contig_f32(n->in[1 + has_w]) : nullptr;
    float *X = contig_f32(x), *Y = fptr(n->out);
    const int64_t D = ln_dim(n), R = D ? nc_numel(x) / D : 0;
    const size_t sbytes = (size_t)(2 * R + 1) * sizeof(float);
    float *stats = (float *)arena_alloc(ctx, sbytes);
    if (!X || !Y || !stats || (has_w && !w) || (has_b && !b)) return NC_ERR_STATE;
    if (!hip_layer_ok(ctx, nc_hip_layer_norm_fwd(R, D, X, w, b, n->p.f[0], Y, stats, stream(ctx)), "layer_norm"))
        return NC_ERR_STATE;
    n->saved = stats;
    n->saved_bytes = sbytes;
    wrote_dev(n->out);
    return NC_OK;
}

static void layer_norm_bwd(nc_node *n) {
    nc_tensor *x = n->in[0];
    nc_ctx *ctx = x->ctx;
    const int has_w = (int)n->p.i[1], has_b = (int)n->p.i[2];
    nc_tensor *wt = has_w ? n->in[1] : nullptr, *bt = has_b ? n->in[1 + has_w] : nullptr;
    float *X = contig_f32(x), *w = wt ? contig_f32(wt) : nullptr, *g = fptr(n->out->grad);
    const int64_t D = ln_dim(n), R = D ? nc_numel(x) / D : 0;
    if (!X || (wt && !w) || !g) return;
    const bool want_x = needs_grad(x), want_w = wt && needs_grad(wt), want_b = bt && needs_grad(bt);
    if ((want_x && !grad_buf(x)) || (want_w && !grad_buf(wt)) || (want_b && !grad_buf(bt))) return;
    const int acc = want_x ? grad_acc(x) : 1;
    float *gx = want_x ? fptr(x->grad) : nullptr;
    // column sums are added into gw / gb: a fresh buffer is given its zeros by fptr
    float *gw = want_w ? fptr(wt->grad) : nullptr;
    float *gb = want_b ? fptr(bt->grad) : nullptr;
    if ((want_x && !gx) || (want_w && !gw) || (want_b && !gb)) return;
    const size_t ws_bytes = (want_w || want_b) ? nc_hip_layer_norm_bwd_workspace(R, D) : 0;
    char *ws = ws_bytes ? arena_alloc(ctx, ws_bytes) : nullptr;
    if (ws_bytes && !ws) return;
    if (!hip_layer_ok(ctx,
                      nc_hip_layer_norm_bwd(R, D, X, w, (const float *)n->saved, g, gx, gw, gb, acc, ws, ws_bytes,
                                            stream(ctx)),
                      "layer_norm"))
        return;
    if (gx) wrote_dev(x->grad);
    if (gw) wrote_dev(wt->grad);
    if (gb) wrote_dev(bt->grad);
}

const OpDef op_layer_norm = {"layer_norm", 0, 0, layer_norm_infer, nullptr, layer_norm_fwd, layer_norm_bwd};

}  // namespace nce

using namespace nce;

extern "C" {
nc_tensor *nc_log_softmax(nc_tensor *x) { return apply(&op_log_softmax, &x, 1, nullptr); }
nc_tensor *nc_softmax(nc_tensor *x) { return apply(&op_softmax, &x, 1, nullptr); }

nc_tensor *nc_layer_norm(nc_tensor *x, int normalized_ndim, nc_tensor *weight, nc_tensor *bias, float eps) {
    nc_tensor *in[3] = {x, nullptr, nullptr};
    int k = 1;
    if (weight) in[k++] = weight;
    if (bias) in[k++] = bias;
    Params p{};
    p.i[0] = normalized_ndim;
    p.i[1] = weight != nullptr;
    p.i[2] = bias != nullptr;
    p.f[0] = eps;
    return apply(&op_layer_norm, in, k, &p);
}
}
