// Reductions over one axis or all.  Reference: engine/src/ops/ops_reduce.c (shape rules :13-58,
// forward :60-116, backward :118-163).  x is viewed as [outer, R, inner].
#include "engine.hpp"

namespace nce {

enum { RED_SUM = NC_HIP_RED_SUM, RED_MEAN = NC_HIP_RED_MEAN, RED_MAX = NC_HIP_RED_MAX, RED_ARGMAX = NC_HIP_RED_ARGMAX };

struct RedDims {
    int64_t outer, R, inner;
};

static RedDims get_dims(const nc_node *n) {
    const nc_tensor *x = n->in[0];
    RedDims d{1, 1, 1};
    int axis = (int)n->p.i[0];
    if (axis == NC_ALL_AXES) {
        d.R = nc_numel(x);
        return d;
    }
    axis = norm_axis(axis, x->ndim);
    for (int i = 0; i < axis; i++) d.outer *= x->shape[i];
    d.R = x->shape[axis];
    for (int i = axis + 1; i < x->ndim; i++) d.inner *= x->shape[i];
    return d;
}

static nc_status reduce_infer(nc_node *n, nc_dtype *dt, int *nd, int64_t *shape) {
    nc_tensor *x = n->in[0];
    const bool int_sum = n->op->kind == RED_SUM && x->dtype == NC_I32;
    if (!int_sum && !expect_f32(n, 0)) return NC_ERR_DTYPE;
    const int axis = (int)n->p.i[0], keep = (int)n->p.i[1];
    *dt = (n->op->kind == RED_ARGMAX || int_sum) ? NC_I32 : NC_F32;
    if (axis == NC_ALL_AXES) {
        if (nc_numel(x) == 0 && n->op->kind >= RED_MAX) {
            error(x->ctx, NC_ERR_SHAPE, "%s: reduction of an empty tensor", n->op->name);
            return NC_ERR_SHAPE;
        }
        *nd = keep ? x->ndim : 0;
        for (int i = 0; i < *nd; i++) shape[i] = 1;
        return NC_OK;
    }
    const int a = norm_axis(axis, x->ndim);
    if (a < 0) {
        error(x->ctx, NC_ERR_ARG, "%s: axis %d out of range for %d-d tensor", n->op->name, axis, x->ndim);
        return NC_ERR_ARG;
    }
    if (x->shape[a] == 0 && n->op->kind >= RED_MAX) {
        error(x->ctx, NC_ERR_SHAPE, "%s: reduction over an empty axis", n->op->name);
        return NC_ERR_SHAPE;
    }
    *nd = 0;
    for (int i = 0; i < x->ndim; i++) {
        if (i != a) shape[(*nd)++] = x->shape[i];
        else if (keep) shape[(*nd)++] = 1;
    }
    return NC_OK;
}

static nc_status reduce_fwd(nc_node *n) {
    nc_ctx *ctx = n->out->ctx;
    const RedDims d = get_dims(n);
    nc_tensor *x = n->in[0];
    if (x->dtype == NC_I32) {
        const int64_t N = nc_numel(x);
        char *src = dptr(x);
        if (!src) return NC_ERR_STATE;
        char *buf = src;
        if (!nc_is_contiguous(x)) {
            buf = arena_alloc(ctx, (size_t)(N ? N : 1) * 4);
            if (!buf || !hip_layer_ok(ctx, nc_hip_copy_strided(4, x->ndim, x->shape, src, x->stride, buf, stream(ctx)),
                                      "sum"))
                return NC_ERR_STATE;
        }
        int32_t *y = (int32_t *)dptr(n->out);
        if (!y || !hip_layer_ok(ctx, nc_hip_reduce_sum_i32(d.outer, d.R, d.inner, (const int32_t *)buf, y, stream(ctx)),
                                "sum"))
            return NC_ERR_STATE;
        wrote_dev(n->out);
        return NC_OK;
    }
    float *xp = contig_f32(x);
    if (!xp) return NC_ERR_STATE;
    const int kind = n->op->kind;
    float *y = kind == RED_ARGMAX ? nullptr : fptr(n->out);
    int32_t *arg = nullptr;
    if (kind == RED_ARGMAX) {
        arg = (int32_t *)dptr(n->out);
    } else if (kind == RED_MAX) {
        const int64_t cells = d.outer * d.inner;
        const size_t bytes = (size_t)(cells > 0 ? cells : 1) * sizeof(int32_t);
        arg = (int32_t *)arena_alloc(ctx, bytes);
        n->saved = arg;
        n->saved_bytes = bytes;
    }
    if ((kind != RED_ARGMAX && !y) || ((kind == RED_ARGMAX || kind == RED_MAX) && !arg)) return NC_ERR_STATE;
    const size_t ws_bytes = nc_hip_reduce_workspace(kind, d.outer, d.R, d.inner);
    char *ws = ws_bytes ? arena_alloc(ctx, ws_bytes) : nullptr;
    if (ws_bytes && !ws) return NC_ERR_STATE;
    if (!hip_layer_ok(ctx, nc_hip_reduce_fwd(kind, d.outer, d.R, d.inner, xp, y, arg, ws, ws_bytes, stream(ctx)),
                      n->op->name))
        return NC_ERR_STATE;
    // workspace goes back to the arena now (stream-ordered): it is not part of the node's saved state
    if (ws && !ctx->bwd_logging) arena_free(ctx, ws, ws_bytes);
    wrote_dev(n->out);
    return NC_OK;
}

static void reduce_bwd(nc_node *n) {
    nc_tensor *x = n->in[0];
    nc_ctx *ctx = x->ctx;
    if (!grad_buf(x)) return;
    const RedDims d = get_dims(n);
    float *g = fptr(n->out->grad);
    if (!g) return;
    const int acc = grad_acc(x);
    float *gi = fptr(x->grad);
    if (!gi) return;
    if (!hip_layer_ok(ctx,
                      nc_hip_reduce_bwd(n->op->kind, d.outer, d.R, d.inner, g, (const int32_t *)n->saved, gi, acc,
                                        stream(ctx)),
                      n->op->name))
        return;
    wrote_dev(x->grad);
}

const OpDef op_sum = {"sum", OPF_REDUCTION, RED_SUM, reduce_infer, nullptr, reduce_fwd, reduce_bwd};
const OpDef op_mean = {"mean", OPF_REDUCTION, RED_MEAN, reduce_infer, nullptr, reduce_fwd, reduce_bwd};
const OpDef op_max = {"max", OPF_REDUCTION, RED_MAX, reduce_infer, nullptr, reduce_fwd, reduce_bwd};
const OpDef op_argmax = {"argmax", OPF_REDUCTION | OPF_NONDIFF, RED_ARGMAX, reduce_infer, nullptr, reduce_fwd, nullptr};

static nc_tensor *reduce(const OpDef *op, nc_tensor *x, int axis, int keepdim) {
    Params p{};
    p.i[0] = axis;
    p.i[1] = keepdim ? 1 : 0;
    return apply(op, &x, 1, &p);
}

}  // namespace nce

using namespace nce;

extern "C" {
nc_tensor *nc_sum(nc_tensor *x, int axis, int keepdim) { return reduce(&op_sum, x, axis, keepdim); }
nc_tensor *nc_mean(nc_tensor *x, int axis, int keepdim) { return reduce(&op_mean, x, axis, keepdim); }
nc_tensor *nc_max(nc_tensor *x, int axis, int keepdim) { return reduce(&op_max, x, axis, keepdim); }
nc_tensor *nc_argmax(nc_tensor *x, int axis) { return reduce(&op_argmax, x, axis, 0); }
}
