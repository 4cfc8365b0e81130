// Reductions over one axis or all of them: sum, mean, max (differentiable) and argmax.
// Reference: engine/src/ops/ops_reduce.c (shape rules :13-58, forward :60-116, backward :118-163);
// the error messages and output shapes are the reference's.  Every kernel sees x as a contiguous
// [outer, R, inner] block reduced over R; an all-axes reduction is the block [1, numel, 1].
#include "engine.hpp"

namespace nce {

enum { RED_SUM = NC_HIP_RED_SUM, RED_MEAN = NC_HIP_RED_MEAN, RED_MAX = NC_HIP_RED_MAX, RED_ARGMAX = NC_HIP_RED_ARGMAX };

// p.i[0]: the axis (NC_ALL_AXES or any index numpy accepts), p.i[1]: keepdim
struct Block {
    int64_t outer = 1, R = 1, inner = 1;
    int64_t cells() const { return outer * inner; }
};

static Block block_of(const nc_node *n) {
    const Dims x = Dims::of(n->in[0]);
    Block b;
    if ((int)n->p.i[0] == NC_ALL_AXES) {
        b.R = x.numel();
        return b;
    }
    const int axis = norm_axis((int)n->p.i[0], x.rank);
    for (int i = 0; i < x.rank; i++) (i < axis ? b.outer : i == axis ? b.R : b.inner) *= x.e[i];
    return b;
}

static bool selects(int kind) { return kind == RED_MAX || kind == RED_ARGMAX; }  // undefined when empty

static nc_status reduce_shape(nc_node *n, OutSpec &out) {
    const Dims x = Dims::of(n->in[0]);
    const int kind = n->op->kind, axis = (int)n->p.i[0];
    const bool keep = n->p.i[1] != 0;
    const bool int_sum = kind == RED_SUM && n->in[0]->dtype == NC_I32;  // i32 sums stay i32
    if (!int_sum && !inputs_f32(n, 0, 1)) return NC_ERR_DTYPE;
    out.dtype = (kind == RED_ARGMAX || int_sum) ? NC_I32 : NC_F32;
    if (axis == NC_ALL_AXES) {
        if (selects(kind) && x.numel() == 0)
            return reject(n, NC_ERR_SHAPE, "%s: reduction of an empty tensor", n->op->name);
        if (keep)
            while (out.dims.rank < x.rank) out.dims.push(1);
        return NC_OK;
    }
    const int a = norm_axis(axis, x.rank);
    if (a < 0) return reject(n, NC_ERR_ARG, "%s: axis %d out of range for %d-d tensor", n->op->name, axis, x.rank);
    if (selects(kind) && x.e[a] == 0)
        return reject(n, NC_ERR_SHAPE, "%s: reduction over an empty axis", n->op->name);
    for (int i = 0; i < x.rank; i++)
        if (i != a || keep) out.dims.push(i == a ? 1 : x.e[i]);
    return NC_OK;
}

// i32 sums: the input gathered when strided, one kernel
static nc_status sum_i32_fwd(nc_node *n, const Block &b) {
    nc_tensor *x = n->in[0];
    nc_ctx *ctx = x->ctx;
    const char *src = dptr(x);
    int32_t *y = (int32_t *)dptr_overwrite(n->out);
    if (!src || !y) return NC_ERR_STATE;
    if (!nc_is_contiguous(x)) {
        char *packed = arena_alloc(ctx, (size_t)(nc_numel(x) ? nc_numel(x) : 1) * sizeof(int32_t));
        if (!packed ||
            !hip_layer_ok(ctx, nc_hip_copy_strided(4, x->ndim, x->shape, src, x->stride, packed, stream(ctx)), "sum"))
            return NC_ERR_STATE;
        src = packed;
    }
    if (!hip_layer_ok(ctx, nc_hip_reduce_sum_i32(b.outer, b.R, b.inner, (const int32_t *)src, y, stream(ctx)), "sum"))
        return NC_ERR_STATE;
    wrote_dev(n->out);
    return NC_OK;
}

// f32: max keeps the index it picked in each cell for its backward (argmax returns it)
static nc_status reduce_fwd(nc_node *n) {
    const Block b = block_of(n);
    if (n->in[0]->dtype == NC_I32) return sum_i32_fwd(n, b);
    nc_ctx *ctx = n->out->ctx;
    const int kind = n->op->kind;
    const float *x = contig_f32(n->in[0]);
    float *y = nullptr;
    int32_t *arg = nullptr;
    if (kind == RED_ARGMAX)
        arg = (int32_t *)dptr_overwrite(n->out);
    else
        y = (float *)dptr_overwrite(n->out);
    if (kind == RED_MAX) arg = (int32_t *)save_state(n, (size_t)(b.cells() ? b.cells() : 1) * sizeof(int32_t));
    if (!x || (kind != RED_ARGMAX && !y) || (selects(kind) && !arg)) return NC_ERR_STATE;
    const size_t ws_bytes = nc_hip_reduce_workspace(kind, b.outer, b.R, b.inner);
    char *ws = ws_bytes ? arena_alloc(ctx, ws_bytes) : nullptr;
    if (ws_bytes && !ws) return NC_ERR_STATE;
    if (!hip_layer_ok(ctx, nc_hip_reduce_fwd(kind, b.outer, b.R, b.inner, x, y, arg, ws, ws_bytes, stream(ctx)),
                      n->op->name))
        return NC_ERR_STATE;
    wrote_dev(n->out);
    return NC_OK;
}

// sum / mean spread g over R (scaled by 1/R for mean); max routes it to the saved index
static void reduce_bwd(nc_node *n) {
    nc_tensor *x = n->in[0];
    nc_ctx *ctx = x->ctx;
    const Block b = block_of(n);
    const float *g = grad_buf(x) ? fptr(n->out->grad) : nullptr;
    if (!g) return;
    const int acc = grad_acc(x);
    float *gx = fptr(x->grad);
    if (!gx || !hip_layer_ok(ctx,
                             nc_hip_reduce_bwd(n->op->kind, b.outer, b.R, b.inner, g, (const int32_t *)n->saved, gx,
                                               acc, stream(ctx)),
                             n->op->name))
        return;
    wrote_dev(x->grad);
}

const OpDef op_sum = {"sum", OPF_REDUCTION, RED_SUM, reduce_shape, nullptr, reduce_fwd, reduce_bwd};
const OpDef op_mean = {"mean", OPF_REDUCTION, RED_MEAN, reduce_shape, nullptr, reduce_fwd, reduce_bwd};
const OpDef op_max = {"max", OPF_REDUCTION, RED_MAX, reduce_shape, nullptr, reduce_fwd, reduce_bwd};
const OpDef op_argmax = {"argmax", OPF_REDUCTION | OPF_NONDIFF, RED_ARGMAX, reduce_shape, nullptr, reduce_fwd, nullptr};

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
