// Elementwise ops: broadcasting binary arithmetic and unary math / activations.
// Reference: engine/src/ops/ops_elementwise.c (binary :60-204, unary :210-411).
// The shape rules keep the reference's error messages; the arithmetic runs in the nc_hip_* kernels
// (include/nc_hip.h) on the context's stream, and op temporaries (gathered operands, reduction
// workspaces) are scratch of the call.
#include <stdio.h>

#include "engine.hpp"

namespace nce {

// ---- binary ----------------------------------------------------------------------------------------
// numpy broadcasting: extents are matched from the last axis back; a pair must agree or one be 1
static nc_status broadcast_shape(nc_node *n, OutSpec &out) {
    if (!inputs_f32(n, 0, 2)) return NC_ERR_DTYPE;
    const Dims a = Dims::of(n->in[0]), b = Dims::of(n->in[1]);
    out.dims.rank = a.rank > b.rank ? a.rank : b.rank;
    for (int k = 0; k < out.dims.rank; k++) {
        const int64_t ea = k < a.rank ? a.back(k) : 1, eb = k < b.rank ? b.back(k) : 1;
        if (ea != eb && ea != 1 && eb != 1) {
            char ta[96], tb[96];
            return reject(n, NC_ERR_SHAPE, "%s: shapes %s and %s are not broadcastable", n->op->name,
                          a.text(ta, sizeof ta), b.text(tb, sizeof tb));
        }
        out.dims.e[out.dims.rank - 1 - k] = ea == 1 ? eb : ea;
    }
    return NC_OK;
}

// Device address and broadcast strides of operand x of output o.  An operand view that the output
// reuses many times over is first gathered into contiguous arena memory: one whose innermost stride is
// not 1 (reused at least 4 times; the broadcast kernels then read it with 128-bit loads rather than
// one cache line per element), or any other non-contiguous view of up to 128 MiB reused at least 8
// times (rows far apart in memory land in few L2 channels; the contiguous copy reads like the plain
// operand: a batch-transposed a[64,512,1,64] broadcast to 2^30 outputs, 827 -> ~700 us with the copy).
static float *operand(nc_tensor *x, const nc_tensor *o, int64_t *sx) {
    const bool strided_inner = x->ndim > 0 && x->shape[x->ndim - 1] > 1 && x->stride[x->ndim - 1] != 1;
    const bool gather_view = !nc_is_contiguous(x) && 8 * nc_numel(x) <= nc_numel(o) &&
                             nc_numel(x) * (int64_t)sizeof(float) <= (int64_t(128) << 20);
    if ((strided_inner && 4 * nc_numel(x) <= nc_numel(o)) || gather_view) {
        float *p = contig_f32(x);
        if (p) bcast_strides_shape(x->ndim, x->shape, o->ndim, o->shape, sx);
        return p;
    }
    bcast_strides(x, o->ndim, o->shape, sx);
    return fptr(x);
}

static nc_status binary_fwd(nc_node *n) {
    nc_tensor *a = n->in[0], *b = n->in[1], *o = n->out;
    nc_ctx *ctx = o->ctx;
    int64_t sa[NC_MAX_DIMS], sb[NC_MAX_DIMS];
    float *pa = operand(a, o, sa), *pb = operand(b, o, sb), *po = fptr(o);
    if (!pa || !pb || !po) return NC_ERR_STATE;
    if (!hip_layer_ok(ctx, nc_hip_binary_fwd(n->op->kind, o->ndim, o->shape, pa, sa, pb, sb, po, o->stride, stream(ctx)),
                      n->op->name))
        return NC_ERR_STATE;
    wrote_dev(o);
    return NC_OK;
}

static void binary_bwd(nc_node *n) {
    nc_tensor *a = n->in[0], *b = n->in[1], *o = n->out;
    nc_ctx *ctx = o->ctx;
    const int nd = o->ndim;
    int64_t sa[NC_MAX_DIMS], sb[NC_MAX_DIMS];
    float *g = fptr(o->grad), *pa = operand(a, o, sa), *pb = operand(b, o, sb);
    if (!g || !pa || !pb) return;
    if (needs_grad(a) && needs_grad(b) && a != b && !same_shape(a, o) && !same_shape(b, o)) {
        // both operands are reduced: one pass over g for both gradients (nc_hip_binary_bwd2)
        if (!grad_buf(a) || !grad_buf(b)) return;
        int64_t sga[NC_MAX_DIMS], sgb[NC_MAX_DIMS];
        bcast_strides_shape(a->ndim, a->shape, nd, o->shape, sga);
        bcast_strides_shape(b->ndim, b->shape, nd, o->shape, sgb);
        const size_t ws_bytes = nc_hip_binary_bwd2_workspace(nd, o->shape, sga, sgb);
        char *ws = ws_bytes ? arena_alloc(ctx, ws_bytes) : nullptr;
        if (ws_bytes && !ws) return;
        int acc_a = grad_acc(a), acc_b = grad_acc(b);
        if (acc_a != acc_b) {  // one fresh buffer: give it its zeros so both accumulate
            if (!fill_zero(acc_a ? b->grad : a->grad)) return;
            acc_a = acc_b = 1;
        }
        float *ga = fptr(a->grad), *gb = fptr(b->grad);
        if (!ga || !gb) return;
        if (!hip_layer_ok(ctx,
                          nc_hip_binary_bwd2(n->op->kind, nd, o->shape, g, o->stride, pa, sa, pb, sb, ga, sga, gb,
                                             sgb, acc_a, ws, ws_bytes, stream(ctx)),
                          n->op->name))
            return;
        wrote_dev(a->grad);
        wrote_dev(b->grad);
        return;
    }
    for (int which = 0; which < 2; which++) {
        nc_tensor *x = n->in[which];
        if (!needs_grad(x)) continue;
        if (!grad_buf(x)) return;
        int64_t sgx[NC_MAX_DIMS];
        bcast_strides_shape(x->ndim, x->shape, nd, o->shape, sgx);
        const size_t ws_bytes = nc_hip_binary_bwd_workspace(nd, o->shape, sgx);
        char *ws = ws_bytes ? arena_alloc(ctx, ws_bytes) : nullptr;
        if (ws_bytes && !ws) return;
        const int acc = grad_acc(x);
        float *gx = fptr(x->grad);
        if (!gx) return;
        if (!hip_layer_ok(ctx,
                          nc_hip_binary_bwd(n->op->kind, which, nd, o->shape, g, o->stride, pa, sa, pb, sb, gx, sgx,
                                            acc, ws, ws_bytes, stream(ctx)),
                          n->op->name))
            return;
        wrote_dev(x->grad);
    }
}

const OpDef op_add = {"add", OPF_ELEMENTWISE, NC_HIP_BIN_ADD, broadcast_shape, nullptr, binary_fwd, binary_bwd};
const OpDef op_sub = {"sub", OPF_ELEMENTWISE, NC_HIP_BIN_SUB, broadcast_shape, nullptr, binary_fwd, binary_bwd};
const OpDef op_mul = {"mul", OPF_ELEMENTWISE, NC_HIP_BIN_MUL, broadcast_shape, nullptr, binary_fwd, binary_bwd};
const OpDef op_div = {"div", OPF_ELEMENTWISE, NC_HIP_BIN_DIV, broadcast_shape, nullptr, binary_fwd, binary_bwd};

static nc_tensor *binary(const OpDef *op, nc_tensor *a, nc_tensor *b) {
    nc_tensor *in[2] = {a, b};
    return apply(op, in, 2, nullptr);
}

// ---- unary -----------------------------------------------------------------------------------------
static nc_status unary_shape(nc_node *n, OutSpec &out) {
    if (!inputs_f32(n, 0, 1)) return NC_ERR_DTYPE;
    out.dims = Dims::of(n->in[0]);
    return NC_OK;
}

static nc_status unary_fwd(nc_node *n) {
    nc_ctx *ctx = n->out->ctx;
    float *x = contig_f32(n->in[0]), *y = fptr(n->out);
    if (!x || !y) return NC_ERR_STATE;
    if (!hip_layer_ok(ctx, nc_hip_unary_fwd(n->op->kind, n->p.f[0], x, y, nc_numel(n->out), stream(ctx)), n->op->name))
        return NC_ERR_STATE;
    wrote_dev(n->out);
    return NC_OK;
}

static bool reads_y(int kind) {
    return kind == NC_HIP_UN_SIGMOID || kind == NC_HIP_UN_TANH || kind == NC_HIP_UN_EXP || kind == NC_HIP_UN_SQRT;
}
static bool reads_x(int kind) {
    return !reads_y(kind) && kind != NC_HIP_UN_NEG && kind != NC_HIP_UN_SCALE && kind != NC_HIP_UN_ADD_SCALAR;
}

static void unary_bwd(nc_node *n) {
    nc_tensor *in = n->in[0];
    nc_ctx *ctx = in->ctx;
    const int kind = n->op->kind;
    if (!grad_buf(in)) return;
    float *x = reads_x(kind) ? contig_f32(in) : nullptr;
    float *y = reads_y(kind) ? fptr(n->out) : nullptr;
    float *g = fptr(n->out->grad);
    if ((reads_x(kind) && !x) || (reads_y(kind) && !y) || !g) return;
    const int acc = grad_acc(in);
    float *gi = fptr(in->grad);
    if (!gi) return;
    if (!hip_layer_ok(ctx, nc_hip_unary_bwd(kind, n->p.f[0], x, y, g, gi, nc_numel(in), acc, stream(ctx)),
                      n->op->name))
        return;
    wrote_dev(in->grad);
}

#define NC_UNARY_DEF(nm, KIND) \
    const OpDef op_##nm = {#nm, OPF_ELEMENTWISE, KIND, unary_shape, nullptr, unary_fwd, unary_bwd};
NC_UNARY_DEF(neg, NC_HIP_UN_NEG)
NC_UNARY_DEF(exp, NC_HIP_UN_EXP)
NC_UNARY_DEF(log, NC_HIP_UN_LOG)
NC_UNARY_DEF(sqrt, NC_HIP_UN_SQRT)
NC_UNARY_DEF(relu, NC_HIP_UN_RELU)
NC_UNARY_DEF(sigmoid, NC_HIP_UN_SIGMOID)
NC_UNARY_DEF(tanh, NC_HIP_UN_TANH)
NC_UNARY_DEF(scale, NC_HIP_UN_SCALE)
NC_UNARY_DEF(add_scalar, NC_HIP_UN_ADD_SCALAR)
NC_UNARY_DEF(pow_scalar, NC_HIP_UN_POW)
NC_UNARY_DEF(leaky_relu, NC_HIP_UN_LEAKY_RELU)
NC_UNARY_DEF(relu6, NC_HIP_UN_RELU6)
NC_UNARY_DEF(hardsigmoid, NC_HIP_UN_HARDSIGMOID)
NC_UNARY_DEF(hardswish, NC_HIP_UN_HARDSWISH)
NC_UNARY_DEF(silu, NC_HIP_UN_SILU)
NC_UNARY_DEF(gelu, NC_HIP_UN_GELU)
NC_UNARY_DEF(gelu_tanh, NC_HIP_UN_GELU_TANH)
#undef NC_UNARY_DEF

static nc_tensor *unary(const OpDef *op, nc_tensor *x, float s) {
    Params p{};
    p.f[0] = s;
    return apply(op, &x, 1, &p);
}

}  // namespace nce

using namespace nce;

extern "C" {
nc_tensor *nc_add(nc_tensor *a, nc_tensor *b) { return binary(&op_add, a, b); }
nc_tensor *nc_sub(nc_tensor *a, nc_tensor *b) { return binary(&op_sub, a, b); }
nc_tensor *nc_mul(nc_tensor *a, nc_tensor *b) { return binary(&op_mul, a, b); }
nc_tensor *nc_div(nc_tensor *a, nc_tensor *b) { return binary(&op_div, a, b); }
nc_tensor *nc_neg(nc_tensor *x) { return unary(&op_neg, x, 0); }
nc_tensor *nc_exp(nc_tensor *x) { return unary(&op_exp, x, 0); }
nc_tensor *nc_log(nc_tensor *x) { return unary(&op_log, x, 0); }
nc_tensor *nc_sqrt(nc_tensor *x) { return unary(&op_sqrt, x, 0); }
nc_tensor *nc_relu(nc_tensor *x) { return unary(&op_relu, x, 0); }
nc_tensor *nc_sigmoid(nc_tensor *x) { return unary(&op_sigmoid, x, 0); }
nc_tensor *nc_tanh(nc_tensor *x) { return unary(&op_tanh, x, 0); }
nc_tensor *nc_scale(nc_tensor *x, float s) { return unary(&op_scale, x, s); }
nc_tensor *nc_add_scalar(nc_tensor *x, float s) { return unary(&op_add_scalar, x, s); }
nc_tensor *nc_pow_scalar(nc_tensor *x, float p) { return unary(&op_pow_scalar, x, p); }
nc_tensor *nc_leaky_relu(nc_tensor *x, float negative_slope) { return unary(&op_leaky_relu, x, negative_slope); }
nc_tensor *nc_relu6(nc_tensor *x) { return unary(&op_relu6, x, 0); }
nc_tensor *nc_hardsigmoid(nc_tensor *x) { return unary(&op_hardsigmoid, x, 0); }
nc_tensor *nc_hardswish(nc_tensor *x) { return unary(&op_hardswish, x, 0); }
nc_tensor *nc_silu(nc_tensor *x) { return unary(&op_silu, x, 0); }
nc_tensor *nc_gelu(nc_tensor *x, int approximate_tanh) {
    return unary(approximate_tanh ? &op_gelu_tanh : &op_gelu, x, 0);
}
}
