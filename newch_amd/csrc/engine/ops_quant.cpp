// int8: symmetric per-row weight quantization and the int8 linear.  Reference: engine/src/ops/ops_quant.c:23-113
// (nc_quantize_rows: not an autograd op; results follow persistent mode like nc_empty).
#include "engine.hpp"

using namespace nce;

extern "C" nc_tensor *nc_quantize_rows(nc_tensor *w, nc_tensor **scale) {
    if (!w) return nullptr;
    nc_ctx *ctx = w->ctx;
    if (w->dtype != NC_F32 || w->ndim != 2) {
        error(ctx, NC_ERR_SHAPE, "quantize_rows: expected a 2-D f32 tensor");
        return nullptr;
    }
    float *W = contig_f32(w);
    nc_tensor *q = nc_empty(ctx, NC_I8, 2, w->shape);
    nc_tensor *s = nc_empty(ctx, NC_F32, 1, w->shape);
    if (!W || !q || !s) return nullptr;
    int8_t *qp = (int8_t *)dptr(q);
    float *sp = fptr(s);
    if (!qp || !sp) return nullptr;
    if (!hip_layer_ok(ctx, nc_hip_quantize_rows(w->shape[0], w->shape[1], W, qp, sp, stream(ctx)), "quantize_rows"))
        return nullptr;
    wrote_dev(q);
    wrote_dev(s);
    if (scale) *scale = s;
    return q;
}

// ---- linear_int8 (ops_quant.c:41-113): y = dequant(quant_rows(x) @ wq^T) + b, inference only ----
// inputs: x f32 [..., in], wq i8 [out, in] (contiguous), w_scale f32 [out], optional bias f32 [out]
static nc_status qlinear_infer(nc_node *n, nc_dtype *dt, int *nd, int64_t *shape) {
    nc_tensor *x = n->in[0], *wq = n->in[1], *ws = n->in[2], *b = n->n_in > 3 ? n->in[3] : nullptr;
    if (x->dtype != NC_F32 || wq->dtype != NC_I8 || ws->dtype != NC_F32 || (b && b->dtype != NC_F32)) {
        error(x->ctx, NC_ERR_DTYPE, "linear_int8: expected x f32, weight i8, scale f32, bias f32");
        return NC_ERR_DTYPE;
    }
    if (x->ndim < 1 || wq->ndim != 2 || x->shape[x->ndim - 1] != wq->shape[1] || ws->ndim != 1 ||
        ws->shape[0] != wq->shape[0] || (b && (b->ndim != 1 || b->shape[0] != wq->shape[0]))) {
        char sx[96], sw[96];
        error(x->ctx, NC_ERR_SHAPE, "linear_int8: expected x [..., in], weight [out, in], scale/bias [out]; got %s, %s",
              shape_str(x->ndim, x->shape, sx, sizeof sx), shape_str(wq->ndim, wq->shape, sw, sizeof sw));
        return NC_ERR_SHAPE;
    }
    *dt = NC_F32;
    *nd = x->ndim;
    memcpy(shape, x->shape, sizeof(int64_t) * (size_t)x->ndim);
    shape[x->ndim - 1] = wq->shape[0];
    return NC_OK;
}

static nc_status qlinear_fwd(nc_node *n) {
    nc_tensor *x = n->in[0], *wq = n->in[1];
    nc_ctx *ctx = x->ctx;
    const int64_t in = wq->shape[1], out = wq->shape[0], M = in ? nc_numel(x) / in : 0;
    const float *X = contig_f32(x), *ws = contig_f32(n->in[2]);
    const float *b = n->n_in > 3 ? contig_f32(n->in[3]) : nullptr;
    if (!X || !ws || (n->n_in > 3 && !b)) return NC_ERR_STATE;
    if (!nc_is_contiguous(wq)) {
        error(ctx, NC_ERR_ARG, "linear_int8: weight must be contiguous");
        return NC_ERR_ARG;
    }
    const int8_t *W = (const int8_t *)dptr(wq);
    float *Y = fptr(n->out);
    const size_t ws_bytes = nc_hip_linear_int8_workspace(M, in);
    char *tmp = ws_bytes ? arena_alloc(ctx, ws_bytes) : nullptr;
    if (!W || !Y || (ws_bytes && !tmp)) return NC_ERR_STATE;
    if (!hip_layer_ok(ctx, nc_hip_linear_int8(M, in, out, X, W, ws, b, Y, tmp, ws_bytes, stream(ctx)), "linear_int8"))
        return NC_ERR_STATE;
    wrote_dev(n->out);
    return NC_OK;
}

static const OpDef op_linear_int8 = {"linear_int8", OPF_NONDIFF, 0, qlinear_infer, nullptr, qlinear_fwd, nullptr};

extern "C" nc_tensor *nc_linear_int8(nc_tensor *x, nc_tensor *wq, nc_tensor *w_scale, nc_tensor *bias) {
    nc_tensor *in[4] = {x, wq, w_scale, bias};
    return apply(&op_linear_int8, in, bias ? 4 : 3, nullptr);
}
