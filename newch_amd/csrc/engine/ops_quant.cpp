// Symmetric per-row int8 weight quantization.  Reference: engine/src/ops/ops_quant.c:23-39
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
