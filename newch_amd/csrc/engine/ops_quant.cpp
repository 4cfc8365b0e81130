// int8: symmetric per-row weight quantization and the int8 linear.  Reference: engine/src/ops/ops_quant.c:23-113.
// nc_quantize_rows is not an autograd op: its two results follow persistent mode like nc_empty.
#include "engine.hpp"

using namespace nce;

// w [rows, cols] f32 -> q i8 [rows, cols] and one f32 scale per row, in one kernel
static bool quantize(nc_tensor *w, nc_tensor *q, nc_tensor *s) {
    nc_ctx *ctx = w->ctx;
    Scratch scratch(ctx);  // a packed copy of a strided w is handed back when the call ends
    const float *W = contig_f32(w);
    int8_t *Q = (int8_t *)dptr_overwrite(q);
    float *S = (float *)dptr_overwrite(s);
    if (!W || !Q || !S ||
        !hip_layer_ok(ctx, nc_hip_quantize_rows(w->shape[0], w->shape[1], W, Q, S, stream(ctx)), "quantize_rows"))
        return false;
    wrote_dev(q);
    wrote_dev(s);
    return true;
}

extern "C" nc_tensor *nc_quantize_rows(nc_tensor *w, nc_tensor **scale) {
    if (!w) return nullptr;
    if (w->dtype != NC_F32 || w->ndim != 2) {
        error(w->ctx, NC_ERR_SHAPE, "quantize_rows: expected a 2-D f32 tensor");
        return nullptr;
    }
    const int64_t rows = w->shape[0];
    nc_tensor *q = nc_empty(w->ctx, NC_I8, 2, w->shape);
    nc_tensor *s = q ? nc_empty(w->ctx, NC_F32, 1, &rows) : nullptr;
    if (!s || !quantize(w, q, s)) return nullptr;
    if (scale) *scale = s;
    return q;
}

// ---- linear_int8 (ops_quant.c:41-113): y = dequant(quant_rows(x) @ wq^T) + b, inference only ----
// inputs: x f32 [..., in], wq i8 [out, in] (contiguous), w_scale f32 [out], optional bias f32 [out]
static nc_status qlinear_shape(nc_node *n, OutSpec &out) {
    const bool has_b = n->n_in > 3;
    const nc_dtype want[4] = {NC_F32, NC_I8, NC_F32, NC_F32};
    for (int i = 0; i < n->n_in; i++)
        if (n->in[i]->dtype != want[i])
            return reject(n, NC_ERR_DTYPE, "linear_int8: expected x f32, weight i8, scale f32, bias f32");
    const Dims x = Dims::of(n->in[0]), w = Dims::of(n->in[1]), sc = Dims::of(n->in[2]);
    const Dims b = has_b ? Dims::of(n->in[3]) : Dims{};
    const auto per_out = [&](const Dims &v) { return v.rank == 1 && v.e[0] == w.e[0]; };
    const bool ok = x.rank >= 1 && w.rank == 2 && x.back(0) == w.e[1] && per_out(sc) && (!has_b || per_out(b));
    if (!ok) {
        char tx[96], tw[96];
        return reject(n, NC_ERR_SHAPE, "linear_int8: expected x [..., in], weight [out, in], scale/bias [out]; got %s, %s",
                      x.text(tx, sizeof tx), w.text(tw, sizeof tw));
    }
    out.dims = x;
    out.dims.e[x.rank - 1] = w.e[0];
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

static const OpDef op_linear_int8 = {"linear_int8", OPF_NONDIFF, 0, qlinear_shape, nullptr, qlinear_fwd, nullptr};

extern "C" nc_tensor *nc_linear_int8(nc_tensor *x, nc_tensor *wq, nc_tensor *w_scale, nc_tensor *bias) {
    nc_tensor *in[4] = {x, wq, w_scale, bias};
    return apply(&op_linear_int8, in, bias ? 4 : 3, nullptr);
}
