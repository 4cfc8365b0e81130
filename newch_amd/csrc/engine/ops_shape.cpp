// Shape ops (views where the layout allows) and dtype conversion.
// Reference: engine/src/ops/ops_shape.c (views :12-294, to_dtype :463-515).
#include "engine.hpp"

namespace nce {

static nc_tensor *alias_with(nc_node *n, int nd, const int64_t *shape, const int64_t *stride, int64_t offset) {
    nc_tensor *t = tensor_alias(n->in[0], false);
    if (!t) return nullptr;
    t->ndim = nd;
    memcpy(t->shape, shape, sizeof(int64_t) * (size_t)nd);
    memcpy(t->stride, stride, sizeof(int64_t) * (size_t)nd);
    t->offset = offset;
    n->out = t;
    return t;
}

static nc_status same_shape_infer(nc_node *n, nc_dtype *dt, int *nd, int64_t *shape) {
    *dt = n->in[0]->dtype;
    *nd = n->in[0]->ndim;
    memcpy(shape, n->in[0]->shape, sizeof(int64_t) * (size_t)*nd);
    return NC_OK;
}

// gather a strided source layout (shape/stride/offset relative to x's storage) into out
static nc_status gather_into(nc_tensor *x, const int64_t *shape, const int64_t *stride, int64_t offset,
                             nc_tensor *out) {
    nc_ctx *ctx = out->ctx;
    nc_tensor *o = owner_of(x);
    if (!dptr(x)) return NC_ERR_STATE;
    const size_t es = dtype_size(x->dtype);
    char *src = o->dev + offset * (int64_t)es;
    char *dst = dptr(out);
    if (!dst) return NC_ERR_STATE;
    if (!hip_layer_ok(ctx, nc_hip_copy_strided((int)es, out->ndim, shape, src, stride, dst, stream(ctx)), "copy"))
        return NC_ERR_STATE;
    wrote_dev(out);
    return NC_OK;
}

static nc_status copy_fwd(nc_node *n) {
    nc_tensor *x = n->in[0];
    return gather_into(x, x->shape, x->stride, x->offset, n->out);
}

// grad layout equals the input's logical layout: a flat accumulate (axpy with alpha 1, as the reference)
static void flat_bwd(nc_node *n) {
    nc_tensor *x = n->in[0];
    nc_ctx *ctx = x->ctx;
    if (!grad_buf(x)) return;
    float *g = fptr(n->out->grad), *gi = fptr(x->grad);  // fptr gives a fresh buffer its zeros
    if (!g || !gi) return;
    if (!hip_layer_ok(ctx, nc_hip_axpy(nc_numel(x), 1.0f, g, gi, stream(ctx)), n->op->name)) return;
    wrote_dev(x->grad);
}

// ---- reshape ---------------------------------------------------------------------------------------
static nc_status reshape_infer(nc_node *n, nc_dtype *dt, int *nd, int64_t *shape) {
    nc_tensor *x = n->in[0];
    const int r = (int)n->p.i[NC_MAX_DIMS];
    int infer_at = -1;
    int64_t known = 1;
    for (int i = 0; i < r; i++) {
        shape[i] = n->p.i[i];
        if (shape[i] == -1 && infer_at < 0) infer_at = i;
        else if (shape[i] < 0) {
            error(x->ctx, NC_ERR_SHAPE, "reshape: invalid dimension %lld", (long long)shape[i]);
            return NC_ERR_SHAPE;
        } else known *= shape[i];
    }
    const int64_t total = nc_numel(x);
    if (infer_at >= 0) shape[infer_at] = known ? total / known : 0;
    if (shape_numel(r, shape) != total) {
        char sa[96], sb[96];
        error(x->ctx, NC_ERR_SHAPE, "reshape: cannot view %s as %s", shape_str(x->ndim, x->shape, sa, sizeof sa),
              shape_str(r, shape, sb, sizeof sb));
        return NC_ERR_SHAPE;
    }
    *dt = x->dtype;
    *nd = r;
    return NC_OK;
}

// Strides that show x's elements in row-major order as `shape`, if such strides exist (the view
// rule of torch's reshape).  x's non-unit dims are grouped into chunks, maximal runs stored back to
// back (innermost first); the new dims, innermost first, must tile those chunks exactly.
static bool view_strides(const nc_tensor *x, int nd, const int64_t *shape, int64_t *st) {
    if (nc_is_contiguous(x) || nc_numel(x) == 0) {
        contig_strides(nd, shape, st);
        return true;
    }
    int64_t chunk_n[NC_MAX_DIMS], chunk_s[NC_MAX_DIMS];
    int nchunks = 0;
    for (int d = x->ndim - 1; d >= 0; d--) {
        if (x->shape[d] == 1) continue;
        if (nchunks > 0 && x->stride[d] == chunk_s[nchunks - 1] * chunk_n[nchunks - 1]) {
            chunk_n[nchunks - 1] *= x->shape[d];
        } else {
            chunk_s[nchunks] = x->stride[d];
            chunk_n[nchunks] = x->shape[d];
            nchunks++;
        }
    }
    int c = 0;
    int64_t run = 1;
    for (int d = nd - 1; d >= 0; d--) {
        if (shape[d] == 1) {
            st[d] = (c < nchunks ? chunk_s[c] : 1) * run;
            continue;
        }
        if (c >= nchunks) return false;
        st[d] = chunk_s[c] * run;
        run *= shape[d];
        if (run > chunk_n[c]) return false;
        if (run == chunk_n[c]) {
            c++;
            run = 1;
        }
    }
    return c == nchunks;
}

static int reshape_view(nc_node *n, int nd, const int64_t *shape) {
    int64_t st[NC_MAX_DIMS];
    if (!view_strides(n->in[0], nd, shape, st)) return 0;
    return alias_with(n, nd, shape, st, n->in[0]->offset) != nullptr;
}

// gather for reshape copies runs over x's own shape (the element order is the same)
static nc_status reshape_copy(nc_node *n) {
    nc_tensor *x = n->in[0], *out = n->out;
    nc_ctx *ctx = out->ctx;
    if (!dptr(x)) return NC_ERR_STATE;
    const size_t es = dtype_size(x->dtype);
    char *dst = dptr(out);
    if (!dst) return NC_ERR_STATE;
    if (!hip_layer_ok(ctx,
                      nc_hip_copy_strided((int)es, x->ndim, x->shape, owner_of(x)->dev + x->offset * (int64_t)es,
                                          x->stride, dst, stream(ctx)),
                      "reshape"))
        return NC_ERR_STATE;
    wrote_dev(out);
    return NC_OK;
}
const OpDef op_reshape = {"reshape", OPF_VIEW, 0, reshape_infer, reshape_view, reshape_copy, flat_bwd};

// ---- transpose -------------------------------------------------------------------------------------
static nc_status transpose_infer(nc_node *n, nc_dtype *dt, int *nd, int64_t *shape) {
    nc_tensor *x = n->in[0];
    const int a0 = norm_axis((int)n->p.i[0], x->ndim), a1 = norm_axis((int)n->p.i[1], x->ndim);
    if (a0 < 0 || a1 < 0) {
        error(x->ctx, NC_ERR_ARG, "transpose: axes (%d, %d) out of range for %d-d tensor", (int)n->p.i[0],
              (int)n->p.i[1], x->ndim);
        return NC_ERR_ARG;
    }
    n->p.i[0] = a0;
    n->p.i[1] = a1;
    *dt = x->dtype;
    *nd = x->ndim;
    memcpy(shape, x->shape, sizeof(int64_t) * (size_t)x->ndim);
    shape[a0] = x->shape[a1];
    shape[a1] = x->shape[a0];
    return NC_OK;
}

static void swapped_strides(const nc_node *n, int64_t *st) {
    const nc_tensor *x = n->in[0];
    memcpy(st, x->stride, sizeof(int64_t) * (size_t)x->ndim);
    const int a0 = (int)n->p.i[0], a1 = (int)n->p.i[1];
    st[a0] = x->stride[a1];
    st[a1] = x->stride[a0];
}

static int transpose_view(nc_node *n, int nd, const int64_t *shape) {
    int64_t st[NC_MAX_DIMS];
    swapped_strides(n, st);
    return alias_with(n, nd, shape, st, n->in[0]->offset) != nullptr;
}

static nc_status transpose_fwd(nc_node *n) {
    int64_t st[NC_MAX_DIMS];
    swapped_strides(n, st);
    return gather_into(n->in[0], n->out->shape, st, n->in[0]->offset, n->out);
}

static void transpose_bwd(nc_node *n) {
    nc_tensor *x = n->in[0], *o = n->out;
    nc_ctx *ctx = x->ctx;
    if (!grad_buf(x)) return;
    // walk the contiguous out grad; write through x's contiguous strides, swapped
    int64_t st[NC_MAX_DIMS];
    contig_strides(x->ndim, x->shape, st);
    const int a0 = (int)n->p.i[0], a1 = (int)n->p.i[1];
    const int64_t t = st[a0];
    st[a0] = st[a1];
    st[a1] = t;
    float *g = fptr(o->grad), *gi = fptr(x->grad);
    if (!g || !gi) return;
    if (!hip_layer_ok(ctx, nc_hip_accumulate_strided(o->ndim, o->shape, g, gi, st, stream(ctx)), "transpose")) return;
    wrote_dev(x->grad);
}

const OpDef op_transpose = {"transpose", OPF_VIEW, 0, transpose_infer, transpose_view, transpose_fwd, transpose_bwd};

// ---- slice: x[..., start : start + len*step : step, ...] along one axis ----------------------------
static nc_status slice_infer(nc_node *n, nc_dtype *dt, int *nd, int64_t *shape) {
    nc_tensor *x = n->in[0];
    const int a = norm_axis((int)n->p.i[0], x->ndim);
    const int64_t start = n->p.i[1], len = n->p.i[2], step = n->p.i[3];
    if (a < 0) {
        error(x->ctx, NC_ERR_ARG, "slice: axis %d out of range for %d-d tensor", (int)n->p.i[0], x->ndim);
        return NC_ERR_ARG;
    }
    if (step < 1 || len < 0 || start < 0 || start > x->shape[a] ||
        (len > 0 && start + (len - 1) * step >= x->shape[a])) {
        error(x->ctx, NC_ERR_ARG, "slice: start %lld, length %lld, step %lld do not fit axis %d of size %lld",
              (long long)start, (long long)len, (long long)step, a, (long long)x->shape[a]);
        return NC_ERR_ARG;
    }
    n->p.i[0] = a;
    *dt = x->dtype;
    *nd = x->ndim;
    memcpy(shape, x->shape, sizeof(int64_t) * (size_t)x->ndim);
    shape[a] = len;
    return NC_OK;
}

static void sliced(const nc_node *n, int64_t *stride, int64_t *offset) {
    const nc_tensor *x = n->in[0];
    const int a = (int)n->p.i[0];
    memcpy(stride, x->stride, sizeof(int64_t) * (size_t)x->ndim);
    *offset = x->offset + (n->p.i[2] > 0 ? n->p.i[1] * x->stride[a] : 0);
    stride[a] = x->stride[a] * n->p.i[3];
}

static int slice_view(nc_node *n, int nd, const int64_t *shape) {
    int64_t st[NC_MAX_DIMS], off;
    sliced(n, st, &off);
    return alias_with(n, nd, shape, st, off) != nullptr;
}

static nc_status slice_fwd(nc_node *n) {
    int64_t st[NC_MAX_DIMS], off;
    sliced(n, st, &off);
    return gather_into(n->in[0], n->out->shape, st, off, n->out);
}

static void slice_bwd(nc_node *n) {
    nc_tensor *x = n->in[0], *o = n->out;
    nc_ctx *ctx = x->ctx;
    if (!grad_buf(x)) return;
    const int a = (int)n->p.i[0];
    if (o->shape[a] == 0) return;
    int64_t st[NC_MAX_DIMS];
    contig_strides(x->ndim, x->shape, st);
    float *g = fptr(o->grad), *gi = fptr(x->grad);
    if (!g || !gi) return;
    gi += n->p.i[1] * st[a];
    st[a] *= n->p.i[3];
    if (!hip_layer_ok(ctx, nc_hip_accumulate_strided(o->ndim, o->shape, g, gi, st, stream(ctx)), "slice")) return;
    wrote_dev(x->grad);
}

const OpDef op_slice = {"slice", OPF_VIEW, 0, slice_infer, slice_view, slice_fwd, slice_bwd};

// ---- contiguous / detach ---------------------------------------------------------------------------
static int contiguous_view(nc_node *n, int nd, const int64_t *shape) {
    if (!nc_is_contiguous(n->in[0])) return 0;
    return alias_with(n, nd, shape, n->in[0]->stride, n->in[0]->offset) != nullptr;
}
const OpDef op_contiguous = {"contiguous", OPF_VIEW, 0, same_shape_infer, contiguous_view, copy_fwd, flat_bwd};

static int detach_view(nc_node *n, int nd, const int64_t *shape) {
    return alias_with(n, nd, shape, n->in[0]->stride, n->in[0]->offset) != nullptr;
}
const OpDef op_detach = {"detach", OPF_VIEW | OPF_NONDIFF, 0, same_shape_infer, detach_view, copy_fwd, nullptr};

// ---- to_dtype --------------------------------------------------------------------------------------
static nc_status to_dtype_infer(nc_node *n, nc_dtype *dt, int *nd, int64_t *shape) {
    const nc_dtype to = (nc_dtype)n->p.i[0], from = n->in[0]->dtype;
    if (to == NC_F16 || from == NC_F16 || dtype_size(to) == 0) {
        error(n->in[0]->ctx, NC_ERR_DTYPE, "to_dtype: %s -> %s is not supported", dtype_name(from), dtype_name(to));
        return NC_ERR_DTYPE;
    }
    *dt = to;
    nc_dtype ignored;
    return same_shape_infer(n, &ignored, nd, shape);
}

static nc_status to_dtype_fwd(nc_node *n) {
    nc_tensor *x = n->in[0], *o = n->out;
    nc_ctx *ctx = o->ctx;
    const size_t es = dtype_size(x->dtype);
    const int64_t N = nc_numel(x);
    char *src = dptr(x);
    if (!src) return NC_ERR_STATE;
    if (!nc_is_contiguous(x)) {
        char *buf = arena_alloc(ctx, (size_t)N * es + 1);
        if (!buf || !hip_layer_ok(ctx, nc_hip_copy_strided((int)es, x->ndim, x->shape, src, x->stride, buf, stream(ctx)),
                                  "to_dtype"))
            return NC_ERR_STATE;
        src = buf;
    }
    char *dst = dptr(o);
    if (!dst || !hip_layer_ok(ctx, nc_hip_convert(x->dtype, o->dtype, N, src, dst, stream(ctx)), "to_dtype"))
        return NC_ERR_STATE;
    wrote_dev(o);
    return NC_OK;
}

const OpDef op_to_dtype = {"to_dtype", 0, 0, to_dtype_infer, nullptr, to_dtype_fwd, flat_bwd};

}  // namespace nce

using namespace nce;

extern "C" {

nc_tensor *nc_reshape(nc_tensor *x, int ndim, const int64_t *shape) {
    if (x && (ndim < 0 || ndim > NC_MAX_DIMS)) {
        error(x->ctx, NC_ERR_SHAPE, "reshape: ndim %d out of range", ndim);
        return nullptr;
    }
    Params p{};
    for (int i = 0; i < ndim; i++) p.i[i] = shape[i];
    p.i[NC_MAX_DIMS] = ndim;
    return apply(&op_reshape, &x, 1, &p);
}

nc_tensor *nc_transpose(nc_tensor *x, int axis0, int axis1) {
    Params p{};
    p.i[0] = axis0;
    p.i[1] = axis1;
    return apply(&op_transpose, &x, 1, &p);
}

nc_tensor *nc_slice(nc_tensor *x, int axis, int64_t start, int64_t length, int64_t step) {
    Params p{};
    p.i[0] = axis;
    p.i[1] = start;
    p.i[2] = length;
    p.i[3] = step;
    return apply(&op_slice, &x, 1, &p);
}

nc_tensor *nc_contiguous(nc_tensor *x) { return apply(&op_contiguous, &x, 1, nullptr); }
nc_tensor *nc_detach(nc_tensor *x) { return apply(&op_detach, &x, 1, nullptr); }

nc_tensor *nc_to_dtype(nc_tensor *x, nc_dtype dt) {
    if (x && dt != NC_F32) x = nc_detach(x);
    Params p{};
    p.i[0] = dt;
    return apply(&op_to_dtype, &x, 1, &p);
}

}  // extern "C"
