// Shape ops (views where the layout allows, copies otherwise) and dtype conversion.
// Reference: engine/src/ops/ops_shape.c (reshape / transpose / slice / contiguous / detach :12-294,
// to_dtype :463-515); the error messages and the view-or-copy results are the reference's.
//
// Every shape op here is described by one function: the Layout of its output over its input's
// storage (extents, element strides, offset of element 0).  The alias rule turns that layout into a
// view; the forward, used when a view is not allowed (persistent mode) or not possible, gathers the
// same layout into new contiguous storage; the backward scatters the output gradient back through
// the layout's strides taken over the contiguous gradient of the input.
#include "engine.hpp"

namespace nce {

struct Layout {
    Dims dims;
    int64_t st[NC_MAX_DIMS] = {};
    int64_t offset = 0;

    static Layout of(const nc_tensor *t) {
        Layout L;
        L.dims = Dims::of(t);
        memcpy(L.st, t->stride, sizeof(int64_t) * (size_t)t->ndim);
        L.offset = t->offset;
        return L;
    }
};

// the output as a view of in[0]'s storage
static bool view_of(nc_node *n, const Layout &L) {
    nc_tensor *t = tensor_alias(n->in[0], false);
    if (!t) return false;
    t->ndim = L.dims.rank;
    memcpy(t->shape, L.dims.e, sizeof(int64_t) * (size_t)L.dims.rank);
    memcpy(t->stride, L.st, sizeof(int64_t) * (size_t)L.dims.rank);
    t->offset = L.offset;
    n->out = t;
    return true;
}

// the elements L shows in in[0]'s storage, in row-major order of L, into the output's new storage
static nc_status gather(nc_node *n, const Layout &L) {
    nc_tensor *x = n->in[0], *out = n->out;
    nc_ctx *ctx = out->ctx;
    const size_t es = dtype_size(x->dtype);
    if (!dptr(x)) return NC_ERR_STATE;
    const char *src = owner_of(x)->dev + L.offset * (int64_t)es;
    char *dst = dptr_overwrite(out);
    if (!dst ||
        !hip_layer_ok(ctx, nc_hip_copy_strided((int)es, L.dims.rank, L.dims.e, src, L.st, dst, stream(ctx)),
                      n->op->name))
        return NC_ERR_STATE;
    wrote_dev(out);
    return NC_OK;
}

// ---- contiguous copy and flat gradient ---------------------------------------------------------
static nc_status copy_fwd(nc_node *n) { return gather(n, Layout::of(n->in[0])); }

// same logical layout on both sides: a flat accumulate (axpy with alpha 1)
static void flat_bwd(nc_node *n) {
    nc_tensor *x = n->in[0];
    const float *g = grad_buf(x) ? fptr(n->out->grad) : nullptr;
    float *gx = g ? fptr(x->grad) : nullptr;  // a fresh buffer gets its zeros here
    if (!gx || !hip_layer_ok(x->ctx, nc_hip_axpy(nc_numel(x), 1.0f, g, gx, stream(x->ctx)), n->op->name)) return;
    wrote_dev(x->grad);
}

// ---- reshape: p.i[0 .. rank) the requested extents (at most one -1), p.i[NC_MAX_DIMS] the rank ------
static nc_status reshape_shape(nc_node *n, OutSpec &out) {
    const Dims x = Dims::of(n->in[0]);
    out.dtype = n->in[0]->dtype;
    int free_at = -1;  // the extent to infer
    int64_t fixed = 1;
    for (int i = 0; i < (int)n->p.i[NC_MAX_DIMS]; i++) {
        const int64_t e = n->p.i[i];
        if (e == -1 && free_at < 0)
            free_at = i;
        else if (e < 0)
            return reject(n, NC_ERR_SHAPE, "reshape: invalid dimension %lld", (long long)e);
        else
            fixed *= e;
        out.dims.push(e);
    }
    if (free_at >= 0) out.dims.e[free_at] = fixed ? x.numel() / fixed : 0;
    if (out.dims.numel() != x.numel()) {
        char tx[96], to[96];
        return reject(n, NC_ERR_SHAPE, "reshape: cannot view %s as %s", x.text(tx, sizeof tx),
                      out.dims.text(to, sizeof to));
    }
    return NC_OK;
}

// Strides that show x's elements in row-major order with the new extents, when they exist (the view
// rule of torch's reshape): x's non-unit axes, innermost first, merge into runs stored back to back;
// the new extents, innermost first, must split those runs exactly.
static bool reshape_layout(const nc_tensor *x, const Dims &to, Layout &L) {
    L.dims = to;
    L.offset = x->offset;
    if (nc_is_contiguous(x) || nc_numel(x) == 0) {
        contig_strides(to.rank, to.e, L.st);
        return true;
    }
    struct Run {
        int64_t len, step;
    } runs[NC_MAX_DIMS];
    int nruns = 0;
    for (int d = x->ndim - 1; d >= 0; d--) {
        if (x->shape[d] == 1) continue;
        Run *last = nruns ? &runs[nruns - 1] : nullptr;
        if (last && x->stride[d] == last->step * last->len)
            last->len *= x->shape[d];
        else
            runs[nruns++] = {x->shape[d], x->stride[d]};
    }
    int r = 0;
    int64_t within = 1;  // elements of run r covered so far
    for (int d = to.rank - 1; d >= 0; d--) {
        const int64_t e = to.e[d];
        if (e == 1) {  // any stride works: the one the next axis would have
            L.st[d] = (r < nruns ? runs[r].step : 1) * within;
            continue;
        }
        if (r == nruns) return false;
        L.st[d] = runs[r].step * within;
        within *= e;
        if (within > runs[r].len || runs[r].len % within) return false;
        if (within == runs[r].len) {
            r++;
            within = 1;
        }
    }
    return r == nruns;
}

static bool reshape_alias(nc_node *n, const OutSpec &out) {
    Layout L;
    return reshape_layout(n->in[0], out.dims, L) && view_of(n, L);
}

// a reshape copy keeps the element order: gather x over its own extents
const OpDef op_reshape = {"reshape", OPF_VIEW, 0, reshape_shape, reshape_alias, copy_fwd, flat_bwd};

// ---- transpose: p.i[0], p.i[1] the two axes (normalized by the shape rule) --------------------------
static nc_status transpose_shape(nc_node *n, OutSpec &out) {
    const Dims x = Dims::of(n->in[0]);
    const int a = norm_axis((int)n->p.i[0], x.rank), b = norm_axis((int)n->p.i[1], x.rank);
    if (a < 0 || b < 0)
        return reject(n, NC_ERR_ARG, "transpose: axes (%d, %d) out of range for %d-d tensor", (int)n->p.i[0],
                      (int)n->p.i[1], x.rank);
    n->p.i[0] = a;
    n->p.i[1] = b;
    out.dtype = n->in[0]->dtype;
    out.dims = x;
    std::swap(out.dims.e[a], out.dims.e[b]);
    return NC_OK;
}

static Layout transposed(const nc_node *n) {
    Layout L = Layout::of(n->in[0]);
    const int a = (int)n->p.i[0], b = (int)n->p.i[1];
    std::swap(L.dims.e[a], L.dims.e[b]);
    std::swap(L.st[a], L.st[b]);
    return L;
}

static bool transpose_alias(nc_node *n, const OutSpec &) { return view_of(n, transposed(n)); }
static nc_status transpose_fwd(nc_node *n) { return gather(n, transposed(n)); }

// ---- slice: x[..., start : start + len*step : step, ...] along one axis ------------------------------
// p.i[0] axis (normalized by the shape rule), p.i[1] start, p.i[2] length, p.i[3] step
static nc_status slice_shape(nc_node *n, OutSpec &out) {
    const Dims x = Dims::of(n->in[0]);
    const int a = norm_axis((int)n->p.i[0], x.rank);
    const int64_t start = n->p.i[1], len = n->p.i[2], step = n->p.i[3];
    if (a < 0) return reject(n, NC_ERR_ARG, "slice: axis %d out of range for %d-d tensor", (int)n->p.i[0], x.rank);
    const bool fits = step >= 1 && len >= 0 && start >= 0 && start <= x.e[a] &&
                      (len == 0 || start + (len - 1) * step < x.e[a]);
    if (!fits)
        return reject(n, NC_ERR_ARG, "slice: start %lld, length %lld, step %lld do not fit axis %d of size %lld",
                      (long long)start, (long long)len, (long long)step, a, (long long)x.e[a]);
    n->p.i[0] = a;
    out.dtype = n->in[0]->dtype;
    out.dims = x;
    out.dims.e[a] = len;
    return NC_OK;
}

static Layout sliced(const nc_node *n) {
    Layout L = Layout::of(n->in[0]);
    const int a = (int)n->p.i[0];
    if (n->p.i[2] > 0) L.offset += n->p.i[1] * L.st[a];
    L.dims.e[a] = n->p.i[2];
    L.st[a] *= n->p.i[3];
    return L;
}

static bool slice_alias(nc_node *n, const OutSpec &) { return view_of(n, sliced(n)); }
static nc_status slice_fwd(nc_node *n) { return gather(n, sliced(n)); }

// transpose / slice backward: the output gradient (contiguous) is added into x's contiguous gradient
// at the places the layout picked, i.e. through the layout rebuilt over x's contiguous strides
static void layout_bwd(nc_node *n, const Layout &over_grad) {
    nc_tensor *x = n->in[0], *o = n->out;
    if (!grad_buf(x) || nc_numel(o) == 0) return;  // an empty output adds nothing to x's (zero) gradient
    const float *g = fptr(o->grad);
    float *gx = g ? fptr(x->grad) : nullptr;
    if (!gx || !hip_layer_ok(x->ctx,
                             nc_hip_accumulate_strided(o->ndim, o->shape, g, gx + over_grad.offset, over_grad.st,
                                                       stream(x->ctx)),
                             n->op->name))
        return;
    wrote_dev(x->grad);
}

// x's layout with contiguous strides and no offset: the layout of x's gradient buffer
static Layout dense_of(const nc_tensor *x) {
    Layout L;
    L.dims = Dims::of(x);
    contig_strides(x->ndim, x->shape, L.st);
    return L;
}

static void transpose_bwd(nc_node *n) {
    Layout L = dense_of(n->in[0]);
    const int a = (int)n->p.i[0], b = (int)n->p.i[1];
    std::swap(L.st[a], L.st[b]);
    layout_bwd(n, L);
}

static void slice_bwd(nc_node *n) {
    Layout L = dense_of(n->in[0]);
    const int a = (int)n->p.i[0];
    if (n->p.i[2] > 0) L.offset = n->p.i[1] * L.st[a];
    L.st[a] *= n->p.i[3];
    layout_bwd(n, L);
}

const OpDef op_transpose = {"transpose", OPF_VIEW, 0, transpose_shape, transpose_alias, transpose_fwd, transpose_bwd};
const OpDef op_slice = {"slice", OPF_VIEW, 0, slice_shape, slice_alias, slice_fwd, slice_bwd};

// ---- contiguous / detach ---------------------------------------------------------------------------
static nc_status keep_shape(nc_node *n, OutSpec &out) {
    out.dtype = n->in[0]->dtype;
    out.dims = Dims::of(n->in[0]);
    return NC_OK;
}

static bool contiguous_alias(nc_node *n, const OutSpec &) {
    return nc_is_contiguous(n->in[0]) && view_of(n, Layout::of(n->in[0]));
}
static bool detach_alias(nc_node *n, const OutSpec &) { return view_of(n, Layout::of(n->in[0])); }

const OpDef op_contiguous = {"contiguous", OPF_VIEW, 0, keep_shape, contiguous_alias, copy_fwd, flat_bwd};
const OpDef op_detach = {"detach", OPF_VIEW | OPF_NONDIFF, 0, keep_shape, detach_alias, copy_fwd, nullptr};

// ---- to_dtype: p.i[0] the target dtype ---------------------------------------------------------------
static nc_status to_dtype_shape(nc_node *n, OutSpec &out) {
    const nc_dtype to = (nc_dtype)n->p.i[0], from = n->in[0]->dtype;
    if (to == NC_F16 || from == NC_F16 || dtype_size(to) == 0)
        return reject(n, NC_ERR_DTYPE, "to_dtype: %s -> %s is not supported", dtype_name(from), dtype_name(to));
    keep_shape(n, out);
    out.dtype = to;
    return NC_OK;
}

static nc_status to_dtype_fwd(nc_node *n) {
    nc_tensor *x = n->in[0], *o = n->out;
    nc_ctx *ctx = o->ctx;
    const size_t es = dtype_size(x->dtype);
    const int64_t N = nc_numel(x);
    const char *src = dptr(x);
    if (src && !nc_is_contiguous(x)) {  // pack first: the converter reads a dense run
        char *packed = arena_alloc(ctx, (size_t)N * es + 1);
        if (!packed ||
            !hip_layer_ok(ctx, nc_hip_copy_strided((int)es, x->ndim, x->shape, src, x->stride, packed, stream(ctx)),
                          "to_dtype"))
            return NC_ERR_STATE;
        src = packed;
    }
    char *dst = dptr_overwrite(o);
    if (!src || !dst || !hip_layer_ok(ctx, nc_hip_convert(x->dtype, o->dtype, N, src, dst, stream(ctx)), "to_dtype"))
        return NC_ERR_STATE;
    wrote_dev(o);
    return NC_OK;
}

// only f32 -> f32 is on the tape (other targets detach first); its gradient passes straight through
const OpDef op_to_dtype = {"to_dtype", 0, 0, to_dtype_shape, nullptr, to_dtype_fwd, flat_bwd};

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
