// Tensors: creation, accessors, residency (device storage + lazy host mirror), broadcasting
// helpers, gradient buffers.  Reference: engine/src/core/tensor.c.
#include <math.h>
#include <stdio.h>
#include <stdlib.h>

#include "engine.hpp"

namespace nce {

size_t dtype_size(nc_dtype dt) {
    switch (dt) {
    case NC_F32: return 4;
    case NC_I32: return 4;
    case NC_F16: return 2;
    case NC_I8: return 1;
    case NC_U8: return 1;
    default: return 0;
    }
}

const char *dtype_name(nc_dtype dt) {
    switch (dt) {
    case NC_F32: return "f32";
    case NC_I32: return "i32";
    case NC_F16: return "f16";
    case NC_I8: return "i8";
    case NC_U8: return "u8";
    default: return "?";
    }
}

int64_t shape_numel(int nd, const int64_t *shape) {
    int64_t n = 1;
    for (int i = 0; i < nd; i++) n *= shape[i];
    return n;
}

void contig_strides(int nd, const int64_t *shape, int64_t *st) {
    int64_t s = 1;
    for (int i = nd - 1; i >= 0; i--) {
        st[i] = s;
        s *= shape[i];
    }
}

int norm_axis(int axis, int nd) {
    if (axis < 0) axis += nd;
    return (axis >= 0 && axis < nd) ? axis : -1;
}

bool same_shape(const nc_tensor *a, const nc_tensor *b) {
    if (a->ndim != b->ndim) return false;
    for (int i = 0; i < a->ndim; i++)
        if (a->shape[i] != b->shape[i]) return false;
    return true;
}

const char *shape_str(int nd, const int64_t *shape, char *buf, size_t size) {
    size_t pos = (size_t)snprintf(buf, size, "[");
    for (int i = 0; i < nd && pos < size; i++)
        pos += (size_t)snprintf(buf + pos, size - pos, i ? ", %lld" : "%lld", (long long)shape[i]);
    if (pos < size) snprintf(buf + pos, size - pos, "]");
    return buf;
}

Dims Dims::of(const nc_tensor *t) {
    Dims d;
    d.rank = t->ndim;
    for (int i = 0; i < t->ndim; i++) d.e[i] = t->shape[i];
    return d;
}

const char *Dims::text(char *buf, size_t size) const { return shape_str(rank, e, buf, size); }

nc_status reject(const nc_node *n, nc_status code, const char *fmt, ...) {
    nc_ctx *ctx = n->in[0]->ctx;
    if (ctx->status == NC_OK) {
        ctx->status = code;
        va_list ap;
        va_start(ap, fmt);
        vsnprintf(ctx->err, sizeof ctx->err, fmt, ap);
        va_end(ap);
    }
    return code;
}

bool inputs_f32(const nc_node *n, int first, int count) {
    for (int i = first; i < first + count; i++)
        if (n->in[i]->dtype != NC_F32) {
            reject(n, NC_ERR_DTYPE, "%s: input %d must be f32, got %s", n->op->name, i, dtype_name(n->in[i]->dtype));
            return false;
        }
    return true;
}

void bcast_strides_shape(int tn, const int64_t *tshape, int nd, const int64_t *shape, int64_t *out) {
    int64_t ts[NC_MAX_DIMS];
    contig_strides(tn, tshape, ts);
    for (int i = 0; i < nd; i++) {
        int j = i - (nd - tn);
        out[i] = (j < 0 || (tshape[j] == 1 && shape[i] != 1)) ? 0 : ts[j];
    }
}

void bcast_strides(const nc_tensor *t, int nd, const int64_t *shape, int64_t *out) {
    for (int i = 0; i < nd; i++) {
        int j = i - (nd - t->ndim);
        out[i] = (j < 0 || (t->shape[j] == 1 && shape[i] != 1)) ? 0 : t->stride[j];
    }
}

static bool check_shape(nc_ctx *ctx, int nd, const int64_t *shape) {
    if (nd < 0 || nd > NC_MAX_DIMS) {
        error(ctx, NC_ERR_SHAPE, "ndim %d out of range [0, %d]", nd, NC_MAX_DIMS);
        return false;
    }
    const int64_t limit = INT64_MAX / 8;
    int64_t n = 1;
    for (int i = 0; i < nd; i++) {
        if (shape[i] < 0) {
            error(ctx, NC_ERR_SHAPE, "negative dimension %lld", (long long)shape[i]);
            return false;
        }
        if (shape[i] && n > limit / shape[i]) {
            char sb[160];
            error(ctx, NC_ERR_SHAPE, "shape %s has too many elements", shape_str(nd, shape, sb, sizeof sb));
            return false;
        }
        n *= shape[i];
    }
    return true;
}

nc_tensor *tensor_new(nc_ctx *ctx, nc_dtype dt, int nd, const int64_t *shape, bool persistent) {
    if (!ctx || !check_shape(ctx, nd, shape)) return nullptr;
    if (dtype_size(dt) == 0) {
        error(ctx, NC_ERR_DTYPE, "unknown dtype %d", (int)dt);
        return nullptr;
    }
    nc_tensor *t = (nc_tensor *)host_alloc(ctx, sizeof(nc_tensor), persistent);
    if (!t) return nullptr;
    t->ctx = ctx;
    t->dtype = dt;
    t->ndim = nd;
    if (nd) memcpy(t->shape, shape, (size_t)nd * sizeof(int64_t));
    contig_strides(nd, t->shape, t->stride);
    t->bytes = (size_t)shape_numel(nd, shape) * dtype_size(dt);
    if (ctx->device >= 0) {
        const bool was = ctx->storage_alloc;
        ctx->storage_alloc = true;  // tensor storage, never an op's scratch
        t->dev = dev_alloc(ctx, t->bytes, persistent);
        ctx->storage_alloc = was;
        if (!t->dev) {
            if (persistent) free(t);
            return nullptr;
        }
        t->res = RES_DEV;
    } else {
        // no device: host storage only (shape logic works, compute ops report the missing device)
        t->host = forced_alloc_failure(ctx) ? nullptr : (char *)calloc(1, t->bytes ? t->bytes : 1);
        if (!t->host) {
            error(ctx, NC_ERR_OOM, "out of host memory");
            return nullptr;
        }
        if (!persistent) ctx->temp_host.push_back(t->host);
        t->res = RES_HOST;
    }
    t->flags |= TF_OWNS_DATA;
    if (persistent) {
        t->flags |= TF_PERSISTENT;
        ctx->persistent.insert(t);
    }
    return t;
}

nc_tensor *tensor_alias(const nc_tensor *src, bool persistent) {
    nc_tensor *t = (nc_tensor *)host_alloc(src->ctx, sizeof(nc_tensor), persistent);
    if (!t) return nullptr;
    *t = *src;
    t->grad = nullptr;
    t->node = nullptr;
    t->name = nullptr;
    t->owner = owner_of(src);
    t->dev = nullptr;
    t->host = nullptr;
    t->bytes = 0;
    t->res = 0;
    t->flags = persistent ? TF_PERSISTENT : 0;
    return t;
}

// ---- residency -------------------------------------------------------------------------------------
// A grad buffer still marked fresh holds no data yet: give it its zeros before anyone reads it.  The
// mark lives on the storage owner, so a view of a lazily zeroed grad (reshape, transpose, slice of
// nc_grad(p) after nc_zero_grad) reads zeros too.
static bool materialize(nc_tensor *t) {
    nc_tensor *o = owner_of(t);
    if (!(o->flags & TF_GRAD_FRESH)) return true;
    return fill_zero(o);
}

// Device address of t's element 0 for a caller about to overwrite every element of t: a write that
// covers the owner's whole storage needs neither the lazy zeros nor the host copy; a partial one
// first makes the rest of the storage current on the device.
char *dptr_overwrite(nc_tensor *t) {
    nc_tensor *o = owner_of(t);
    if (!need_device(t->ctx, "op")) return nullptr;
    const size_t span = (size_t)shape_numel(t->ndim, t->shape) * dtype_size(t->dtype);
    if (t->offset == 0 && span == o->bytes && nc_is_contiguous(t) && o->dev) {
        o->flags &= ~TF_GRAD_FRESH;
        return o->dev;
    }
    return dptr(t);
}

char *dptr(nc_tensor *t) {
    nc_tensor *o = owner_of(t);
    nc_ctx *ctx = t->ctx;
    if (!need_device(ctx, "op")) return nullptr;
    if (!materialize(t)) return nullptr;
    if (!o->dev) {
        error(ctx, NC_ERR_STATE, "tensor has no device storage (released?)");
        return nullptr;
    }
    if (!(o->res & RES_DEV) || (o->res & RES_MAPPED)) {
        // the host copy is authoritative: upload it (stream-ordered before the consumer)
        if (!hip_ok(ctx, hipMemcpyAsync(o->dev, o->host, o->bytes, hipMemcpyHostToDevice, ctx->stream), "upload"))
            return nullptr;
        if (!hip_ok(ctx, hipStreamSynchronize(ctx->stream), "upload")) return nullptr;
        if (!(o->res & RES_MAPPED)) o->res |= RES_DEV;
    }
    return o->dev + t->offset * (int64_t)dtype_size(t->dtype);
}

void wrote_dev(nc_tensor *t) {
    nc_tensor *o = owner_of(t);
    o->res = RES_DEV;
    o->wgen++;
}

char *hptr(nc_tensor *t, bool write) {
    nc_tensor *o = owner_of(t);
    nc_ctx *ctx = t->ctx;
    if (!materialize(t)) return nullptr;
    if (!o->host) {
        o->host = (char *)malloc(o->bytes ? o->bytes : 1);
        if (!o->host) {
            error(ctx, NC_ERR_OOM, "out of host memory (mirror of %zu bytes)", o->bytes);
            return nullptr;
        }
        if (!(o->flags & TF_PERSISTENT)) ctx->temp_host.push_back(o->host);
    }
    if (!(o->res & RES_HOST)) {
        if (!o->dev) return nullptr;
        if (!hip_ok(ctx, hipMemcpyAsync(o->host, o->dev, o->bytes, hipMemcpyDeviceToHost, ctx->stream), "download") ||
            !hip_ok(ctx, hipStreamSynchronize(ctx->stream), "download"))
            return nullptr;
        o->res |= RES_HOST;
    }
    if (write && o->dev) o->res = RES_HOST | RES_MAPPED;
    if (write) o->wgen++;
    return o->host + t->offset * (int64_t)dtype_size(t->dtype);
}

bool fill_zero(nc_tensor *t) {
    t->flags &= ~TF_GRAD_FRESH;
    if (t->ctx->device < 0) {
        char *h = hptr(t, true);
        if (h) memset(h, 0, t->bytes);
        return h != nullptr;
    }
    char *p = dptr(t);
    if (!p) return false;
    const int64_t n = shape_numel(t->ndim, t->shape);
    if (!hip_layer_ok(t->ctx, nc_hip_fill(p, (int)dtype_size(t->dtype), 0, n, t->ctx->stream), "zero fill"))
        return false;
    wrote_dev(t);
    return true;
}

float *contig_f32(nc_tensor *t) {
    if (nc_is_contiguous(t)) return fptr(t);
    nc_ctx *ctx = t->ctx;
    const int64_t n = shape_numel(t->ndim, t->shape);
    char *src = dptr(t);
    if (!src) return nullptr;
    float *buf = (float *)arena_alloc(ctx, (size_t)n * sizeof(float));
    if (!buf) return nullptr;
    if (!hip_layer_ok(ctx, nc_hip_copy_strided(4, t->ndim, t->shape, src, t->stride, buf, ctx->stream),
                      "contiguous copy"))
        return nullptr;
    return buf;
}

nc_tensor *grad_buf(nc_tensor *t) {
    if (t->grad && (t->flags & TF_GRAD_CLEARED)) {
        if (!fill_zero(t->grad)) return nullptr;
        t->flags &= ~TF_GRAD_CLEARED;
        t->grad->flags |= TF_GRAD_FRESH;
    }
    if (!t->grad) {
        const bool persistent = (t->flags & TF_PERSISTENT) != 0;
        t->grad = tensor_new(t->ctx, NC_F32, t->ndim, t->shape, persistent);
        if (!t->grad) return nullptr;
        // zeroed lazily: the first kernel writing it stores instead of accumulating (grad_acc)
        t->grad->flags |= TF_GRAD_FRESH;
    }
    return t->grad;
}

int grad_acc(nc_tensor *x) {
    nc_tensor *g = x->grad;
    if (g->flags & TF_GRAD_FRESH) {
        g->flags &= ~TF_GRAD_FRESH;
        return 0;
    }
    return 1;
}

}  // namespace nce

using namespace nce;

extern "C" {

nc_tensor *nc_empty(nc_ctx *ctx, nc_dtype dt, int ndim, const int64_t *shape) {
    return tensor_new(ctx, dt, ndim, shape, persistent_mode(ctx));
}

nc_tensor *nc_zeros(nc_ctx *ctx, nc_dtype dt, int ndim, const int64_t *shape) {
    nc_tensor *t = nc_empty(ctx, dt, ndim, shape);
    if (t && !fill_zero(t)) return nullptr;
    return t;
}

nc_tensor *nc_full(nc_ctx *ctx, float value, int ndim, const int64_t *shape) {
    nc_tensor *t = nc_empty(ctx, NC_F32, ndim, shape);
    if (!t) return nullptr;
    if (ctx->device < 0) {
        float *h = (float *)hptr(t, true);
        for (int64_t i = 0, n = shape_numel(ndim, shape); i < n; i++) h[i] = value;
        return t;
    }
    uint32_t bits;
    memcpy(&bits, &value, 4);
    if (!hip_layer_ok(ctx, nc_hip_fill(t->dev, 4, bits, shape_numel(ndim, shape), ctx->stream), "nc_full"))
        return nullptr;
    wrote_dev(t);
    return t;
}

nc_tensor *nc_randn(nc_ctx *ctx, float stddev, int ndim, const int64_t *shape) {
    nc_tensor *t = nc_empty(ctx, NC_F32, ndim, shape);
    if (!t) return nullptr;
    float *h = (float *)hptr(t, true);
    if (!h) return nullptr;
    for (int64_t i = 0, n = shape_numel(ndim, shape); i < n; i++) h[i] = stddev * rand_normal(ctx);
    return t;
}

nc_tensor *nc_rand_uniform(nc_ctx *ctx, float lo, float hi, int ndim, const int64_t *shape) {
    nc_tensor *t = nc_empty(ctx, NC_F32, ndim, shape);
    if (!t) return nullptr;
    float *h = (float *)hptr(t, true);
    if (!h) return nullptr;
    for (int64_t i = 0, n = shape_numel(ndim, shape); i < n; i++) h[i] = lo + (hi - lo) * rand_uniform01(ctx);
    return t;
}

nc_tensor *nc_from_data(nc_ctx *ctx, nc_dtype dt, const void *data, int ndim, const int64_t *shape) {
    nc_tensor *t = nc_empty(ctx, dt, ndim, shape);
    if (!t || !data) return t;
    if (ctx->device < 0) {
        memcpy(hptr(t, true), data, t->bytes);
        return t;
    }
    if (!hip_ok(ctx, hipMemcpyAsync(t->dev, data, t->bytes, hipMemcpyHostToDevice, ctx->stream), "nc_from_data") ||
        !hip_ok(ctx, hipStreamSynchronize(ctx->stream), "nc_from_data"))
        return nullptr;
    wrote_dev(t);
    return t;
}

nc_tensor *nc_from_device(nc_ctx *ctx, nc_dtype dt, const void *device_data, int ndim, const int64_t *shape) {
    if (!ctx || !need_device(ctx, "nc_from_device")) return nullptr;
    nc_tensor *t = nc_empty(ctx, dt, ndim, shape);
    if (!t || !device_data) return t;
    if (!hip_ok(ctx, hipMemcpyAsync(t->dev, device_data, t->bytes, hipMemcpyDeviceToDevice, ctx->stream),
                "nc_from_device"))
        return nullptr;
    wrote_dev(t);
    return t;
}

nc_tensor *nc_scalar(nc_ctx *ctx, float value) { return nc_full(ctx, value, 0, nullptr); }

nc_tensor *nc_parameter(nc_ctx *ctx, const nc_tensor *init, int ndim, const int64_t *shape) {
    nc_tensor *t = tensor_new(ctx, NC_F32, ndim, shape, true);
    if (!t) return nullptr;
    if (init) {
        if (init->dtype != NC_F32 || nc_numel(init) != nc_numel(t)) {
            error(ctx, NC_ERR_SHAPE, "parameter init has %lld elements, expected %lld", (long long)nc_numel(init),
                  (long long)nc_numel(t));
            return nullptr;
        }
        nc_tensor *src = const_cast<nc_tensor *>(init);
        if (ctx->device < 0) {
            if (!nc_copy_to(src, hptr(t, true), t->bytes)) return nullptr;
        } else {
            char *sp = dptr(src);
            if (!sp) return nullptr;
            if (!hip_layer_ok(ctx, nc_hip_copy_strided(4, src->ndim, src->shape, sp, src->stride, t->dev, ctx->stream),
                              "nc_parameter"))
                return nullptr;
            wrote_dev(t);
        }
    } else if (!fill_zero(t)) {
        return nullptr;
    }
    t->flags |= TF_REQUIRES_GRAD;
    return t;
}

int nc_ndim(const nc_tensor *t) { return t ? t->ndim : 0; }
const int64_t *nc_shape(const nc_tensor *t) { return t ? t->shape : nullptr; }
int64_t nc_numel(const nc_tensor *t) { return t ? shape_numel(t->ndim, t->shape) : 0; }
nc_dtype nc_get_dtype(const nc_tensor *t) { return t ? t->dtype : NC_F32; }
int nc_requires_grad(const nc_tensor *t) { return t ? needs_grad(t) : 0; }
nc_tensor *nc_grad(const nc_tensor *t) { return (t && !(t->flags & TF_GRAD_CLEARED)) ? t->grad : nullptr; }
int nc_is_persistent(const nc_tensor *t) { return t && (t->flags & TF_PERSISTENT) != 0; }

int64_t nc_dim(const nc_tensor *t, int axis) {
    if (!t) return 0;
    int a = norm_axis(axis, t->ndim);
    return a < 0 ? 0 : t->shape[a];
}

void nc_release(nc_tensor *t) {
    if (!t || !(t->flags & TF_PERSISTENT)) return;
    nc_ctx *ctx = t->ctx;
    if (t->grad) nc_release(t->grad);
    if (t->flags & TF_OWNS_DATA) {
        if (t->dev) {
            (void)hipStreamSynchronize(ctx->stream);  // queued kernels may still read it
            dev_free(ctx, t->dev, t->bytes, true);
        }
        free(t->host);
    }
    ctx->persistent.erase(t);
    free(t);
}

void nc_set_name(nc_tensor *t, const char *name) {
    if (t) t->name = name;
}
const char *nc_name(const nc_tensor *t) { return t && t->name ? t->name : ""; }

void nc_set_requires_grad(nc_tensor *t, int on) {
    if (!t) return;
    if (on && t->dtype != NC_F32) {
        error(t->ctx, NC_ERR_DTYPE, "only f32 tensors can require grad");
        return;
    }
    if (on) t->flags |= TF_REQUIRES_GRAD;
    else t->flags &= ~TF_REQUIRES_GRAD;
}

int nc_is_contiguous(const nc_tensor *t) {
    if (!t) return 0;
    int64_t s = 1;
    for (int i = t->ndim - 1; i >= 0; i--) {
        if (t->shape[i] != 1 && t->stride[i] != s) return 0;
        s *= t->shape[i];
    }
    return 1;
}

float *nc_data_f32(nc_tensor *t) {
    if (!t || t->dtype != NC_F32 || !nc_is_contiguous(t)) return nullptr;
    return (float *)hptr(t, true);
}

int32_t *nc_data_i32(nc_tensor *t) {
    if (!t || t->dtype != NC_I32 || !nc_is_contiguous(t)) return nullptr;
    return (int32_t *)hptr(t, true);
}

void *nc_device_ptr(nc_tensor *t) {
    if (!t) return nullptr;
    return dptr(t);
}

float nc_get(const nc_tensor *t, const int64_t *index) {
    if (!t) return NAN;
    nc_tensor *tt = const_cast<nc_tensor *>(t);
    if (!materialize(tt)) return NAN;
    nc_tensor *o = owner_of(tt);
    int64_t off = 0;
    for (int i = 0; i < t->ndim; i++) off += index[i] * t->stride[i];
    const size_t es = dtype_size(t->dtype);
    unsigned char buf[8] = {0};
    if ((o->res & RES_HOST) && o->host) {
        memcpy(buf, o->host + (t->offset + off) * (int64_t)es, es);
    } else {
        nc_ctx *ctx = t->ctx;
        if (!o->dev) return NAN;
        if (!hip_ok(ctx, hipMemcpyAsync(buf, o->dev + (t->offset + off) * (int64_t)es, es, hipMemcpyDeviceToHost,
                                        ctx->stream),
                    "nc_get") ||
            !hip_ok(ctx, hipStreamSynchronize(ctx->stream), "nc_get"))
            return NAN;
    }
    float f;
    switch (t->dtype) {
    case NC_F32: memcpy(&f, buf, 4); return f;
    case NC_I32: { int32_t v; memcpy(&v, buf, 4); return (float)v; }
    case NC_I8: return (float)(int8_t)buf[0];
    case NC_U8: return (float)buf[0];
    default: return NAN;
    }
}

float nc_item(const nc_tensor *t) {
    if (!t || nc_numel(t) != 1) return NAN;
    int64_t zero[NC_MAX_DIMS] = {0};
    return nc_get(t, zero);
}

int nc_copy_to(const nc_tensor *t, void *dst, size_t dst_bytes) {
    if (!t || !dst) return 0;
    nc_tensor *tt = const_cast<nc_tensor *>(t);
    nc_ctx *ctx = t->ctx;
    const int64_t n = nc_numel(t);
    const size_t es = dtype_size(t->dtype), need = (size_t)n * es;
    if (dst_bytes < need) {
        error(ctx, NC_ERR_ARG, "nc_copy_to: buffer has %zu bytes, need %zu", dst_bytes, need);
        return 0;
    }
    if (n == 0) return 1;
    if (!materialize(tt)) return 0;
    nc_tensor *o = owner_of(tt);
    if ((o->res & RES_HOST) && o->host) {
        // gather from the host copy
        const unsigned char *s = (const unsigned char *)o->host + t->offset * (int64_t)es;
        unsigned char *d = (unsigned char *)dst;
        if (nc_is_contiguous(t)) {
            memcpy(d, s, need);
            return 1;
        }
        int64_t idx[NC_MAX_DIMS] = {0};
        for (int64_t i = 0; i < n; i++) {
            int64_t off = 0;
            for (int k = 0; k < t->ndim; k++) off += idx[k] * t->stride[k];
            memcpy(d + i * es, s + off * es, es);
            for (int k = t->ndim - 1; k >= 0; k--) {
                if (++idx[k] < t->shape[k]) break;
                idx[k] = 0;
            }
        }
        return 1;
    }
    char *src = dptr(tt);
    if (!src) return 0;
    const void *from = src;
    if (!nc_is_contiguous(t)) {
        char *buf = arena_alloc(ctx, need);
        if (!buf) return 0;
        if (!hip_layer_ok(ctx, nc_hip_copy_strided((int)es, t->ndim, t->shape, src, t->stride, buf, ctx->stream),
                          "nc_copy_to"))
            return 0;
        from = buf;
    }
    if (!hip_ok(ctx, hipMemcpyAsync(dst, from, need, hipMemcpyDeviceToHost, ctx->stream), "nc_copy_to") ||
        !hip_ok(ctx, hipStreamSynchronize(ctx->stream), "nc_copy_to"))
        return 0;
    if (from != src) arena_free(ctx, (char *)from, need);
    return 1;
}

int nc_copy_from(nc_tensor *t, const void *src, size_t src_bytes) {
    if (!t || !src) return 0;
    nc_ctx *ctx = t->ctx;
    const size_t need = (size_t)nc_numel(t) * dtype_size(t->dtype);
    if (!nc_is_contiguous(t) || src_bytes != need) {
        error(ctx, NC_ERR_ARG, "nc_copy_from: need a contiguous tensor and exactly %zu bytes (got %zu)", need,
              src_bytes);
        return 0;
    }
    if (ctx->device < 0) {
        memcpy(hptr(t, true), src, need);
        return 1;
    }
    char *d = dptr_overwrite(t);
    if (!d) return 0;
    if (!hip_ok(ctx, hipMemcpyAsync(d, src, need, hipMemcpyHostToDevice, ctx->stream), "nc_copy_from") ||
        !hip_ok(ctx, hipStreamSynchronize(ctx->stream), "nc_copy_from"))
        return 0;
    wrote_dev(t);
    return 1;
}

void nc_print(const nc_tensor *t) {
    if (!t) {
        printf("tensor(NULL)\n");
        return;
    }
    printf("tensor(%s%s%s, %s, shape=[", t->name ? "\"" : "", t->name ? t->name : "", t->name ? "\"" : "",
           dtype_name(t->dtype));
    for (int i = 0; i < t->ndim; i++) printf(i ? ", %lld" : "%lld", (long long)t->shape[i]);
    printf("]%s)\n  ", needs_grad(t) ? ", grad" : "");
    const int64_t n = nc_numel(t), shown = n < 32 ? n : 32;
    int64_t idx[NC_MAX_DIMS] = {0};
    for (int64_t i = 0; i < shown; i++) {
        printf("%.5g ", nc_get(t, idx));
        for (int k = t->ndim - 1; k >= 0; k--) {
            if (++idx[k] < t->shape[k]) break;
            idx[k] = 0;
        }
    }
    printf(n > shown ? "... (%lld total)\n" : "\n", (long long)n);
}

}  // extern "C"
