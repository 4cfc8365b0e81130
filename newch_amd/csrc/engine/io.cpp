// NCW1 named-tensor files (reference: engine/src/core/io.c; format docs/FORMAT.md).  The bytes are
// the reference's, so files move freely between the two engines:
//
//   char[4] "NCW1" | u32 version (1) | u32 count
//   count x { u32 name_len | name | u32 dtype | u32 ndim | i64 shape[ndim] | u64 nbytes | row-major data }
//
// Tensor data moves between HBM and the file through a pinned staging buffer in two halves: the
// device-to-host copy of the next chunk runs while the current one is written, and the upload of a
// chunk runs while the next one is read.  Views are gathered on the device first.  Readers skip
// entries they were not asked for; validation and messages follow the reference.
#if !defined(_FILE_OFFSET_BITS)
#define _FILE_OFFSET_BITS 64
#endif
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "engine.hpp"

namespace nce {

constexpr uint32_t kFileVersion = 1;
constexpr uint32_t kMaxName = 4096;
constexpr size_t kStageHalf = (size_t)16 << 20;

static bool put(FILE *f, const void *p, size_t n) { return fwrite(p, 1, n, f) == n; }
static bool get(FILE *f, void *p, size_t n) { return fread(p, 1, n, f) == n; }

static char *stage(nc_ctx *ctx) {
    if (!ctx->io_stage && !hip_ok(ctx, hipHostMalloc((void **)&ctx->io_stage, 2 * kStageHalf, hipHostMallocDefault),
                                  "pinned staging buffer"))
        ctx->io_stage = nullptr;
    return ctx->io_stage;
}

// device bytes [src, src + bytes) to the file, two staging halves in flight
static bool write_device(nc_ctx *ctx, FILE *f, const char *src, size_t bytes) {
    char *st = stage(ctx);
    if (!st) return false;
    size_t off = 0;
    int cur = 0;
    if (bytes && !hip_ok(ctx, hipMemcpyAsync(st, src, std::min(kStageHalf, bytes), hipMemcpyDeviceToHost, ctx->stream),
                         "nc_save"))
        return false;
    while (off < bytes) {
        const size_t n = std::min(kStageHalf, bytes - off);
        if (!hip_ok(ctx, hipStreamSynchronize(ctx->stream), "nc_save")) return false;
        const size_t next = off + n;
        if (next < bytes &&
            !hip_ok(ctx, hipMemcpyAsync(st + (cur ^ 1) * kStageHalf, src + next, std::min(kStageHalf, bytes - next),
                                        hipMemcpyDeviceToHost, ctx->stream),
                    "nc_save"))
            return false;
        if (!put(f, st + cur * kStageHalf, n)) {
            (void)hipStreamSynchronize(ctx->stream);
            return false;
        }
        off = next;
        cur ^= 1;
    }
    return true;
}

// file bytes to device [dst, dst + bytes): a half is refilled only after its previous upload finished
static int read_device(nc_ctx *ctx, FILE *f, char *dst, size_t bytes) {  // 1 ok, 0 short read, -1 device
    char *st = stage(ctx);
    if (!st) return -1;
    hipEvent_t ev[2];
    bool pending[2] = {false, false};
    if (!hip_ok(ctx, hipEventCreateWithFlags(&ev[0], hipEventDisableTiming), "nc_load")) return -1;
    if (!hip_ok(ctx, hipEventCreateWithFlags(&ev[1], hipEventDisableTiming), "nc_load")) {
        (void)hipEventDestroy(ev[0]);
        return -1;
    }
    int rc = 1;
    size_t off = 0;
    int cur = 0;
    while (off < bytes) {
        const size_t n = std::min(kStageHalf, bytes - off);
        if (pending[cur] && !hip_ok(ctx, hipEventSynchronize(ev[cur]), "nc_load")) {
            rc = -1;
            break;
        }
        char *h = st + cur * kStageHalf;
        if (!get(f, h, n)) {
            rc = 0;
            break;
        }
        if (!hip_ok(ctx, hipMemcpyAsync(dst + off, h, n, hipMemcpyHostToDevice, ctx->stream), "nc_load") ||
            !hip_ok(ctx, hipEventRecord(ev[cur], ctx->stream), "nc_load")) {
            rc = -1;
            break;
        }
        pending[cur] = true;
        off += n;
        cur ^= 1;
    }
    if (!hip_ok(ctx, hipStreamSynchronize(ctx->stream), "nc_load")) rc = -1;
    (void)hipEventDestroy(ev[0]);
    (void)hipEventDestroy(ev[1]);
    return rc;
}

// host gather of a strided view (no device: storage is host memory)
static void gather_host(const nc_tensor *t, const char *base, char *dst) {
    const size_t es = dtype_size(t->dtype);
    const int64_t n = nc_numel(t);
    int64_t idx[NC_MAX_DIMS] = {0};
    for (int64_t i = 0; i < n; i++) {
        int64_t off = 0;
        for (int d = 0; d < t->ndim; d++) off += idx[d] * t->stride[d];
        memcpy(dst + (size_t)i * es, base + off * (int64_t)es, es);
        for (int d = t->ndim - 1; d >= 0; d--) {
            if (++idx[d] < t->shape[d]) break;
            idx[d] = 0;
        }
    }
}

static bool write_tensor(nc_ctx *ctx, FILE *f, nc_tensor *t, size_t bytes) {
    if (bytes == 0) return true;
    nc_tensor *o = owner_of(t);
    const bool on_device = ctx->device >= 0 && o->dev && (o->res & RES_DEV) && !(o->res & RES_MAPPED) &&
                           !(o->flags & TF_GRAD_FRESH);
    if (on_device) {
        const char *src = dptr(t);
        if (!src) return false;
        if (nc_is_contiguous(t)) return write_device(ctx, f, src, bytes);
        char *tmp = arena_alloc(ctx, bytes);
        if (!tmp || !hip_layer_ok(ctx, nc_hip_copy_strided((int)dtype_size(t->dtype), t->ndim, t->shape, src, t->stride,
                                                           tmp, ctx->stream),
                                  "nc_save"))
            return false;
        const bool ok = write_device(ctx, f, tmp, bytes);
        arena_free(ctx, tmp, bytes);
        return ok;
    }
    const char *h = hptr(t, false);  // host copy authoritative (or the only storage)
    if (!h) return false;
    if (nc_is_contiguous(t)) return put(f, h, bytes);
    char *tmp = (char *)malloc(bytes);
    if (!tmp) return false;
    gather_host(t, h, tmp);
    const bool ok = put(f, tmp, bytes);
    free(tmp);
    return ok;
}

}  // namespace nce

using namespace nce;

extern "C" {

nc_status nc_save(nc_ctx *ctx, const char *path, int n, const char *const *names, nc_tensor *const *tensors) {
    if (ctx->status != NC_OK) return ctx->status;
    for (int i = 0; i < n; i++) {
        if (!tensors[i] || !names[i]) {
            error(ctx, NC_ERR_ARG, "nc_save: entry %d has a NULL name or tensor", i);
            return ctx->status;
        }
    }
    FILE *f = fopen(path, "wb");
    if (!f) {
        error(ctx, NC_ERR_ARG, "nc_save: cannot open '%s' for writing", path);
        return ctx->status;
    }
    const uint32_t version = kFileVersion, count = (uint32_t)n;
    bool ok = put(f, "NCW1", 4) && put(f, &version, 4) && put(f, &count, 4);
    for (int i = 0; ok && i < n; i++) {
        nc_tensor *t = tensors[i];
        const uint32_t len = (uint32_t)strlen(names[i]), dt = (uint32_t)t->dtype, nd = (uint32_t)t->ndim;
        const uint64_t bytes = (uint64_t)nc_numel(t) * dtype_size(t->dtype);
        ok = put(f, &len, 4) && put(f, names[i], len) && put(f, &dt, 4) && put(f, &nd, 4) &&
             put(f, t->shape, sizeof(int64_t) * nd) && put(f, &bytes, 8) && write_tensor(ctx, f, t, (size_t)bytes);
    }
    if (fclose(f) != 0) ok = false;
    if (!ok && ctx->status == NC_OK) error(ctx, NC_ERR_ARG, "nc_save: write to '%s' failed", path);
    return ctx->status;
}

nc_status nc_load(nc_ctx *ctx, const char *path, int n, const char *const *names, nc_tensor *const *tensors) {
    if (ctx->status != NC_OK) return ctx->status;
    FILE *f = fopen(path, "rb");
    if (!f) {
        error(ctx, NC_ERR_ARG, "nc_load: cannot open '%s'", path);
        return ctx->status;
    }
    std::vector<unsigned char> found((size_t)(n > 0 ? n : 1), 0);
    std::vector<char> name(kMaxName + 1);
    char magic[4];
    uint32_t version = 0, count = 0;
    if (!get(f, magic, 4) || memcmp(magic, "NCW1", 4) != 0 || !get(f, &version, 4) || !get(f, &count, 4)) {
        error(ctx, NC_ERR_ARG, "nc_load: '%s' is not an NCW1 tensor file", path);
        fclose(f);
        return ctx->status;
    }
    if (version != kFileVersion) {
        error(ctx, NC_ERR_ARG, "nc_load: '%s' has unsupported version %u", path, version);
        fclose(f);
        return ctx->status;
    }
    for (uint32_t e = 0; e < count; e++) {
        uint32_t len, dt, nd;
        int64_t shape[NC_MAX_DIMS];
        uint64_t bytes;
        if (!get(f, &len, 4) || len > kMaxName || !get(f, name.data(), len) || !get(f, &dt, 4) || !get(f, &nd, 4) ||
            nd > NC_MAX_DIMS || !get(f, shape, sizeof(int64_t) * nd) || !get(f, &bytes, 8)) {
            error(ctx, NC_ERR_ARG, "nc_load: '%s' is truncated or corrupt", path);
            break;
        }
        name[len] = '\0';
        int idx = -1;
        for (int i = 0; i < n; i++)
            if (!found[i] && strcmp(names[i], name.data()) == 0) idx = i;
        if (idx < 0) {
            if (fseeko(f, (off_t)bytes, SEEK_CUR) != 0) {
                error(ctx, NC_ERR_ARG, "nc_load: '%s' is truncated", path);
                break;
            }
            continue;
        }
        nc_tensor *t = tensors[idx];
        bool same = t->dtype == (nc_dtype)dt && t->ndim == (int)nd;
        for (uint32_t d = 0; same && d < nd; d++) same = t->shape[d] == shape[d];
        if (!same) {
            char want[96], got[96];
            error(ctx, NC_ERR_SHAPE, "nc_load: '%s' is %s %s in the file but %s %s in the model", name.data(),
                  dtype_name((nc_dtype)dt), shape_str((int)nd, shape, got, sizeof got), dtype_name(t->dtype),
                  shape_str(t->ndim, t->shape, want, sizeof want));
            break;
        }
        // the byte count must be exactly the tensor's size: a larger one would overrun the storage
        if (bytes != (uint64_t)nc_numel(t) * dtype_size(t->dtype)) {
            error(ctx, NC_ERR_ARG, "nc_load: '%s' in '%s' is corrupt (%llu data bytes for %s)", name.data(), path,
                  (unsigned long long)bytes, dtype_name(t->dtype));
            break;
        }
        bool ok = nc_is_contiguous(t);
        if (ok && bytes) {
            if (ctx->device >= 0) {
                // every byte of t is about to be written; the rest of its owner is made current first
                char *dst = dptr_overwrite(t);
                const int rc = dst ? read_device(ctx, f, dst, (size_t)bytes) : 0;
                if (rc < 0) break;
                ok = rc == 1;
                if (ok) wrote_dev(t);
            } else {
                char *h = hptr(t, true);
                ok = h && get(f, h, (size_t)bytes);
            }
        }
        if (!ok) {
            error(ctx, NC_ERR_ARG, "nc_load: cannot read '%s' (truncated file or non-contiguous tensor)", name.data());
            break;
        }
        found[idx] = 1;
    }
    if (ctx->status == NC_OK) {
        for (int i = 0; i < n; i++) {
            if (!found[i]) {
                error(ctx, NC_ERR_ARG, "nc_load: '%s' not found in '%s'", names[i], path);
                break;
            }
        }
    }
    fclose(f);
    return ctx->status;
}

}  // extern "C"
