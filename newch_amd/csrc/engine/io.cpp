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

#include <string>

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


// ---- the file, entry by entry -------------------------------------------------------------------------
// One entry's header as stored: name, dtype, shape and the data byte count that follows it.
struct EntryHeader {
    std::string name;
    uint32_t dtype = 0;
    Dims dims;
    uint64_t bytes = 0;
};

class NcwWriter {
  public:
    NcwWriter(nc_ctx *ctx, FILE *f) : ctx_(ctx), f_(f) {}
    bool header(uint32_t count) {
        const uint32_t version = kFileVersion;
        return put(f_, "NCW1", 4) && put(f_, &version, 4) && put(f_, &count, 4);
    }
    bool entry(const char *name, nc_tensor *t) {
        const uint32_t len = (uint32_t)strlen(name), dt = (uint32_t)t->dtype, nd = (uint32_t)t->ndim;
        const uint64_t bytes = (uint64_t)nc_numel(t) * dtype_size(t->dtype);
        return put(f_, &len, 4) && put(f_, name, len) && put(f_, &dt, 4) && put(f_, &nd, 4) &&
               put(f_, t->shape, sizeof(int64_t) * nd) && put(f_, &bytes, 8) && write_tensor(ctx_, f_, t, (size_t)bytes);
    }

  private:
    nc_ctx *ctx_;
    FILE *f_;
};

class NcwReader {
  public:
    explicit NcwReader(FILE *f) : f_(f) {}
    // magic and version; on failure the reference's message for the problem found
    bool open(const char *path, nc_ctx *ctx) {
        char magic[4];
        uint32_t version = 0;
        if (!get(f_, magic, 4) || memcmp(magic, "NCW1", 4) != 0 || !get(f_, &version, 4) || !get(f_, &count_, 4)) {
            error(ctx, NC_ERR_ARG, "nc_load: '%s' is not an NCW1 tensor file", path);
            return false;
        }
        if (version != kFileVersion) {
            error(ctx, NC_ERR_ARG, "nc_load: '%s' has unsupported version %u", path, version);
            return false;
        }
        return true;
    }
    uint32_t count() const { return count_; }
    bool next(EntryHeader &h) {
        uint32_t len = 0, nd = 0;
        if (!get(f_, &len, 4) || len > kMaxName) return false;
        h.name.resize(len);
        if (!get(f_, &h.name[0], len) || !get(f_, &h.dtype, 4) || !get(f_, &nd, 4) || nd > NC_MAX_DIMS) return false;
        h.dims.rank = (int)nd;
        return get(f_, h.dims.e, sizeof(int64_t) * nd) && get(f_, &h.bytes, 8);
    }
    bool skip(uint64_t bytes) { return fseeko(f_, (off_t)bytes, SEEK_CUR) == 0; }
    // the entry's data into t (contiguous, exactly its size): 1 ok, 0 short read, -1 device error
    int read_into(nc_ctx *ctx, nc_tensor *t, uint64_t bytes) {
        if (!bytes) return 1;
        if (ctx->device < 0) {
            char *h = hptr(t, true);
            return h && get(f_, h, (size_t)bytes) ? 1 : 0;
        }
        // every byte of t is about to be written; the rest of its owner is made current first
        char *dst = dptr_overwrite(t);
        if (!dst) return 0;
        const int rc = read_device(ctx, f_, dst, (size_t)bytes);
        if (rc == 1) wrote_dev(t);
        return rc;
    }

  private:
    FILE *f_;
    uint32_t count_ = 0;
};

// The requested tensors by name.  A name asked for twice takes the file's entries from its last
// request backwards, as the reference's lookup does.
class Wanted {
  public:
    Wanted(int n, const char *const *names) : done_((size_t)(n > 0 ? n : 0), 0) {
        for (int i = 0; i < n; i++) by_name_[names[i]].push_back(i);
    }
    int claim(const std::string &name) {  // the index an entry of this name fills, or -1
        auto it = by_name_.find(name);
        if (it == by_name_.end()) return -1;
        for (auto k = it->second.rbegin(); k != it->second.rend(); ++k)
            if (!done_[(size_t)*k]) return *k;
        return -1;
    }
    void fill(int i) { done_[(size_t)i] = 1; }
    int first_missing() const {
        for (size_t i = 0; i < done_.size(); i++)
            if (!done_[i]) return (int)i;
        return -1;
    }

  private:
    std::unordered_map<std::string, std::vector<int>> by_name_;
    std::vector<char> done_;
};

// Why entry h cannot go into t, as the reference reports it (NC_OK when it can).
static nc_status check_entry(nc_ctx *ctx, const char *path, const EntryHeader &h, const nc_tensor *t) {
    const Dims want = Dims::of(t);
    bool same = t->dtype == (nc_dtype)h.dtype && want.rank == h.dims.rank;
    for (int d = 0; same && d < want.rank; d++) same = want.e[d] == h.dims.e[d];
    if (!same) {
        char tw[96], tg[96];
        error(ctx, NC_ERR_SHAPE, "nc_load: '%s' is %s %s in the file but %s %s in the model", h.name.c_str(),
              dtype_name((nc_dtype)h.dtype), h.dims.text(tg, sizeof tg), dtype_name(t->dtype), want.text(tw, sizeof tw));
        return NC_ERR_SHAPE;
    }
    // the byte count must be exactly the tensor's size: a larger one would overrun the storage
    if (h.bytes != (uint64_t)want.numel() * dtype_size(t->dtype)) {
        error(ctx, NC_ERR_ARG, "nc_load: '%s' in '%s' is corrupt (%llu data bytes for %s)", h.name.c_str(), path,
              (unsigned long long)h.bytes, dtype_name(t->dtype));
        return NC_ERR_ARG;
    }
    return NC_OK;
}

static nc_status load_entries(nc_ctx *ctx, const char *path, NcwReader &rd, Wanted &wanted, nc_tensor *const *tensors) {
    EntryHeader h;
    for (uint32_t e = 0; e < rd.count(); e++) {
        if (!rd.next(h)) {
            error(ctx, NC_ERR_ARG, "nc_load: '%s' is truncated or corrupt", path);
            return ctx->status;
        }
        const int idx = wanted.claim(h.name);
        if (idx < 0) {
            if (!rd.skip(h.bytes)) {
                error(ctx, NC_ERR_ARG, "nc_load: '%s' is truncated", path);
                return ctx->status;
            }
            continue;
        }
        nc_tensor *t = tensors[idx];
        if (check_entry(ctx, path, h, t) != NC_OK) return ctx->status;
        const int rc = nc_is_contiguous(t) ? rd.read_into(ctx, t, h.bytes) : 0;
        if (rc < 0) return ctx->status;  // the device error is recorded
        if (rc == 0) {
            error(ctx, NC_ERR_ARG, "nc_load: cannot read '%s' (truncated file or non-contiguous tensor)", h.name.c_str());
            return ctx->status;
        }
        wanted.fill(idx);
    }
    return NC_OK;
}

}  // namespace nce

using namespace nce;

extern "C" {

nc_status nc_save(nc_ctx *ctx, const char *path, int n, const char *const *names, nc_tensor *const *tensors) {
    if (ctx->status != NC_OK) return ctx->status;
    for (int i = 0; i < n; i++)
        if (!tensors[i] || !names[i]) {
            error(ctx, NC_ERR_ARG, "nc_save: entry %d has a NULL name or tensor", i);
            return ctx->status;
        }
    FILE *f = fopen(path, "wb");
    if (!f) {
        error(ctx, NC_ERR_ARG, "nc_save: cannot open '%s' for writing", path);
        return ctx->status;
    }
    NcwWriter w(ctx, f);
    bool ok = w.header((uint32_t)n);
    for (int i = 0; ok && i < n; i++) ok = w.entry(names[i], tensors[i]);
    ok = fclose(f) == 0 && ok;
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
    NcwReader rd(f);
    Wanted wanted(n, names);
    if (rd.open(path, ctx) && load_entries(ctx, path, rd, wanted, tensors) == NC_OK) {
        const int miss = wanted.first_missing();
        if (miss >= 0) error(ctx, NC_ERR_ARG, "nc_load: '%s' not found in '%s'", names[miss], path);
    }
    fclose(f);
    return ctx->status;
}

}  // extern "C"
