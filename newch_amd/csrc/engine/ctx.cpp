// Context: device selection and stream, host metadata arena, device step arena, persistent
// allocations, sticky errors, RNG, statistics.  Reference: engine/src/core/ctx.c.
#include <stdio.h>
#include <stdlib.h>
#include <unistd.h>

#include <algorithm>
#include <cmath>

#include "engine.hpp"

namespace nce {

static size_t align_up(size_t v, size_t a) { return (v + a - 1) & ~(a - 1); }

void error(nc_ctx *ctx, nc_status code, const char *fmt, ...) {
    if (!ctx || ctx->status != NC_OK) return;  // the first error sticks (ctx.c:375-382)
    ctx->status = code;
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(ctx->err, sizeof ctx->err, fmt, ap);
    va_end(ap);
}

bool hip_ok(nc_ctx *ctx, hipError_t e, const char *what) {
    if (e == hipSuccess) return true;
    error(ctx, e == hipErrorOutOfMemory ? NC_ERR_OOM : NC_ERR_STATE, "%s: HIP error %s", what, hipGetErrorString(e));
    return false;
}

bool hip_layer_ok(nc_ctx *ctx, int rc, const char *what) {
    if (rc == NC_HIP_OK) return true;
    error(ctx, rc == NC_HIP_ERR_ARG ? NC_ERR_ARG : NC_ERR_STATE, "%s: %s", what, nc_hip_last_error());
    return false;
}

bool need_device(nc_ctx *ctx, const char *what) {
    if (ctx->device >= 0) return true;
    error(ctx, NC_ERR_STATE, "%s: no HIP device (this engine computes on an MI355X only)", what);
    return false;
}

bool persistent_mode(const nc_ctx *ctx) { return ctx->persistent_depth > 0; }

// ---- host metadata ---------------------------------------------------------------------------------
void *host_alloc(nc_ctx *ctx, size_t bytes, bool persistent) {
    if (persistent) {
        void *p = calloc(1, bytes ? bytes : 1);
        if (!p) error(ctx, NC_ERR_OOM, "out of host memory (%zu bytes)", bytes);
        return p;
    }
    HostArena &h = ctx->harena;
    const size_t need = align_up(bytes ? bytes : 1, 64);
    if (need > kHostChunk / 4) {
        void *p = calloc(1, need);
        if (!p) {
            error(ctx, NC_ERR_OOM, "out of host memory (%zu bytes)", bytes);
            return nullptr;
        }
        h.big.push_back((char *)p);
        return p;
    }
    while (h.cur < h.chunks.size() && kHostChunk - h.used < need) {
        h.cur++;
        h.used = 0;
    }
    if (h.cur == h.chunks.size()) {
        char *c = (char *)malloc(kHostChunk);
        if (!c) {
            error(ctx, NC_ERR_OOM, "out of host memory");
            return nullptr;
        }
        h.chunks.push_back(c);
        h.used = 0;
    }
    char *p = h.chunks[h.cur] + h.used;
    h.used += need;
    memset(p, 0, need);
    return p;
}

void host_free(nc_ctx *, void *p) { free(p); }

// ---- device arena ------------------------------------------------------------------------------------
// NC_DEBUG_POISON=1 at nc_init (the reference's debug switch, ctx.c:41-56): every device block the
// context gives back -- a step-arena block on free, a persistent tensor before hipFree -- is filled
// with 0xCD bytes on the context's stream, so a kernel that reads released memory sees garbage
// instead of stale values.
static bool poison_env() {
    const char *v = getenv("NC_DEBUG_POISON");
    return v && v[0] && v[0] != '0';
}

static void poison(nc_ctx *ctx, char *p, size_t bytes) {
    if (ctx->poison && p && bytes && ctx->device >= 0) (void)nc_hip_fill(p, 1, 0xCD, (int64_t)bytes, ctx->stream);
}

// NC_FAIL_ALLOC_AT=N (read at nc_init): the context's N-th storage allocation request -- device
// allocations and, without a device, host tensor storage, counted from 1 -- fails as out of memory,
// so the sticky NC_ERR_OOM path and the recovery after it (nc_clear_error, nc_step_end) can be tested
// without exhausting the device.
static uint64_t fail_alloc_env() {
    const char *v = getenv("NC_FAIL_ALLOC_AT");
    return v && *v ? strtoull(v, nullptr, 10) : 0;
}

bool forced_alloc_failure(nc_ctx *ctx) { return ++ctx->storage_requests == ctx->fail_alloc_at; }

// every device allocation the context makes goes through here (counted for nc_device_alloc_count)
static hipError_t device_malloc(nc_ctx *ctx, char **p, size_t bytes) {
    if (forced_alloc_failure(ctx)) return hipErrorOutOfMemory;
    const hipError_t e = hipMalloc((void **)p, bytes);
    if (e == hipSuccess) ctx->device_allocs++;
    return e;
}

static void large_trim(nc_ctx *ctx) {
    DevArena &a = ctx->darena;
    const size_t budget = std::max(a.large_peak, a.large_prev_peak);
    while (!a.large_cache.empty() && a.large_live_bytes + a.large_cache_bytes > budget) {
        auto it = std::prev(a.large_cache.end());  // largest first
        (void)hipFree(it->second);
        a.large_cache_bytes -= it->first;
        a.reserved -= it->first;
        a.large_cache.erase(it);
    }
}

static void note_use(DevArena &a, size_t n) {
    a.in_use += n;
    a.peak = std::max(a.peak, a.in_use);
}

char *arena_alloc(nc_ctx *ctx, size_t bytes) {
    if (!need_device(ctx, "arena")) return nullptr;
    DevArena &a = ctx->darena;
    const size_t need = align_up(bytes ? bytes : 1, kDevAlign);
    char *p = nullptr;
    if (need >= a.chunk_bytes / 4) {
        // a cached block of the same size (up to 1/4 larger), else a new one
        auto it = a.large_cache.lower_bound(need);
        if (it != a.large_cache.end() && it->first <= need + need / 4) {
            p = it->second;
            const size_t sz = it->first;
            a.large_cache.erase(it);
            a.large_cache_bytes -= sz;
            a.large_live[p] = sz;
            a.large_live_bytes += sz;
            note_use(a, sz);
        } else {
            hipError_t e = device_malloc(ctx, &p, need);
            if (e == hipErrorOutOfMemory && !a.large_cache.empty()) {  // give cached blocks back, retry
                for (auto &kv : a.large_cache) (void)hipFree(kv.second), a.reserved -= kv.first;
                a.large_cache.clear();
                a.large_cache_bytes = 0;
                (void)hipGetLastError();
                e = device_malloc(ctx, &p, need);
            }
            if (!hip_ok(ctx, e, "device arena (large block)")) return nullptr;
            a.reserved += need;
            a.large_live[p] = need;
            a.large_live_bytes += need;
            note_use(a, need);
        }
        a.large_peak = std::max(a.large_peak, a.large_live_bytes);
        large_trim(ctx);
    } else {
        // best fit among blocks freed during this step (<= 1/4 slack)
        size_t best = SIZE_MAX;
        for (size_t i = 0; i < a.free_small.size(); i++) {
            const size_t sz = a.free_small[i].second;
            if (sz >= need && sz <= need + need / 4 && (best == SIZE_MAX || sz < a.free_small[best].second)) {
                best = i;
                if (sz == need) break;
            }
        }
        if (best != SIZE_MAX) {
            p = a.free_small[best].first;
            note_use(a, a.free_small[best].second);
            a.free_small[best] = a.free_small.back();
            a.free_small.pop_back();
        } else {
            while (a.cur < a.chunks.size() && a.chunks[a.cur].cap - a.chunks[a.cur].used < need) a.cur++;
            if (a.cur == a.chunks.size()) {
                char *base = nullptr;
                if (!hip_ok(ctx, device_malloc(ctx, &base, a.chunk_bytes), "device arena (chunk)")) return nullptr;
                a.chunks.push_back({base, a.chunk_bytes, 0});
                a.reserved += a.chunk_bytes;
            }
            DevArena::Chunk &c = a.chunks[a.cur];
            p = c.base + c.used;
            c.used += need;
            note_use(a, need);
        }
    }
    if (ctx->scratch && !ctx->storage_alloc) ctx->scratch->add(p, need);
    return p;
}

void arena_free(nc_ctx *ctx, char *p, size_t bytes) {
    if (!p) return;
    DevArena &a = ctx->darena;
    auto it = a.large_live.find(p);
    if (it != a.large_live.end()) {
        const size_t sz = it->second;
        poison(ctx, p, sz);
        a.large_live.erase(it);
        a.large_live_bytes -= sz;
        a.large_cache.insert({sz, p});
        a.large_cache_bytes += sz;
        a.in_use -= sz;
        large_trim(ctx);
        return;
    }
    const size_t need = align_up(bytes ? bytes : 1, kDevAlign);
    poison(ctx, p, need);
    a.free_small.push_back({p, need});
    a.in_use -= need;
}

char *dev_alloc(nc_ctx *ctx, size_t bytes, bool persistent) {
    if (!persistent) return arena_alloc(ctx, bytes);
    if (!need_device(ctx, "allocation")) return nullptr;
    char *p = nullptr;
    if (!hip_ok(ctx, device_malloc(ctx, &p, align_up(bytes ? bytes : 1, kDevAlign)), "device allocation (persistent)"))
        return nullptr;
    ctx->persistent_bytes += bytes;
    return p;
}

void dev_free(nc_ctx *ctx, char *p, size_t bytes, bool persistent) {
    if (!p) return;
    if (persistent) {
        if (ctx->poison) {
            poison(ctx, p, bytes);
            (void)hipStreamSynchronize(ctx->stream);
        }
        (void)hipFree(p);
        ctx->persistent_bytes -= bytes;
    } else {
        arena_free(ctx, p, bytes);
    }
}

// ---- RNG: xoshiro256** seeded by splitmix64 (the reference's generator, ctx.c:295-298,414-435) ----
static uint64_t splitmix64(uint64_t *x) {
    uint64_t z = (*x += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

static inline uint64_t rotl(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }

static uint64_t rng_next(nc_ctx *ctx) {
    uint64_t *s = ctx->rng;
    const uint64_t r = rotl(s[1] * 5, 7) * 9;
    const uint64_t t = s[1] << 17;
    s[2] ^= s[0];
    s[3] ^= s[1];
    s[1] ^= s[2];
    s[0] ^= s[3];
    s[2] ^= t;
    s[3] = rotl(s[3], 45);
    return r;
}

float rand_uniform01(nc_ctx *ctx) { return (float)(rng_next(ctx) >> 40) * (1.0f / 16777216.0f); }

float rand_normal(nc_ctx *ctx) {
    float u1 = rand_uniform01(ctx), u2 = rand_uniform01(ctx);
    if (u1 < 1e-7f) u1 = 1e-7f;
    return sqrtf(-2.0f * logf(u1)) * cosf(6.2831853f * u2);
}

void detect_cpu(nc_cpu_info *info) {
    memset(info, 0, sizeof *info);
    info->arch = "x86_64";
#if defined(__x86_64__)
    __builtin_cpu_init();
    info->has_avx2 = __builtin_cpu_supports("avx2");
    info->has_fma = __builtin_cpu_supports("fma");
#endif
    long n = sysconf(_SC_NPROCESSORS_ONLN);
    info->n_cores = n > 0 ? (int)n : 1;
    info->n_big_cores = info->n_cores;
}

static int env_device() {
    const char *v = getenv("NC_DEVICE");
    if (!v || !*v) return 0;
    if (!strncmp(v, "hip:", 4)) v += 4;
    return atoi(v);
}

static void release_device(nc_ctx *ctx) {
    if (ctx->own_stream && ctx->stream) (void)hipStreamDestroy(ctx->stream);
    ctx->stream = nullptr;
    ctx->own_stream = false;
}

static bool bind_device(nc_ctx *ctx, int dev) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) {
        (void)hipGetLastError();
        ctx->device = -1;
        snprintf(ctx->backend, sizeof ctx->backend, "hip:none");
        return false;
    }
    if (dev < 0 || dev >= n) {
        error(ctx, NC_ERR_ARG, "device %d out of range (%d visible)", dev, n);
        return false;
    }
    if (!hip_ok(ctx, hipSetDevice(dev), "hipSetDevice")) return false;
    release_device(ctx);
    hipStream_t s = nullptr;
    // a default-priority non-blocking stream of our own
    if (!hip_ok(ctx, hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "hipStreamCreate")) return false;
    ctx->stream = s;
    ctx->own_stream = true;
    ctx->device = dev;
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, dev) == hipSuccess)
        snprintf(ctx->backend, sizeof ctx->backend, "hip:%.40s", prop.gcnArchName);
    else
        snprintf(ctx->backend, sizeof ctx->backend, "hip");
    return true;
}

}  // namespace nce

using namespace nce;

extern "C" {

nc_ctx *nc_init(const nc_config *cfg) {
    nc_ctx *ctx = new (std::nothrow) nc_ctx();
    if (!ctx) return nullptr;
    nc_config c{};
    if (cfg) c = *cfg;
    if (c.arena_chunk_bytes) ctx->darena.chunk_bytes = align_up(c.arena_chunk_bytes, kDevAlign);
    nc_manual_seed(ctx, c.seed);
    ctx->poison = poison_env();
    ctx->fail_alloc_at = fail_alloc_env();
    detect_cpu(&ctx->cpu);
    ctx->n_threads = c.threads > 0 ? c.threads : ctx->cpu.n_cores;
    ctx->n_threads = std::min(std::max(ctx->n_threads, 1), 64);
    bind_device(ctx, env_device());
    return ctx;
}

void nc_manual_seed(nc_ctx *ctx, uint64_t seed) {
    uint64_t s = seed ? seed : 0x6E63u;
    for (int i = 0; i < 4; i++) ctx->rng[i] = splitmix64(&s);
}

void nc_step_end(nc_ctx *ctx) {
    HostArena &h = ctx->harena;
    h.cur = 0;
    h.used = 0;
    for (char *p : h.big) free(p);
    h.big.clear();
    for (void *p : ctx->temp_host) free(p);
    ctx->temp_host.clear();
    DevArena &a = ctx->darena;
    for (auto &c : a.chunks) c.used = 0;
    a.cur = 0;
    a.free_small.clear();
    for (auto &kv : a.large_live) {
        a.large_cache.insert({kv.second, kv.first});
        a.large_cache_bytes += kv.second;
    }
    a.large_live.clear();
    a.large_live_bytes = 0;
    a.in_use = 0;
    a.large_prev_peak = a.large_peak;
    a.large_peak = 0;
    large_trim(ctx);
    ctx->tape.clear();
}

void nc_arena_trim(nc_ctx *ctx) {
    DevArena &a = ctx->darena;
    std::vector<DevArena::Chunk> keep;
    for (auto &c : a.chunks) {
        if (c.used == 0) {
            (void)hipFree(c.base);
            a.reserved -= c.cap;
        } else {
            keep.push_back(c);
        }
    }
    a.chunks.swap(keep);
    a.cur = 0;
    for (auto &kv : a.large_cache) {
        (void)hipFree(kv.second);
        a.reserved -= kv.first;
    }
    a.large_cache.clear();
    a.large_cache_bytes = 0;
}

void nc_free_ctx(nc_ctx *ctx) {
    if (!ctx) return;
    if (ctx->device >= 0) {
        (void)hipSetDevice(ctx->device);
        (void)hipStreamSynchronize(ctx->stream);
    }
    nc_step_end(ctx);
    while (!ctx->optims.empty()) nc_optim_free(ctx->optims.back());
    if (ctx->io_stage) (void)hipHostFree(ctx->io_stage);
    if (ctx->loss_flag) (void)hipHostFree(ctx->loss_flag);
    for (nc_tensor *t : ctx->persistent) {
        if (t->dev && (t->flags & TF_OWNS_DATA)) (void)hipFree(t->dev);
        free(t->host);
        free(t);
    }
    ctx->persistent.clear();
    nc_arena_trim(ctx);
    for (auto &c : ctx->darena.chunks) (void)hipFree(c.base);
    for (auto &kv : ctx->darena.large_live) (void)hipFree(kv.first);
    for (char *c : ctx->harena.chunks) free(c);
    release_device(ctx);
    delete ctx;
}

int nc_num_threads(const nc_ctx *ctx) { return ctx->n_threads; }
void nc_persistent_begin(nc_ctx *ctx) { ctx->persistent_depth++; }
void nc_persistent_end(nc_ctx *ctx) {
    if (ctx->persistent_depth > 0) ctx->persistent_depth--;
}
int nc_set_grad_enabled(nc_ctx *ctx, int enabled) {
    int prev = ctx->grad_enabled;
    ctx->grad_enabled = enabled ? 1 : 0;
    return prev;
}
int nc_ok(const nc_ctx *ctx) { return ctx->status == NC_OK; }
nc_status nc_status_code(const nc_ctx *ctx) { return ctx->status; }
const char *nc_error(const nc_ctx *ctx) { return ctx->status == NC_OK ? "" : ctx->err; }
void nc_clear_error(nc_ctx *ctx) {
    ctx->status = NC_OK;
    ctx->err[0] = '\0';
}

nc_mem_stats nc_get_mem_stats(const nc_ctx *ctx) {
    nc_mem_stats s;
    s.persistent_bytes = ctx->persistent_bytes;
    s.arena_bytes_in_use = ctx->darena.in_use;
    s.arena_bytes_reserved = ctx->darena.reserved;
    s.arena_peak_bytes = ctx->darena.peak;
    return s;
}
void nc_reset_peak(nc_ctx *ctx) { ctx->darena.peak = ctx->darena.in_use; }
const nc_cpu_info *nc_cpu(const nc_ctx *ctx) { return &ctx->cpu; }
const char *nc_kernel_backend(const nc_ctx *ctx) { return ctx->backend; }

// ---- device extensions -------------------------------------------------------------------------------
int nc_device_count(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) {
        (void)hipGetLastError();
        return 0;
    }
    return n;
}

int nc_set_device(nc_ctx *ctx, int device) {
    if (!ctx) return 0;
    if (!ctx->persistent.empty() || ctx->darena.in_use) {
        error(ctx, NC_ERR_STATE, "nc_set_device: the context already holds tensors");
        return 0;
    }
    return bind_device(ctx, device) ? 1 : 0;
}

int nc_get_device(const nc_ctx *ctx) { return ctx ? ctx->device : -1; }

uint64_t nc_device_alloc_count(const nc_ctx *ctx) { return ctx ? ctx->device_allocs : 0; }

void nc_set_stream(nc_ctx *ctx, void *stream) {
    if (!ctx || ctx->device < 0) return;
    if (!stream) {
        bind_device(ctx, ctx->device);
        return;
    }
    (void)hipStreamSynchronize(ctx->stream);
    release_device(ctx);
    ctx->stream = (hipStream_t)stream;
    ctx->own_stream = false;
}

void *nc_get_stream(const nc_ctx *ctx) { return ctx ? (void *)ctx->stream : nullptr; }

nc_status nc_synchronize(nc_ctx *ctx) {
    if (!ctx) return NC_ERR_ARG;
    if (ctx->device < 0) return ctx->status;
    hip_ok(ctx, hipStreamSynchronize(ctx->stream), "nc_synchronize");
    return ctx->status;
}

}  // extern "C"
