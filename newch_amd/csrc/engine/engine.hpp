// Internal definitions of the MI355X newch engine (not installed).
//
// The engine behind the reference's C API (include/nc.h): tensors whose storage is device memory
// (HBM), ops that enqueue nc_hip_* kernels (include/nc_hip.h) on the context's HIP stream, and
// reverse-mode autograd over a tape of recorded calls.  The pieces:
//   * nc_tensor: shape / element strides / offset over an owner's storage; the storage is device
//     memory with a lazily created host mirror and residency bits, so host-visible accessors copy
//     on demand and host writes are uploaded before device use;
//   * OpDef: an op's shape rule (validate the inputs, describe the output as an OutSpec), an
//     optional alias rule (the output as a view of the input), and forward / backward launchers;
//   * Scratch: the arena blocks one op call allocates for itself (workspaces, gathered operands),
//     returned when the call ends; only state an op declares saved outlives its forward;
//   * the tape: the recorded nodes in call order, walked newest to oldest by the backward pass;
//   * DevArena: a device bump arena freed in O(1) by nc_step_end, with a size-keyed cache of large
//     blocks so steady-state steps never call hipMalloc.
#pragma once

#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdint.h>
#include <string.h>

#include <map>
#include <unordered_map>
#include <unordered_set>
#include <utility>
#include <vector>

#include "nc.h"
#include "nc_hip.h"

namespace nce {

constexpr size_t kDevAlign = 256;
constexpr int kMaxInputs = 6;
constexpr size_t kDefaultDevChunk = size_t(64) << 20;
constexpr size_t kHostChunk = size_t(1) << 20;

// tensor flags (same meaning as the reference's NC_TF_*, nc_internal.h:19-30) plus GRAD_FRESH
enum : uint32_t {
    TF_REQUIRES_GRAD = 1u << 0,
    TF_PERSISTENT = 1u << 1,
    TF_OWNS_DATA = 1u << 2,
    TF_GRAD_CLEARED = 1u << 3,
    TF_ON_TAPE = 1u << 4,
    TF_GRAD_FRESH = 1u << 5,  // grad buffer is all zeros and unwritten: kernels may store instead of add
};
// residency of an owner's storage
// RES_MAPPED: a host pointer was handed out (nc_data_f32 / nc_data_i32) and the host copy stays
// authoritative: every device read re-uploads it, until a kernel writes the storage.
enum : uint32_t { RES_DEV = 1u, RES_HOST = 2u, RES_MAPPED = 4u };

enum : uint32_t { OPF_ELEMENTWISE = 1u, OPF_REDUCTION = 2u, OPF_VIEW = 4u, OPF_NONDIFF = 8u };

}  // namespace nce

struct nc_node;

struct nc_tensor {
    nc_ctx *ctx;
    nc_dtype dtype;
    int ndim;
    uint32_t flags;
    int64_t shape[NC_MAX_DIMS];
    int64_t stride[NC_MAX_DIMS];  // elements
    int64_t offset;               // elements from the owner's storage base to this view's element 0
    // storage (meaningful on owners: owner == NULL)
    char *dev;        // device base (NULL when the context has no device)
    char *host;       // host mirror base (lazily allocated)
    size_t bytes;     // storage bytes
    uint32_t res;     // RES_DEV | RES_HOST: which copies are current
    uint64_t wgen;    // write generation: bumped by every device write and every host pointer handed out for writing
    nc_tensor *grad;  // contiguous, same logical shape
    nc_node *node;
    nc_tensor *owner;  // views: the storage owner
    const char *name;
};

namespace nce {

struct Params {
    int64_t i[NC_MAX_DIMS + 2];
    float f[4];
};

// A shape as a value: rank and extents (the right-aligned view of numpy broadcasting is `back`).
struct Dims {
    int rank = 0;
    int64_t e[NC_MAX_DIMS] = {};

    static Dims of(const nc_tensor *t);
    int64_t numel() const {
        int64_t n = 1;
        for (int i = 0; i < rank; i++) n *= e[i];
        return n;
    }
    int64_t back(int k) const { return e[rank - 1 - k]; }  // k-th extent from the last
    void push(int64_t v) { e[rank++] = v; }
    // the reference's text for a shape, "[2, 3]"
    const char *text(char *buf, size_t size) const;
};

// Output description produced by an op's shape rule.
struct OutSpec {
    nc_dtype dtype = NC_F32;
    Dims dims;
};

struct OpDef {
    const char *name;
    uint32_t flags;
    int kind;
    nc_status (*shape)(nc_node *n, OutSpec &out);          // validate the inputs, describe the output
    bool (*alias)(nc_node *n, const OutSpec &out);         // set n->out to a view of in[0]; may be NULL
    nc_status (*forward)(nc_node *n);
    void (*backward)(nc_node *n);  // NULL = not differentiable
};

}  // namespace nce

struct nc_node {
    const nce::OpDef *op;
    nc_tensor *in[nce::kMaxInputs];
    int n_in;
    nc_tensor *out;
    nce::Params p;
    void *saved;  // state the backward needs (declared by the forward with save_state)
    size_t saved_bytes;
    uint32_t seq;   // position on the context's tape
    bool released;  // a FREE_GRAPH backward freed its activation
};

namespace nce {

// Device step arena: bump allocation from large device chunks, a within-step free list for small
// blocks and dedicated cached blocks for large ones (the reference's arena policy, ctx.c:68-264,
// sized for HBM).
struct DevArena {
    size_t chunk_bytes = kDefaultDevChunk;
    struct Chunk {
        char *base;
        size_t cap, used;
    };
    std::vector<Chunk> chunks;
    size_t cur = 0;
    std::vector<std::pair<char *, size_t>> free_small;
    std::multimap<size_t, char *> large_cache;
    std::unordered_map<char *, size_t> large_live;
    size_t large_live_bytes = 0, large_cache_bytes = 0, large_peak = 0, large_prev_peak = 0;
    size_t in_use = 0, reserved = 0, peak = 0;
};

struct HostArena {
    std::vector<char *> chunks;
    size_t cur = 0, used = 0;
    std::vector<char *> big;  // oversize requests, freed at step end
};

// The arena blocks one op call allocates for itself (workspaces, gathered operands): every raw
// arena_alloc made while the scope is open is recorded and handed back when it closes.  The return
// is stream-ordered -- the kernels that use a block are already queued on the context's stream -- so
// the next op may reuse it at once.  Blocks that must outlive the call (a forward's saved state)
// are claimed with keep(); tensor storage never counts as scratch.  Scopes nest (an op calling
// another op's entry point): each closes its own blocks.
class Scratch {
  public:
    explicit Scratch(nc_ctx *ctx);
    ~Scratch();
    Scratch(const Scratch &) = delete;
    Scratch &operator=(const Scratch &) = delete;
    void add(char *p, size_t bytes) { blocks_.push_back({p, bytes}); }
    void keep(const void *p);

  private:
    nc_ctx *ctx_;
    Scratch *outer_;
    std::vector<std::pair<char *, size_t>> blocks_;
};

}  // namespace nce

struct nc_ctx {
    nce::HostArena harena;
    nce::DevArena darena;
    size_t persistent_bytes = 0;
    std::unordered_set<nc_tensor *> persistent;  // owned headers, freed at nc_free_ctx
    std::vector<void *> temp_host;               // host mirrors of temporaries, freed at step end

    int persistent_depth = 0;
    int grad_enabled = 1;
    std::vector<nc_node *> tape;      // recorded nodes in call order, cleared by nc_step_end
    nce::Scratch *scratch = nullptr;  // the innermost open op call's scratch
    bool storage_alloc = false;       // tensor storage is being allocated: never scratch

    nc_status status = NC_OK;
    char err[256] = {0};

    uint64_t rng[4] = {0, 0, 0, 0};
    nc_cpu_info cpu{};
    int n_threads = 1;

    std::vector<nc_optim *> optims;  // live optimizers, freed at nc_free_ctx
    char *io_stage = nullptr;        // pinned staging for NCW1 file I/O (two halves), allocated on first use
    uint64_t *loss_flag = nullptr;   // pinned, device-mapped word: the loss forwards' first-bad-label key
    uint64_t *loss_flag_dev = nullptr;  // the same word as the kernels address it

    uint64_t device_allocs = 0;  // hipMalloc calls made for this context (arena chunks, large blocks, persistent)
    bool poison = false;         // NC_DEBUG_POISON: released device blocks are filled with 0xCD
    uint64_t storage_requests = 0;  // storage allocations asked for (device allocations, host storage)
    uint64_t fail_alloc_at = 0;     // NC_FAIL_ALLOC_AT: this request fails as out of memory (0: none)
    int device = -1;  // -1: no HIP device
    hipStream_t stream = nullptr;
    bool own_stream = false;
    char backend[64] = {0};
};

namespace nce {

// ---- context / memory (ctx.cpp) --------------------------------------------------------------------
void error(nc_ctx *ctx, nc_status code, const char *fmt, ...);
bool hip_ok(nc_ctx *ctx, hipError_t e, const char *what);  // records a device error, returns e == success
bool hip_layer_ok(nc_ctx *ctx, int rc, const char *what);   // same for nc_hip_* return codes
bool need_device(nc_ctx *ctx, const char *what);
void *host_alloc(nc_ctx *ctx, size_t bytes, bool persistent);  // tensor headers and nodes
void host_free(nc_ctx *ctx, void *p);
char *dev_alloc(nc_ctx *ctx, size_t bytes, bool persistent);
void dev_free(nc_ctx *ctx, char *p, size_t bytes, bool persistent);
char *arena_alloc(nc_ctx *ctx, size_t bytes);  // recorded as scratch while a Scratch scope is open
void arena_free(nc_ctx *ctx, char *p, size_t bytes);
bool persistent_mode(const nc_ctx *ctx);
float rand_uniform01(nc_ctx *ctx);
float rand_normal(nc_ctx *ctx);
void detect_cpu(nc_cpu_info *info);

// ---- tensors (tensor.cpp) --------------------------------------------------------------------------
size_t dtype_size(nc_dtype dt);
const char *dtype_name(nc_dtype dt);
int64_t shape_numel(int nd, const int64_t *shape);
void contig_strides(int nd, const int64_t *shape, int64_t *st);
int norm_axis(int axis, int nd);
bool same_shape(const nc_tensor *a, const nc_tensor *b);
const char *shape_str(int nd, const int64_t *shape, char *buf, size_t size);
// Records an op's failure on its context (the first error sticks) and returns the code.
nc_status reject(const nc_node *n, nc_status code, const char *fmt, ...);
// Every listed input is f32, else the reference's dtype error for the first that is not.
bool inputs_f32(const nc_node *n, int first, int count);
nc_tensor *tensor_new(nc_ctx *ctx, nc_dtype dt, int nd, const int64_t *shape, bool persistent);
nc_tensor *tensor_alias(const nc_tensor *src, bool persistent);
inline nc_tensor *owner_of(const nc_tensor *t) { return t->owner ? t->owner : const_cast<nc_tensor *>(t); }
// device address of element 0, uploading a host-authoritative copy first (NULL + error on failure)
char *dptr(nc_tensor *t);
inline float *fptr(nc_tensor *t) { return (float *)dptr(t); }
// device address of element 0 for a caller that overwrites every element of t (the rest of the
// owner's storage made current first when t does not cover it)
char *dptr_overwrite(nc_tensor *t);
// marks a tensor's storage as written on the device (host mirror stale)
void wrote_dev(nc_tensor *t);
// counts a storage allocation request; true for the one NC_FAIL_ALLOC_AT names (a forced failure)
bool forced_alloc_failure(nc_ctx *ctx);
// host address of element 0 with the host copy current; write = the caller may write through it
char *hptr(nc_tensor *t, bool write);
void bcast_strides(const nc_tensor *t, int nd, const int64_t *shape, int64_t *out);
void bcast_strides_shape(int tn, const int64_t *tshape, int nd, const int64_t *shape, int64_t *out);
// contiguous device copy of t (t itself when contiguous; else an arena temporary)
float *contig_f32(nc_tensor *t);
// gradient buffer, zero on first use (TF_GRAD_FRESH set while it is untouched)
nc_tensor *grad_buf(nc_tensor *t);
// accumulate flag for kernels writing into t's grad buffer: 0 if fresh (and clears the flag)
int grad_acc(nc_tensor *x);
bool fill_zero(nc_tensor *t);

// ---- dispatch and autograd (dispatch.cpp) ----------------------------------------------------------
nc_tensor *apply(const OpDef *op, nc_tensor **in, int n_in, const Params *p);
// Device memory for state a node's backward reads, held with the node: released with the node's
// activation by a FREE_GRAPH backward, at once when the call is not recorded, else at step end.
void *save_state(nc_node *n, size_t bytes);

inline bool needs_grad(const nc_tensor *t) { return (t->flags & TF_REQUIRES_GRAD) != 0; }
inline hipStream_t stream(const nc_ctx *ctx) { return ctx->stream; }

}  // namespace nce
