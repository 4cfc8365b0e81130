// Optimizers and gradient clipping on the device (reference: engine/src/optim/optim.c).
//
// An optimizer is a list of parameter slots.  Each slot holds its parameter and up to two state
// buffers in persistent device memory next to it (momentum, or Adam's m, in slot 0; Adam's v, or
// RMSprop's square average, in slot 1), zeroed at creation.  A step updates every parameter that
// has a gradient with the reference's update expressions (bit-identical results): up to 32
// parameters with 128-bit aligned arrays per nc_hip_optim_step_multi launch, the others one
// nc_hip_optim_step launch each; gradient accumulation (every n-th step updates, with the mean of
// the summed gradients), the step count and Adam's bias corrections (host powf, as the reference)
// are host logic with the reference's semantics and messages.  clip_grad_norm sums and rescales 32
// gradients per launch.  nc_optim_state hands out a host copy of a
// state buffer, read back on request and authoritative until the next step, which uploads it first
// (the contract nc_data_f32 has for tensors): checkpoint code that reads or writes it keeps working.
#include <math.h>

#include "engine.hpp"

namespace nce {

struct ParamSlot {
    nc_tensor *p = nullptr;
    int64_t n = 0;
    float *dev[2] = {nullptr, nullptr};   // device state buffers (nullptr: not kept)
    float *host[2] = {nullptr, nullptr};  // host copies handed out by nc_optim_state
    bool mapped[2] = {false, false};      // the host copy is authoritative
};

static bool is_adam(int kind) { return kind == NC_HIP_OPT_ADAM || kind == NC_HIP_OPT_ADAMW; }

// which state buffers a kind keeps: slot 0 for Adam's m or a momentum, slot 1 for Adam's v or
// RMSprop's square average
static bool keeps(int kind, int slot, const nc_optim_opts &o) {
    if (is_adam(kind)) return true;
    return slot == 0 ? o.momentum != 0.0f : kind == NC_HIP_OPT_RMSPROP;
}

// unset (zero) hyper-parameters take the kind's defaults
static nc_optim_opts with_defaults(int kind, nc_optim_opts o) {
    auto fill = [](float &v, float d) {
        if (v == 0.0f) v = d;
    };
    if (is_adam(kind)) {
        fill(o.beta1, 0.9f);
        fill(o.beta2, 0.999f);
        fill(o.eps, 1e-8f);
    } else if (kind == NC_HIP_OPT_RMSPROP) {
        fill(o.beta2, 0.99f);
        fill(o.eps, 1e-8f);
    }
    return o;
}

static bool usable_param(const nc_tensor *p) {
    return (p->flags & TF_PERSISTENT) && needs_grad(p) && p->dtype == NC_F32 && nc_is_contiguous(p);
}

}  // namespace nce

using namespace nce;

struct nc_optim {
    nc_ctx *ctx = nullptr;
    int kind = 0;
    nc_optim_opts o{};
    std::vector<ParamSlot> slots;
    int64_t t = 0;
    int accum_every = 1, accum_seen = 0;  // update on every accum_every-th step; steps summed so far
    int eps_inside_sqrt = 0;

    // the kept state buffers, zeroed
    bool allocate() {
        for (ParamSlot &s : slots)
            for (int k = 0; k < 2; k++) {
                if (!keeps(kind, k, o)) continue;
                s.dev[k] = (float *)dev_alloc(ctx, (size_t)s.n * 4, true);
                if (!s.dev[k] || !hip_layer_ok(ctx, nc_hip_fill(s.dev[k], 4, 0, s.n, ctx->stream), "optimizer state"))
                    return false;
            }
        return true;
    }
    void release() {
        for (ParamSlot &s : slots)
            for (int k = 0; k < 2; k++) {
                if (s.dev[k]) dev_free(ctx, (char *)s.dev[k], (size_t)s.n * 4, true);
                free(s.host[k]);
            }
    }
    // accumulation: true when this call updates the weights
    bool due() {
        if (accum_every > 1 && ++accum_seen < accum_every) return false;
        accum_seen = 0;
        return true;
    }
    // host copies the caller may have written go back to the device first
    bool upload_mapped() {
        for (ParamSlot &s : slots)
            for (int k = 0; k < 2; k++) {
                if (!s.mapped[k]) continue;
                if (!hip_ok(ctx, hipMemcpyAsync(s.dev[k], s.host[k], (size_t)s.n * 4, hipMemcpyHostToDevice, ctx->stream),
                            "optimizer state upload") ||
                    !hip_ok(ctx, hipStreamSynchronize(ctx->stream), "optimizer state upload"))
                    return false;
                s.mapped[k] = false;
            }
        return true;
    }
};

namespace nce {

static nc_optim *create(nc_ctx *ctx, int kind, nc_tensor **params, int n, nc_optim_opts opts) {
    if (!ctx) return nullptr;
    for (int i = 0; i < n; i++) {
        nc_tensor *p = params ? params[i] : nullptr;
        if (!p) return nullptr;
        if (!usable_param(p)) {
            error(ctx, NC_ERR_ARG, "optimizer: param %d must be a contiguous f32 nc_parameter", i);
            return nullptr;
        }
    }
    if (!need_device(ctx, "optimizer")) return nullptr;
    nc_optim *o = new nc_optim();
    o->ctx = ctx;
    o->kind = kind;
    o->o = opts;
    o->slots.resize((size_t)(n > 0 ? n : 0));
    for (int i = 0; i < n; i++) {
        o->slots[(size_t)i].p = params[i];
        o->slots[(size_t)i].n = nc_numel(params[i]);
    }
    if (!o->allocate()) {
        o->release();
        delete o;
        return nullptr;
    }
    ctx->optims.push_back(o);
    return o;
}

}  // namespace nce

extern "C" {

nc_optim *nc_sgd(nc_ctx *ctx, nc_tensor **params, int n, nc_optim_opts opts) {
    return create(ctx, NC_HIP_OPT_SGD, params, n, with_defaults(NC_HIP_OPT_SGD, opts));
}
nc_optim *nc_adam(nc_ctx *ctx, nc_tensor **params, int n, nc_optim_opts opts) {
    return create(ctx, NC_HIP_OPT_ADAM, params, n, with_defaults(NC_HIP_OPT_ADAM, opts));
}
nc_optim *nc_adamw(nc_ctx *ctx, nc_tensor **params, int n, nc_optim_opts opts) {
    return create(ctx, NC_HIP_OPT_ADAMW, params, n, with_defaults(NC_HIP_OPT_ADAMW, opts));
}
nc_optim *nc_rmsprop(nc_ctx *ctx, nc_tensor **params, int n, nc_optim_opts opts, int eps_inside_sqrt) {
    nc_optim *o = create(ctx, NC_HIP_OPT_RMSPROP, params, n, with_defaults(NC_HIP_OPT_RMSPROP, opts));
    if (o) o->eps_inside_sqrt = eps_inside_sqrt ? 1 : 0;
    return o;
}

void nc_optim_free(nc_optim *o) {
    if (!o) return;
    auto &live = o->ctx->optims;
    for (auto it = live.begin(); it != live.end(); ++it)
        if (*it == o) {
            live.erase(it);
            break;
        }
    if (o->ctx->device >= 0) (void)hipStreamSynchronize(o->ctx->stream);  // queued steps may use the state
    o->release();
    delete o;
}

void nc_optim_set_accumulation(nc_optim *o, int steps) {
    if (!o) return;
    if (steps < 1) {
        error(o->ctx, NC_ERR_ARG, "gradient accumulation steps must be >= 1, got %d", steps);
        return;
    }
    o->accum_every = steps;
    o->accum_seen = 0;
}

// while summing toward an update the gradients are kept
void nc_optim_zero_grad(nc_optim *o) {
    if (!o || o->accum_seen != 0) return;
    for (ParamSlot &s : o->slots) nc_zero_grad(s.p);
}

void nc_optim_clear_grad(nc_optim *o) {
    if (!o || o->accum_seen != 0) return;
    for (ParamSlot &s : o->slots) nc_clear_grad(s.p);
}

void nc_optim_set_lr(nc_optim *o, float lr) {
    if (o) o->o.lr = lr;
}

float *nc_optim_state(nc_optim *o, int param, int slot) {
    if (!o || param < 0 || param >= (int)o->slots.size() || slot < 0 || slot > 1) return nullptr;
    ParamSlot &s = o->slots[(size_t)param];
    if (!s.dev[slot]) return nullptr;
    const size_t bytes = (size_t)s.n * 4;
    if (!s.host[slot] && !(s.host[slot] = (float *)malloc(bytes ? bytes : 4))) {
        error(o->ctx, NC_ERR_OOM, "out of host memory");
        return nullptr;
    }
    if (!s.mapped[slot]) {
        nc_ctx *ctx = o->ctx;
        if (!hip_ok(ctx, hipMemcpyAsync(s.host[slot], s.dev[slot], bytes, hipMemcpyDeviceToHost, ctx->stream),
                    "optimizer state") ||
            !hip_ok(ctx, hipStreamSynchronize(ctx->stream), "optimizer state"))
            return nullptr;
        s.mapped[slot] = true;
    }
    return s.host[slot];
}

int64_t nc_optim_get_step(const nc_optim *o) { return o ? o->t : 0; }

void nc_optim_set_step(nc_optim *o, int64_t t) {
    if (!o) return;
    if (t < 0) {
        error(o->ctx, NC_ERR_ARG, "optimizer step count must be >= 0, got %lld", (long long)t);
        return;
    }
    o->t = t;
    o->accum_seen = 0;
}

// the state buffers were sized at creation: a momentum cannot appear or vanish later
void nc_optim_set_opts(nc_optim *o, nc_optim_opts opts) {
    if (!o) return;
    if (!is_adam(o->kind) && keeps(o->kind, 0, o->o) != keeps(o->kind, 0, opts)) {
        error(o->ctx, NC_ERR_ARG, "optimizer: momentum cannot switch between zero and non-zero (%g -> %g)",
              (double)o->o.momentum, (double)opts.momentum);
        return;
    }
    o->o = opts;
}

// [p, p + n) and [q, q + m) share an element
static bool overlaps(const float *p, int64_t n, const float *q, int64_t m) { return p < q + m && q < p + n; }

void nc_optim_step(nc_optim *o) {
    if (!o || !nc_ok(o->ctx) || !o->due()) return;
    const nc_optim_opts &c = o->o;
    const float gs = 1.0f / (float)o->accum_every;  // the mean of the summed gradients
    o->t++;
    const float bc1 = is_adam(o->kind) ? 1.0f - powf(c.beta1, (float)o->t) : 1.0f;
    const float bc2 = is_adam(o->kind) ? 1.0f - powf(c.beta2, (float)o->t) : 1.0f;
    if (!o->upload_mapped()) return;
    nc_ctx *ctx = o->ctx;
    // parameters whose arrays allow 128-bit access go up to NC_HIP_OPT_MULTI_MAX per launch, the rest
    // one launch each (the same arithmetic either way).  A parameter listed again (or sharing memory
    // with one already in the batch) first flushes the batch: the reference updates the slots in
    // turn, so the later slot reads the earlier one's result (optim.c:172-213).
    nc_hip_opt_param batch[NC_HIP_OPT_MULTI_MAX];
    int nb = 0;
    auto flush = [&]() {
        const int k = nb;
        nb = 0;
        return k == 0 || hip_layer_ok(ctx,
                                      nc_hip_optim_step_multi(o->kind, k, batch, c.lr, c.momentum, c.weight_decay,
                                                              c.beta1, c.beta2, c.eps, gs, bc1, bc2,
                                                              o->eps_inside_sqrt, ctx->stream),
                                      "optimizer step");
    };
    auto a16 = [](const void *p) { return p == nullptr || ((uintptr_t)p & 15u) == 0; };
    for (ParamSlot &s : o->slots) {
        nc_tensor *gt = nc_grad(s.p);
        if (!gt) continue;  // no gradient (never reached, or cleared)
        float *w = fptr(s.p), *g = fptr(gt);
        if (!w || !g) return;
        if (s.n % 4 == 0 && a16(w) && a16(g) && a16(s.dev[0]) && a16(s.dev[1])) {
            for (int i = 0; i < nb; i++)
                if (overlaps(batch[i].w, batch[i].n, w, s.n) || overlaps(batch[i].w, batch[i].n, g, s.n) ||
                    overlaps(batch[i].g, batch[i].n, w, s.n)) {
                    if (!flush()) return;
                    break;
                }
            batch[nb++] = nc_hip_opt_param{w, g, s.dev[0], s.dev[1], s.n};
            if (nb == NC_HIP_OPT_MULTI_MAX && !flush()) return;
        } else if (!hip_layer_ok(ctx,
                                 nc_hip_optim_step(o->kind, s.n, w, g, s.dev[0], s.dev[1], c.lr, c.momentum,
                                                   c.weight_decay, c.beta1, c.beta2, c.eps, gs, bc1, bc2,
                                                   o->eps_inside_sqrt, ctx->stream),
                                 "optimizer step")) {
            return;
        }
        wrote_dev(s.p);
    }
    flush();
}

// torch.nn.utils.clip_grad_norm_: the 2-norm over all gradients together, from an fp64 sum of
// squares accumulated on the device; gradients still lazily zero add nothing and are not scaled
float nc_clip_grad_norm(nc_tensor **params, int n, float max_norm) {
    nc_ctx *ctx = nullptr;
    for (int i = 0; i < n && !ctx; i++)
        if (params[i]) ctx = params[i]->ctx;
    auto live_grad = [&](int i) -> nc_tensor * {
        nc_tensor *g = params[i] ? nc_grad(params[i]) : nullptr;
        return g && !(g->flags & TF_GRAD_FRESH) ? g : nullptr;
    };
    // the gradients go to the device NC_HIP_OPT_MULTI_MAX at a time: one sum of squares (or one
    // rescale) launch per group, with the bits of one call per gradient in parameter order
    float *xs[NC_HIP_OPT_MULTI_MAX];
    int64_t ns[NC_HIP_OPT_MULTI_MAX];
    double ss = 0.0;
    if (ctx && need_device(ctx, "clip_grad_norm")) {
        Scratch scratch(ctx);
        double *dss = (double *)arena_alloc(ctx, sizeof(double));
        if (!dss) return 0.0f;
        int cnt = 0;
        bool first = true;  // the first group overwrites *dss, the later ones add to it
        auto flush = [&]() {
            const size_t wsb = nc_hip_sumsq_multi_workspace(cnt, ns);
            char *ws = wsb ? arena_alloc(ctx, wsb) : nullptr;
            if (wsb && !ws) return false;
            const int rc = nc_hip_sumsq_multi(cnt, (const float *const *)xs, ns, dss, first ? 0 : 1, ws, wsb,
                                              ctx->stream);
            first = false;
            cnt = 0;
            return hip_layer_ok(ctx, rc, "clip_grad_norm");
        };
        for (int i = 0; i < n; i++) {
            nc_tensor *g = live_grad(i);
            if (!g) continue;
            if (!(xs[cnt] = fptr(g))) return 0.0f;
            ns[cnt] = nc_numel(g);
            if (++cnt == NC_HIP_OPT_MULTI_MAX && !flush()) return 0.0f;
        }
        if ((cnt || first) && !flush()) return 0.0f;  // no gradient at all: *dss = 0
        if (!hip_ok(ctx, hipMemcpyAsync(&ss, dss, sizeof ss, hipMemcpyDeviceToHost, ctx->stream), "clip_grad_norm") ||
            !hip_ok(ctx, hipStreamSynchronize(ctx->stream), "clip_grad_norm"))
            return 0.0f;
    }
    const float total = (float)sqrt(ss);
    const float coef = max_norm / (total + 1e-6f);
    if (coef < 1.0f && ctx) {
        // a gradient listed twice is scaled twice, in turn, as the reference's loop does
        // (optim.c:216-233): it goes into a later launch than its first listing
        int cnt = 0;
        auto flush = [&]() {
            const int rc = nc_hip_scale_multi(cnt, xs, ns, coef, ctx->stream);
            cnt = 0;
            return hip_layer_ok(ctx, rc, "clip_grad_norm");
        };
        for (int i = 0; i < n; i++) {
            nc_tensor *g = live_grad(i);
            if (!g) continue;
            float *gp = fptr(g);
            if (!gp) return total;
            const int64_t gn = nc_numel(g);
            for (int j = 0; j < cnt; j++)
                if (overlaps(xs[j], ns[j], gp, gn)) {
                    if (!flush()) return total;
                    break;
                }
            xs[cnt] = gp;
            ns[cnt] = gn;
            wrote_dev(g);
            if (++cnt == NC_HIP_OPT_MULTI_MAX && !flush()) return total;
        }
        if (cnt && !flush()) return total;
    }
    return total;
}

}  // extern "C"
