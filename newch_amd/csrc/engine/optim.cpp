// Optimizers and gradient clipping on device (reference: engine/src/optim/optim.c).
//
// State (momentum / Adam m and v / RMSprop square average) lives in persistent device memory next
// to the parameters and is zeroed at creation.  nc_optim_step runs one nc_hip_optim_step launch per
// parameter with a gradient, in the reference's update expressions (bit-identical results);
// gradient accumulation, the step count and Adam's bias corrections (host powf, as the reference)
// are host logic identical to the reference's.  nc_optim_state hands out a host copy of a state
// buffer, read back on request and authoritative until the next step, which uploads it first (the
// same contract as nc_data_f32 for tensors): checkpoint code that reads or writes it keeps working.
#include <math.h>

#include "engine.hpp"

struct nc_optim {
    nc_ctx *ctx;
    int kind;  // NC_HIP_OPT_*
    int n;
    std::vector<nc_tensor *> params;
    std::vector<int64_t> numel;
    std::vector<float *> s[2];  // device state per parameter (nullptr when not kept)
    std::vector<float *> h[2];  // host copies handed out by nc_optim_state
    std::vector<char> mapped[2];
    nc_optim_opts o;
    int64_t t = 0;
    int accum_steps = 1, accum_count = 0, eps_inside_sqrt = 0;
};

namespace nce {

static void free_optim(nc_optim *o) {
    for (int k = 0; k < 2; k++) {
        for (int i = 0; i < o->n; i++) {
            if (o->s[k].size() > (size_t)i) dev_free(o->ctx, (char *)o->s[k][i], (size_t)o->numel[i] * 4, true);
            if (o->h[k].size() > (size_t)i) free(o->h[k][i]);
        }
    }
    delete o;
}

static nc_optim *create(nc_ctx *ctx, int kind, nc_tensor **params, int n, nc_optim_opts opts) {
    if (!ctx) return nullptr;
    for (int i = 0; i < n; i++) {
        nc_tensor *p = params ? params[i] : nullptr;
        if (!p) return nullptr;
        if (!(p->flags & TF_PERSISTENT) || !needs_grad(p) || p->dtype != NC_F32 || !nc_is_contiguous(p)) {
            error(ctx, NC_ERR_ARG, "optimizer: param %d must be a contiguous f32 nc_parameter", i);
            return nullptr;
        }
    }
    if (!need_device(ctx, "optimizer")) return nullptr;
    nc_optim *o = new nc_optim();
    o->ctx = ctx;
    o->kind = kind;
    o->n = n;
    o->o = opts;
    o->params.assign(params, params + n);
    const bool adam = kind == NC_HIP_OPT_ADAM || kind == NC_HIP_OPT_ADAMW;
    const bool need[2] = {adam || opts.momentum != 0.0f, adam || kind == NC_HIP_OPT_RMSPROP};
    for (int i = 0; i < n; i++) o->numel.push_back(nc_numel(params[i]));
    for (int k = 0; k < 2; k++) {
        o->h[k].assign(n, nullptr);
        o->mapped[k].assign(n, 0);
        if (!need[k]) continue;
        for (int i = 0; i < n; i++) {
            float *d = (float *)dev_alloc(ctx, (size_t)o->numel[i] * 4, true);
            o->s[k].push_back(d);
            if (!d || !hip_layer_ok(ctx, nc_hip_fill(d, 4, 0, o->numel[i], ctx->stream), "optimizer state")) {
                free_optim(o);
                return nullptr;
            }
        }
    }
    ctx->optims.push_back(o);
    return o;
}

static nc_optim_opts adam_defaults(nc_optim_opts opts) {
    if (opts.beta1 == 0.0f) opts.beta1 = 0.9f;
    if (opts.beta2 == 0.0f) opts.beta2 = 0.999f;
    if (opts.eps == 0.0f) opts.eps = 1e-8f;
    return opts;
}

// a host copy of state (k, i) that the caller may have written goes back to the device first
static bool upload_mapped(nc_optim *o) {
    for (int k = 0; k < 2; k++)
        for (int i = 0; i < o->n; i++)
            if (o->mapped[k][i]) {
                if (!hip_ok(o->ctx, hipMemcpyAsync(o->s[k][i], o->h[k][i], (size_t)o->numel[i] * 4,
                                                   hipMemcpyHostToDevice, o->ctx->stream),
                            "optimizer state upload") ||
                    !hip_ok(o->ctx, hipStreamSynchronize(o->ctx->stream), "optimizer state upload"))
                    return false;
                o->mapped[k][i] = 0;
            }
    return true;
}

}  // namespace nce

using namespace nce;

extern "C" {

nc_optim *nc_sgd(nc_ctx *ctx, nc_tensor **params, int n, nc_optim_opts opts) {
    return create(ctx, NC_HIP_OPT_SGD, params, n, opts);
}
nc_optim *nc_adam(nc_ctx *ctx, nc_tensor **params, int n, nc_optim_opts opts) {
    return create(ctx, NC_HIP_OPT_ADAM, params, n, adam_defaults(opts));
}
nc_optim *nc_adamw(nc_ctx *ctx, nc_tensor **params, int n, nc_optim_opts opts) {
    return create(ctx, NC_HIP_OPT_ADAMW, params, n, adam_defaults(opts));
}
nc_optim *nc_rmsprop(nc_ctx *ctx, nc_tensor **params, int n, nc_optim_opts opts, int eps_inside_sqrt) {
    if (opts.beta2 == 0.0f) opts.beta2 = 0.99f;
    if (opts.eps == 0.0f) opts.eps = 1e-8f;
    nc_optim *o = create(ctx, NC_HIP_OPT_RMSPROP, params, n, opts);
    if (o) o->eps_inside_sqrt = eps_inside_sqrt ? 1 : 0;
    return o;
}

void nc_optim_free(nc_optim *o) {
    if (!o) return;
    auto &v = o->ctx->optims;
    for (size_t i = 0; i < v.size(); i++)
        if (v[i] == o) {
            v.erase(v.begin() + (long)i);
            break;
        }
    if (o->ctx->device >= 0) (void)hipStreamSynchronize(o->ctx->stream);  // queued steps may use the state
    free_optim(o);
}

void nc_optim_set_accumulation(nc_optim *o, int steps) {
    if (!o) return;
    if (steps < 1) {
        error(o->ctx, NC_ERR_ARG, "gradient accumulation steps must be >= 1, got %d", steps);
        return;
    }
    o->accum_steps = steps;
    o->accum_count = 0;
}

void nc_optim_zero_grad(nc_optim *o) {
    if (!o || o->accum_count != 0) return;  // still summing toward an update
    for (nc_tensor *p : o->params) nc_zero_grad(p);
}

void nc_optim_clear_grad(nc_optim *o) {
    if (!o || o->accum_count != 0) return;
    for (nc_tensor *p : o->params) nc_clear_grad(p);
}

void nc_optim_set_lr(nc_optim *o, float lr) {
    if (o) o->o.lr = lr;
}

float *nc_optim_state(nc_optim *o, int param, int slot) {
    if (!o || param < 0 || param >= o->n || slot < 0 || slot > 1 || o->s[slot].empty()) return nullptr;
    const size_t bytes = (size_t)o->numel[param] * 4;
    float *&h = o->h[slot][param];
    if (!h && !(h = (float *)malloc(bytes ? bytes : 4))) {
        error(o->ctx, NC_ERR_OOM, "out of host memory");
        return nullptr;
    }
    if (!o->mapped[slot][param]) {
        if (!hip_ok(o->ctx, hipMemcpyAsync(h, o->s[slot][param], bytes, hipMemcpyDeviceToHost, o->ctx->stream),
                    "optimizer state") ||
            !hip_ok(o->ctx, hipStreamSynchronize(o->ctx->stream), "optimizer state"))
            return nullptr;
        o->mapped[slot][param] = 1;
    }
    return h;
}

int64_t nc_optim_get_step(const nc_optim *o) { return o ? o->t : 0; }

void nc_optim_set_step(nc_optim *o, int64_t t) {
    if (!o) return;
    if (t < 0) {
        error(o->ctx, NC_ERR_ARG, "optimizer step count must be >= 0, got %lld", (long long)t);
        return;
    }
    o->t = t;
    o->accum_count = 0;
}

void nc_optim_set_opts(nc_optim *o, nc_optim_opts opts) {
    if (!o) return;
    const bool adam = o->kind == NC_HIP_OPT_ADAM || o->kind == NC_HIP_OPT_ADAMW;
    const bool has_momentum = !adam && !o->s[0].empty();
    if (!adam && has_momentum != (opts.momentum != 0.0f)) {
        error(o->ctx, NC_ERR_ARG, "optimizer: momentum cannot switch between zero and non-zero (%g -> %g)",
              (double)o->o.momentum, (double)opts.momentum);
        return;
    }
    o->o = opts;
}

void nc_optim_step(nc_optim *o) {
    if (!o || !nc_ok(o->ctx)) return;
    if (o->accum_steps > 1 && ++o->accum_count < o->accum_steps) return;
    o->accum_count = 0;
    const nc_optim_opts &c = o->o;
    const float gs = 1.0f / (float)o->accum_steps;  // average the summed grads
    o->t++;
    float bc1 = 1.0f, bc2 = 1.0f;
    if (o->kind == NC_HIP_OPT_ADAM || o->kind == NC_HIP_OPT_ADAMW) {
        bc1 = 1.0f - powf(c.beta1, (float)o->t);
        bc2 = 1.0f - powf(c.beta2, (float)o->t);
    }
    if (!upload_mapped(o)) return;
    nc_ctx *ctx = o->ctx;
    for (int i = 0; i < o->n; i++) {
        nc_tensor *p = o->params[i];
        nc_tensor *gt = nc_grad(p);
        if (!gt) continue;  // no gradient (never reached, or cleared)
        float *w = fptr(p), *g = fptr(gt);
        if (!w || !g) return;
        float *s1 = o->s[0].empty() ? nullptr : o->s[0][i], *s2 = o->s[1].empty() ? nullptr : o->s[1][i];
        if (!hip_layer_ok(ctx,
                          nc_hip_optim_step(o->kind, o->numel[i], w, g, s1, s2, c.lr, c.momentum, c.weight_decay,
                                            c.beta1, c.beta2, c.eps, gs, bc1, bc2, o->eps_inside_sqrt, ctx->stream),
                          "optimizer step"))
            return;
        wrote_dev(p);
    }
}

// torch.nn.utils.clip_grad_norm_: 2-norm over all grads together, fp64 sum of squares
float nc_clip_grad_norm(nc_tensor **params, int n, float max_norm) {
    nc_ctx *ctx = nullptr;
    for (int i = 0; i < n && !ctx; i++)
        if (params[i]) ctx = params[i]->ctx;
    double ss = 0.0;
    if (ctx && need_device(ctx, "clip_grad_norm")) {
        double *dss = (double *)arena_alloc(ctx, sizeof(double));
        if (!dss || !hip_layer_ok(ctx, nc_hip_fill(dss, 8, 0, 1, ctx->stream), "clip_grad_norm")) return 0.0f;
        for (int i = 0; i < n; i++) {
            nc_tensor *g = params[i] ? nc_grad(params[i]) : nullptr;
            if (!g || (g->flags & TF_GRAD_FRESH)) continue;  // a lazily zeroed grad adds nothing
            const int64_t N = nc_numel(g);
            float *d = fptr(g);
            if (!d) return 0.0f;
            const size_t wsb = nc_hip_sumsq_workspace(N);
            char *ws = wsb ? arena_alloc(ctx, wsb) : nullptr;
            if ((wsb && !ws) || !hip_layer_ok(ctx, nc_hip_sumsq(N, d, dss, 1, ws, wsb, ctx->stream), "clip_grad_norm"))
                return 0.0f;
        }
        if (!hip_ok(ctx, hipMemcpyAsync(&ss, dss, sizeof ss, hipMemcpyDeviceToHost, ctx->stream), "clip_grad_norm") ||
            !hip_ok(ctx, hipStreamSynchronize(ctx->stream), "clip_grad_norm"))
            return 0.0f;
    }
    const float total = (float)sqrt(ss);
    const float coef = max_norm / (total + 1e-6f);
    if (coef < 1.0f && ctx) {
        for (int i = 0; i < n; i++) {
            nc_tensor *g = params[i] ? nc_grad(params[i]) : nullptr;
            if (!g || (g->flags & TF_GRAD_FRESH)) continue;
            float *d = fptr(g);
            if (!d || !hip_layer_ok(ctx, nc_hip_unary_fwd(NC_HIP_UN_SCALE, coef, d, d, nc_numel(g), ctx->stream),
                                    "clip_grad_norm"))
                return total;
            wrote_dev(g);
        }
    }
    return total;
}

}  // extern "C"
